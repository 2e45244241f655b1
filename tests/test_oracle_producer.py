"""CPU pins of the producer oracle (oracle/producer.py): golden vectors written by the reference's AxialRoPE,
closed forms of the rotation, the window layout and the e4m3 quantisation convention."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import producer as P

GOLDEN = os.path.join(os.path.dirname(__file__), 'golden')


def _golden_rope():
    meta = json.load(open(os.path.join(GOLDEN, 'axial_rope.json')))
    data = np.load(os.path.join(GOLDEN, 'axial_rope.npz'))
    for m in meta:
        n = m['name']
        yield (torch.from_numpy(data[n + '/x']).view(torch.bfloat16), torch.from_numpy(data[n + '/positions']),
               torch.from_numpy(data[n + '/frequencies']), torch.from_numpy(data[n + '/out']).view(torch.bfloat16))


def test_axial_rope_equals_reference_golden_bits():
    for x, pos, freq, want in _golden_rope():
        assert torch.equal(P.rope_frequencies(x.shape[-1]), freq)
        got = P.axial_rope(x, pos, freq)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_rope_frequencies_closed_form():
    f = P.rope_frequencies(48)
    assert f.dtype == torch.float32 and f.numel() == 8
    for i in range(8):
        assert abs(float(f[i]) - 10000.0 ** (-2 * i / 16)) <= 1e-6 * 10000.0 ** (-2 * i / 16)
    with pytest.raises(ValueError):
        P.rope_frequencies(64)


def test_axial_rope_known_answers_in_float64():
    """A unit pair (1, 0) in axis t, pair i, turns to (cos p, sin p) with p = pos[t] * freq[i]; position 0 is the
    identity; other axes' dims do not move; norms of every pair are kept; rotations compose."""
    D = 24
    freq = P.rope_frequencies(D)
    pos = torch.tensor([[[3.5, -7.25, 40.0]]])
    for axis in range(3):
        for i in range(D // 6):
            x = torch.zeros(1, 1, 1, D, dtype=torch.float64)
            d = axis * (D // 3) + 2 * i
            x[..., d] = 1.0
            out = P.axial_rope(x, pos, freq)
            p = np.float32(np.float32(pos[0, 0, axis]) * np.float32(freq[i]))
            assert abs(float(out[..., d]) - float(np.float32(np.cos(p)))) < 1e-7
            assert abs(float(out[..., d + 1]) - float(np.float32(np.sin(p)))) < 1e-7
            others = [e for e in range(D) if e not in (d, d + 1)]
            assert torch.all(out[..., others] == 0)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 5, D, generator=g, dtype=torch.float64)
    assert torch.equal(P.axial_rope(x, torch.zeros(2, 5, 3), freq), x)
    p1 = torch.randn(2, 5, 3, generator=g) * 3
    p2 = torch.randn(2, 5, 3, generator=g) * 3
    y = P.axial_rope(x, p1, freq)
    pairs = lambda t: t.reshape(*t.shape[:-1], D // 2, 2).pow(2).sum(-1)
    assert torch.allclose(pairs(y), pairs(x), rtol=1e-6)
    assert torch.allclose(P.axial_rope(y, p2, freq), P.axial_rope(x, p1 + p2, freq), atol=1e-5)


def test_window_kv_layout_and_e4m3_convention():
    g = torch.Generator().manual_seed(1)
    H, Pn, L, D, cap = 2, 5, 7, 24, 16
    pk, pv = (torch.randn(H, Pn, D, generator=g).to(torch.bfloat16) for _ in range(2))
    lk, lv = (torch.randn(H, L, D, generator=g).to(torch.bfloat16) for _ in range(2))
    pos = torch.randn(L, 3, generator=g) * 10
    freq = P.rope_frequencies(D)
    k, v = P.window_kv(pk, pv, lk, lv, pos, freq, cap)
    assert torch.equal(k[:, :Pn], pk) and torch.equal(v[:, :Pn], pv)
    assert torch.equal(k[:, Pn:Pn + L], P.axial_rope(lk[None], pos[None], freq)[0])
    assert torch.equal(v[:, Pn:Pn + L], lv)
    assert torch.all(k[:, Pn + L:] == 0) and torch.all(v[:, Pn + L:] == 0)
    k0, _ = P.window_kv(pk, pv, lk, lv, None, freq, cap)
    assert torch.equal(k0[:, Pn:Pn + L], lk)
    with pytest.raises(ValueError):
        P.window_kv(pk, pv, lk, lv, pos, freq, Pn + L - 1)
    codes, scale = P.quantize_e4m3(k, Pn + L)
    amax = k[:, :Pn + L].float().abs().amax(dim=(1, 2))
    assert torch.equal(scale, torch.clamp(amax / 448.0, min=1e-12))
    deq = A.dequant_e4m3(codes, 1.0) * scale[:, None, None].double()
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 above the subnormal range, and the max maps to 448.
    big = k.float().abs() > scale[:, None, None] * 2 ** -6
    assert torch.all((deq - k.double()).abs()[big] <= k.double().abs()[big] * 2 ** -4 + 1e-12)
    assert torch.all(codes[:, Pn + L:] == 0)
    top = (k.float().abs() == amax[:, None, None])
    assert torch.all((codes[top] & 0x7f) == 0x7e)                # 448 = 1.75 * 2^8
