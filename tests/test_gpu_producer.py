"""GPU parity of the operand producers (svhip_axial_rope, svhip_kv_write) through the C ABI.

Bars: AxialRoPE bf16 bits equal the reference module's (golden vectors) and the oracle's, except where the device
and host fp32 sin / cos differ by an ulp right at a bf16 rounding boundary (then one bf16 ulp; counted and bounded
below 0.1 % of the elements); the cache write is bit-exact to the oracle's window layout (bf16), and the e4m3
codes and scales are bit-exact to torch's float8_e4m3fn conversion of x / (amax / 448)."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import producer as P

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), 'golden')


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def _ulps(a, b):
    """Per-element distance in bf16 ulps (same-sign finite values)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


def _close_bits(got, want, what):
    d = _ulps(got.cpu(), want.cpu())
    frac = float((d != 0).float().mean())
    print(f'[gpu-case] {what}: {int((d != 0).sum())} of {d.numel()} elements differ, max {int(d.max())} ulp',
          flush=True)
    assert int(d.max()) <= 1 and frac <= 1e-3, (what, int(d.max()), frac)


def test_axial_rope_matches_reference_golden(dev):
    from streamvoxel_amd.stream.producer import axial_rope
    meta = json.load(open(os.path.join(GOLDEN, 'axial_rope.json')))
    data = np.load(os.path.join(GOLDEN, 'axial_rope.npz'))
    for m in meta:
        n = m['name']
        _case(f'axial_rope golden {n} {m["shape"]}')
        x = torch.from_numpy(data[n + '/x']).view(torch.bfloat16)
        pos = torch.from_numpy(data[n + '/positions'])
        freq = torch.from_numpy(data[n + '/frequencies'])
        want = torch.from_numpy(data[n + '/out']).view(torch.bfloat16)
        got = axial_rope(x.to(dev), pos.to(dev), freq.to(dev))
        torch.cuda.synchronize()
        _close_bits(got, want, n)


def test_axial_rope_in_place_on_strided_view(dev):
    """The Q producer's form: the projection's [B, N, H, D] buffer rotated in place through its [B, H, N, D] view;
    equal to the out-of-place result on a contiguous copy and to the oracle."""
    from streamvoxel_amd.stream.producer import axial_rope, rope_frequencies
    _case('axial_rope in place, strided [B,N,H,D] view')
    B, N, H, D = 3, 257, 8, 48
    g = torch.Generator().manual_seed(3)
    buf = torch.randn(B, N, H, D, generator=g).to(torch.bfloat16)
    pos = (torch.randint(0, 2048, (B, N, 3), generator=g).float() / 8)
    freq = rope_frequencies(D)
    want = P.axial_rope(buf.transpose(1, 2), pos, freq)
    dbuf = buf.to(dev)
    view = dbuf.transpose(1, 2)
    contig = axial_rope(view.contiguous(), pos.to(dev), freq.to(dev))
    axial_rope(view, pos.to(dev), freq.to(dev), out=view)
    torch.cuda.synchronize()
    assert torch.equal(view, contig)
    _close_bits(view, want, 'strided in place')


def test_cross_query_and_local_kv(dev):
    from streamvoxel_amd.stream.producer import cross_query, local_kv, rope_frequencies

    class Rope(torch.nn.Module):
        def __init__(self, D):
            super().__init__()
            self.register_buffer('frequencies', rope_frequencies(D))

    class Cross(torch.nn.Module):
        def __init__(self, width, heads):
            super().__init__()
            self.heads = heads
            self.query = torch.nn.Linear(width, width)
            self.key_value = torch.nn.Linear(width, 2 * width)
            self.norm = torch.nn.LayerNorm(width, elementwise_affine=False, eps=1e-6)
            self.rope = Rope(width // heads)

    _case('cross_query / local_kv, width 384, 8 heads')
    torch.manual_seed(4)
    cross = Cross(384, 8).to(dev).to(torch.bfloat16)
    value = torch.randn(2, 100, 384, device=dev, dtype=torch.bfloat16)
    positions = torch.randint(0, 1024, (2, 100, 3), device=dev).float() / 4
    q = cross_query(cross, value, positions)
    base = cross.query(cross.norm(value)).reshape(2, 100, 8, 48).transpose(1, 2)
    want = P.axial_rope(base.cpu(), positions.cpu(), cross.rope.frequencies.cpu())
    _close_bits(q, want, 'cross_query')
    local = torch.randn(1, 77, 384, device=dev, dtype=torch.bfloat16)
    lpos = torch.randint(0, 1024, (1, 77, 3), device=dev).float() / 4
    k, v = local_kv(cross, local, lpos)
    kv = cross.key_value(local).reshape(1, 77, 2, 8, 48)
    _close_bits(k, P.axial_rope(kv[:, :, 0].transpose(1, 2).cpu(), lpos.cpu(), cross.rope.frequencies.cpu()),
                'local_kv K')
    assert torch.equal(v, kv[:, :, 1].transpose(1, 2))


@pytest.mark.parametrize('rotate', [False, True])
def test_cached_context_window_write_bf16(dev, rotate):
    """CachedContext.write (svhip_kv_write): prefix + local keys, V stored transposed, zeros after the window's
    keys (stale contents are overwritten); windows of 0 keys, exactly the capacity, and a tail inside a block."""
    from streamvoxel_amd.stream.step import CachedContext
    H, D = 4, 48
    ctx = CachedContext(1, 3, H, D, 300, dev)
    for t in ctx.k + ctx.vt:
        t.fill_(7.0)                                   # stale contents that must not survive
    g = torch.Generator().manual_seed(5)
    freq = P.rope_frequencies(D)
    for index, (Pn, L) in enumerate([(0, 0), (64, 256 - 64 + 64), (17, 100)]):
        _case(f'kv_write bf16 rotate={rotate} window={index} P={Pn} L={L}')
        pk = torch.randn(H, Pn, D, generator=g).to(torch.bfloat16)
        pv = torch.randn(H, Pn, D, generator=g).to(torch.bfloat16)
        lk = torch.randn(H, L, D, generator=g).to(torch.bfloat16)
        lv = torch.randn(H, L, D, generator=g).to(torch.bfloat16)
        pos = torch.randint(0, 4096, (L, 3), generator=g).float() / 8 if rotate else None
        ctx.write(0, index, lk.to(dev), lv.to(dev), prefix=(pk.to(dev), pv.to(dev)),
                  positions=None if pos is None else pos.to(dev), frequencies=freq.to(dev) if rotate else None)
        wk, wv = P.window_kv(pk, pv, lk, lv, pos, freq, ctx.kv_cap)
        torch.cuda.synchronize()
        got_k = ctx.k[0][index].cpu()
        got_v = ctx.vt[0][index].cpu().transpose(1, 2)
        assert ctx.host_lengths[index] == Pn + L and int(ctx.lengths[index]) == Pn + L
        assert torch.equal(got_v, wv)
        if rotate:
            _close_bits(got_k, wk, f'window {index} K')
        else:
            assert torch.equal(got_k, wk)


def test_kv_write_row_major_v_and_e4m3_codes(dev):
    """svhip_kv_write with V rows and e4m3: every positive bf16 value up to 1 (and its negative) in one head, so
    x / scale runs over all e4m3 codes, their rounding midpoints and the subnormals; codes and scales bit-exact to
    torch's conversion; V^T and V-row layouts agree."""
    from streamvoxel_amd import _lib
    H, D, L = 2, 64, 256
    bits = torch.arange(0, 0x3F81, dtype=torch.int32)                 # 0 .. 1.0 in bf16
    vals = bits.to(torch.int16).view(torch.bfloat16)
    flat = torch.cat([vals, -vals])
    flat = torch.cat([flat, torch.zeros(H * L * D - flat.numel(), dtype=torch.bfloat16)])
    k = flat.reshape(H, L, D)
    g = torch.Generator().manual_seed(6)
    v = (torch.randn(H, L, D, generator=g) * 3).to(torch.bfloat16)
    kcap = 320
    lib = _lib.load()
    nbytes = int(lib.svhip_kv_write_workspace_bytes(H, kcap))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    outs = {}
    for vt in (False, True):
        _case(f'kv_write e4m3 V transposed={vt}')
        ck = torch.full((H, kcap, D), 0x55, dtype=torch.uint8, device=dev)
        cv = torch.full((H, D, kcap) if vt else (H, kcap, D), 0x55, dtype=torch.uint8, device=dev)
        ks = torch.zeros(H, device=dev)
        vs = torch.zeros(H, device=dev)
        kd, vd = k.to(dev), v.to(dev)
        scv = (cv.stride(0), cv.stride(2), cv.stride(1)) if vt else (cv.stride(0), cv.stride(1), cv.stride(2))
        _lib.check(lib.svhip_kv_write(
            None, None, 0, 0, 0, 0, 0, _lib.ptr(kd), _lib.ptr(vd), L, kd.stride(0), kd.stride(1), vd.stride(0),
            vd.stride(1), None, 0, None, H, D, _lib.ptr(ck), ck.stride(0), ck.stride(1), _lib.ptr(cv), *scv, kcap,
            _lib.SVHIP_FP8_E4M3, _lib.ptr(ks), _lib.ptr(vs), _lib.ptr(ws), nbytes, _lib.stream_of(kd)),
            'svhip_kv_write')
        torch.cuda.synchronize()
        wk, wv = P.window_kv(torch.zeros(H, 0, D, dtype=torch.bfloat16), torch.zeros(H, 0, D, dtype=torch.bfloat16),
                             k, v, None, None, kcap)
        ck_want, ks_want = P.quantize_e4m3(wk, L)
        cv_want, vs_want = P.quantize_e4m3(wv, L)
        assert torch.equal(ks.cpu(), ks_want) and torch.equal(vs.cpu(), vs_want)
        assert torch.equal(ck.cpu(), ck_want)
        got_v = cv.cpu().transpose(1, 2) if vt else cv.cpu()
        assert torch.equal(got_v, cv_want)
        outs[vt] = got_v
    assert torch.equal(outs[False], outs[True])
    # Every e4m3 magnitude code 0..0x7e appears among the K codes.
    assert set(range(0x7f)) <= set(np.unique(ck_want.numpy() & 0x7f).tolist())
