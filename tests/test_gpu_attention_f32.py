"""fp32 cross attention (svhip_xattn_fwd_f32) against the float64 oracle (oracle.attention.cross_attention, the
reference's masked SDPA) at fp32 tolerances: padded and packed windows, row-major V and V^T views, window lengths
that end inside a 16-key block, shorter than one block and empty, every head width the kernel takes."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def qkv(B, H, Q, kcap, D, seed, spread=1.0):
    g = torch.Generator().manual_seed(seed)
    s = spread / math.sqrt(D)
    return (torch.randn(B, H, Q, D, generator=g) * s, torch.randn(B, H, kcap, D, generator=g) * s,
            torch.randn(B, H, kcap, D, generator=g) / math.sqrt(D))


def check(got, ref, atol, rtol):
    err = (got.double().cpu() - ref).abs().max().item()
    assert err <= atol, err
    assert err <= rtol * ref.abs().max().item(), (err, ref.abs().max().item())


@pytest.mark.parametrize('D', [16, 32, 48, 64])
@pytest.mark.parametrize('transposed', [False, True])
def test_padded_windows_match_the_oracle(dev, D, transposed):
    from streamvoxel_amd.stream.attention import attention
    lengths = [700, 1, 15, 0, 17, 128, 333]
    B, H, Q, kcap = len(lengths), 2, 150, 704
    _case(f'xattn fp32 padded D={D} transposed={transposed} lengths={lengths}')
    q, k, v = qkv(B, H, Q, kcap, D, seed=D + 7 * transposed)
    ref = A.cross_attention(q, k, v, lengths)
    vv = v.transpose(2, 3).contiguous().to(dev).transpose(2, 3) if transposed else v.to(dev)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    out = attention(q.to(dev), k.to(dev), vv, lengths=lt)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    assert torch.equal(out[3].cpu(), torch.zeros_like(out[3].cpu()))     # the empty window gives zeros
    check(out, ref, 2e-5, 1e-4)


def test_packed_equals_padded_and_the_oracle(dev):
    from streamvoxel_amd.stream.attention import attention
    lengths = [700, 33, 0, 256, 95]
    B, H, Q, D, kcap = len(lengths), 3, 96, 64, 704
    _case(f'xattn fp32 packed vs padded lengths={lengths}')
    q, k, v = qkv(B, H, Q, kcap, D, seed=11)
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    padded = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)
    kp = torch.cat([k[b, :, :L] for b, L in enumerate(lengths)], 1).to(dev)
    vp = torch.cat([v[b, :, :L] for b, L in enumerate(lengths)], 1).to(dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=dev)
    packed = attention(q.to(dev), kp, vp, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert torch.equal(packed, padded)
    check(packed, ref, 2e-5, 1e-4)


def test_sharp_rows_and_a_dominant_key(dev):
    """Logits with standard deviation about 8 (one key far above the rest in many rows): the running max moves
    often and a dominant key returns its value row."""
    from streamvoxel_amd.stream.attention import attention
    lengths = [999, 64]
    B, H, Q, D, kcap = 2, 2, 64, 64, 1024
    _case(f'xattn fp32 sharp rows lengths={lengths}')
    q, k, v = qkv(B, H, Q, kcap, D, seed=5, spread=8.0)
    k[0, 0, 517] = q[0, 0, 3] * 40.0                 # query 3 of window 0, head 0 sees one key far above the rest
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    out = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    check(out, ref, 2e-5, 1e-4)
    assert torch.allclose(out[0, 0, 3].cpu(), v[0, 0, 517], atol=1e-5)


def test_fp32_inputs_are_checked(dev):
    from streamvoxel_amd.stream.attention import attention
    q, k, v = qkv(1, 1, 8, 64, 64, seed=1)
    lt = torch.tensor([64], dtype=torch.int32, device=dev)
    with pytest.raises(TypeError):
        attention(q.to(dev), k.to(dev).bfloat16(), v.to(dev), lengths=lt)
    with pytest.raises(TypeError):
        attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt, key_mask=torch.ones(1, 64, dtype=torch.bool,
                                                                                   device=dev))
    with pytest.raises(RuntimeError, match='head_dim'):
        q2, k2, v2 = qkv(1, 1, 8, 64, 96, seed=2)
        attention(q2.to(dev), k2.to(dev), v2.to(dev), lengths=lt)
