"""fp32 cross attention (svhip_xattn_fwd_f32, svhip_xattn_fwd_f32_masked) against the float64 oracle
(oracle.attention.cross_attention, the reference's masked SDPA) at fp32 tolerances: padded and packed windows,
row-major V and V^T views, window lengths that end inside a 16-key block, shorter than one block and empty, every
head width the kernel takes, key masks with holes (SlotCrossAttention's prefix ++ local mask)."""
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


def _masked_reference(q, k, v, mask, lengths=None):
    """float64 attention of every window over exactly its attended keys (mask True, below the length): the
    oracle's attention over the gathered keys; a query with no attended key gets zeros."""
    B, H, Q, D = q.shape
    out = torch.zeros((B, H, Q, D), dtype=torch.float64)
    for b in range(B):
        keep = mask[b].clone()
        if lengths is not None:
            keep[int(lengths[b]):] = False
        idx = keep.nonzero().squeeze(1)
        if len(idx):
            out[b:b + 1] = A.cross_attention(q[b:b + 1], k[b:b + 1, :, idx], v[b:b + 1, :, idx], [len(idx)])
    return out


@pytest.mark.parametrize('D', [16, 32, 48, 64])
@pytest.mark.parametrize('transposed', [False, True])
def test_key_mask_matches_the_oracle(dev, D, transposed):
    """svhip_xattn_fwd_f32_masked: random masks with holes, a window whose first blocks hold no attended key, a
    window with none (zeros), one key only in the last block; with and without lengths. The oracle's reference is
    also checked against the reference's SDPA call itself (float64 on the CPU), which gives zeros for the window
    with no attended key too."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 4, 2, 100, 300
    _case(f'xattn fp32 key mask D={D} transposed={transposed}')
    q, k, v = qkv(B, H, Q, kcap, D, seed=40 + D + transposed)
    g = torch.Generator().manual_seed(D)
    mask = torch.rand(B, kcap, generator=g) < 0.5
    mask[1, :70] = False                     # four blocks and more of 16 keys without an attended key
    mask[2] = False                          # nothing attended: zeros
    mask[3] = False
    mask[3, 299] = True                      # one key, in the last block
    vv = v.transpose(2, 3).contiguous().to(dev).transpose(2, 3) if transposed else v.to(dev)
    sdpa = A.masked_sdpa_mask(q.double(), k.double(), v.double(), mask)
    for lengths in (None, [300, 250, 10, 300]):
        lt = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=dev)
        out = attention(q.to(dev), k.to(dev), vv, lengths=lt, key_mask=mask.to(dev))
        torch.cuda.synchronize()
        assert out.dtype == torch.float32
        ref = _masked_reference(q, k, v, mask, lengths)
        check(out, ref, 2e-5, 1e-4)
        assert torch.all(out[2] == 0)
        if lengths is None:
            assert (ref - sdpa).abs().max() < 1e-12


def test_slot_attention_mask_and_prefix_mask(dev):
    """The mask of SlotCrossAttention.forward (streamvoxel/stream/engine.py:44-46): the valid keys of a padded
    prefix followed by the valid keys of the padded local keys, a hole between them, in fp32 against the oracle;
    a prefix mask gives the bits of the lengths form; the packed layout takes the mask per window."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, D, pcap, lcap = 3, 4, 64, 48, 400, 128
    kcap = pcap + lcap
    _case('xattn fp32 slot-attention mask (prefix ++ local), prefix mask == lengths, packed + mask')
    q, k, v = qkv(B, H, Q, kcap, D, seed=77)
    prefix_valid = torch.arange(pcap)[None] < torch.tensor([400, 137, 0])[:, None]
    local_valid = torch.arange(lcap)[None] < torch.tensor([128, 64, 100])[:, None]
    mask = torch.cat((prefix_valid, local_valid), 1)
    out = attention(q.to(dev), k.to(dev), v.to(dev), key_mask=mask.to(dev))
    torch.cuda.synchronize()
    check(out, _masked_reference(q, k, v, mask), 2e-5, 1e-4)
    lengths = [528, 300, 1]
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    prefix = torch.arange(kcap, device=dev)[None] < lt[:, None]
    a = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)
    b = attention(q.to(dev), k.to(dev), v.to(dev), key_mask=prefix)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    kp = torch.cat([k[i, :, :lengths[i]] for i in range(B)], 1).to(dev)
    vp = torch.cat([v[i, :, :lengths[i]] for i in range(B)], 1).to(dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=dev)
    packed = attention(q.to(dev), kp, vp, cu_seqlens=cu, key_mask=mask.to(dev))
    torch.cuda.synchronize()
    check(packed, _masked_reference(q, k, v, mask, lengths), 2e-5, 1e-4)


def test_fp32_inputs_are_checked(dev):
    from streamvoxel_amd.stream.attention import attention
    q, k, v = qkv(1, 1, 8, 64, 64, seed=1)
    lt = torch.tensor([64], dtype=torch.int32, device=dev)
    with pytest.raises(TypeError):
        attention(q.to(dev), k.to(dev).bfloat16(), v.to(dev), lengths=lt)
    with pytest.raises(TypeError):
        attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt, k_scale=torch.ones(1, 1, device=dev),
                  v_scale=torch.ones(1, 1, device=dev))
    with pytest.raises(ValueError):
        attention(q.to(dev), k.to(dev), v.to(dev), key_mask=torch.ones(1, 32, dtype=torch.bool, device=dev))
    with pytest.raises(RuntimeError, match='head_dim'):
        q2, k2, v2 = qkv(1, 1, 8, 64, 96, seed=2)
        attention(q2.to(dev), k2.to(dev), v2.to(dev), lengths=lt)
