"""The reference-named entry points of streamvoxel_amd.stream.fast_ops on the GPU: cross_flex / cross_sdpa (query
projection, AxialRoPE, cached-key attention, output projection) against the oracle's rotation and float64
attention; entropy_triton, top_mask_nosync and quota_select_nosync against the functions they name."""
import pytest
import torch

from oracle import attention as A
from oracle import producer as P

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


class _Rope(torch.nn.Module):
    def __init__(self, head_dim):
        super().__init__()
        from streamvoxel_amd.stream.producer import rope_frequencies
        self.register_buffer('frequencies', rope_frequencies(head_dim))


class _Cross(torch.nn.Module):
    """The attributes RotaryCrossAttention exposes to fast_ops (streaming_controlnet.py): norm, query, key_value,
    proj, heads, rope."""

    def __init__(self, width, heads):
        super().__init__()
        self.heads = heads
        self.norm = torch.nn.LayerNorm(width, elementwise_affine=False, eps=1e-6)
        self.query = torch.nn.Linear(width, width)
        self.key_value = torch.nn.Linear(width, 2 * width)
        self.proj = torch.nn.Linear(width, width)
        self.rope = _Rope(width // heads)


def test_cross_flex_and_sdpa(dev):
    from streamvoxel_amd.stream.fast_ops import cross_flex, cross_sdpa
    torch.manual_seed(12)
    n, Q, W, H, kcap = 3, 96, 384, 8, 320
    D = W // H
    cross = _Cross(W, H).to(dev).to(torch.bfloat16)
    value = torch.randn(n, Q, W, device=dev, dtype=torch.bfloat16)
    positions = torch.randint(0, 512, (n, Q, 3), device=dev).float() / 4
    lengths = [320, 77, 1]
    key = (torch.randn(n, H, kcap, D, device=dev) / 4).bfloat16()
    val = (torch.randn(n, H, kcap, D, device=dev) / 4).bfloat16()
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    valid = torch.arange(kcap, device=dev)[None] < lt[:, None]
    out_flex = cross_flex(cross, value, positions, key, val, lt)
    out_sdpa = cross_sdpa(cross, value, positions, key, val, valid)
    torch.cuda.synchronize()
    assert torch.equal(out_flex, out_sdpa)
    # Expected: the same projections in torch, the oracle's AxialRoPE, float64 attention over the first L_b keys.
    with torch.no_grad():
        q = cross.query(cross.norm(value)).reshape(n, Q, H, D).transpose(1, 2)
        q = P.axial_rope(q.cpu(), positions.cpu(), cross.rope.frequencies.cpu())
        att = A.cross_attention(q, key.cpu(), val.cpu(), lengths)                  # [n, H, Q, D] float64
        want = cross.proj(att.to(dev).transpose(1, 2).reshape(n, Q, W).to(torch.bfloat16)).float()
    err = (out_flex.float() - want).abs().max().item()
    assert err <= 3e-2 * max(1.0, want.abs().max().item()), err
    # A key mask that is not a prefix (masked SDPA takes any boolean mask): the True keys of each window exactly,
    # as torch's masked SDPA over the same projections in float64.
    holes = torch.rand(n, kcap, device=dev, generator=torch.Generator(dev).manual_seed(4)) < 0.6
    holes[:, 0] = True
    out_holes = cross_sdpa(cross, value, positions, key, val, holes)
    torch.cuda.synchronize()
    with torch.no_grad():
        ref = A.masked_sdpa_mask(q.double(), key.cpu().double(), val.cpu().double(), holes.cpu())
        want = cross.proj(ref.to(dev).transpose(1, 2).reshape(n, Q, W).to(torch.bfloat16)).float()
    err = (out_holes.float() - want).abs().max().item()
    assert err <= 3e-2 * max(1.0, want.abs().max().item()), err


def test_selection_names(dev):
    from streamvoxel_amd import synth
    from streamvoxel_amd.sampling.block_quota import quota_select, top_mask
    from streamvoxel_amd.sampling.entropy import entropy_scores
    from streamvoxel_amd.stream.fast_ops import (entropy_torch, entropy_triton, quota_select_nosync,
                                                 top_mask_nosync)
    shape = (32, 16, 16)
    N = 32 * 16 * 16
    logits = synth.bimodal_logits(N, 64, 0.6, seed=5, device=dev).t().reshape(64, *shape).bfloat16()
    s = entropy_scores(logits)
    assert torch.equal(entropy_triton(logits, block_n=128, block_c=8), s)
    assert torch.equal(entropy_torch(logits), s)
    eligible = torch.rand(shape, device=dev) < 0.7
    count = torch.tensor(1000, device=dev)
    first = top_mask_nosync(s, eligible, count)
    assert torch.equal(first, top_mask(s, eligible, 1000)) and int(first.sum()) == 1000
    nb = N // 64
    pos = torch.randperm(nb, generator=torch.Generator().manual_seed(1)).to(dev)
    n_total = torch.full((nb,), 64, dtype=torch.int64, device=dev)
    mask = torch.ones(shape, dtype=torch.bool, device=dev)
    a = quota_select_nosync(s, mask, torch.tensor(700, device=dev), 4, pos, torch.tensor(700 / N, device=dev,
                                                                                          dtype=torch.float64),
                            n_total, torch.tensor(0, device=dev))
    b = quota_select(s, mask, 700, 4, pos, 700 / N, n_total, 0)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and int(a.sum()) == 700


def test_one_window_selection_functions_allocate_nothing_with_caller_buffers(dev):
    """quota_select / block_quota_select / top_mask with `out=` and `buffers=` (caller-owned SelectBuffers): once
    warm, repeated eager calls make no allocation of the caching allocator, and give the default calls' results."""
    from streamvoxel_amd.sampling.block_quota import SelectBuffers, block_quota_select, quota_select, top_mask
    shape = (64, 16, 16)
    N = 64 * 16 * 16
    nb = N // 64
    g = torch.Generator(dev).manual_seed(8)
    s = torch.rand(shape, device=dev, generator=g)
    mask = torch.rand(shape, device=dev, generator=g) < 0.8
    order = torch.randperm(nb, device=dev, generator=g)
    pos = torch.empty_like(order)
    pos[order] = torch.arange(nb, device=dev)
    n_total = torch.full((nb,), 64, dtype=torch.int64, device=dev)
    k_dev = torch.tensor(500, device=dev)
    frac_dev = torch.tensor((N - int(mask.sum()) + 500) / N, device=dev, dtype=torch.float64)
    com_dev = torch.tensor(N - int(mask.sum()), device=dev)
    count = torch.tensor(300, device=dev)
    frac_h, com_h = float(frac_dev), int(com_dev)
    buffers = SelectBuffers(shape, 4, dev)
    outs = [torch.empty(shape, dtype=torch.bool, device=dev) for _ in range(4)]

    def calls():
        a = quota_select(s, mask, k_dev, 4, pos, frac_dev, n_total, com_dev, out=outs[0], buffers=buffers)
        b = quota_select(s, mask, 500, 4, pos, frac_h, n_total, com_h, out=outs[1], buffers=buffers)
        c = block_quota_select(s, mask, 500, 4, order, frac_h, n_total, out=outs[2], buffers=buffers)
        d = top_mask(s, mask, count, out=outs[3])
        return a, b, c, d

    want = [quota_select(s, mask, 500, 4, pos, frac_h, n_total, com_h), top_mask(s, mask, 300)]
    calls()
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(dev)['allocation.all.allocated']
    for _ in range(5):
        a, b, c, d = calls()
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats(dev)['allocation.all.allocated'] == before
    assert all(t is o for t, o in zip((a, b, c, d), outs))
    assert torch.equal(a, want[0]) and torch.equal(b, want[0]) and torch.equal(c, want[0])
    assert torch.equal(d, want[1]) and int(c.sum()) == 500 and int(d.sum()) == 300


def test_selection_results_are_fresh_and_chain_like_the_reference(dev):
    """The reference's callers keep selection results and chain them: `top_mask(score, top_mask(draw, mask, c), k)`
    (eval/samplers.py:27-28) and a held quota_select result across a second call. Every default call returns a
    tensor of its own, so both equal the oracle bit for bit; an `out` that aliases an input is refused."""
    import numpy as np
    from oracle import sampling as S
    from streamvoxel_amd.sampling.block_quota import SelectBuffers, block_quota_select, quota_select, top_mask
    shape = (32, 16, 16)
    N = 32 * 16 * 16
    nb = N // 64
    rng = np.random.default_rng(3)
    score = (rng.integers(-40, 1, shape) / 8).astype(np.float32)
    draw = rng.random(shape).astype(np.float32)
    mask = rng.random(shape) < 0.75
    sd, dd, md = (torch.from_numpy(a).to(dev) for a in (score, draw, mask))
    c, k = 1500, 600
    got = top_mask(sd, top_mask(dd, md, c), k)
    want = S.top_mask(score, S.top_mask(draw, mask, c), k)
    assert np.array_equal(got.cpu().numpy(), want)

    order = rng.permutation(nb)
    pos = S.order_to_pos(order)
    n_total = np.full(nb, 64, np.int64)
    committed = int(N - mask.sum())
    results = []
    for kk in (300, 900):
        frac = (committed + kk) / N
        results.append((kk, frac, quota_select(sd, md, kk, 4, torch.from_numpy(pos).to(dev), frac,
                                               torch.from_numpy(n_total).to(dev), committed)))
    held = [block_quota_select(sd, md, kk, 4, torch.from_numpy(order).to(dev), (committed + kk) / N,
                               torch.from_numpy(n_total).to(dev)) for kk in (300, 900)]
    for (kk, frac, res), blk in zip(results, held):
        expect = S.quota_select_nosync(score, mask, kk, 4, pos, frac, n_total, committed)
        assert np.array_equal(res.cpu().numpy(), expect), kk
        assert np.array_equal(blk.cpu().numpy(), expect), kk
    assert results[0][2].data_ptr() != results[1][2].data_ptr()

    eligible = md.clone()
    with pytest.raises(ValueError, match='shares memory'):
        top_mask(sd, eligible, 10, out=eligible)
    with pytest.raises(ValueError, match='shares memory'):
        quota_select(sd, eligible, 10, 4, torch.from_numpy(pos).to(dev), 0.5, torch.from_numpy(n_total).to(dev),
                     committed, out=eligible)
    with pytest.raises(ValueError, match='buffers are for'):
        quota_select(sd, md, 10, 4, torch.from_numpy(pos).to(dev), 0.5, torch.from_numpy(n_total).to(dev),
                     committed, buffers=SelectBuffers((64, 16, 16), 4, dev))