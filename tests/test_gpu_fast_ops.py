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
    first = top_mask_nosync(s, eligible, count).clone()     # results live in reused buffers: keep a copy
    assert torch.equal(first, top_mask(s, eligible, 1000)) and int(first.sum()) == 1000
    nb = N // 64
    pos = torch.randperm(nb, generator=torch.Generator().manual_seed(1)).to(dev)
    n_total = torch.full((nb,), 64, dtype=torch.int64, device=dev)
    mask = torch.ones(shape, dtype=torch.bool, device=dev)
    a = quota_select_nosync(s, mask, torch.tensor(700, device=dev), 4, pos, torch.tensor(700 / N, device=dev,
                                                                                          dtype=torch.float64),
                            n_total, torch.tensor(0, device=dev)).clone()
    b = quota_select(s, mask, 700, 4, pos, 700 / N, n_total, 0)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and int(a.sum()) == 700


def test_one_window_selection_functions_allocate_nothing_when_repeated(dev):
    """quota_select / block_quota_select / top_mask keep their workspace and outputs per (device, shape, block):
    once warm, repeated eager calls make no allocation of the caching allocator."""
    from streamvoxel_amd.sampling.block_quota import block_quota_select, quota_select, top_mask
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

    def calls():
        a = quota_select(s, mask, k_dev, 4, pos, frac_dev, n_total, com_dev)
        b = quota_select(s, mask, 500, 4, pos, frac_h, n_total, com_h)
        c = block_quota_select(s, mask, 500, 4, order, frac_h, n_total)
        d = top_mask(s, mask, count)
        return a, b, c, d

    want = [t.clone() for t in calls()[:1]]
    calls()
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(dev)['allocation.all.allocated']
    for _ in range(5):
        a, b, c, d = calls()
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats(dev)['allocation.all.allocated'] == before
    assert torch.equal(c, want[0]) and int(c.sum()) == 500 and int(d.sum()) == 300
