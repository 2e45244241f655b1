"""GPU parity of reading the class head's output in place (svhip_entropy_patches, svhip_air_prob_patches,
svhip_ease_select_patches through the C ABI, and the PatchLogits paths of EaseSelect and the slot classes).

Bar: bit-exact against the same kernels over the same logits copied into (y, z, x) voxel-major rows (the voxel
rows are read in another order, the per-voxel arithmetic is the same); the entropy also against the oracle in
float64; a whole window of slot steps (marking + 25 solid steps, select graphs captured over PatchLogits) gives the
same commits and tokens as the slot fed the permuted logits."""
import numpy as np
import pytest
import torch

from oracle import sampling as S

pytestmark = pytest.mark.gpu

SHAPE, P = (256, 16, 16), 4
N = SHAPE[0] * SHAPE[1] * SHAPE[2]


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def _to_patches(flat, classes):
    """[n, N, C] rows in (y, z, x) order -> PatchLogits holding the same logits in the class head's order."""
    from streamvoxel_amd.stream.patches import PatchLogits
    n = flat.shape[0]
    out = PatchLogits(torch.empty(n, N // P ** 3, P ** 3 * classes, dtype=flat.dtype, device=flat.device), SHAPE, P,
                      classes)
    out.rows[:, out.row_index(torch.arange(N, device=flat.device))] = flat
    return out


@pytest.mark.parametrize('dtype,classes', [(torch.float32, 256), (torch.bfloat16, 304)])
def test_entropy_and_air_prob_equal_yzx_rows(dev, dtype, classes):
    from streamvoxel_amd import _lib, synth
    from streamvoxel_amd.sampling.entropy import air_prob, entropy_batched, entropy_scores
    n = 3
    _case(f'entropy / air prob patches {dtype} C={classes} n={n}')
    flat = synth.bimodal_logits(n * N, classes, 0.7, seed=11, device=dev).reshape(n, N, classes).to(dtype)
    pl = _to_patches(flat, classes)
    assert torch.equal(pl.class_major(), flat.transpose(1, 2).reshape(n, classes, *SHAPE))
    got = entropy_scores(pl)
    want = entropy_batched(flat, layout='voxel_major')
    torch.cuda.synchronize()
    assert got.shape == (n, *SHAPE)
    assert torch.equal(got.reshape(n, N), want)
    ref = S.entropy_scores(flat[1, ::97].double().cpu().t())
    err = (got.reshape(n, N)[1, ::97].double().cpu() - torch.as_tensor(np.asarray(ref))).abs().max().item()
    assert err <= 2e-5, err
    air_ids = torch.tensor([0, 5, classes - 1], dtype=torch.int32, device=dev)
    got_air = air_prob(pl, None, air_index=air_ids)
    want_air = torch.empty(n, N, device=dev)
    lib = _lib.load()
    _lib.check(lib.svhip_air_prob(_lib.ptr(flat), _lib.dtype_code(dtype), n, classes, N, flat.stride(0),
                                  flat.stride(2), flat.stride(1), _lib.ptr(air_ids), 3, _lib.ptr(want_air),
                                  _lib.stream_of(flat)), 'svhip_air_prob')
    torch.cuda.synchronize()
    assert torch.equal(got_air.reshape(n, N), want_air)


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_ease_select_and_mark_equal_yzx_rows(dev, dtype):
    """EaseSelect over 8 windows with deferred voxels and committed tokens: chosen, scores, bad and the marking
    pass's deferred masks are the same bits from PatchLogits and from (y, z, x) rows."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.step import EaseSelect
    B, C, block = 8, 256, 4
    _case(f'ease select patches {dtype} B={B}')
    flat = synth.bimodal_logits(B * N, C, 0.75, seed=21, device=dev).reshape(B, N, C).to(dtype)
    flat[:, :, 0] += 25.0 * (torch.rand(B, N, device=dev, generator=torch.Generator(device=dev).manual_seed(3)) < 0.3)
    pl = _to_patches(flat, C)
    sels = [EaseSelect(B, SHAPE, C, block, dev, air_ids=(0,)) for _ in range(2)]
    g = torch.Generator().manual_seed(9)
    last = torch.rand(B, N, generator=g) < 0.2
    tokens = torch.where(torch.rand(B, N, generator=g) < 0.1, torch.randint(0, C, (B, N), generator=g),
                         torch.full((B, N), C))
    for sel in sels:
        sel.tokens.copy_(tokens.to(dev))
        for b in range(B):
            sel.bind_window(b, torch.randperm(N // 64, generator=torch.Generator().manual_seed(40 + b)),
                            last=last[b].to(dev))
            committed = int(((tokens[b] != C) & ~last[b]).sum())
            k = 1500 + 37 * b
            sel.set_step(b, k, committed, (committed + k) / int((~last[b]).sum()))
    sels[0].run(pl, keep_scores=True)
    sels[1].run(flat.reshape(B * N, C), keep_scores=True)
    torch.cuda.synchronize()
    assert torch.equal(sels[0].scores, sels[1].scores)
    assert torch.equal(sels[0].chosen, sels[1].chosen)
    assert not bool(sels[0].bad.any()) and not bool(sels[1].bad.any())
    assert torch.equal(sels[0].chosen.sum(1).cpu(), torch.tensor([1500 + 37 * b for b in range(B)]))
    for sel in sels:
        sel.last.zero_()
    sels[0].mark(pl, 1e-4)
    sels[1].mark(flat.reshape(B * N, C), 1e-4)
    torch.cuda.synchronize()
    assert torch.equal(sels[0].air, sels[1].air)
    assert torch.equal(sels[0].last, sels[1].last)
    assert int(sels[0].last.sum()) > 0


def test_slot_window_from_patch_logits(dev):
    """Two slots fed PatchLogits (select graphs captured over them, staged by consume_batch) and two fed the
    permuted [C, Y, Z, X] logits: the same commits every step and the same tokens and records at the end."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.patches import PatchLogits
    from streamvoxel_amd.stream.slot import LowEntropyLastSlot, SelectGraphs, consume_batch
    C, cap, slots_n = 256, 25, 2
    _case(f'slot window from patch logits, block=4, slots={slots_n}')

    class Engine:
        def __init__(self):
            self.device = dev
            self.outputs = {slots_n: PatchLogits(torch.zeros(slots_n, N // 64, 64 * C, device=dev), SHAPE, P, C)}
            self.tokens = torch.full((slots_n, *SHAPE), C, dtype=torch.int64, device=dev)
            self.graphs = True

    engine = Engine()
    a = [LowEntropyLastSlot(SHAPE, C, (0,), 0, 1e-4, 4, dev) for _ in range(slots_n)]
    b = [LowEntropyLastSlot(SHAPE, C, (0,), 0, 1e-4, 4, dev) for _ in range(slots_n)]
    graphs = SelectGraphs(engine, a)
    assert len(graphs.graphs) == slots_n
    for i in range(slots_n):
        a[i].arm(seed=77 + i, cap=cap, target=(i, 0, 0))
        b[i].arm(seed=77 + i, cap=cap, target=(i, 0, 0))
    out = engine.outputs[slots_n]
    flat = torch.empty(slots_n, N, C, device=dev)
    tokens_b = engine.tokens.clone()
    records_a, records_b = {}, {}
    for step in range(cap + 1):
        for i in range(slots_n):
            if step == 0:
                x = synth.bimodal_logits(N, C, 0.7, seed=300 + i, device=dev)
                heights = torch.randint(96, 224, (SHAPE[1], SHAPE[2]), device=dev,
                                        generator=torch.Generator(device=dev).manual_seed(i))
                ys = torch.arange(SHAPE[0], device=dev)[:, None, None]
                x[:, 0] += 40.0 * (ys >= heights[None]).reshape(-1)
            else:
                share = 0.30 + (0.05 - 0.30) * step / cap
                x = synth.bimodal_logits(N, C, 1.0 - share, seed=1000 * i + step, device=dev)
            flat[i].copy_(x)
        out.rows[:, out.row_index(torch.arange(N, device=dev))] = flat
        got_a = consume_batch(a, out, engine.tokens, slots_n, graphs)
        permuted = out.class_major()                # the reference's permuted copy: contiguous class planes
        got_b = consume_batch(b, permuted, tokens_b, slots_n)
        assert sorted(got_a) == sorted(got_b), step
        for i in got_a:
            (ra, ca), (rb, cb) = got_a[i], got_b[i]
            assert (ca is None) == (cb is None), (step, i)
            if ca is not None:
                assert ca['step'] == cb['step']
                assert np.array_equal(ca['positions'], cb['positions']), (step, i)
                assert np.array_equal(ca['values'], cb['values']), (step, i)
            if ra is not None:
                records_a[i], records_b[i] = ra, rb
        assert torch.equal(engine.tokens, tokens_b), step
    assert sorted(records_a) == list(range(slots_n))
    for i in range(slots_n):
        assert records_a[i]['last_count'] == records_b[i]['last_count'] > 0
        assert torch.equal(records_a[i]['step_map'], records_b[i]['step_map'])
        assert torch.equal(records_a[i]['values'], records_b[i]['values'])
    assert int((engine.tokens == C).sum()) == 0
