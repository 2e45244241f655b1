"""GPU parity of the counter-based sampling tail (`svhip_sample_chosen`, streamvoxel_amd.stream.sampler) against
the oracle (oracle/sampler.py), through the C ABI.

The uniforms are integer work and must agree exactly; the class is the inversion of a floating-point softmax CDF,
so the bar is stated per draw: the kernel's class c must satisfy CDF64(c - 1) - EPS <= u <= CDF64(c) + EPS for the
oracle's float64 CDF (fp32 exponentials and sums over up to 1000 classes stay well inside EPS = 1e-4), and at least
99.9 % of the draws must equal the oracle's class outright."""
import numpy as np
import pytest
import torch

from oracle import sampler as S

pytestmark = pytest.mark.gpu

EPS = 1e-4


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def _buffers(n, shape, dev, seed=0, step=0):
    values = torch.empty((n, *shape), dtype=torch.int16, device=dev)
    seeds = torch.full((n,), seed, dtype=torch.int64, device=dev)
    steps = torch.full((n,), step, dtype=torch.int64, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    return values, seeds, steps, err


def _check_draws(got, rows64, chosen, seed, step, where):
    """got: int [N] classes (-1 where not chosen); rows64 [N, C] float64 logits as the kernel read them."""
    want, idx, u, cdf = S.sample_chosen(rows64, chosen, seed, step)
    assert np.array_equal(got < 0, ~chosen), where
    g = got[idx].astype(np.int64)
    r = np.arange(len(idx))
    lo = np.where(g > 0, cdf[r, np.maximum(g - 1, 0)], 0.0)
    hi = cdf[r, g]
    assert np.all((lo - EPS <= u) & (u <= hi + EPS)), (where, np.flatnonzero(~((lo - EPS <= u) & (u <= hi + EPS)))[:5])
    same = np.mean(g == want[idx]) if len(idx) else 1.0
    assert same >= 0.999, (where, same)
    return same


@pytest.mark.parametrize('classes', [5, 100, 256, 304, 500, 1000])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_class_major_and_patch_layouts_match_oracle(dev, classes, dtype):
    from streamvoxel_amd.stream.patches import PatchLogits
    from streamvoxel_amd.stream.sampler import sample_chosen
    n, shape, p = 2, (16, 8, 32), 2
    N = shape[0] * shape[1] * shape[2]
    _case(f'sample_chosen C={classes} dtype={dtype} windows={n} shape={shape}')
    g = torch.Generator().manual_seed(classes)
    cm = (torch.randn(n, classes, *shape, generator=g) * 2.5).to(dtype)     # class-major [n, C, Y, Z, X]
    chosen = torch.rand(n, *shape, generator=g) < 0.3
    tokens0 = torch.randint(0, classes, (n, *shape), generator=g)
    gy, gz, gx = (s // p for s in shape)
    patches = (cm.reshape(n, classes, gy, p, gz, p, gx, p).permute(0, 2, 4, 6, 3, 5, 7, 1)
               .reshape(n, gy * gz * gx, p ** 3 * classes).contiguous())
    seeds = [11, 2 ** 63 - 5]
    outs = []
    for form in ('class-major', 'patches'):
        logits = cm.to(dev) if form == 'class-major' else PatchLogits(patches.to(dev), shape, p, classes)
        values, _, steps, err = _buffers(n, shape, dev, step=7)
        seed_t = torch.tensor(seeds, dtype=torch.int64, device=dev)
        tokens = tokens0.to(dev)
        sample_chosen(logits, chosen.to(dev), seed_t, steps, values, err, tokens)
        torch.cuda.synchronize()
        assert int(err) == 0
        v = values.cpu()
        t = tokens.cpu()
        assert torch.equal(t[~chosen], tokens0[~chosen])          # untouched where not chosen
        assert torch.equal(t[chosen], v[chosen].long())           # the draws, in place
        outs.append(v)
    assert torch.equal(outs[0], outs[1])                          # same rows, same arithmetic, same classes
    for b in range(n):
        rows64 = cm[b].reshape(classes, N).t().double().numpy()
        same = _check_draws(outs[0][b].reshape(-1).numpy(), rows64, chosen[b].reshape(-1).numpy(), seeds[b], 7,
                            f'C={classes} window={b}')
        print(f'[gpu-case] C={classes} {dtype} window {b}: {same:.5f} of the draws equal the oracle class', flush=True)


@pytest.mark.parametrize('shape,share', [((5, 7, 9), 1.0), ((10, 10, 10), 1.0), ((8, 8, 20), 0.6)])
@pytest.mark.parametrize('classes,dtype', [(64, torch.bfloat16), (64, torch.float32), (100, torch.float32),
                                           (256, torch.float32), (304, torch.bfloat16), (512, torch.bfloat16),
                                           (1000, torch.float32)])
def test_ragged_windows_and_dense_choices_match_oracle(dev, shape, share, classes, dtype):
    """Windows whose voxel count is not a multiple of the kernel's 512-voxel workgroup (315: one partial group;
    1000: one full and one partial; 1280: two full and one partial), up to every voxel chosen, from voxel rows (a
    class-major view with unit class stride, the 16-byte row loads where they apply)."""
    from streamvoxel_amd.stream.sampler import sample_chosen
    n = 2
    N = shape[0] * shape[1] * shape[2]
    _case(f'sample_chosen ragged C={classes} dtype={dtype} shape={shape} share={share}')
    g = torch.Generator().manual_seed(N + classes)
    rows = (torch.randn(n, N, classes, generator=g) * 2.0).to(dtype)          # voxel rows [n, N, C]
    chosen = torch.rand(n, *shape, generator=g) < share
    cm = rows.to(dev).transpose(1, 2).reshape(n, classes, *shape)              # view, class stride 1
    assert cm.stride(1) == 1
    values, _, steps, err = _buffers(n, shape, dev, step=3)
    seeds = [5, 77]
    sample_chosen(cm, chosen.to(dev), torch.tensor(seeds, dtype=torch.int64, device=dev), steps, values, err)
    torch.cuda.synchronize()
    assert int(err) == 0
    v = values.cpu()
    for b in range(n):
        _check_draws(v[b].reshape(-1).numpy(), rows[b].double().numpy(), chosen[b].reshape(-1).numpy(), seeds[b], 3,
                     f'ragged C={classes} window={b}')


def test_equal_logits_draw_floor_u_times_classes(dev):
    """Equal logits: the CDF is (c + 1) / C, so the class is floor(u C) (up to the fp32 rounding of u * total at
    the boundaries)."""
    from streamvoxel_amd.stream.sampler import sample_chosen
    C, shape = 304, (32, 32, 32)
    N = 32 ** 3
    _case(f'sample_chosen equal logits C={C} N={N}')
    logits = torch.zeros(1, C, *shape, device=dev)
    chosen = torch.ones(1, *shape, dtype=torch.bool, device=dev)
    values, seeds, steps, err = _buffers(1, shape, dev, seed=123, step=4)
    sample_chosen(logits, chosen, seeds, steps, values, err)
    got = values.cpu().reshape(-1).numpy().astype(np.int64)
    u = S.uniforms(123, 4, np.arange(N))
    want = np.floor(u * C).astype(np.int64)
    near = np.abs(u * C - np.round(u * C)) < 1e-3
    assert np.all((got == want) | near)
    assert np.mean(got == want) > 0.999
    # Frequencies: every class about N / C times.
    counts = np.bincount(got, minlength=C)
    assert counts.min() > 0.6 * N / C and counts.max() < 1.4 * N / C


def test_non_finite_rows_set_the_error_flag(dev):
    from streamvoxel_amd.stream.sampler import sample_chosen
    C, shape = 16, (4, 4, 4)
    _case('sample_chosen NaN and all -inf rows')
    for bad in ('nan', '-inf'):
        logits = torch.randn(C, *shape, device=dev)
        if bad == 'nan':
            logits[3, 1, 2, 3] = float('nan')
        else:
            logits[:, 1, 2, 3] = float('-inf')
        chosen = torch.zeros(*shape, dtype=torch.bool, device=dev)
        values, seeds, steps, err = _buffers(1, shape, dev)
        sample_chosen(logits, chosen, seeds, steps, values, err)       # the bad voxel not chosen: no error
        assert int(err) == 0
        chosen[1, 2, 3] = True
        chosen[0, 0, 0] = True
        tokens = torch.full(shape, C, dtype=torch.int64, device=dev)
        sample_chosen(logits, chosen, seeds, steps, values, err, tokens)
        assert int(err) != 0, bad
        # the bad row draws nothing: its token stays the mask token and its value reads -1; the good one is drawn
        assert int(tokens[1, 2, 3]) == C and int(values.view(shape)[1, 2, 3]) == -1, bad
        assert 0 <= int(tokens[0, 0, 0]) < C and int(values.view(shape)[0, 0, 0]) == int(tokens[0, 0, 0])
        # A -inf class among finite ones is a zero-probability class, not an error.
    logits = torch.randn(C, *shape, device=dev)
    logits[:5] = float('-inf')
    chosen = torch.ones(*shape, dtype=torch.bool, device=dev)
    values, seeds, steps, err = _buffers(1, shape, dev)
    sample_chosen(logits, chosen, seeds, steps, values, err)
    assert int(err) == 0 and int(values.min()) >= 5


def test_graph_replays_equal_eager_draws(dev):
    """A captured launch replayed with new step and seed values gives the eager draws of those values (the tail
    inside a captured step); eager work and synchronisations run between the replays."""
    from streamvoxel_amd.stream.sampler import sample_chosen
    C, shape = 256, (64, 16, 16)
    _case(f'sample_chosen graph replays C={C}')
    g = torch.Generator(device=dev).manual_seed(5)
    logits = torch.randn(1, C, *shape, device=dev, generator=g)
    chosen = torch.rand(1, *shape, device=dev, generator=g) < 0.05
    values, seeds, steps, err = _buffers(1, shape, dev)
    tokens = torch.zeros(1, *shape, dtype=torch.int64, device=dev)
    sample_chosen(logits, chosen, seeds, steps, values, err, tokens)     # warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sample_chosen(logits, chosen, seeds, steps, values, err, tokens)
    for step, seed in [(0, 1), (1, 1), (2, 99), (25, 2 ** 40)]:
        steps.fill_(step)
        seeds.fill_(seed)
        graph.replay()
        torch.cuda.synchronize()
        replayed = values.clone()
        eager_v, _, _, eager_err = _buffers(1, shape, dev)
        sample_chosen(logits, chosen, seeds, steps, eager_v, eager_err)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager_v), (step, seed)
        assert torch.equal(tokens[chosen], replayed[chosen].long())
    assert int(err) == 0


def test_philox_slot_window_eager_equals_graph_and_oracle_draws(dev):
    """A whole window on the 'philox' sampler: the per-slot eager `consume` over voxel-row views and the graph-staged
    batch over class planes (selection and sampling captured together through SelectGraphs) commit the same
    positions and values at every step, every
    step commits exactly its quota, and the committed values are the oracle's counter-based draws on that step's
    logits."""
    from streamvoxel_amd.stream.slot import LowEntropyLastSlot, SelectGraphs, consume_batch
    from tests.test_gpu_slot import (AIR, AIR_TOKEN, CAP, CLASSES, EPS as LEL_EPS, SHAPE, _Engine, _compare_commit,
                                     _compare_record, marking_logits, solid_logits)
    _case('philox slot window, eager vs staged, block=4')
    engine = _Engine(2, dev)
    eager = LowEntropyLastSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, LEL_EPS, 4, dev, sampler='philox')
    staged = [LowEntropyLastSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, LEL_EPS, 4, dev, sampler='philox') for _ in range(2)]
    graphs = SelectGraphs(engine, staged)
    assert int((engine.tokens != CLASSES).sum()) == 0                 # capture drew nothing into the token rows
    seed = 2024
    eager.arm(seed=seed, cap=CAP, target=(0, 0, 0))
    staged[0].arm(seed=seed, cap=CAP, target=(0, 0, 0))
    tok_e = torch.full(SHAPE, CLASSES, dtype=torch.int64, device=dev)
    out = engine.outputs[2]
    rec_e = rec_s = None
    commits = 0
    N = SHAPE[0] * SHAPE[1] * SHAPE[2]
    for step in range(CAP + 1):
        out[0].copy_(marking_logits(3, dev) if step == 0 else solid_logits(50 + step, step, CAP + 1, dev))
        # the eager slot reads the same logits as a view of voxel rows (class stride 1), the staged ones the class
        # planes: the scores, selections and draws do not depend on the layout
        rows_view = out[0].permute(1, 2, 3, 0).contiguous().permute(3, 0, 1, 2)
        assert rows_view.stride(0) == 1
        r_e, c_e = eager.consume(rows_view, tok_e)
        got = consume_batch(staged, out, engine.tokens, 2, graphs)
        r_s, c_s = got.get(0, (None, None))
        _compare_commit(c_e, c_s, f'step={step}')
        if c_e is not None:
            commits += 1
            assert len(c_e['positions']) == eager.quotas[c_e['step'] - 2]
            rows64 = out[0].reshape(CLASSES, N).t()[torch.as_tensor(c_e['positions'], device=dev).long()]
            rows64 = rows64.double().cpu().numpy()
            full = np.zeros((N, CLASSES))
            full[c_e['positions']] = rows64
            chosen = np.zeros(N, dtype=bool)
            chosen[c_e['positions']] = True
            drawn = np.full(N, -1, dtype=np.int64)
            drawn[c_e['positions']] = c_e['values']
            _check_draws(drawn, full, chosen, seed, c_e['step'] - 2, f'step={step}')
        rec_e = rec_e or r_e
        rec_s = rec_s or r_s
    _compare_record(rec_e, rec_s, 'finish')
    assert torch.equal(tok_e, engine.tokens[0])
    assert commits == len(eager.quotas) and rec_e is not None
    assert int((tok_e == CLASSES).sum()) == 0


def test_philox_slot_reads_voxel_row_views(dev):
    """Logits handed to a 'philox' slot as a view of voxel rows (class stride 1) are sampled where the selection
    read them: the slot's draws equal `sample_chosen` over the same values in class planes on the slot's own
    chosen mask, seed and step."""
    from streamvoxel_amd.stream.sampler import sample_chosen
    from streamvoxel_amd.stream.slot import LowEntropyLastSlot
    from tests.test_gpu_slot import AIR, AIR_TOKEN, CAP, CLASSES, EPS as LEL_EPS, SHAPE, marking_logits, solid_logits
    _case('philox slot, voxel-row view of the logits')
    slot = LowEntropyLastSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, LEL_EPS, 4, dev, sampler='philox')
    slot.arm(seed=77, cap=CAP, target=(0, 0, 0))
    tokens = torch.full(SHAPE, CLASSES, dtype=torch.int64, device=dev)
    slot.consume(marking_logits(9, dev), tokens)                      # the marking forward
    planes = solid_logits(901, 1, CAP + 1, dev).contiguous()           # [C, Y, Z, X]
    rows_view = planes.permute(1, 2, 3, 0).contiguous().permute(3, 0, 1, 2)
    assert rows_view.stride(0) == 1
    k = slot.prepare()
    before = tokens.clone()
    slot.select(rows_view, tokens)
    torch.cuda.synchronize()
    assert int(slot.chosen.sum()) == k and int(slot.sample_err) == 0
    values, _, _, err = _buffers(1, SHAPE, dev)
    want_tokens = before.clone()
    sample_chosen(planes, slot.chosen, slot.seed_dev, slot.step_dev, values, err, want_tokens.view(1, *SHAPE))
    torch.cuda.synchronize()
    assert torch.equal(slot.drawn, values.view(SHAPE))
    assert torch.equal(tokens, want_tokens)
