"""Whole-window trajectories of the product slots (streamvoxel_amd.stream.slot) against the oracle slot
(oracle/slot.py, the restatement of stream/slot.py:50-176), on the GPU with the same seeds.

The oracle is fed the kernels' own fp32 scores and air probabilities (the split contract: selection and deferral
masks are bit-exact given identical scores); its selection is the numpy restatement, its categorical draws are
torch's multinomial on the same device and generator. Every step's commit (positions and values), the token
buffers and the finish records must be identical. Block sizes 1, 4 and 16 (the block sweep of the EASE-loop
configuration): 8 windows x 26 forwards (the marking forward and 25 solid steps), logits regenerated every step
with the uncertain share drifting from 30 % to 5 %, solid steps graph-captured through SelectGraphs and staged
for the whole batch by consume_batch."""
import numpy as np
import pytest
import torch

from oracle.slot import LowEntropyLastSlot as OracleSlot

pytestmark = pytest.mark.gpu

SHAPE, CLASSES, AIR, AIR_TOKEN, EPS, CAP = (256, 16, 16), 256, (0,), 0, 1e-4, 25
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


def marking_logits(seed, dev):
    """[C,Y,Z,X]: N(0,1), and in every (z, x) column the voxels from a random height up carry air at +40 (air
    probability ~1: they are deferred); a few of them are made uncertain so that the deferred run stops early."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(CLASSES, *SHAPE, device=dev, generator=g)
    tops = torch.randint(100, 257, (SHAPE[1], SHAPE[2]), device=dev, generator=g)
    ys = torch.arange(SHAPE[0], device=dev)[:, None, None]
    clean = ys >= tops[None]
    holes = torch.rand(SHAPE, device=dev, generator=g) < 0.002
    x[AIR[0]] += 40.0 * (clean & ~holes)
    return x


def solid_logits(seed, step, steps, dev):
    from streamvoxel_amd import synth
    share = 0.30 + (0.05 - 0.30) * step / max(steps - 1, 1)
    flat = synth.bimodal_logits(N, CLASSES, 1.0 - share, seed, device=dev)      # [N, C]
    return flat.t().reshape(CLASSES, *SHAPE)


class _Engine:
    """The engine attributes SelectGraphs reads: static per-bucket logits and token rows."""

    def __init__(self, slots, dev):
        self.device = dev
        self.outputs = {slots: torch.zeros(slots, CLASSES, *SHAPE, device=dev)}
        self.tokens = torch.full((slots, *SHAPE), CLASSES, dtype=torch.int64, device=dev)
        self.graphs = True


def _compare_commit(a, b, where):
    assert (a is None) == (b is None), where
    if a is not None:
        assert a['step'] == b['step'], where
        assert np.array_equal(a['positions'], b['positions']), where
        assert np.array_equal(a['values'], b['values']), where


def _compare_record(a, b, where):
    assert (a is None) == (b is None), where
    if a is not None:
        for key in ('target', 'seed', 'cap', 'nfe', 'actual', 'last_count'):
            assert a[key] == b[key], (where, key, a[key], b[key])
        assert torch.equal(a['step_map'], b['step_map']), where
        assert torch.equal(a['values'], b['values']), where


@pytest.mark.parametrize('block', [1, 4, 16])
def test_window_trajectories_match_oracle_slot(dev, block):
    from streamvoxel_amd.stream.slot import FastLowEntropyLastSlot, SelectGraphs, consume_batch
    slots_n = 8
    _case(f'slot trajectories block={block} slots={slots_n} forwards={CAP + 1}')
    engine = _Engine(slots_n, dev)
    prod = [FastLowEntropyLastSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, EPS, block, dev, keep_scores=True)
            for _ in range(slots_n)]
    graphs = SelectGraphs(engine, prod)
    assert len(graphs.graphs) == slots_n
    orac = []
    for i in range(slots_n):
        p = prod[i]
        orac.append(OracleSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, EPS, block, dev,
                               score_fn=lambda logits, p=p: p.scores.cpu().numpy(),
                               air_prob_fn=lambda logits, air, p=p: p.air_p.cpu().numpy()))
    tokens_o = engine.tokens.clone()
    for i in range(slots_n):
        prod[i].arm(seed=1000 + 17 * i + block, cap=CAP, target=(i, 0, 0))
        orac[i].arm(seed=1000 + 17 * i + block, cap=CAP, target=(i, 0, 0))
    out = engine.outputs[slots_n]
    finished = commits = 0
    records = []
    for step in range(CAP + 1):
        for i in range(slots_n):
            src = marking_logits(7 * i + 1, dev) if step == 0 else solid_logits(100 * i + step, step, CAP + 1, dev)
            out[i].copy_(src)
        got = consume_batch(prod, out, engine.tokens, slots_n, graphs)
        for i in range(slots_n):
            want = orac[i].consume(out[i], tokens_o[i])
            rec, commit = got.get(i, (None, None))
            where = f'block={block} step={step} slot={i}'
            _compare_commit(commit, want[1], where)
            _compare_record(rec, want[0], where)
            finished += rec is not None
            commits += commit is not None
            if rec is not None:
                records.append(rec)
        assert torch.equal(engine.tokens, tokens_o), f'tokens differ after step {step}'
    assert finished == slots_n
    # The windows are not trivial: a fifth to a half of each is deferred, the rest committed over >= 20 steps.
    lasts = [r['last_count'] for r in records]
    print(f'[gpu-case] block={block} commits={commits} last_counts={lasts} actual={[r["actual"] for r in records]}',
          flush=True)
    assert all(0.15 * N < c < 0.5 * N for c in lasts), lasts
    assert all(r['actual'] >= 20 for r in records)
    assert commits == sum(r['actual'] for r in records)
    assert all(p.idle for p in prod)
    assert int((engine.tokens == CLASSES).sum()) == 0      # every voxel filled (air for the deferred ones)


def test_eager_consume_equals_staged_graph_path(dev):
    """The per-slot `consume` (eager select) and the graph-staged batch give the same window, and `time()`
    follows the committed fraction."""
    from streamvoxel_amd.stream.slot import LowEntropyLastSlot, SelectGraphs, consume_batch
    _case('slot eager vs staged, block=4, 2 slots')
    engine = _Engine(2, dev)
    eager = LowEntropyLastSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, EPS, 4, dev)
    staged = [LowEntropyLastSlot(SHAPE, CLASSES, AIR, AIR_TOKEN, EPS, 4, dev) for _ in range(2)]
    graphs = SelectGraphs(engine, staged)
    eager.arm(seed=5, cap=CAP, target=(0, 0, 0))
    staged[0].arm(seed=5, cap=CAP, target=(0, 0, 0))
    tok_e = torch.full(SHAPE, CLASSES, dtype=torch.int64, device=dev)
    out = engine.outputs[2]
    times = [eager.time()]
    rec_e = rec_s = None
    for step in range(CAP + 1):
        out[0].copy_(marking_logits(3, dev) if step == 0 else solid_logits(50 + step, step, CAP + 1, dev))
        r_e, c_e = eager.consume(out[0], tok_e)
        got = consume_batch(staged, out, engine.tokens, 2, graphs)
        r_s, c_s = got.get(0, (None, None))
        _compare_commit(c_e, c_s, f'step={step}')
        rec_e = rec_e or r_e
        rec_s = rec_s or r_s
        if not eager.idle:
            times.append(eager.time())
        assert 1 not in got                                  # the second slot is idle
    _compare_record(rec_e, rec_s, 'finish')
    assert torch.equal(tok_e, engine.tokens[0])
    assert eager.idle and eager.time() == 1.0
    assert all(a > b for a, b in zip(times[1:], times[2:]))  # model time falls as voxels are committed
