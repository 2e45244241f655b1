"""The slot engine (`SlotEngine`, the reference's `FastSlotForward` surface) on the GPU: slot loads into the cache,
the captured step against the float64 oracle step over the engine's own cache, one graph per bucket equal to the
eager step bit for bit, the numerical gate, and whole windows driven the way the reference's worker drives them
(`replay(timesteps, count)` + `SelectGraphs` + `consume_batch`) equal to the eager path (`eager` + per-slot
`consume`) commit for commit."""
import numpy as np
import pytest
import torch

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


def _model(dev, **kw):
    from streamvoxel_amd import synth
    model = synth.StepModel(**kw)
    for p in model.parameters():
        p.data = p.data.to(torch.bfloat16)
    return model.to(dev)


SMALL = dict(classes=40, voxel_shape=(64, 16, 16), width=192, depth=4, heads=8, control_width=192, control_depth=2,
             seed=3)


def _small_engine(dev, batch=5, capture=True):
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.engine import SlotEngine
    model = _model(dev, **SMALL)
    spec = synth.WindowSpec(height=64, tile=16, num_classes=40)
    return model, spec, SlotEngine(model, spec, dev, batch, l1_cap=2, l2_cap=8, capture=capture)


def test_engine_layout_and_loads(dev):
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.producer import axial_rope
    _case('engine small: capacity, lengths, cache rows after load_slot')
    model, spec, engine = _small_engine(dev, capture=False)
    # l1 = 16 x 16, l2 = 4, biome (halo 4, patch 2) = 8 x 3 x 3; caps 2 / 8
    assert (engine.l1_tokens, engine.l2_tokens, engine.biome_tokens) == (256, 4, 72)
    assert (engine.prefix_len, engine.local_len) == (32, 584)
    assert engine.context.kv_cap == 640 and engine.sizes == [1, 2, 4, 5]
    sizes = [(32, 584), (0, 72), (5, 300), (32, 0), (17, 1)]
    conds = [synth.condition(model, P, L, seed=40 + i, device=dev) for i, (P, L) in enumerate(sizes)]
    for i, c in enumerate(conds):
        engine.load_slot(i, c)
    engine.wait_loads()
    torch.cuda.synchronize()
    assert engine.packed.lengths.tolist() == [P + L for P, L in sizes]
    assert bool((engine.tokens == spec.num_classes).all())
    for j, cross in enumerate(model.cross):
        H, D = cross.heads, cross.width // cross.heads
        for i, ((P, L), c) in enumerate(zip(sizes, conds)):
            k = engine.context.k[j][i]                     # [H, Kcap, D]
            vt = engine.context.vt[j][i]                   # [H, D, Kcap]
            assert torch.equal(k[:, :P], c.prefix[j][0]) and torch.equal(vt[:, :, :P].transpose(1, 2), c.prefix[j][1])
            assert not bool(k[:, P + L:].any()) and not bool(vt[:, :, P + L:].any())
            if L == 0:
                continue
            with torch.autocast('cuda', dtype=torch.bfloat16):
                kv = cross.key_value(c.local[0]).to(torch.bfloat16).view(L, 2, H, D)
            lk = axial_rope(kv[:, 0].transpose(0, 1)[None].contiguous(), c.positions.float(),
                            cross.rope.frequencies.float())[0]
            assert torch.equal(k[:, P:P + L], lk)
            assert torch.equal(vt[:, :, P:P + L].transpose(1, 2), kv[:, 1].transpose(0, 1))
    with pytest.raises(ValueError):
        engine.load_slot(0, synth.condition(model, 33, 10, seed=1, device=dev))
    with pytest.raises(IndexError):
        engine.load_slot(5, conds[0])


def test_engine_replay_against_oracle(dev):
    """The engine's captured step over slots it loaded itself (the prefix keys, and the local keys it projected and
    rotated) against the float64 oracle step over the cache it wrote: the engine's numbers pinned to the oracle, not
    only to its own eager path. Tolerances as the step forward's (tests/test_gpu_forward.py): the class-head rows
    within 4e-2 of max |reference| (max-abs) and 1e-2 of mean |reference| (mean-abs)."""
    from oracle import backbone as O
    from streamvoxel_amd import synth
    _case('engine small: replay against the float64 oracle step over the engine\'s own cache')
    model, spec, engine = _small_engine(dev, batch=2)
    sizes = [(32, 300), (5, 61)]
    for i, (P, L) in enumerate(sizes):
        engine.load_slot(i, synth.condition(model, P, L, seed=70 + i, device=dev))
    engine.wait_loads()
    g = torch.Generator().manual_seed(12)
    tokens = torch.randint(0, spec.num_classes + 1, tuple(engine.tokens.shape), generator=g)
    engine.tokens.copy_(tokens.to(dev))
    times = [0.35, 0.8]
    got = engine.replay(times).patches.float().cpu().double()
    torch.cuda.synchronize()
    keys = [engine.context.k[j].cpu() for j in range(len(model.cross))]
    values = [engine.context.vt[j].cpu().transpose(2, 3) for j in range(len(model.cross))]
    params = {k: v.cpu() for k, v in model.state_dict().items()}
    ref = O.step_forward(params, tokens, torch.tensor(times), engine.origin.cpu(), engine.group_origin.cpu(), keys,
                         values, [P + L for P, L in sizes], depth=SMALL['depth'], heads=SMALL['heads'],
                         control_heads=int(model.cross[0].heads), layer_map=model.layer_map, patch=4,
                         y_range=model.backbone.y_range, time_dim=model.backbone.time_dim,
                         voxel_shape=SMALL['voxel_shape'])
    err = (got - ref).abs()
    assert float(err.max()) <= 4e-2 * float(ref.abs().max()), (float(err.max()), float(ref.abs().max()))
    assert float(err.mean()) <= 1e-2 * float(ref.abs().mean()), (float(err.mean()), float(ref.abs().mean()))


def test_engine_bucket_graphs_equal_eager(dev):
    from streamvoxel_amd import synth
    _case('engine small: replay(t, count) per bucket == eager forward, twice')
    model, spec, engine = _small_engine(dev)
    assert engine.graph_ok and sorted(engine.graphs) == [1, 2, 4, 5] and engine.graph is engine.graphs[5]
    for i in range(engine.batch):
        engine.load_slot(i, synth.condition(model, 8 * i, 100 + 90 * i, seed=i, device=dev))
    engine.wait_loads()
    g = torch.Generator(device=dev).manual_seed(9)
    engine.tokens.copy_(torch.randint(0, spec.num_classes + 1, engine.tokens.shape, device=dev, generator=g))
    times = [0.9, 0.5, 0.3, 0.7, 1.0]
    for count in (1, 2, 3, 4, 5):
        size = engine.bucket(count)
        got = engine.replay(times, count)
        assert len(got) == size
        first = got.class_major().clone()
        again = engine.replay(times, count).class_major()
        want = engine.forward(size).class_major()
        assert torch.equal(first, again), count
        assert torch.equal(first, want), count
        assert torch.isfinite(first.float()).all()
    # the full batch: replay == eager
    full = engine.replay(times).class_major().clone()
    assert torch.equal(full, engine.eager(times).class_major())
    # one timestep for all slots
    assert torch.equal(engine.replay(0.5).class_major(), engine.eager([0.5] * 5).class_major())


def test_engine_numerical_gate(dev):
    from streamvoxel_amd import synth
    _case('engine small: numerical_gate')
    model, spec, engine = _small_engine(dev, batch=4)
    item = synth.condition(model, 32, 584, seed=11, device=dev)
    other = synth.condition(model, 12, 200, seed=12, device=dev)
    report = engine.numerical_gate(item, other)
    for key in ('graph_equal', 'graph_used', 'padded_close', 'bucket_close', 'bucket_match', 'buckets', 'max_abs',
                'mean_abs', 'argmax_match', 'batch', 'prefix_len', 'local_len', 'options'):
        assert key in report, key
    assert report['graph_used'] and report['graph_equal'], report
    assert report['padded_close'] and report['bucket_close'], report
    assert report['buckets'] == [1, 2, 4] and report['reference'] == 'one_slot_exact_cache'
    assert engine.packed.lengths.tolist()[:2] == [32 + 584, 12 + 200]



@pytest.mark.parametrize('config', [dict(patchify='conv', attention='sdpa', compile=False),
                                    dict(patchify='conv', attention='flex', compile=False),
                                    dict(patchify='gather', attention='sdpa', compile=False),
                                    dict(patchify='gather', attention='flex', compile=True)])
def test_engine_reference_option_sets_give_the_default_forward(dev, config):
    """The reference's FastSlotForward option sets (scripts/bench_ops.py:201-206) construct on the GPU and give the
    default engine's forward bit for bit: 'conv' and 'gather' are one sum (the gather kernel), 'sdpa' and 'flex' one
    masked attention over the valid keys (the attention kernel)."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.engine import SlotEngine
    _case(f'engine small: options {config}')
    model = _model(dev, **SMALL)
    spec = synth.WindowSpec(height=64, tile=16, num_classes=40)
    engines = [SlotEngine(model, spec, dev, 2, l1_cap=2, l2_cap=8, capture=False),
               SlotEngine(model, spec, dev, 2, l1_cap=2, l2_cap=8, capture=False, **config)]
    g = torch.Generator(device=dev).manual_seed(4)
    tokens = torch.randint(0, spec.num_classes + 1, engines[0].tokens.shape, device=dev, generator=g)
    outs = []
    for engine in engines:
        for i in range(2):
            engine.load_slot(i, synth.condition(model, 10 * i, 150 + 60 * i, seed=20 + i, device=dev))
        engine.wait_loads()
        engine.tokens.copy_(tokens)
        outs.append(engine.eager([0.8, 0.4]).class_major().clone())
    assert engines[1].options['patchify'] == config['patchify']
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize('entropy', ['torch', 'triton'])
def test_slot_reference_entropy_names_select_like_hip(dev, entropy):
    """FastLowEntropyLastSlot(..., entropy='torch' | 'triton') (fast_ops.py:491-496) runs the HIP entropy kernel: the
    marking forward and two solid steps commit exactly what entropy='hip' commits on the same logits."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.slot import FastLowEntropyLastSlot
    _case(f'slot entropy={entropy}')
    shape, classes = (64, 16, 16), 40
    N = 64 * 16 * 16
    runs = []
    for name in ('hip', entropy):
        slot = FastLowEntropyLastSlot(shape, classes, (0,), 0, 1e-4, 4, dev, entropy=name)
        slot.arm(77, 10, (0, 0))
        tokens = torch.full(shape, classes, dtype=torch.int64, device=dev)
        commits = []
        for step in range(3):
            logits = synth.bimodal_logits(N, classes, 0.7, seed=50 + step, device=dev).t().reshape(classes, *shape)
            commits.append(slot.consume(logits, tokens)[1])
        runs.append((commits, tokens.clone()))
    (c_a, t_a), (c_b, t_b) = runs
    assert torch.equal(t_a, t_b) and c_a[0] is None and c_b[0] is None
    for x, y in zip(c_a[1:], c_b[1:]):
        assert np.array_equal(x['positions'], y['positions']) and np.array_equal(x['values'], y['values'])

def _drive(engine, slots, seeds, cap, staged):
    """The worker's loop (streamvoxel/stream/worker.py:378-397): arm every slot, then forward / consume until all
    windows finish. staged: graph replays + SelectGraphs + consume_batch; else eager forwards + per-slot consume."""
    from streamvoxel_amd.stream.slot import SelectGraphs, consume_batch
    select = SelectGraphs(engine, slots) if staged else None
    for i, slot in enumerate(slots):
        slot.arm(seeds[i], cap, (i, 0))
    engine.clear_tokens()
    commits = {i: [] for i in range(len(slots))}
    records = {}
    forwards = 0
    while any(not s.idle for s in slots):
        count = 1 + max(i for i, s in enumerate(slots) if not s.idle)
        times = [s.time(engine.tokens[i]) if i < count else 1.0 for i, s in enumerate(slots)]
        if staged:
            logits = engine.replay(times, count)
            results = consume_batch(slots, logits, engine.tokens, count, select)
        else:
            logits = engine.eager(times)
            results = {i: slots[i].consume(logits[i], engine.tokens[i]) for i in range(count) if not slots[i].idle}
        forwards += 1
        for i, (finished, commit) in results.items():
            if commit is not None:
                commits[i].append(commit)
            if finished is not None:
                records[i] = finished
        assert forwards <= cap + 2
    return commits, records, engine.tokens.clone(), forwards


@pytest.mark.parametrize('sampler', ['multinomial', 'philox'])
def test_engine_whole_window_staged_equals_eager_shipped_shape(dev, sampler):
    """8 slots of the shipped model's shape (304 classes, 256 x 16 x 16, 25 x 768 backbone, 13 x 384 control) with
    full-capacity-class conditions; 26 forwards per window (marking + 25 solid steps). With the reference's
    multinomial tail the staged path runs one captured selection per slot; with the counter-based sampler
    SelectGraphs keeps the slots in one PhiloxBatch and a forward selects and samples all 8 windows in one graph."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.engine import SlotEngine
    from streamvoxel_amd.stream.slot import LowEntropyLastSlot
    _case(f'engine shipped shape: whole window staged vs eager, sampler={sampler}')
    model = _model(dev, seed=1)
    spec = synth.WindowSpec()
    engine = SlotEngine(model, spec, dev, 8, l1_cap=8, l2_cap=256)
    assert engine.graph_ok
    g = torch.Generator().manual_seed(5)
    for i in range(8):
        P = int(torch.randint(0, 4097, (1,), generator=g))
        L = 288 + 1024 * int(torch.randint(0, 9, (1,), generator=g))
        engine.load_slot(i, synth.condition(model, P, L, seed=100 + i, device=dev, scale=0.3))
    engine.wait_loads()
    cap = 25
    seeds = [1000 + 7 * i for i in range(8)]
    runs = []
    for staged in (True, False):
        slots = [LowEntropyLastSlot(engine.shape, spec.num_classes, (0,), air_token=0, last_eps=1e-4, block_size=4,
                                    device=dev, sampler=sampler) for _ in range(8)]
        runs.append(_drive(engine, slots, seeds, cap, staged))
        if staged:
            from streamvoxel_amd.stream.slot import PhiloxBatch
            assert PhiloxBatch.fits(slots, engine.tokens) == (sampler == 'philox')
    (c_a, r_a, t_a, f_a), (c_b, r_b, t_b, f_b) = runs
    assert f_a == f_b == cap + 1
    assert torch.equal(t_a, t_b)
    assert not bool((t_a == spec.num_classes).any())              # every voxel committed or deferred to air
    for i in range(8):
        assert r_a[i]['nfe'] == r_b[i]['nfe'] == cap + 1
        assert torch.equal(r_a[i]['values'], r_b[i]['values'])
        assert torch.equal(r_a[i]['step_map'], r_b[i]['step_map'])
        assert len(c_a[i]) == len(c_b[i]) == cap
        for x, y in zip(c_a[i], c_b[i]):
            assert x['step'] == y['step']
            assert np.array_equal(x['positions'], y['positions']) and np.array_equal(x['values'], y['values'])
        total = sum(len(x['positions']) for x in c_a[i]) + r_a[i]['last_count']
        assert total == 256 * 16 * 16
