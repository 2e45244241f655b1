"""Host logic of the slot engine: condition widths and capacities, batch buckets, option checking, the drop-in
names; no GPU."""
import pytest
import torch


class _Spec:
    def __init__(self, height, tile, num_classes=3, y_origin=-64.0):
        self.height, self.tile, self.num_classes, self.y_origin = height, tile, num_classes, y_origin


class _Model:
    def __init__(self, halo, patch):
        self.biome_halo, self.biome_patch = halo, patch


def test_condition_widths():
    from streamvoxel_amd.stream.engine import condition_widths
    # the reference's tiny live-test model (16^3 windows, halo 4, biome patch 2): its packed lengths are
    # 2 + 64 + 18 for one L1 tile and two L2 tiles (tests/stream/test_live_fast_ops.py:147)
    assert condition_widths(_Model(4, 2), _Spec(16, 16)) == (64, 1, 18)
    # the shipped model (256 x 16 x 16, halo 4, patch 2): 8 L1 tiles + 256 L2 tiles + biome = 12 576 keys
    l1, l2, biome = condition_widths(_Model(4, 2), _Spec(256, 16))
    assert (l1, l2, biome) == (1024, 16, 288) and 8 * l1 + 256 * l2 + biome == 12576
    assert condition_widths(_Model(16, 1), _Spec(256, 16))[2] == 64 * 144
    assert condition_widths(_Model(16, 4), _Spec(256, 16))[2] == 16 * 9
    assert condition_widths(_Model(4, 4), _Spec(256, 16))[2] == 16 * 4


def test_buckets():
    from streamvoxel_amd.stream.engine import buckets
    assert buckets(1) == [1]
    assert buckets(8) == [1, 2, 4, 8]
    assert buckets(6) == [1, 2, 4, 6]
    assert buckets(64) == [1, 2, 4, 8, 16, 32, 64]


def test_engine_options_and_device_checked_before_any_work():
    from streamvoxel_amd.stream.engine import SlotEngine
    spec = _Spec(16, 16)
    with pytest.raises(ValueError):
        SlotEngine(None, spec, 'cuda', 2, 1, 1, patchify='onehot')
    with pytest.raises(ValueError):
        SlotEngine(None, spec, 'cuda', 2, 1, 1, attention='math')
    with pytest.raises(ValueError):
        SlotEngine(None, spec, 'cuda', 2, 1, 1, compile='max-autotune')
    with pytest.raises(RuntimeError, match='no CPU path'):
        SlotEngine(None, spec, 'cpu', 2, 1, 1)


def test_drop_in_names():
    from streamvoxel_amd.stream import fast_ops
    from streamvoxel_amd.stream.engine import SlotEngine
    assert fast_ops.FastSlotForward is SlotEngine
    assert fast_ops.RECOMMENDED == dict(patchify='gather', attention='flex', compile='emulate')
    for name in ('load_slot', 'wait_loads', 'clear_tokens', 'bucket', 'replay', 'eager', 'numerical_gate'):
        assert callable(getattr(SlotEngine, name))
    for name in ('graphs', 'outputs', 'packed', 'graph_ok'):
        assert isinstance(getattr(SlotEngine, name), property)


def test_synthetic_condition_layout():
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.engine import Encoded
    model = synth.StepModel(classes=8, voxel_shape=(64, 16, 16), width=96, depth=2, heads=4, control_width=48,
                            control_depth=1)
    c = synth.condition(model, 5, 7, seed=0, device='cpu')
    assert isinstance(c, Encoded) and len(c.prefix) == 1
    assert c.prefix[0][0].shape == (4, 5, 12) and c.prefix[0][0].dtype == torch.bfloat16
    assert c.local.shape == (1, 7, 48) and c.positions.shape == (1, 7, 3)


def test_default_encoder_is_the_reference_packages_encode_item(monkeypatch):
    """A worker constructs the engine without an encoder (worker.py:272): for a model with `encode_group` the engine
    takes the reference package's `encode_item` when that package is importable (here a stand-in module), and
    wraps its (prefix, local, positions) as an Encoded; a model without `encode_group`, or no package, gives None."""
    import sys
    import types
    from streamvoxel_amd.stream.engine import Encoded, default_encoder

    calls = []

    def encode_item(model, item, spec, device):
        calls.append((model, item, spec, device))
        return ['prefix'], 'local', 'positions'

    class RefModel:
        def encode_group(self, group):
            return group

    pkg, sub, mod = types.ModuleType('streamvoxel'), types.ModuleType('streamvoxel.stream'), \
        types.ModuleType('streamvoxel.stream.engine')
    mod.encode_item = encode_item
    monkeypatch.setitem(sys.modules, 'streamvoxel', pkg)
    monkeypatch.setitem(sys.modules, 'streamvoxel.stream', sub)
    monkeypatch.setitem(sys.modules, 'streamvoxel.stream.engine', mod)
    model, spec = RefModel(), object()
    enc = default_encoder(model, spec, 'cuda:0')
    out = enc('item')
    assert isinstance(out, Encoded) and out.prefix == ['prefix'] and out.local == 'local'
    assert calls == [(model, 'item', spec, 'cuda:0')]
    assert default_encoder(object(), spec, 'cuda:0') is None          # not a reference model
    monkeypatch.setitem(sys.modules, 'streamvoxel.stream.engine', None)  # the package is not importable
    assert default_encoder(model, spec, 'cuda:0') is None


def test_deferred_commit_runs_its_host_work_once_on_first_read():
    """A batched solid step's commit: nothing is written to the slot's maps until it is read or settled; then the
    positions are the drawn voxels in ascending flat order, the values their classes, the maps updated at those
    voxels only, and the slot's pending reference cleared. A drawn count that misses the quota raises then."""
    import types

    import numpy as np

    from streamvoxel_amd.stream.slot import DeferredCommit
    shape = (2, 4, 4)
    slot = types.SimpleNamespace(_step_map=torch.zeros(shape, dtype=torch.int16),
                                 _values=torch.full(shape, -1, dtype=torch.int16), _pending=None)
    drawn = np.full(32, -1, np.int16)
    drawn[[3, 7, 8, 30]] = [5, 0, 17, 2]
    commit = DeferredCommit(slot, drawn, 4, 6)
    slot._pending = commit
    assert int((slot._step_map != 0).sum()) == 0 and int((slot._values != -1).sum()) == 0
    assert commit['step'] == 6
    assert slot._pending is None
    assert np.array_equal(commit['positions'], [3, 7, 8, 30]) and commit['positions'].dtype == np.int32
    assert np.array_equal(commit['values'], [5, 0, 17, 2])
    copied = dict(commit, target=(1, 0))                   # the reference worker's progressive record
    assert sorted(copied) == ['positions', 'step', 'target', 'values']
    assert copied['positions'] is commit['positions'] and copied['values'] is commit['values']
    assert sorted(commit) == ['positions', 'step', 'values'] and len(commit) == 3
    assert np.array_equal(np.flatnonzero(slot._step_map.numpy().reshape(-1)), [3, 7, 8, 30])
    assert set(slot._step_map.numpy().reshape(-1)[[3, 7, 8, 30]]) == {6}
    assert np.array_equal(slot._values.numpy().reshape(-1)[[3, 7, 8, 30]], [5, 0, 17, 2])
    drawn[0] = 1                                            # the row is no longer read once materialised
    assert np.array_equal(commit['positions'], [3, 7, 8, 30])
    short = DeferredCommit(slot, np.full(32, -1, np.int16), 2, 7)
    with pytest.raises(AssertionError, match='0 voxels drawn for a quota of 2'):
        short.materialize()
