"""streamvoxel_amd.stream.fast_ops exports the reference's names on this path (stream/fast_ops.py) and refuses
host tensors: there is no CPU fallback."""
import pytest
import torch

from streamvoxel_amd.stream import fast_ops


def test_reference_names_exported():
    want = {'local_kv', 'cross_query', 'cross_flex', 'cross_sdpa', 'entropy_torch', 'entropy_triton',
            'top_mask_nosync', 'quota_select_nosync', 'FastLowEntropyLastSlot', 'SelectGraphs', 'consume_batch',
            'FastSlotForward', 'RECOMMENDED'}
    assert want == set(fast_ops.__all__)
    assert all(callable(getattr(fast_ops, name)) for name in want - {'RECOMMENDED'})


def test_host_tensors_are_refused():
    with pytest.raises((RuntimeError, ValueError, TypeError)):
        fast_ops.entropy_triton(torch.zeros(4, 8))
    with pytest.raises((RuntimeError, ValueError, TypeError)):
        fast_ops.top_mask_nosync(torch.zeros(8), torch.ones(8, dtype=torch.bool), 3)


# The option sets the reference's own callers pass: FastSlotForward(**CONFIGS[...]) (scripts/bench_ops.py:201-206)
# and FastLowEntropyLastSlot(..., entropy=) (fast_ops.py:491-496, bench_ops.py:359-371).
REFERENCE_ENGINE_CONFIGS = [
    dict(patchify='conv', attention='sdpa', compile=False),
    dict(patchify='conv', attention='flex', compile=False),
    dict(patchify='gather', attention='sdpa', compile=False),
    dict(patchify='gather', attention='flex', compile=False),
    dict(patchify='gather', attention='flex', compile=True),
]


@pytest.mark.parametrize('config', REFERENCE_ENGINE_CONFIGS)
def test_engine_accepts_every_reference_option_set(config):
    """Every option set passes validation; constructing on the host then stops only at the device check (the engine
    has no CPU path), never at an option."""
    from streamvoxel_amd.stream.engine import SlotEngine, check_engine_options
    check_engine_options(**config)
    with pytest.raises(RuntimeError, match='no CPU path'):
        fast_ops.FastSlotForward(None, None, 'cpu', 8, 8, 256, **config)
    assert fast_ops.FastSlotForward is SlotEngine


@pytest.mark.parametrize('bad', [dict(patchify='onehot'), dict(attention='triton'), dict(compile='max'),
                                 dict(kv_dtype='fp16')])
def test_engine_refuses_unknown_options(bad):
    with pytest.raises(ValueError):
        fast_ops.FastSlotForward(None, None, 'cpu', 8, 8, 256, **bad)


@pytest.mark.parametrize('entropy', ['torch', 'triton', 'hip'])
def test_slot_accepts_the_reference_entropy_names(entropy):
    from streamvoxel_amd.stream.slot import check_slot_options
    check_slot_options(entropy, 'multinomial')
    with pytest.raises(RuntimeError, match='no CPU path'):
        fast_ops.FastLowEntropyLastSlot((64, 16, 16), 40, (0,), air_token=0, last_eps=1e-4, block_size=4,
                                        device='cpu', entropy=entropy)


def test_slot_refuses_unknown_options():
    with pytest.raises(ValueError):
        fast_ops.FastLowEntropyLastSlot((64, 16, 16), 40, (0,), 0, 1e-4, 4, 'cpu', entropy='numpy')
    with pytest.raises(ValueError):
        fast_ops.FastLowEntropyLastSlot((64, 16, 16), 40, (0,), 0, 1e-4, 4, 'cpu', sampler='gumbel')
