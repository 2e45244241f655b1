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
