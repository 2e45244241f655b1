"""Host side of reading the class head's output in place (streamvoxel_amd/stream/patches.py): the row map and the
reference's permute, against the loop restatement in oracle/patches.py and the 4^3 block order."""
import numpy as np
import pytest
import torch

from oracle import patches as OP
from oracle import sampling as S
from streamvoxel_amd.stream.patches import PatchLogits


@pytest.mark.parametrize('shape,p', [((16, 8, 8), 4), ((8, 4, 16), 2), ((4, 4, 4), 4), ((8, 8, 8), 1)])
def test_class_major_matches_loop_restatement(shape, p):
    Y, Z, X = shape
    C, n = 3, 2
    P = (Y // p) * (Z // p) * (X // p)
    patches = torch.arange(n * P * p ** 3 * C, dtype=torch.float32).reshape(n, P, p ** 3 * C)
    logits = PatchLogits(patches, shape, p, C)
    want = OP.to_class_major(patches.numpy(), shape, p, C)
    assert np.array_equal(logits.class_major().numpy(), want)
    # row_index: voxel (y, z, x) of window b reads rows[b, row_index(flat)].
    flat = torch.arange(Y * Z * X)
    rows = logits.row_index(flat)
    assert sorted(rows.tolist()) == list(range(Y * Z * X))
    got = logits.rows[1][rows].t().reshape(C, Y, Z, X)
    assert np.array_equal(got.numpy(), want[1])
    assert torch.equal(logits.gather(flat[::7], window=1), logits.rows[1][rows[::7]])


def test_patch_order_is_the_block_order_at_block_size_p():
    """With p = b the rows of patch j are block j of block_view (in-block order (dy, dz, dx))."""
    shape, p = (16, 8, 8), 4
    n_vox = 16 * 8 * 8
    logits = PatchLogits(torch.zeros(1, n_vox // 64, 64), shape, p, 1)
    rows = logits.row_index(torch.arange(n_vox)).numpy().reshape(shape)
    assert np.array_equal(S.block_view(rows, p), np.arange(n_vox).reshape(-1, 64))


def test_window_views_and_validation():
    shape, p, C = (8, 4, 4), 2, 5
    patches = torch.randn(3, 16, 8 * C)
    logits = PatchLogits(patches, shape, p, C)
    assert len(logits) == 3 and logits[2].rows.shape == (1, 128, C)
    assert logits[-1].data_ptr() == patches[2].data_ptr()
    with pytest.raises(ValueError):
        PatchLogits(patches, (8, 4, 6), p, C)            # not a power of two
    with pytest.raises(ValueError):
        PatchLogits(patches, shape, 4, C)                # patch > Z
    with pytest.raises(ValueError):
        PatchLogits(patches, shape, p, C + 1)            # row width
    with pytest.raises(TypeError):
        PatchLogits(patches.double(), shape, p, C)
    with pytest.raises(TypeError):
        logits[0:1]
