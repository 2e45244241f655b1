"""The class head's output, read where it lies.

The reference's forward ends with the class head writing `patches` [n, GY*GZ*GX, p^3*C] (one row of C logits per
voxel, patches in (y/p, z/p, x/p) order, the voxels of a patch in (y%p, z%p, x%p) order), then copies it into
[n, C, Y, Z, X]:
    patches.reshape(n, gy, gz, gx, p, p, p, C).permute(0, 7, 1, 4, 2, 5, 3, 6).reshape(n, C, Y, Z, X)
(stream/fast_ops.py:305-308, models/unconditional_md4.py:126-129). `PatchLogits` wraps `patches` with its window
shape and patch size; the selection (`EaseSelect`, the slot classes), the entropy and the air probability read it
in place through the `*_patches` kernels, so the permuted copy is never made. Voxel-indexed results (scores,
chosen, tokens) stay in (y, z, x) order.
"""
from __future__ import annotations

import torch


def _pow2(v):
    return v > 0 and (v & (v - 1)) == 0


class PatchLogits:
    """patches [n, GY*GZ*GX, p^3 * classes] (fp32 or bf16, class axis contiguous) of [Y, Z, X] windows."""

    def __init__(self, patches, voxel_shape, patch_size, classes):
        Y, Z, X = (int(v) for v in voxel_shape)
        p = int(patch_size)
        if patches.dim() != 3:
            raise ValueError(f'patches must be [n, patches, p^3 * classes], got {tuple(patches.shape)}')
        if not all(_pow2(v) for v in (p, Y, Z, X)) or p > min(Y, Z, X):
            raise ValueError(f'patch order needs power-of-two patch and window extents, got {p} and {(Y, Z, X)}')
        n, P, W = patches.shape
        if P != (Y // p) * (Z // p) * (X // p) or W != p ** 3 * classes:
            raise ValueError(f'patches {tuple(patches.shape)} do not hold [{Y},{Z},{X}] windows of {classes} '
                             f'classes in patches of {p}^3')
        if patches.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError('patch logits must be fp32 or bf16')
        self.patches = patches
        self.rows = patches.view(n, P * p ** 3, classes)   # [n, N, C], row r = voxel in patch order
        self.shape = (Y, Z, X)
        self.patch = p
        self.classes = classes

    def __len__(self):
        return self.patches.shape[0]

    def __getitem__(self, i):
        """Window i as a PatchLogits of one window (the slot API's per-window logits)."""
        if not isinstance(i, int):
            raise TypeError('index a PatchLogits with an int window index')
        i = range(len(self))[i]
        return PatchLogits(self.patches[i:i + 1], self.shape, self.patch, self.classes)

    def data_ptr(self):
        return self.patches.data_ptr()

    @property
    def dtype(self):
        return self.patches.dtype

    @property
    def device(self):
        return self.patches.device

    def row_index(self, index):
        """Rows of the (y, z, x)-flat voxel indices `index` (int64 tensor, any device)."""
        _, Z, X = self.shape
        p = self.patch
        y, z, x = index // (Z * X), (index // X) % Z, index % X
        patch = ((y // p) * (Z // p) + z // p) * (X // p) + x // p
        return patch * p ** 3 + ((y % p) * p + z % p) * p + x % p

    def gather(self, index, window=0):
        """[len(index), classes] logits of window `window` at the (y, z, x)-flat voxel indices `index`."""
        return self.rows[window].index_select(0, self.row_index(index))

    def class_major(self):
        """The reference's permuted copy [n, C, Y, Z, X] (fast_ops.py:305-308)."""
        Y, Z, X = self.shape
        p = self.patch
        n = len(self)
        return self.patches.reshape(n, Y // p, Z // p, X // p, p, p, p, self.classes).permute(
            0, 7, 1, 4, 2, 5, 3, 6).reshape(n, self.classes, Y, Z, X)
