"""Oracle restatement of the class head's output order (test infrastructure only, see oracle/__init__.py).

`to_class_major`: the reshape / permute that turns the head's patches [n, GY*GZ*GX, p^3*C] into logits
[n, C, Y, Z, X] (stream/fast_ops.py:305-308, models/unconditional_md4.py:126-129), written as explicit loops over
patches and in-patch offsets, so that it pins the product's row map independently of torch's permute.
"""
from __future__ import annotations

import numpy as np


def to_class_major(patches, voxel_shape, p, classes):
    """patches (numpy [n, P, p^3*C]) -> numpy [n, C, Y, Z, X]."""
    Y, Z, X = voxel_shape
    GY, GZ, GX = Y // p, Z // p, X // p
    n = patches.shape[0]
    out = np.empty((n, classes, Y, Z, X), dtype=patches.dtype)
    for gy in range(GY):
        for gz in range(GZ):
            for gx in range(GX):
                patch = (gy * GZ + gz) * GX + gx
                for py in range(p):
                    for pz in range(p):
                        for px in range(p):
                            off = (py * p + pz) * p + px
                            out[:, :, gy * p + py, gz * p + pz, gx * p + px] = \
                                patches[:, patch, off * classes:(off + 1) * classes]
    return out
