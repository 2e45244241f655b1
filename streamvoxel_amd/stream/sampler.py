"""Counter-based sampling of a solid step's chosen voxels (`svhip_sample_chosen`), a fixed-size form of the tail.

The reference's tail after the selection (stream/fast_ops.py:548-553) runs `nonzero_static(size=k)`, a gather of
the k rows, `softmax`, `torch.multinomial` on the slot's generator and `index_copy_`: its sizes follow the step's k
and its draws the generator's position, so it stays outside the captured selection. `sample_chosen` draws voxel v
of step `step` of the window seeded `seed` from its own Philox4x64-10 counter (v, step) and inverts the row's
softmax CDF, in one launch over the whole window that reads the `chosen` mask where the selection left it. The
selection and this tail then replay as one graph; the host copies back one int16 per voxel.

The draws are a different random stream from `torch.multinomial`'s (same distribution: the categorical of the
row's softmax). `LowEntropyLastSlot(sampler='multinomial')` keeps the reference's stream.
"""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.stream.patches import PatchLogits

__all__ = ['sample_chosen']


def _voxel_strides(logits, shape):
    """(batch stride, class stride, voxel stride) of class-major logits [n, C, Y, Z, X] whose voxels flatten."""
    Y, Z, X = shape
    sn = logits.stride(-1)
    if logits.stride(-2) != X * sn or logits.stride(-3) != Z * X * sn:
        raise ValueError('the voxel axes of the logits must flatten to one strided axis')
    return logits.stride(0), logits.stride(1), sn


def sample_chosen(logits, chosen, seed, step, values, err, tokens=None):
    """Draw the class of every chosen voxel (graph-capturable, no host sync).

    logits: PatchLogits of n windows, or class-major [n, C, Y, Z, X] / [C, Y, Z, X] fp32 or bf16.
    chosen: bool [n, Y, Z, X] (or [Y, Z, X]); values: int16 of the same shape, gets the class of each chosen voxel
    and -1 elsewhere; tokens: int64 of the same shape or None, gets the class of each chosen voxel in place.
    seed, step: device int64 [n]; err: device int32 [1], set non-zero when a chosen row has no finite maximum or
    holds a NaN (the reference's multinomial raises there)."""
    if isinstance(logits, PatchLogits):
        rows = logits.rows
        _lib.require_gpu(rows, chosen, values, seed, step, err, tokens)
        n, shape, classes, patch = len(logits), logits.shape, logits.classes, logits.patch
        x, sb, sc, sn = rows, rows.stride(0), rows.stride(2), rows.stride(1)
    else:
        _lib.require_gpu(logits, chosen, values, seed, step, err, tokens)
        x = logits if logits.dim() == 5 else logits.unsqueeze(0)
        if x.dim() != 5:
            raise ValueError('class-major logits are [n, C, Y, Z, X] or [C, Y, Z, X]')
        n, classes, shape, patch = x.shape[0], x.shape[1], tuple(x.shape[2:]), 0
        sb, sc, sn = _voxel_strides(x, shape)
    Y, Z, X = shape
    for name, t, dtype in (('chosen', chosen, torch.bool), ('values', values, torch.int16),
                           ('tokens', tokens, torch.int64)):
        if t is None:
            continue
        if t.dtype != dtype or t.numel() != n * Y * Z * X or not t.is_contiguous():
            raise ValueError(f'{name} must be a contiguous {dtype} tensor of {n} x {shape} voxels')
    for name, t in (('seed', seed), ('step', step)):
        if t.dtype != torch.int64 or t.numel() != n or not t.is_contiguous():
            raise ValueError(f'{name} must be a contiguous device int64 tensor of {n} entries')
    if err.dtype != torch.int32 or err.numel() < 1:
        raise ValueError('err must be a device int32 tensor')
    lib = _lib.load()
    _lib.check(lib.svhip_sample_chosen(_lib.ptr(x), _lib.dtype_code(x.dtype), classes, patch, sb, sc, sn,
                                       _lib.ptr(chosen.view(torch.uint8)), _lib.ptr(tokens), _lib.ptr(values),
                                       _lib.ptr(seed), _lib.ptr(step), _lib.ptr(err), n, Y, Z, X,
                                       _lib.stream_of(x)), 'svhip_sample_chosen')
    return values
