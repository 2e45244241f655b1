"""Negative Shannon entropy per voxel on the GPU (mirror of streamvoxel/sampling/entropy.py:1-4)."""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.stream.patches import PatchLogits


def _as_kernel_input(logits):
    if logits.dtype in (torch.float32, torch.bfloat16):
        return logits
    # fp16 / fp64 logits are promoted on the device (the reference also computes in fp32).
    return logits.float()


def entropy_scores(logits):
    """sum_c p_c log p_c over axis 0 (nats, fp32 arithmetic). logits [C, ...] on the GPU -> fp32 [...]; a
    PatchLogits (the class head's output in place) -> fp32 [n, Y, Z, X]."""
    if isinstance(logits, PatchLogits):
        return _patch_stats(logits, None)
    _lib.require_gpu(logits)
    classes = logits.shape[0]
    x = _as_kernel_input(logits).reshape(classes, -1)
    n = x.shape[1]
    out = torch.empty(n, device=logits.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.svhip_entropy(_lib.ptr(x), _lib.dtype_code(x.dtype), 1, classes, n, 0, x.stride(0), x.stride(1),
                                 _lib.ptr(out), _lib.stream_of(x)), 'svhip_entropy')
    return out.reshape(logits.shape[1:])


def entropy_batched(logits, layout='class_major', out=None):
    """Scores for a batch of windows in one launch.

    layout 'class_major': logits [B, C, *spatial] (the class head's output); 'voxel_major': logits [B, N, C] or
    [B * N, C] together with out [B, N]. Returns fp32 [B, N]."""
    _lib.require_gpu(logits)
    x = _as_kernel_input(logits)
    if layout == 'class_major':
        B, C = x.shape[0], x.shape[1]
        x = x.reshape(B, C, -1)
        n = x.shape[2]
        sb, sc, sn = x.stride(0), x.stride(1), x.stride(2)
    elif layout == 'voxel_major':
        if x.dim() == 2:
            if out is None:
                raise ValueError('voxel_major [B*N, C] logits need `out` [B, N] to give the batch split')
            B, n = out.shape
            C = x.shape[1]
            x3 = x.reshape(B, n, C)
        else:
            x3 = x
            B, n, C = x3.shape
        sb, sn, sc = x3.stride(0), x3.stride(1), x3.stride(2)
        x = x3
    else:
        raise ValueError(layout)
    if out is None:
        out = torch.empty((B, n), device=logits.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.svhip_entropy(_lib.ptr(x), _lib.dtype_code(x.dtype), B, C, n, sb, sc, sn, _lib.ptr(out),
                                 _lib.stream_of(x)), 'svhip_entropy')
    return out


def _patch_stats(logits, air_index):
    rows = logits.rows
    _lib.require_gpu(rows)
    Y, Z, X = logits.shape
    n = len(logits)
    out = torch.empty((n, Y, Z, X), device=rows.device, dtype=torch.float32)
    lib = _lib.load()
    if air_index is None:
        _lib.check(lib.svhip_entropy_patches(_lib.ptr(rows), _lib.dtype_code(rows.dtype), n, logits.classes, Y, Z, X,
                                             logits.patch, rows.stride(0), rows.stride(1), _lib.ptr(out),
                                             _lib.stream_of(rows)), 'svhip_entropy_patches')
    else:
        _lib.check(lib.svhip_air_prob_patches(_lib.ptr(rows), _lib.dtype_code(rows.dtype), n, logits.classes, Y, Z,
                                              X, logits.patch, rows.stride(0), rows.stride(1), _lib.ptr(air_index),
                                              int(air_index.numel()), _lib.ptr(out), _lib.stream_of(rows)),
                   'svhip_air_prob_patches')
    return out


def air_prob(logits, air_ids, air_index=None):
    """sum over the air classes of softmax(logits, 0) (stream/slot.py:126). logits [C, ...] -> fp32 [...]; a
    PatchLogits -> fp32 [n, Y, Z, X]. `air_index` may carry the ids as a device int32 tensor (graph capture needs
    a fixed buffer)."""
    if isinstance(logits, PatchLogits):
        if air_index is None:
            air_index = torch.as_tensor(list(air_ids), dtype=torch.int32, device=logits.device)
        return _patch_stats(logits, air_index)
    _lib.require_gpu(logits)
    classes = logits.shape[0]
    x = _as_kernel_input(logits).reshape(classes, -1)
    n = x.shape[1]
    if air_index is None:
        air_index = torch.as_tensor(list(air_ids), dtype=torch.int32, device=logits.device)
    out = torch.empty(n, device=logits.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.svhip_air_prob(_lib.ptr(x), _lib.dtype_code(x.dtype), 1, classes, n, 0, x.stride(0), x.stride(1),
                                  _lib.ptr(air_index), int(air_index.numel()), _lib.ptr(out), _lib.stream_of(x)),
               'svhip_air_prob')
    return out.reshape(logits.shape[1:])
