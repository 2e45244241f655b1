"""Producers of the cross-attention operands on the HIP kernels.

Reference counterparts: AxialRoPE (streamvoxel/models/unconditional_md4.py:10-24), cross_query and local_kv
(streamvoxel/stream/fast_ops.py:90-101), RotaryCrossAttention.encode_kv (streamvoxel/models/streaming_controlnet.py:
31-35), FastSlotForward.encode / _write (streamvoxel/stream/fast_ops.py:228-250). The projections (LayerNorm,
Linear) stay torch modules, as in the reference; the rotation and the cache write are `svhip_axial_rope` and
`svhip_kv_write`.
"""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib


def rope_frequencies(head_dim, base=10000.0, device=None):
    """The AxialRoPE `frequencies` buffer: fp32 base^(-2i / (head_dim / 3)), i < head_dim / 6, computed on the host
    like the module's buffer and then moved to `device`."""
    if head_dim % 6:
        raise ValueError('Each head must allocate an even width to each XYZ axis')
    axis = head_dim // 3
    freq = base ** (-torch.arange(0, axis, 2).float() / axis)
    return freq if device is None else freq.to(device)


def axial_rope(x, positions, frequencies, out=None):
    """AxialRoPE of x [B,H,N,D] bf16 (head_dim contiguous, any other strides) at fp32 positions [B,N,3].
    `out` (optional, may be x) receives the result; returns it."""
    _lib.require_gpu(x, positions, frequencies, out)
    if x.dtype != torch.bfloat16:
        raise TypeError('x must be bfloat16 (the autocast dtype of the reference)')
    B, H, N, D = x.shape
    if positions.shape != (B, N, 3):
        raise ValueError(f'positions must be [B, N, 3], got {tuple(positions.shape)}')
    if frequencies.numel() * 6 != D or frequencies.dtype != torch.float32:
        raise ValueError('frequencies must be the fp32 [head_dim / 6] buffer')
    pos = positions if positions.dtype == torch.float32 and positions.stride(-1) == 1 else positions.float()
    pos = pos if pos.stride(-1) == 1 else pos.contiguous()
    freq = frequencies.contiguous()
    if out is None:
        out = torch.empty_like(x)
    if out.shape != x.shape or out.dtype != torch.bfloat16 or out.stride(-1) != 1 or x.stride(-1) != 1:
        raise ValueError('x and out need a contiguous head_dim')
    lib = _lib.load()
    _lib.check(lib.svhip_axial_rope(_lib.ptr(x), _lib.ptr(out), _lib.ptr(pos), _lib.ptr(freq), B, H, N, D,
                                    x.stride(0), x.stride(1), x.stride(2), out.stride(0), out.stride(1),
                                    out.stride(2), pos.stride(0), pos.stride(1), _lib.stream_of(x)),
               'svhip_axial_rope')
    return out


def _frequencies_of(cross):
    return cross.rope.frequencies.to(device=cross.query.weight.device, dtype=torch.float32)


def cross_query(cross, value, positions):
    """fast_ops.py:98-101: Q = RoPE(query(norm(value))) as [B,H,N,D] bf16; `cross` is the layer's
    RotaryCrossAttention (its `norm`, `query`, `heads`, `rope.frequencies`)."""
    batch, queries, width = value.shape
    query = cross.query(cross.norm(value)).reshape(batch, queries, cross.heads, width // cross.heads)
    query = query.to(torch.bfloat16).transpose(1, 2)
    return axial_rope(query, positions, _frequencies_of(cross), out=query)


def local_kv(cross, local, positions):
    """fast_ops.py:90-95: the local keys' ([1,H,L,D] rotated K, [1,H,L,D] V) of one unpadded item [1, L, W]."""
    batch, keys, width = local.shape
    kv = cross.key_value(local).to(torch.bfloat16).reshape(batch, keys, 2, cross.heads, width // cross.heads)
    key, value = kv.unbind(2)
    key, value = key.transpose(1, 2), value.transpose(1, 2)
    return axial_rope(key, positions, _frequencies_of(cross)), value
