"""Entropy-ranked selection on the GPU (mirror of streamvoxel/sampling/block_quota.py:1-38)."""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib


def block_view(a, b):
    """[Y,Z,X] -> [(Y/b)(Z/b)(X/b), b^3]: blocks in (by,bz,bx) order, in-block entries (dy,dz,dx)
    (streamvoxel/sampling/block_quota.py:15-17). A pure re-indexing (torch view/permute), any device."""
    y, z, x = a.shape
    return a.reshape(y // b, b, z // b, b, x // b, b).permute(0, 2, 4, 1, 3, 5).reshape(-1, b ** 3)


def _bytes(mask):
    if mask.dtype != torch.bool:
        raise TypeError('masks are torch.bool')
    return mask.contiguous().view(torch.uint8)


def top_mask(scores, eligible, count):
    """The `count` largest scores among `eligible`, ties to the lower flat index
    (streamvoxel/sampling/block_quota.py:4-12). `count` is a host int or a 0-dim device int64 tensor."""
    _lib.require_gpu(scores, eligible)
    s = scores.contiguous().float().reshape(-1)
    e = _bytes(eligible).reshape(-1)
    out = torch.empty(eligible.shape, dtype=torch.bool, device=scores.device)
    lib = _lib.load()
    if torch.is_tensor(count):
        cnt = count.to(device=scores.device, dtype=torch.int64).reshape(1)
        rc = lib.svhip_top_mask(_lib.ptr(s), _lib.ptr(e), 1, s.numel(), _lib.ptr(cnt), 0,
                                _lib.ptr(out.view(torch.uint8)), _lib.stream_of(s))
    else:
        rc = lib.svhip_top_mask(_lib.ptr(s), _lib.ptr(e), 1, s.numel(), None, int(count),
                                _lib.ptr(out.view(torch.uint8)), _lib.stream_of(s))
    _lib.check(rc, 'svhip_top_mask')
    return out


class QuotaWorkspace:
    """Device workspace for the quota selection of `batch` windows of `shape` with block size `b` (allocated once;
    launches allocate nothing)."""

    def __init__(self, batch, shape, b, device, fused=False):
        lib = _lib.load()
        Y, Z, X = shape
        query = lib.svhip_ease_select_workspace_bytes if fused else lib.svhip_quota_select_workspace_bytes
        nbytes = int(query(batch, Y, Z, X, b))
        if nbytes == 0:
            raise ValueError(f'unsupported selection geometry batch={batch} shape={shape} block={b}: '
                             + lib.svhip_last_error().decode(errors='replace'))
        self.buffer = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self.key = (batch, tuple(shape), b, fused)


def quota_select_into(score, mask, k, b, pos, frac, n_total, committed, chosen, bad, workspace):
    """Batched no-sync selection writing `chosen` [B,Y,Z,X] bool and `bad` [B] bool in place.

    score fp32 [B,Y,Z,X]; mask bool [B,Y,Z,X]; k, committed int64 [B]; frac float64 [B]; pos, n_total int64 [B,nb]
    (all device tensors)."""
    _lib.require_gpu(score, mask, k, pos, frac, n_total, committed, chosen, bad)
    B, Y, Z, X = score.shape
    lib = _lib.load()
    _lib.check(lib.svhip_quota_select(
        _lib.ptr(score), _lib.ptr(mask.view(torch.uint8)), B, Y, Z, X, b, _lib.ptr(k), _lib.ptr(pos), _lib.ptr(frac),
        _lib.ptr(n_total), _lib.ptr(committed), _lib.ptr(chosen.view(torch.uint8)), _lib.ptr(bad.view(torch.uint8)),
        _lib.ptr(workspace.buffer), workspace.buffer.numel(), _lib.stream_of(score)), 'svhip_quota_select')


def _device_scalar(v, dtype, device):
    if torch.is_tensor(v):
        return v.to(device=device, dtype=dtype).reshape(1)
    return torch.full((1,), v, dtype=dtype, device=device)


def quota_select(score, mask, k, b, pos, frac, n_total, committed):
    """One window, like `quota_select_nosync` (streamvoxel/stream/fast_ops.py:442-473): k, frac and committed are
    host numbers or 0-dim device tensors; pos is the inverse block order."""
    _lib.require_gpu(score, mask)
    device = score.device
    shape = tuple(score.shape)
    chosen = torch.empty((1, *shape), dtype=torch.bool, device=device)
    bad = torch.empty(1, dtype=torch.bool, device=device)
    ws = QuotaWorkspace(1, shape, b, device)
    quota_select_into(score.contiguous().float().reshape(1, *shape), mask.contiguous().reshape(1, *shape),
                      _device_scalar(k, torch.int64, device), b, pos.to(device=device, dtype=torch.int64).reshape(1, -1),
                      _device_scalar(frac, torch.float64, device),
                      n_total.to(device=device, dtype=torch.int64).reshape(1, -1),
                      _device_scalar(committed, torch.int64, device), chosen, bad, ws)
    return chosen[0]


def block_quota_select(score, mask, k, b, order, frac, n_total):
    """Exactly k voxels of `mask`, balanced over b^3 blocks (streamvoxel/sampling/block_quota.py:20-38). `order` is
    the seeded block order; the committed count is derived on the device as sum(n_total) - sum(mask)."""
    _lib.require_gpu(score, mask, order, n_total)
    device = score.device
    pos = torch.empty_like(order)
    pos[order] = torch.arange(len(order), device=device, dtype=order.dtype)
    n_total = n_total.to(dtype=torch.int64)
    committed = (n_total.sum() - mask.sum()).reshape(1)
    return quota_select(score, mask, k, b, pos, frac, n_total, committed)
