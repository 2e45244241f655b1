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


def _check_out(out, shape, device, *inputs):
    """`out` must be a contiguous bool tensor of `shape` on `device` that shares no memory with an input (the
    kernels read their inputs while they write the output)."""
    if out.dtype != torch.bool or tuple(out.shape) != tuple(shape) or out.device != device:
        raise ValueError(f'out must be a bool tensor of shape {tuple(shape)} on {device}')
    if not out.is_contiguous():
        raise ValueError('out must be contiguous')
    if any(_lib.overlaps(out, t) for t in inputs):
        raise ValueError('out shares memory with an input; pass a separate buffer')


def top_mask(scores, eligible, count, out=None):
    """The `count` largest scores among `eligible`, ties to the lower flat index
    (streamvoxel/sampling/block_quota.py:4-12). `count` is a host int or a 0-dim device int64 tensor (no host
    read). Returns a new bool tensor, as the reference does; `out` (a bool tensor of eligible's shape that shares no
    memory with the inputs) takes the result instead, and then a call with contiguous fp32 scores, a contiguous
    mask and a device int64 count allocates nothing."""
    _lib.require_gpu(scores, eligible, out)
    s = scores.contiguous().float().reshape(-1)
    e = _bytes(eligible).reshape(-1)
    if out is None:
        out = torch.empty(eligible.shape, dtype=torch.bool, device=scores.device)
    else:
        _check_out(out, eligible.shape, scores.device, s, e)
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
    (all device tensors). committed None: derived on the device as sum(n_total) - sum(mask) per window."""
    _lib.require_gpu(score, mask, k, pos, frac, n_total, committed, chosen, bad)
    B, Y, Z, X = score.shape
    lib = _lib.load()
    _lib.check(lib.svhip_quota_select(
        _lib.ptr(score), _lib.ptr(mask.view(torch.uint8)), B, Y, Z, X, b, _lib.ptr(k), _lib.ptr(pos), _lib.ptr(frac),
        _lib.ptr(n_total), _lib.ptr(committed), _lib.ptr(chosen.view(torch.uint8)), _lib.ptr(bad.view(torch.uint8)),
        _lib.ptr(workspace.buffer), workspace.buffer.numel(), _lib.stream_of(score)), 'svhip_quota_select')


class SelectBuffers:
    """Caller-owned device buffers of the one-window selection functions below: the workspace, the per-call
    scalars (k, frac, committed), the `bad` flag and the block positions, for windows of `shape` with block size
    `b`. Passed as `buffers=` together with `out=`, a call allocates nothing (the reference keeps such buffers on its
    slot, fast_ops.py:501-510). The object is the caller's: calls that share one must not run concurrently on
    different streams."""

    def __init__(self, shape, b, device):
        shape = tuple(int(s) for s in shape)
        b = int(b)
        nb = (shape[0] // b) * (shape[1] // b) * (shape[2] // b)
        self.shape, self.b, self.device = shape, b, torch.device(device)
        self.ws = QuotaWorkspace(1, shape, b, device)
        self.bad = torch.empty(1, dtype=torch.bool, device=device)
        self.k = torch.empty(1, dtype=torch.int64, device=device)
        self.committed = torch.empty(1, dtype=torch.int64, device=device)
        self.frac = torch.empty(1, dtype=torch.float64, device=device)
        self.pos = torch.empty(nb, dtype=torch.int64, device=device)
        self.arange = torch.arange(nb, dtype=torch.int64, device=device)

    def fits(self, shape, b, device):
        return self.shape == tuple(shape) and self.b == int(b) and self.device == torch.device(device)


def _select_buffers(buffers, shape, b, device):
    if buffers is None:
        return SelectBuffers(shape, b, device)
    if not buffers.fits(shape, b, device):
        raise ValueError(f'buffers are for {buffers.shape} windows, block {buffers.b} on {buffers.device}; the call '
                         f'has {tuple(shape)}, block {b} on {device}')
    return buffers


def _set_scalar(dst, v):
    """A host number or a 0-dim / one-element device tensor into the one-element device buffer `dst`, without an
    allocation and without a host read."""
    if torch.is_tensor(v):
        dst.copy_(v.reshape(1))
    else:
        dst.fill_(v)
    return dst


def quota_select(score, mask, k, b, pos, frac, n_total, committed, out=None, buffers=None):
    """One window, like `quota_select_nosync` (streamvoxel/stream/fast_ops.py:442-473): k, frac and committed are
    host numbers or 0-dim device tensors (committed None: derived on the device as sum(n_total) - sum(mask)); pos
    is the inverse block order. Returns a new bool mask, as the reference does. `out` (bool, the window's shape,
    no memory shared with an input) takes the result instead, and `buffers` (a `SelectBuffers` of this geometry)
    holds the workspace and scalars; with both, fp32 contiguous scores, int64 pos / n_total and a contiguous mask,
    a call allocates nothing."""
    _lib.require_gpu(score, mask, out)
    device = score.device
    shape = tuple(score.shape)
    buf = _select_buffers(buffers, shape, b, device)
    s = score.contiguous().float().reshape(1, *shape)
    m = mask.contiguous().reshape(1, *shape)
    if out is None:
        out = torch.empty(shape, dtype=torch.bool, device=device)
    else:
        _check_out(out, shape, device, s, m)
    quota_select_into(s, m, _set_scalar(buf.k, k), b, pos.to(device=device, dtype=torch.int64).reshape(1, -1),
                      _set_scalar(buf.frac, frac), n_total.to(device=device, dtype=torch.int64).reshape(1, -1),
                      None if committed is None else _set_scalar(buf.committed, committed), out.view(1, *shape),
                      buf.bad, buf.ws)
    return out


def block_quota_select(score, mask, k, b, order, frac, n_total, out=None, buffers=None):
    """Exactly k voxels of `mask`, balanced over b^3 blocks (streamvoxel/sampling/block_quota.py:20-38). `order` is
    the seeded block order; the committed count is derived on the device as sum(n_total) - sum(mask). Returns a
    new bool mask (or fills `out`; `buffers` as for `quota_select`)."""
    _lib.require_gpu(score, mask, order, n_total)
    buf = _select_buffers(buffers, tuple(score.shape), b, score.device)
    pos = buf.pos.scatter_(0, order.to(torch.int64), buf.arange)
    return quota_select(score, mask, k, b, pos, frac, n_total, None, out=out, buffers=buf)
