"""Low-entropy-last deferral (mirror of streamvoxel/sampling/low_entropy_last.py:1-33)."""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.sampling.schedule import counts

STRATA_BAND = 8


def low_entropy_last_update(last, mask, air, solid, eps, band, col=False):
    """last | the top run of clean units, where bad = (mask & air <= 1-eps) | solid (fp32 compare).

    col=True: `last` [Y,Z,X], every (z,x) column defers its own top run of clean voxels; otherwise `last` [Y] and
    units are layers (or 8-layer bands with band=True). Returns a new tensor (the input is not modified)."""
    _lib.require_gpu(last, mask, air, solid)
    Y, Z, X = air.shape
    out = last.clone().contiguous()
    a = air.contiguous().float()
    m = mask.contiguous().view(torch.uint8) if mask is not None else None
    s = solid.contiguous().view(torch.uint8) if solid is not None else None
    mode = _lib.SVHIP_LEL_COLUMN if col else (_lib.SVHIP_LEL_BAND if band else _lib.SVHIP_LEL_LAYER)
    lib = _lib.load()
    _lib.check(lib.svhip_lel_update(_lib.ptr(out.view(torch.uint8)), _lib.ptr(m), _lib.ptr(a), _lib.ptr(s),
                                    float(eps), mode, 1, Y, Z, X, _lib.stream_of(a)), 'svhip_lel_update')
    return out


def low_entropy_last_quotas(total, steps, n_last, schedule='quartercos'):
    """Quarter-cosine quotas of length `steps` with the `n_last` deferred voxels taken from the tail steps; only
    the positive quotas are returned, summing to total - n_last (streamvoxel/sampling/low_entropy_last.py:20-33)."""
    n_last = int(n_last)
    if steps < 1 or not 0 <= n_last <= total:
        raise ValueError((total, steps, n_last))
    quotas = counts(total, dict(steps=int(steps), schedule=schedule, rounding='positive'))
    deferred = n_last
    solid = [0] * len(quotas)
    for i in range(len(quotas) - 1, -1, -1):
        take = min(quotas[i], deferred)
        deferred -= take
        solid[i] = quotas[i] - take
    if deferred != 0 or sum(solid) != total - n_last:
        raise AssertionError((total, steps, n_last))
    return [q for q in solid if q > 0]
