"""Oracle restatement of `streamvoxel/sampling/*.py` and the no-sync selection in `streamvoxel/stream/fast_ops.py`.

Test infrastructure only (see oracle/__init__.py). Integer and ordering work is numpy; reference-form float reductions
use torch fp32 on the CPU (the same operator sequence as the reference); `*_f64` forms are numpy float64.

Ordering conventions restated here:
  * "descending, stable" sorts (reference `torch.argsort(..., descending=True, stable=True)`) are numpy stable sorts
    of the negated key, so equal scores keep ascending flat-index order; -0.0 and +0.0 compare equal.
  * The apportionment sort `torch.argsort(-(ideal-base)*1e6 + pos)` (block_quota.py:28, fast_ops.py:459) is not
    stable in the reference. Keys only collide when two blocks' fractional parts differ by exactly an integer / 1e6;
    the oracle (and the HIP kernel) break such collisions by ascending block index.
"""
from __future__ import annotations

import math

import numpy as np

# --------------------------------------------------------------------------------------------------- entropy (E1)


def entropy_scores(logits):
    """Reference form of `entropy_scores` (sampling/entropy.py:1-4): fp32 log_softmax over axis 0, then sum p*logp.

    `logits` is a torch tensor [C, ...] (any float dtype); returns a torch fp32 tensor [...]."""
    logp = logits.float().log_softmax(0)
    return (logp.exp() * logp).sum(0)


def entropy_scores_f64(logits):
    """Same quantity in float64 (numpy): sum_c p_c log p_c, the high-precision target for tolerance checks.

    `logits` is array-like [C, ...]."""
    x = np.asarray(logits, dtype=np.float64)
    peak = x.max(axis=0, keepdims=True)
    shifted = x - peak
    e = np.exp(shifted)
    total = e.sum(axis=0)
    return (e * shifted).sum(axis=0) / total - np.log(total)


def air_prob(logits, air_ids):
    """Reference form of the marking pass's air probability (stream/slot.py:126):
    `logits.float().softmax(0)[air].sum(0)` (torch fp32)."""
    import torch
    air = torch.as_tensor(list(air_ids), dtype=torch.long)
    return logits.float().softmax(0)[air].sum(0)


def air_prob_f64(logits, air_ids):
    x = np.asarray(logits, dtype=np.float64)
    e = np.exp(x - x.max(axis=0, keepdims=True))
    return e[list(air_ids)].sum(axis=0) / e.sum(axis=0)


# ------------------------------------------------------------------------------------------------ top_mask (E3)


def top_mask(scores, eligible, count):
    """`top_mask` (sampling/block_quota.py:4-12): the `count` largest scores among `eligible`, ties to the lower flat
    (YZX) index. `count` is clamped to the number of eligible voxels; count <= 0 selects nothing."""
    scores = np.asarray(scores)
    eligible = np.asarray(eligible, dtype=bool)
    result = np.zeros(eligible.shape, dtype=bool)
    indices = np.flatnonzero(eligible)
    count = min(int(count), len(indices))
    if count > 0:
        key = -scores.reshape(-1)[indices].astype(np.float64)
        key[key == 0] = 0.0                                   # -0.0 == +0.0
        order = np.argsort(key, kind='stable')
        result.reshape(-1)[indices[order[:count]]] = True
    return result


def top_mask_nosync(scores, eligible, count):
    """`top_mask_nosync` (stream/fast_ops.py:433-439). For finite scores it equals `top_mask`; restated separately
    because the reference ranks over all voxels with non-eligible ones filled by -inf."""
    scores = np.asarray(scores, dtype=np.float64).reshape(-1)
    eligible = np.asarray(eligible, dtype=bool)
    flat = np.where(eligible.reshape(-1), scores, -np.inf)
    key = -flat
    key[key == 0] = 0.0
    order = np.argsort(key, kind='stable')
    rank = np.empty_like(order)
    rank[order] = np.arange(len(order))
    return ((rank < int(count)) & eligible.reshape(-1)).reshape(eligible.shape)


# ---------------------------------------------------------------------------------------------- block view (E4)


def block_view(a, b):
    """`block_view` (sampling/block_quota.py:15-17): [Y,Z,X] -> [(Y/b)(Z/b)(X/b), b^3], blocks in (by,bz,bx) order,
    in-block entries in (dy,dz,dx) order."""
    a = np.asarray(a)
    y, z, x = a.shape
    return a.reshape(y // b, b, z // b, b, x // b, b).transpose(0, 2, 4, 1, 3, 5).reshape(-1, b ** 3)


def block_unview(blocks, b, shape):
    """Inverse of `block_view` (the permute at sampling/block_quota.py:34)."""
    y, z, x = shape
    return np.asarray(blocks).reshape(y // b, z // b, x // b, b, b, b).transpose(0, 3, 1, 4, 2, 5).reshape(shape)


# ---------------------------------------------------------------------------------------- block quota select (E5)


def apportion(mask, n_total, pos, frac, goal, b):
    """Per-block quota of `block_quota_select` (sampling/block_quota.py:24-30) / `quota_select_nosync`
    (stream/fast_ops.py:451-463).

    Returns (quota, target, legal, already) as int64 [nb]. `goal` is committed + k."""
    mb = block_view(mask, b).astype(bool)
    legal = mb.sum(1).astype(np.int64)
    n_total = np.asarray(n_total, dtype=np.int64)
    already = n_total - legal
    ideal = np.float64(frac) * n_total.astype(np.float64)
    base = np.floor(ideal + 1e-9).astype(np.int64)
    extra = max(int(goal) - int(base.sum()), 0)
    key = -(ideal - base.astype(np.float64)) * 1e6 + np.asarray(pos, dtype=np.int64).astype(np.float64)
    frac_rank = np.argsort(key, kind='stable')
    target = base.copy()
    target[frac_rank[:extra]] += 1
    quota = np.minimum(np.maximum(target - already, 0), legal)
    return quota, target, legal, already


def in_block_select(score, mask, quota, b):
    """The in-block top-`quota` by (score desc, in-block index asc) among masked voxels
    (sampling/block_quota.py:31-34), returned in [Y,Z,X] layout and intersected with the mask."""
    mb = block_view(mask, b).astype(bool)
    sm = np.where(mb, block_view(score, b).astype(np.float64), -np.inf)
    key = -sm
    key[key == 0] = 0.0
    ranks = np.argsort(key, axis=1, kind='stable')
    bc = np.zeros_like(mb)
    take = np.arange(b ** 3)[None, :] < np.asarray(quota)[:, None]
    np.put_along_axis(bc, ranks, take, axis=1)
    return block_unview(bc, b, np.shape(mask)) & np.asarray(mask, dtype=bool)


def order_to_pos(order):
    """`pos[order] = arange(nb)` (sampling/block_quota.py:26, stream/fast_ops.py:527)."""
    order = np.asarray(order, dtype=np.int64)
    pos = np.empty_like(order)
    pos[order] = np.arange(len(order))
    return pos


def block_quota_select(score, mask, k, b, order, frac, n_total):
    """`block_quota_select` (sampling/block_quota.py:20-38): exactly k voxels of `mask` balanced over b^3 blocks,
    global entropy trim / top-up when the clamped quotas miss k."""
    mask = np.asarray(mask, dtype=bool)
    mb = block_view(mask, b)
    already_sum = int((np.asarray(n_total, dtype=np.int64) - mb.sum(1)).sum())
    quota, *_ = apportion(mask, n_total, order_to_pos(order), frac, already_sum + int(k), b)
    sel = in_block_select(score, mask, quota, b)
    got = int(sel.sum())
    if got > k:
        sel = top_mask(score, sel, k)
    elif got < k:
        sel = sel | top_mask(score, mask & ~sel, k - got)
    return sel


def quota_select_nosync(score, mask, k, b, pos, frac, n_total, committed):
    """`quota_select_nosync` (stream/fast_ops.py:442-473): as `block_quota_select` with goal = committed + k and
    `pos` (the inverse block order) given directly."""
    mask = np.asarray(mask, dtype=bool)
    k = int(k)
    quota, *_ = apportion(mask, n_total, pos, frac, int(committed) + k, b)
    sel = in_block_select(score, mask, quota, b)
    got = int(sel.sum())
    if got > k:
        return top_mask_nosync(score, sel, k)
    if got < k:
        return sel | top_mask_nosync(score, mask & ~sel, k - got)
    return sel


def select_bad(chosen, selectable, k):
    """The quota-violation flag (stream/fast_ops.py:540): chosen.sum() != k or chosen outside selectable."""
    chosen = np.asarray(chosen, dtype=bool)
    return bool(int(chosen.sum()) != int(k) or (chosen & ~np.asarray(selectable, dtype=bool)).any())


# ------------------------------------------------------------------------------------- low-entropy-last (E6, E7)

STRATA_BAND = 8


def low_entropy_last_update(last, mask, air, solid, eps, band, col=False):
    """`low_entropy_last_update` (sampling/low_entropy_last.py:8-17).

    bad = (mask & air <= 1-eps) | solid, where the compare is done in fp32 against fp32(1-eps) like a torch fp32
    tensor compared with a Python float. col=True: every (z,x) column defers its top run of clean voxels; otherwise
    per layer (or per STRATA_BAND-layer band) on a [Y] `last`."""
    air = np.asarray(air, dtype=np.float32)
    threshold = np.float32(1 - eps)
    bad = (np.asarray(mask, dtype=bool) & (air <= threshold)) | np.asarray(solid, dtype=bool)
    last = np.asarray(last, dtype=bool)
    if col:
        clean = ~bad
        run = np.cumprod(clean[::-1].astype(np.int64), axis=0)[::-1].astype(bool)
        return last | run
    clean = ~bad.reshape(bad.shape[0], -1).any(1)
    if band:
        clean = np.repeat(clean.reshape(-1, STRATA_BAND).all(1), STRATA_BAND)
    top_run = np.cumprod(clean[::-1].astype(np.int64))[::-1].astype(bool)
    return last | top_run


def actual_time(mask_fraction):
    """`actual_time` (sampling/schedule.py:4-5)."""
    return 2 * math.asin(min(1., max(0., mask_fraction))) / math.pi


def reveal_fraction(u, schedule):
    """`reveal_fraction` (sampling/schedule.py:8-12)."""
    if schedule == 'linear':
        return u
    if schedule == 'halfcos':
        return (1 - math.cos(math.pi * u)) / 2
    if schedule == 'reversequarter':
        return math.sin(math.pi * u / 2)
    raise ValueError(schedule)


def quota_counts(total, steps, schedule):
    """Legacy rounding (sampling/schedule.py:15-18)."""
    cumulative = [0] + [min(total, max(0, math.floor(total * reveal_fraction(s / steps, schedule) + 1e-9)))
                        for s in range(1, steps + 1)]
    cumulative[-1] = total
    return [b - a for a, b in zip(cumulative, cumulative[1:])]


def curve(u, name):
    """`curve` (sampling/schedule.py:21-29)."""
    if name == 'linear':
        return u
    if name == 'quartercos':
        return 1 - math.cos(math.pi * u / 2)
    if name == 'reversequarter':
        return math.sin(math.pi * u / 2)
    if name == 'halfcos':
        return (1 - math.cos(math.pi * u)) / 2
    if name == 'arccos':
        return 2 / math.pi * math.acos(1 - u)
    if name.startswith('front'):
        return 1 - (1 - u) ** float(name[5:])
    if name.startswith('power'):
        return u ** float(name[5:])
    raise ValueError(name)


def counts(total, spec):
    """`counts` (sampling/schedule.py:32-38): 'positive' rounding guarantees every step reveals >= 1."""
    if spec['schedule'] == 'native_quarter':
        return None
    if spec.get('rounding') == 'legacy':
        return quota_counts(total, spec['steps'], spec['schedule'])
    steps = spec['steps']
    assert 1 <= steps <= total
    cumulative = [0] + [s + math.floor((total - steps) * curve(s / steps, spec['schedule']) + 1e-10)
                        for s in range(1, steps + 1)]
    cumulative[-1] = total
    q = [b - a for a, b in zip(cumulative, cumulative[1:])]
    assert min(q) >= 1 and sum(q) == total
    return q


def low_entropy_last_quotas(total, steps, n_last, schedule='quartercos'):
    """`low_entropy_last_quotas` (sampling/low_entropy_last.py:20-33): the deferred count is taken from the tail
    steps; only positive quotas are returned."""
    n_last = int(n_last)
    if steps < 1 or not 0 <= n_last <= total:
        raise ValueError((total, steps, n_last))
    quotas = counts(total, dict(steps=int(steps), schedule=schedule, rounding='positive'))
    air = n_last
    solid = []
    for q in reversed(quotas):
        take = min(q, air)
        air -= take
        solid.append(q - take)
    solid.reverse()
    assert air == 0 and sum(solid) == total - n_last
    return [q for q in solid if q > 0]
