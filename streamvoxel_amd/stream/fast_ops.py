"""The names of the reference's `streamvoxel/stream/fast_ops.py` on this path, backed by the HIP library.

A caller of the reference imports these in place of its own module: same names, argument order and meaning; the
attention takes the windows' key lengths (int32, device) where the reference builds a FlexAttention BlockMask from
the same lengths (`PackedKeys.lengths`, fast_ops.py:122-159).
"""
from __future__ import annotations

import torch

from streamvoxel_amd.sampling.block_quota import quota_select, top_mask
from streamvoxel_amd.sampling.entropy import entropy_scores
from streamvoxel_amd.stream.attention import attention
from streamvoxel_amd.stream.engine import RECOMMENDED, SlotEngine
from streamvoxel_amd.stream.producer import cross_query, local_kv
from streamvoxel_amd.stream.slot import FastLowEntropyLastSlot, SelectGraphs, consume_batch

__all__ = ['RECOMMENDED', 'FastSlotForward', 'local_kv', 'cross_query', 'cross_flex', 'cross_sdpa', 'entropy_torch',
           'entropy_triton', 'top_mask_nosync', 'quota_select_nosync', 'FastLowEntropyLastSlot', 'SelectGraphs',
           'consume_batch']

# fast_ops.py:164-375: the slot engine the worker drives (tokens, load_slot, wait_loads, replay, numerical_gate).
FastSlotForward = SlotEngine


def _project(cross, out, batch, queries, width):
    return cross.proj(out.transpose(1, 2).reshape(batch, queries, width))


def cross_flex(cross, value, positions, key, val, lengths):
    """fast_ops.py:104-108: RoPE'd query of `value` [n, Q, W] at `positions` against the cached key / val
    [n, H, Kcap, D] (bf16, or e4m3 with per-(window, head) scales through `attention`), the first lengths[b] keys
    of window b, then the output projection. `lengths` int32 [n] on the device replaces the BlockMask."""
    batch, queries, width = value.shape
    query = cross_query(cross, value, positions)
    out = attention(query, key, val, lengths=lengths)
    return _project(cross, out, batch, queries, width)


def cross_sdpa(cross, value, positions, key, val, valid):
    """fast_ops.py:111-115 with `valid` [n, Kcap] bool, the key mask of the masked SDPA (any pattern: the
    kernel attends exactly the True keys of each window)."""
    batch, queries, width = value.shape
    query = cross_query(cross, value, positions)
    out = attention(query, key, val, key_mask=valid.contiguous())
    return _project(cross, out, batch, queries, width)


def entropy_torch(logits):
    """fast_ops.py:380-382."""
    return entropy_scores(logits)


def entropy_triton(logits, block_n=256, block_c=16):
    """fast_ops.py:420-430: sum p log p over the class axis of logits [C, ...] in one HBM pass with fp32 math. The
    tile sizes of the reference's Triton kernel do not apply to the HIP kernel and are accepted for the signature's
    sake."""
    del block_n, block_c
    return entropy_scores(logits)


def top_mask_nosync(scores, eligible, count):
    """fast_ops.py:433-439: `count` may be a host int or a 0-dim device tensor; no host read."""
    return top_mask(scores, eligible, count)


def quota_select_nosync(score, mask, k, b, pos, frac, n_total, committed):
    """fast_ops.py:442-473: k, frac, committed host numbers or 0-dim device tensors (long, double, long); no host
    read, capturable."""
    return quota_select(score, mask, k, b, pos, frac, n_total, committed)
