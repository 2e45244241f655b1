"""Seeded synthetic inputs of the hot-path workloads (the trained weights are not published).

  * cached cross-attention context: per-window key counts L_b = 1552 + 1024 k_b (k_b ~ U{0..8} present
    neighbours of 1024 tokens, 81 wider columns x 16 tokens and 256 biome tokens);
  * bimodal class logits: a `peaked` share of voxels has one class raised by `gap` over N(0,1), the rest is N(0,1).
"""
from __future__ import annotations

import torch

NEIGHBOUR_TOKENS = 1024
WIDE_TOKENS = 81 * 16
BIOME_TOKENS = 256
BASE_KEYS = WIDE_TOKENS + BIOME_TOKENS      # 1552
MAX_KEYS = 8 * NEIGHBOUR_TOKENS + BASE_KEYS  # 9744


def kv_lengths(slots, seed):
    g = torch.Generator().manual_seed(seed)
    neighbours = torch.randint(0, 9, (slots,), generator=g)
    return (BASE_KEYS + NEIGHBOUR_TOKENS * neighbours).tolist()


def bimodal_logits_(out, peaked, gap=12.0, generator=None):
    """Fill `out` [N, C] (voxel-major, any float dtype, on any device) in place."""
    n, c = out.shape
    out.normal_(generator=generator)
    dev = out.device
    hot = torch.rand(n, device=dev, generator=generator) < peaked
    cls = torch.randint(c, (n,), device=dev, generator=generator)
    rows = torch.arange(n, device=dev)
    out[rows[hot], cls[hot]] += gap
    return out


def bimodal_logits(n, classes, peaked, seed, device='cpu', dtype=torch.float32, gap=12.0):
    g = torch.Generator(device=device).manual_seed(seed)
    out = torch.empty((n, classes), dtype=dtype, device=device)
    return bimodal_logits_(out, peaked, gap, g)


def high_entropy_share(step, steps, start=0.30, end=0.05):
    """Linear drift of the uncertain share over a window (30% -> 5%)."""
    if steps <= 1:
        return start
    return start + (end - start) * step / (steps - 1)
