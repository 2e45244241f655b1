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


def patch_positions(voxel_shape=(256, 16, 16), patch=4):
    """Self-attention positions of a window's patch tokens, fp32 [N, 3] in XYZ order: the patch centres divided by
    the patch size (unconditional_md4.py:74-76, fast_ops.py:280): token (gy, gz, gx) in row-major YZX order sits at
    (gx + 1/2, gy + 1/2, gz + 1/2)."""
    gy, gz, gx = (v // patch for v in voxel_shape)
    grid = torch.stack(torch.meshgrid(torch.arange(gy).float(), torch.arange(gz).float(), torch.arange(gx).float(),
                                      indexing='ij'), -1).reshape(-1, 3)
    return (grid[:, [2, 0, 1]] * patch + patch / 2) / patch


class _Rope(torch.nn.Module):
    def __init__(self, head_dim):
        super().__init__()
        axis = head_dim // 3
        self.register_buffer('frequencies', 10000.0 ** (-torch.arange(0, axis, 2).float() / axis))


class _Attention(torch.nn.Module):
    def __init__(self, width, heads):
        super().__init__()
        self.heads = heads
        self.qkv = torch.nn.Linear(width, 3 * width)
        self.proj = torch.nn.Linear(width, width)
        self.rope = _Rope(width // heads)


class BlockWeights(torch.nn.Module):
    """Random-initialised parameters in the layout of the reference's UnconditionalBlock (the trained weights are
    not published): `norm1` / `norm2` (LayerNorm, eps 1e-6; affine only without AdaLN), `attn.qkv`, `attn.proj`,
    `attn.heads`, `attn.rope.frequencies`, `mlp` = Linear, GELU, Linear and, when `timed`, `ada` = SiLU, Linear(W, 6W)
    (unconditional_md4_timefree.py:33-63; unconditional_md4.py:27-56). Holds parameters only: the forward is
    `streamvoxel_amd.stream.backbone.block_forward`. Linear weights xavier-uniform, biases and the AdaLN
    projection N(0, 0.02^2) so that every gate and shift is non-zero."""

    def __init__(self, width, heads, ratio=4.0, timed=True, seed=0):
        super().__init__()
        if width % heads or (width // heads) % 6:
            raise ValueError('heads must split the width into head_dim multiples of 6')
        g = torch.Generator().manual_seed(seed)
        self.norm1 = torch.nn.LayerNorm(width, elementwise_affine=not timed, eps=1e-6)
        self.norm2 = torch.nn.LayerNorm(width, elementwise_affine=not timed, eps=1e-6)
        self.attn = _Attention(width, heads)
        hidden = int(width * ratio)
        self.mlp = torch.nn.Sequential(torch.nn.Linear(width, hidden), torch.nn.GELU(), torch.nn.Linear(hidden, width))
        if timed:
            self.ada = torch.nn.Sequential(torch.nn.SiLU(), torch.nn.Linear(width, 6 * width))
        with torch.no_grad():
            for m in self.modules():
                if isinstance(m, torch.nn.Linear):
                    bound = (6.0 / (m.in_features + m.out_features)) ** 0.5
                    m.weight.copy_((torch.rand(m.weight.shape, generator=g) * 2 - 1) * bound)
                    m.bias.copy_(torch.randn(m.bias.shape, generator=g) * 0.02)
            if timed:
                self.ada[1].weight.copy_(torch.randn(self.ada[1].weight.shape, generator=g) * 0.02)
                self.ada[1].bias.copy_(torch.randn(self.ada[1].bias.shape, generator=g) * 0.02)
            else:
                for n in (self.norm1, self.norm2):
                    n.weight.copy_(1 + torch.randn(width, generator=g) * 0.1)
                    n.bias.copy_(torch.randn(width, generator=g) * 0.1)
