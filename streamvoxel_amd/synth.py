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


class _Cross(torch.nn.Module):
    """RotaryCrossAttention's parameters (streaming_controlnet.py:19-28): norm, query, key_value, proj, heads, width,
    rope."""

    def __init__(self, width, heads):
        super().__init__()
        self.heads, self.width = heads, width
        self.query = torch.nn.Linear(width, width)
        self.key_value = torch.nn.Linear(width, 2 * width)
        self.proj = torch.nn.Linear(width, width)
        self.rope = _Rope(width // heads)
        self.norm = torch.nn.LayerNorm(width, elementwise_affine=False, eps=1e-6)


class Trunk(torch.nn.Module):
    """The time-conditioned patch DiT's parameters in the reference's layout (unconditional_md4_timefree.py:66-125):
    target_patch (Conv3d), patch_centers_xyz, y_embed, time_mlp / time_projection, blocks, final_norm / final_ada /
    class_head (`head=True`), and its sizes; `time_encoding` as the reference computes it."""

    def __init__(self, classes, voxel_shape, patch, width, depth, heads, time_dim=256, y_range=(-64.0, 192.0),
                 head=True, seed=0):
        super().__init__()
        self.num_classes, self.voxel_shape, self.patch_size = classes, tuple(voxel_shape), patch
        self.hidden_dim, self.depth, self.num_heads, self.time_dim = width, depth, heads, time_dim
        self.y_range, self.time_free = tuple(y_range), False
        self.patch_shape = tuple(v // patch for v in self.voxel_shape)
        self.target_patch = torch.nn.Conv3d(classes + 1, width, patch, stride=patch)
        self.register_buffer('patch_centers_xyz', patch_positions(self.voxel_shape, patch) * patch)
        self.y_embed = torch.nn.Sequential(torch.nn.Linear(1, width), torch.nn.SiLU(), torch.nn.Linear(width, width))
        self.time_mlp = torch.nn.Sequential(torch.nn.Linear(time_dim // 4, time_dim), torch.nn.GELU(),
                                            torch.nn.Linear(time_dim, time_dim))
        self.time_projection = torch.nn.Sequential(torch.nn.SiLU(), torch.nn.Linear(time_dim, width))
        self.blocks = torch.nn.ModuleList(BlockWeights(width, heads, seed=seed * 1000 + i) for i in range(depth))
        if head:
            self.final_norm = torch.nn.LayerNorm(width, elementwise_affine=False, eps=1e-6)
            self.final_ada = torch.nn.Sequential(torch.nn.SiLU(), torch.nn.Linear(width, 2 * width))
            self.class_head = torch.nn.Linear(width, patch ** 3 * classes)
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for m in [self.target_patch, *self.y_embed, *self.time_mlp, *self.time_projection,
                      *([self.final_ada[1], self.class_head] if head else [])]:
                if isinstance(m, (torch.nn.Linear, torch.nn.Conv3d)):
                    fan = m.weight[0].numel() + m.weight.shape[0]
                    m.weight.copy_((torch.rand(m.weight.shape, generator=g) * 2 - 1) * (6.0 / fan) ** 0.5)
                    m.bias.copy_(torch.randn(m.bias.shape, generator=g) * 0.02)

    def time_encoding(self, t):
        """unconditional_md4_timefree.py:119-125 (time_free False)."""
        import math
        half = self.time_dim // 8
        freq = torch.exp(-math.log(10000.0) * torch.arange(half, device=t.device).float() / half)
        phase = t.float()[:, None] * freq
        return self.time_projection(self.time_mlp(torch.cat((phase.sin(), phase.cos()), -1)))


class StepModel(torch.nn.Module):
    """Random-initialised parameters of the streaming ControlNet a generation step runs (the trained weights are
    not published), in the reference's layout (streaming_controlnet.py:64-115, compact_controlnet.py:10-33):
    `backbone` (Trunk with the class head), `control` (Trunk of its own width and depth, no head), `cross`
    (one _Cross per control block, at the control width), `zero` (Linear control width -> backbone width) and
    `layer_map` (backbone block -> control block, the uniformly spaced injections of the compact model).
    Defaults: the shipped model (304 classes, 256 x 16 x 16 windows, patch 4, 25 x 768 backbone, 13 x 384
    control, 8 heads)."""

    def __init__(self, classes=304, voxel_shape=(256, 16, 16), patch=4, width=768, depth=25, heads=8,
                 control_width=384, control_depth=13, seed=0):
        super().__init__()
        self.backbone = Trunk(classes, voxel_shape, patch, width, depth, heads, seed=seed + 1)
        self.control = Trunk(classes, voxel_shape, patch, control_width, control_depth, heads, head=False,
                             seed=seed + 2)
        self.cross = torch.nn.ModuleList(_Cross(control_width, heads) for _ in range(control_depth))
        self.zero = torch.nn.ModuleList(torch.nn.Linear(control_width, width) for _ in range(control_depth))
        indices = [0] if control_depth == 1 else [round(i * (depth - 1) / (control_depth - 1))
                                                  for i in range(control_depth)]
        self.layer_map = {idx: j for j, idx in enumerate(indices)}
        # The condition layout of the shipped model (biome window of halo 4 pooled by 2: 288 local biome keys).
        self.biome_halo, self.biome_patch = 4, 2
        g = torch.Generator().manual_seed(seed + 3)
        with torch.no_grad():
            for m in [*self.cross.modules(), *self.zero]:
                if isinstance(m, torch.nn.Linear):
                    bound = (6.0 / (m.in_features + m.out_features)) ** 0.5
                    m.weight.copy_((torch.rand(m.weight.shape, generator=g) * 2 - 1) * bound)
                    m.bias.copy_(torch.randn(m.bias.shape, generator=g) * 0.02)


class WindowSpec:
    """The window geometry the slot engine reads from the reference's ModelSpec (streamvoxel/stream/condition.py):
    height, tile (windows of height x tile x tile voxels), num_classes and y_origin. Defaults: the shipped model."""

    def __init__(self, height=256, tile=16, num_classes=304, y_origin=-64.0):
        self.height, self.tile, self.num_classes, self.y_origin = int(height), int(tile), int(num_classes), y_origin


def condition(model, prefix_keys, local_keys, seed, device, scale=1.0):
    """A seeded synthetic window condition in the layout the reference's encoders produce (the encoders and their
    inputs are not part of this library): per cross-attention layer a prefix (K, V) [H, P, D] bf16 (K of unit
    variance times `scale`), local context features [1, L, W] ~ N(0, 1) (the encoders end in a LayerNorm) and their
    XYZ positions [1, L, 3] in patch units (x, z in [-8, 8), y in [0, 64))."""
    from streamvoxel_amd.stream.engine import Encoded
    g = torch.Generator().manual_seed(seed)
    cross = model.cross[0]
    H, W = int(cross.heads), int(cross.width)
    D = W // H
    prefix = []
    for _ in model.cross:
        k = (torch.randn(H, prefix_keys, D, generator=g) * scale).to(torch.bfloat16)
        v = torch.randn(H, prefix_keys, D, generator=g).to(torch.bfloat16)
        prefix.append((k.to(device), v.to(device)))
    local = torch.randn(1, local_keys, W, generator=g)
    positions = torch.rand(1, local_keys, 3, generator=g) * torch.tensor([16.0, 64.0, 16.0]) - torch.tensor(
        [8.0, 0.0, 8.0])
    return Encoded(prefix, local.to(device), positions.to(device))
