"""The forward of one generation step of the streaming ControlNet on the HIP kernels.

Reference counterpart: `FastSlotForward.forward` (streamvoxel/stream/fast_ops.py:274-308) with `GatherPatch`
(:58-75), `run_block` (:118-119) and `cross_flex` (:104-108): gather patchify of both branches, the 25 backbone
blocks, the 13 control blocks each followed by its cross-attention over the window's cached context and the zero
projection into the backbone, the final AdaLN LayerNorm and the class head, whose rows are returned in patch order
(`PatchLogits`) for the selection to read in place.

Kernels: `svhip_patch_embed` (patchify), the block path of `backbone` (`svhip_layer_norm`, `svhip_qkv_rope`,
`svhip_xattn_fwd`, `svhip_residual_norm`), `svhip_axial_rope` + `svhip_xattn_fwd` over `CachedContext` (cross
attention), `svhip_residual_norm` for every residual sum and `svhip_layer_norm` for the final norm. The Linear
layers and the small time / height embeddings stay the model's torch modules, run under bf16 autocast as in the
reference (fast_ops.py:312); the blocks' AdaLN projections of a trunk run as one GEMM per step (they share the
time vector). The control branch (13 control blocks, each with its cross attention and zero projection) never
reads the backbone, so it runs on a second stream from the start of the step while the backbone's 25 blocks run on
the current one; the backbone waits only for each zero projection it adds (an event per injection). Same kernels,
same bits; a step captured in a graph keeps the two branches.
"""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.stream.backbone import block_forward, layer_norm, residual_norm
from streamvoxel_amd.stream.patches import PatchLogits
from streamvoxel_amd.stream.producer import axial_rope

__all__ = ['GatherPatch', 'StepForward']


class GatherPatch:
    """fast_ops.py:58-75: the patch Conv3d of one-hot tokens as a sum of the weight rows the tokens pick
    (`svhip_patch_embed`). `bad` (device int32) becomes non-zero when a token lies outside [0, classes + 1)."""

    def __init__(self, conv, dtype=torch.bfloat16):
        weight = conv.weight.detach()
        hidden, inputs, patch = weight.shape[0], weight.shape[1], weight.shape[2]
        self.patch, self.hidden, self.inputs = patch, hidden, inputs
        self.table = weight.permute(1, 2, 3, 4, 0).reshape(inputs * patch ** 3, hidden).to(dtype).contiguous()
        self.bias = None if conv.bias is None else conv.bias.detach().to(dtype).contiguous()
        self.bad = torch.zeros(1, dtype=torch.int32, device=weight.device)

    def __call__(self, tokens, out=None):
        _lib.require_gpu(tokens, self.table, out)
        if tokens.dim() != 4 or tokens.dtype != torch.int64:
            raise ValueError('tokens must be int64 [B, Y, Z, X]')
        tokens = tokens if tokens.stride(-1) == 1 and tokens[0].is_contiguous() else tokens.contiguous()
        B, Y, Z, X = tokens.shape
        p = self.patch
        n = (Y // p) * (Z // p) * (X // p)
        if out is None:
            out = torch.empty((B, n, self.hidden), dtype=self.table.dtype, device=tokens.device)
        lib = _lib.load()
        _lib.check(lib.svhip_patch_embed(_lib.ptr(tokens), _lib.ptr(self.table), _lib.ptr(self.bias), _lib.ptr(out),
                                         _lib.ptr(self.bad), B, Y, Z, X, p, self.inputs, self.hidden,
                                         tokens.stride(0), out.stride(0), out.stride(1), _lib.stream_of(tokens)),
                   'svhip_patch_embed')
        return out


def cross_step(cross, value, positions, context, layer):
    """`value + cross_flex(cross, value, positions, key, val, lengths)` (fast_ops.py:104-108, 296) over layer
    `layer` of `context` (a CachedContext, its first n windows): LayerNorm (kernel), query projection, AxialRoPE
    (kernel, in place), attention (kernel) into [n, N, H, D], output projection, residual sum (kernel)."""
    n, N, W = value.shape
    H = cross.heads
    D = W // H
    q = cross.query(layer_norm(value, cross.norm)).view(n, N, H, D).transpose(1, 2)
    freq = cross.rope.frequencies.to(device=value.device, dtype=torch.float32)
    axial_rope(q, positions, freq, out=q)
    out = torch.empty((n, N, H, D), dtype=torch.bfloat16, device=value.device)
    context.attend(layer, q, out=out.transpose(1, 2), n=n)
    return residual_norm(value, cross.proj(out.view(n, N, W)))


class _AdaStack:
    """The AdaLN projections (`ada` = SiLU, Linear(W, 6W)) of every block of a trunk, stacked into one weight: they
    all act on the same time vector, so one GEMM per step gives every block's gates, shifts and scales."""

    def __init__(self, blocks):
        self.width = blocks[0].ada[1].in_features
        self.weight = torch.cat([b.ada[1].weight.detach() for b in blocks], 0)
        self.bias = torch.cat([b.ada[1].bias.detach() for b in blocks], 0)

    def __call__(self, time):
        out = torch.nn.functional.linear(torch.nn.functional.silu(time), self.weight, self.bias)
        return out.view(len(time), -1, 6 * self.width).unbind(1)


def _ada_stack(trunk):
    blocks = list(trunk.blocks)
    if not blocks or not all(hasattr(b, 'ada') and isinstance(b.ada[0], torch.nn.SiLU) for b in blocks):
        return None
    return _AdaStack(blocks)


class StepForward:
    """FastSlotForward.forward for the model `model` (the reference's StreamingControlNet / compact form, or a
    module with the same attributes: backbone, control, cross, zero, layer_map) over the cached context `context`
    (one layer per control block). Weights are used in their own dtype under bf16 autocast. The patch tables and
    the stacked AdaLN projections are taken from the weights when the object is built (as the reference's
    GatherPatch tables are); build a new one after loading other weights."""

    def __init__(self, model, context, concurrent=True):
        self.model, self.context = model, context
        self.side = torch.cuda.Stream(device=context.lengths.device) if concurrent else None
        bb, cc = model.backbone, model.control
        self.patch_b, self.patch_c = GatherPatch(bb.target_patch), GatherPatch(cc.target_patch)
        self.layer_map = getattr(model, 'layer_map', None) or {i: i for i in range(bb.depth)}
        self.timed = hasattr(bb, 'time_encoding')
        self.ada_b = _ada_stack(bb) if self.timed else None
        self.ada_c = _ada_stack(cc) if self.timed else None
        if len(model.cross) != context.layers:
            raise ValueError('the context needs one layer per cross-attention')

    @torch.inference_mode()
    def __call__(self, tokens, timestep, origin, group_origin):
        """tokens int64 [n, Y, Z, X], timestep [n], origin [n, 3], group_origin [3] (XYZ) -> PatchLogits of the
        class head (n windows)."""
        with torch.autocast('cuda', dtype=torch.bfloat16):
            return self._forward(tokens, timestep, origin, group_origin)

    def _injection(self, i, j, b, c, bt, ct, sa_positions, positions, mod_b, mod_c):
        """Backbone block i with control block j injected (fast_ops.py:293-298): the control branch on the side
        stream (when there is one) while the backbone block runs on the current stream."""
        model = self.model
        bb, cc = model.backbone, model.control

        def control(c):
            c = block_forward(cc.blocks[j], c, ct, sa_positions, mod_c)
            c = cross_step(model.cross[j], c, positions, self.context, j)
            return c, model.zero[j](c).to(torch.bfloat16)

        if self.side is None:
            c, z = control(c)
            return residual_norm(block_forward(bb.blocks[i], b, bt, sa_positions, mod_b), z), c
        main = torch.cuda.current_stream()
        self.side.wait_stream(main)
        with torch.cuda.stream(self.side):
            c, z = control(c)
        b = block_forward(bb.blocks[i], b, bt, sa_positions, mod_b)
        main.wait_stream(self.side)
        c.record_stream(main)
        z.record_stream(main)
        return residual_norm(b, z), c

    def _two_streams(self, b, c, bt, ct, sa_positions, positions, mod_b, mod_c):
        """The control chain on the side stream, an event after each zero projection; the backbone on the current
        stream, waiting for event j before adding projection j after backbone block layer_map^-1(j)."""
        model = self.model
        bb, cc = model.backbone, model.control
        main = torch.cuda.current_stream()
        self.side.wait_stream(main)
        zs = []
        with torch.cuda.stream(self.side):
            for j in range(len(cc.blocks)):
                c = block_forward(cc.blocks[j], c, ct, sa_positions, mod_c[j])
                c = cross_step(model.cross[j], c, positions, self.context, j)
                z = model.zero[j](c).to(torch.bfloat16)
                done = torch.cuda.Event()
                done.record(self.side)
                zs.append((z, done))
        for i in range(bb.depth):
            b = block_forward(bb.blocks[i], b, bt, sa_positions, mod_b[i])
            j = self.layer_map.get(i)
            if j is not None:
                z, done = zs[j]
                main.wait_event(done)
                z.record_stream(main)
                b = residual_norm(b, z)
        main.wait_stream(self.side)
        return b

    def _forward(self, tokens, timestep, origin, group_origin):
        model = self.model
        bb, cc = model.backbone, model.control
        n = len(tokens)
        centers = bb.patch_centers_xyz[None] + origin[:, None]
        positions = (centers - group_origin[None, None]) / 4
        sa_positions = bb.patch_centers_xyz[None].expand(n, -1, -1) / 4
        y = 2 * (centers[..., 1:2] - bb.y_range[0]) / (bb.y_range[1] - bb.y_range[0]) - 1
        b = residual_norm(self.patch_b(tokens), bb.y_embed(y).to(torch.bfloat16))
        c = residual_norm(self.patch_c(tokens), cc.y_embed(y).to(torch.bfloat16))
        bt = bb.time_encoding(timestep) if self.timed else None
        ct = cc.time_encoding(timestep) if self.timed else None
        mod_b = self.ada_b(bt) if self.ada_b is not None else [None] * bb.depth
        mod_c = self.ada_c(ct) if self.ada_c is not None else [None] * len(cc.blocks)
        if self.side is None:
            for i in range(bb.depth):
                j = self.layer_map.get(i)
                if j is None:
                    b = block_forward(bb.blocks[i], b, bt, sa_positions, mod_b[i])
                    continue
                b, c = self._injection(i, j, b, c, bt, ct, sa_positions, positions, mod_b[i], mod_c[j])
        else:
            b = self._two_streams(b, c, bt, ct, sa_positions, positions, mod_b, mod_c)
        if self.timed:
            shift, gain = bb.final_ada(bt).chunk(2, -1)
            h = layer_norm(b, bb.final_norm, shift, gain)
        else:
            h = layer_norm(b, bb.final_norm)
        patches = bb.class_head(h)
        return PatchLogits(patches, bb.voxel_shape, bb.patch_size, bb.num_classes)
