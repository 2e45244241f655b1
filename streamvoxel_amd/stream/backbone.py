"""Transformer blocks of the MD4 backbone and of the ControlNet branch on the HIP kernels.

Reference counterparts: `RotaryAttention.forward` and `UnconditionalBlock.forward`
(streamvoxel/models/unconditional_md4_timefree.py:33-63, time-conditioned AdaLN; streamvoxel/models/
unconditional_md4.py:27-56, affine LayerNorm) and `run_block` (streamvoxel/stream/fast_ops.py:118-119), which
`FastSlotForward.forward` calls for the 25 backbone and 13 control blocks of a step (fast_ops.py:288-298).

What runs where: LayerNorm with the AdaLN modulation is `svhip_layer_norm` (one HBM pass); the gated residual
after the attention and the second LayerNorm are one `svhip_residual_norm` pass, the gated residual after the MLP
another; the qkv split, the two AxialRoPE rotations and V's transposed layout are `svhip_qkv_rope` (one pass); the
attention is `svhip_xattn_fwd` over the window's own tokens (every window attends all N keys; V^T staged straight
into LDS). The Linear layers (qkv, proj, the MLP, the AdaLN projection) and the MLP's GELU stay the block's torch
modules, as in the reference: plain library GEMMs.
"""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.stream.attention import attention

__all__ = ['layer_norm', 'residual_norm', 'qkv_rope', 'rotary_attention', 'block_forward', 'run_block']

_full_lengths = {}


def _lengths(batch, tokens, device):
    """int32 [batch] filled with `tokens` (cached: a self-attention window attends all of its tokens)."""
    key = (batch, tokens, device)
    t = _full_lengths.get(key)
    if t is None:
        t = torch.full((batch,), tokens, dtype=torch.int32, device=device)
        _full_lengths[key] = t
    return t


def _f32(p):
    return None if p is None else p.detach().to(torch.float32).contiguous()


def _rows(t, name):
    if t.dtype != torch.bfloat16 or t.dim() != 3 or t.stride(-1) != 1:
        raise ValueError(f'{name} must be bf16 [B, N, W] with a contiguous last axis')


def _window_rows(t, B, W, name):
    """A per-window [B, W] operand (gate, shift, scale) as bf16 with a contiguous last axis."""
    t = t.to(torch.bfloat16)
    if t.shape != (B, W) or t.stride(-1) != 1:
        raise ValueError(f'{name} must be [B, W] with a contiguous last axis')
    return t


def residual_norm(x, branch, gate=None, norm=None, shift=None, scale=None):
    """r = x + gate[:, None] * branch (x + branch without gate; bf16 roundings as the reference's tensors), and,
    when `norm` is given, y = norm(r) modulated by shift / scale as `layer_norm` does, in one pass. Returns r, or
    (r, y) with a norm."""
    _lib.require_gpu(x, branch, gate, shift, scale)
    _rows(x, 'x')
    _rows(branch, 'branch')
    if branch.shape != x.shape:
        raise ValueError('branch must match x')
    B, N, W = x.shape
    if gate is not None:
        gate = _window_rows(gate, B, W, 'gate')
    if (shift is None) != (scale is None):
        raise ValueError('shift and scale come together')
    if shift is not None:
        if norm is None:
            raise ValueError('shift / scale modulate the norm')
        shift, scale = _window_rows(shift, B, W, 'shift'), _window_rows(scale, B, W, 'scale')
        if shift.stride(0) != scale.stride(0):
            shift, scale = shift.contiguous(), scale.contiguous()
    r = torch.empty_like(x)
    y = None
    weight = bias = None
    eps = 0.0
    if norm is not None:
        if tuple(norm.normalized_shape) != (W,):
            raise ValueError(f'LayerNorm over {tuple(norm.normalized_shape)} does not match width {W}')
        y = torch.empty_like(x)
        weight, bias, eps = _f32(norm.weight), _f32(norm.bias), float(norm.eps)
    lib = _lib.load()
    _lib.check(lib.svhip_residual_norm(
        _lib.ptr(x), _lib.ptr(branch), _lib.ptr(gate), 0 if gate is None else gate.stride(0), _lib.ptr(r),
        _lib.ptr(y), _lib.ptr(weight), _lib.ptr(bias), _lib.ptr(shift), _lib.ptr(scale),
        0 if shift is None else shift.stride(0), B, N, W, x.stride(0), x.stride(1), branch.stride(0),
        branch.stride(1), r.stride(0), r.stride(1), 0 if y is None else y.stride(0), 0 if y is None else y.stride(1),
        eps, _lib.stream_of(x)), 'svhip_residual_norm')
    return r if y is None else (r, y)


def layer_norm(x, norm, shift=None, scale=None, out=None):
    """`norm(x)` for x [B,N,W] bf16 (nn.LayerNorm over W: its eps, and its weight / bias when affine), followed by
    the AdaLN `modulate(., shift, scale)` (unconditional_md4_timefree.py:12-13) when shift / scale [B,W] are given.
    `out` (optional, may be x) receives the bf16 result; returns it."""
    _lib.require_gpu(x, shift, scale, out)
    if x.dtype != torch.bfloat16:
        raise TypeError('x must be bfloat16')
    if x.dim() != 3 or x.stride(-1) != 1:
        raise ValueError('x must be [B, N, W] with a contiguous last axis')
    B, N, W = x.shape
    if tuple(norm.normalized_shape) != (W,):
        raise ValueError(f'LayerNorm over {tuple(norm.normalized_shape)} does not match width {W}')
    if (shift is None) != (scale is None):
        raise ValueError('shift and scale come together')
    if shift is not None:
        shift, scale = shift.to(torch.bfloat16), scale.to(torch.bfloat16)
        if shift.shape != (B, W) or scale.shape != (B, W) or shift.stride(-1) != 1 or scale.stride(-1) != 1:
            raise ValueError('shift / scale must be [B, W] with a contiguous last axis')
        if shift.stride(0) != scale.stride(0):
            scale = scale.contiguous()
            shift = shift.contiguous()
    if out is None:
        out = torch.empty_like(x)
    if out.shape != x.shape or out.dtype != torch.bfloat16 or out.stride(-1) != 1:
        raise ValueError('out must be bf16 like x')
    weight, bias = _f32(norm.weight), _f32(norm.bias)
    lib = _lib.load()
    _lib.check(lib.svhip_layer_norm(_lib.ptr(x), _lib.ptr(out), _lib.ptr(weight), _lib.ptr(bias), _lib.ptr(shift),
                                    _lib.ptr(scale), B, N, W, x.stride(0), x.stride(1), out.stride(0),
                                    out.stride(1), 0 if shift is None else shift.stride(0), float(norm.eps),
                                    _lib.stream_of(x)),
               'svhip_layer_norm')
    return out


def qkv_rope(qkv, positions, frequencies, heads):
    """The attention operands from the fused projection qkv [B,N,3W] bf16: Q and K [B,H,N,D] rotated in place
    (views of qkv) and V^T [B,H,D,Ncap] (Ncap = N rounded up to 8, its tail unused). Returns (q, k, vt)."""
    _lib.require_gpu(qkv, positions, frequencies)
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 3 or qkv.stride(-1) != 1:
        raise ValueError('qkv must be bf16 [B, N, 3W] with a contiguous last axis')
    B, N, W3 = qkv.shape
    if W3 % (3 * heads):
        raise ValueError('qkv width must be 3 * heads * head_dim')
    D = W3 // (3 * heads)
    if positions.shape != (B, N, 3):
        raise ValueError(f'positions must be [B, N, 3], got {tuple(positions.shape)}')
    if frequencies.numel() * 6 != D or frequencies.dtype != torch.float32:
        raise ValueError('frequencies must be the fp32 [head_dim / 6] buffer')
    pos = positions.float()
    pos = pos if pos.stride(-1) == 1 else pos.contiguous()
    freq = frequencies.contiguous()
    view = qkv.view(B, N, 3, heads, D)
    q, k = view[:, :, 0].transpose(1, 2), view[:, :, 1].transpose(1, 2)
    ncap = (N + 7) // 8 * 8
    vt = torch.empty((B, heads, D, ncap), dtype=torch.bfloat16, device=qkv.device)
    lib = _lib.load()
    _lib.check(lib.svhip_qkv_rope(_lib.ptr(qkv), _lib.ptr(pos), _lib.ptr(freq), B, N, heads, D, qkv.stride(0),
                                  qkv.stride(1), pos.stride(0), pos.stride(1), _lib.ptr(q), q.stride(0), q.stride(1),
                                  q.stride(2), _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2), _lib.ptr(vt),
                                  vt.stride(0), vt.stride(1), vt.stride(2), _lib.stream_of(qkv)),
               'svhip_qkv_rope')
    return q, k, vt


def rotary_attention(attn, x, positions):
    """RotaryAttention.forward (unconditional_md4_timefree.py:41-47): qkv projection, AxialRoPE of Q and K at
    `positions` [B,N,3], softmax(Q K^T / sqrt(D)) V over the window's N tokens, output projection. `attn` is the
    block's RotaryAttention (its `qkv`, `proj`, `heads`, `rope.frequencies`)."""
    b, n, d = x.shape
    heads = attn.heads
    qkv = attn.qkv(x)
    if qkv.dtype != torch.bfloat16:
        qkv = qkv.to(torch.bfloat16)
    freq = attn.rope.frequencies.to(device=qkv.device, dtype=torch.float32)
    q, k, vt = qkv_rope(qkv, positions, freq, heads)
    out = torch.empty((b, n, heads, d // heads), dtype=torch.bfloat16, device=x.device)
    attention(q, k, vt[..., :n].transpose(2, 3), lengths=_lengths(b, n, x.device), out=out.transpose(1, 2))
    return attn.proj(out.view(b, n, d))


def block_forward(block, x, time, positions, modulation=None):
    """UnconditionalBlock.forward: with `time` [B,W] the AdaLN block (unconditional_md4_timefree.py:60-63), with
    time None the affine-LayerNorm block (unconditional_md4.py:52-56). x [B,N,W] bf16, positions [B,N,3].
    `modulation` [B, 6W] (optional) is `block.ada(time)` computed beforehand (a step batches the projections of all
    blocks into one GEMM: they share the time vector)."""
    if time is None and modulation is None:
        x, h = residual_norm(x, rotary_attention(block.attn, layer_norm(x, block.norm1), positions), None, block.norm2)
        return residual_norm(x, block.mlp(h))
    s1, c1, g1, s2, c2, g2 = (block.ada(time) if modulation is None else modulation).chunk(6, -1)
    a = rotary_attention(block.attn, layer_norm(x, block.norm1, s1, c1), positions)
    x, h = residual_norm(x, a, g1, block.norm2, s2, c2)
    return residual_norm(x, block.mlp(h), g2)


def run_block(block, x, time, positions):
    """fast_ops.py:118-119."""
    return block_forward(block, x, time, positions)
