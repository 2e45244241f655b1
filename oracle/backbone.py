"""Oracle restatement of the transformer blocks (test infrastructure only, see oracle/__init__.py).

Everything in float64 on the CPU from a block's parameters, given as the reference module's state-dict names
(`norm1.weight`, `attn.qkv.weight`, `attn.proj.bias`, `mlp.0.weight`, `mlp.2.bias`, `ada.1.weight`, ...):

* `layer_norm`: nn.LayerNorm, (x - mean) / sqrt(biased var + eps) [* weight + bias].
* `modulate`: x * (1 + scale) + shift per window (models/unconditional_md4_timefree.py:12-13).
* `gelu`: nn.GELU's exact form 0.5 x (1 + erf(x / sqrt 2)); `silu`: x / (1 + e^-x).
* `rotary_attention`: RotaryAttention.forward (unconditional_md4_timefree.py:41-47): qkv projection split as
  [3, H, D], AxialRoPE of Q and K (producer.axial_rope, here in float64), softmax(Q K^T / sqrt D) V over all tokens,
  output projection.
* `block`: UnconditionalBlock.forward with time (AdaLN, unconditional_md4_timefree.py:60-63) or without
  (affine LayerNorm, unconditional_md4.py:52-56).
* `patch_embed`: the patchify Conv3d of the one-hot tokens (unconditional_md4_timefree.py:141-147) as the sum of
  the weight columns the tokens pick (stream/fast_ops.py:54-75, GatherPatch), by explicit loops over the patches.
* `time_encoding`, `step_forward`: the time features (unconditional_md4_timefree.py:119-125) and one generation
  step's forward of the streaming ControlNet (stream/fast_ops.py:274-308), composed from the functions above.
"""
from __future__ import annotations

import math

import torch

from oracle import attention as A
from oracle import producer as P

F64 = torch.float64


def _d(t):
    return None if t is None else t.detach().to(F64)


def layer_norm(x, eps, weight=None, bias=None):
    x = _d(x)
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    y = (x - mean) / torch.sqrt(var + eps)
    if weight is not None:
        y = y * _d(weight)
        if bias is not None:
            y = y + _d(bias)
    return y


def modulate(x, shift, scale):
    return _d(x) * (1 + _d(scale)[:, None]) + _d(shift)[:, None]


def gelu(x):
    x = _d(x)
    return 0.5 * x * (1 + torch.erf(x / math.sqrt(2.0)))


def silu(x):
    x = _d(x)
    return x / (1 + torch.exp(-x))


def linear(x, weight, bias=None):
    y = torch.matmul(_d(x), _d(weight).t())
    return y if bias is None else y + _d(bias)


def rotary_attention(x, positions, params, heads, prefix='attn.'):
    """x [B,N,W] -> [B,N,W] float64; positions [B,N,3]."""
    b, n, w = x.shape
    D = w // heads
    qkv = linear(x, params[prefix + 'qkv.weight'], params[prefix + 'qkv.bias']).reshape(b, n, 3, heads, D)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    freq = params.get(prefix + 'rope.frequencies', P.rope_frequencies(D))
    q = P.axial_rope(q, positions, freq)
    k = P.axial_rope(k, positions, freq)
    o = A.cross_attention(q, k, v, [n] * b)
    return linear(o.transpose(1, 2).reshape(b, n, w), params[prefix + 'proj.weight'], params[prefix + 'proj.bias'])


def mlp(x, params):
    return linear(gelu(linear(x, params['mlp.0.weight'], params['mlp.0.bias'])), params['mlp.2.weight'],
                  params['mlp.2.bias'])


def block(x, time, positions, params, heads, eps=1e-6):
    """UnconditionalBlock.forward in float64. time [B,W] or None."""
    x = _d(x)
    if time is None:
        h = layer_norm(x, eps, params.get('norm1.weight'), params.get('norm1.bias'))
        x = x + rotary_attention(h, positions, params, heads)
        return x + mlp(layer_norm(x, eps, params.get('norm2.weight'), params.get('norm2.bias')), params)
    s1, c1, g1, s2, c2, g2 = linear(silu(time), params['ada.1.weight'], params['ada.1.bias']).chunk(6, -1)
    x = x + g1[:, None] * rotary_attention(modulate(layer_norm(x, eps), s1, c1), positions, params, heads)
    return x + g2[:, None] * mlp(modulate(layer_norm(x, eps), s2, c2), params)


def patch_embed(tokens, weight, bias, patch):
    """tokens int [B,Y,Z,X] in [0, C+1); weight [W, C+1, p, p, p]; bias [W] or None -> [B, N, W] float64 with patch
    token n row-major over (Y/p, Z/p, X/p): bias + sum over the kernel offsets (dy, dz, dx) of
    weight[:, tokens[p*gy + dy, p*gz + dz, p*gx + dx], dy, dz, dx]."""
    B, Y, Z, X = tokens.shape
    W = weight.shape[0]
    w = _d(weight)
    gy, gz, gx = Y // patch, Z // patch, X // patch
    out = torch.zeros(B, gy * gz * gx, W, dtype=F64)
    for b in range(B):
        for n in range(gy * gz * gx):
            py, pz, px = n // (gz * gx), (n // gx) % gz, n % gx
            acc = torch.zeros(W, dtype=F64)
            for dy in range(patch):
                for dz in range(patch):
                    for dx in range(patch):
                        cell = int(tokens[b, py * patch + dy, pz * patch + dz, px * patch + dx])
                        acc += w[:, cell, dy, dz, dx]
            out[b, n] = acc if bias is None else acc + _d(bias)
    return out


def _sub(params, prefix):
    return {k[len(prefix):]: v for k, v in params.items() if k.startswith(prefix)}


def time_encoding(t, params, time_dim, time_free=False):
    """UnconditionalMD4DiT.time_encoding (unconditional_md4_timefree.py:119-125): sinusoidal features of t formed
    in fp32 as the module forms them, then time_mlp (Linear, GELU, Linear) and time_projection (SiLU, Linear) in
    float64; a time-free model returns its `constant_time` for every window."""
    if time_free:
        return _d(params['constant_time'])[None].expand(len(t), -1)
    half = time_dim // 8
    # The module forms the frequencies, the phases and their sines and cosines in fp32.
    freq = torch.exp(-math.log(10000.0) * torch.arange(half).float() / half)
    phase = torch.as_tensor(t).float()[:, None] * freq
    h = _d(torch.cat((phase.sin(), phase.cos()), -1))
    h = linear(gelu(linear(h, params['time_mlp.0.weight'], params['time_mlp.0.bias'])), params['time_mlp.2.weight'],
               params['time_mlp.2.bias'])
    return linear(silu(h), params['time_projection.1.weight'], params['time_projection.1.bias'])


def step_forward(params, tokens, timestep, origin, group_origin, keys, values, lengths, *, depth, heads,
                 control_heads, layer_map, patch, y_range, time_dim, voxel_shape, timed=True, time_free=False):
    """FastSlotForward.forward (stream/fast_ops.py:274-308) in float64 from the model's state dict `params`
    (backbone.*, control.*, cross.*, zero.*): gather patchify + height embedding, the backbone blocks with the
    control block, cross attention over keys[j] / values[j] [n, H, Kcap, D] (first lengths[b] keys of window b)
    and zero projection at every mapped block, final LayerNorm (AdaLN-modulated when `timed`, affine otherwise),
    class head. timed: the AdaLN blocks of unconditional_md4_timefree.py (time_free: the constant time), else the
    affine blocks of unconditional_md4.py. Returns the head's rows [n, N, p^3 C]."""
    bb, cc = _sub(params, 'backbone.'), _sub(params, 'control.')
    centers = _d(bb['patch_centers_xyz'])[None] + _d(origin)[:, None]
    positions = (centers - _d(group_origin)[None, None]) / 4
    n = len(tokens)
    sa_positions = _d(bb['patch_centers_xyz'])[None].expand(n, -1, -1) / 4
    y = 2 * (centers[..., 1:2] - y_range[0]) / (y_range[1] - y_range[0]) - 1

    def embed(tp):
        x = patch_embed(tokens, tp['target_patch.weight'], tp['target_patch.bias'], patch)
        e = linear(silu(linear(y, tp['y_embed.0.weight'], tp['y_embed.0.bias'])), tp['y_embed.2.weight'],
                   tp['y_embed.2.bias'])
        return x + e

    b, c = embed(bb), embed(cc)
    bt = time_encoding(timestep, bb, time_dim, time_free) if timed else None
    ct = time_encoding(timestep, cc, time_dim, time_free) if timed else None
    for i in range(depth):
        b_next = block(b, bt, sa_positions.float(), _sub(bb, f'blocks.{i}.'), heads)
        j = layer_map.get(i)
        if j is not None:
            c = block(c, ct, sa_positions.float(), _sub(cc, f'blocks.{j}.'), control_heads)
            cp = _sub(params, f'cross.{j}.')
            W = c.shape[-1]
            D = W // control_heads
            q = linear(layer_norm(c, 1e-6), cp['query.weight'], cp['query.bias'])
            q = q.reshape(n, -1, control_heads, D).transpose(1, 2)
            q = P.axial_rope(q, positions.float(), cp.get('rope.frequencies', P.rope_frequencies(D)))
            o = A.cross_attention(q, keys[j], values[j], lengths)
            c = c + linear(o.transpose(1, 2).reshape(n, -1, W), cp['proj.weight'], cp['proj.bias'])
            b_next = b_next + linear(c, params[f'zero.{j}.weight'], params[f'zero.{j}.bias'])
        b = b_next
    if timed:
        shift, gain = linear(silu(bt), bb['final_ada.1.weight'], bb['final_ada.1.bias']).chunk(2, -1)
        h = modulate(layer_norm(b, 1e-6), shift, gain)
    else:
        h = layer_norm(b, 1e-6, bb.get('final_norm.weight'), bb.get('final_norm.bias'))
    return linear(h, bb['class_head.weight'], bb['class_head.bias'])
