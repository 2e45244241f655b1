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
    freq = P.rope_frequencies(D)
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
