"""Oracle restatement of the cross-attention operand producers (test infrastructure only, see oracle/__init__.py).

* `rope_frequencies`, `axial_rope`: AxialRoPE (models/unconditional_md4.py:10-24). Phases are fp32 products of the
  fp32 positions and frequencies; sin and cos are evaluated in fp32 and cast to the activations' dtype; the
  rotation is computed in that dtype, one rounding per product and per sum, which is what the module does under
  bf16 autocast.
* `window_kv`: one window of the cached context as FastSlotForward.encode + _write build it
  (stream/fast_ops.py:90-95, 228-250): [prefix keys ; local keys, K rotated at the local positions], zeros after.
* `quantize_e4m3`: per-head scale amax / 448 clamped at 1e-12, codes = (x / scale) in float8_e4m3fn
  (scripts/bench_ops.py:505-522 for the convention).
"""
from __future__ import annotations

import torch


def rope_frequencies(head_dim, base=10000.0):
    """fp32 [head_dim / 6]: base^(-2i / (head_dim / 3)), i < head_dim / 6 (unconditional_md4.py:11-16)."""
    if head_dim % 6:
        raise ValueError('head_dim must give every axis an even width')
    axis = head_dim // 3
    return base ** (-torch.arange(0, axis, 2).float() / axis)


def axial_rope(x, positions, frequencies):
    """x [B,H,N,D] (float dtype), positions [B,N,3] -> rotated x in x's dtype (unconditional_md4.py:18-24). The
    phases are the fp32 positions times the frequencies buffer in the promotion of fp32 and the buffer's dtype, as
    the module computes them: fp32 for the fp32 buffer, fp64 for a module cast to double."""
    n_freq = frequencies.numel()
    D = x.shape[-1]
    if D != 6 * n_freq:
        raise ValueError((D, n_freq))
    out = torch.empty_like(x)
    if not frequencies.is_floating_point() or frequencies.dtype.itemsize < 4:
        frequencies = frequencies.float()
    for axis in range(3):
        theta = positions[..., axis].float()[..., None] * frequencies      # [B, N, n_freq]
        s = theta.sin()[:, None].to(x.dtype)
        c = theta.cos()[:, None].to(x.dtype)
        lo = axis * 2 * n_freq
        first = x[..., lo:lo + 2 * n_freq:2]
        second = x[..., lo + 1:lo + 2 * n_freq:2]
        out[..., lo:lo + 2 * n_freq:2] = first * c - second * s
        out[..., lo + 1:lo + 2 * n_freq:2] = first * s + second * c
    return out


def window_kv(prefix_k, prefix_v, local_k, local_v, positions, frequencies, kv_cap):
    """[H,P,D] prefix banks, [H,L,D] local projections (bf16), positions [L,3] or None -> K, V [H, kv_cap, D] with
    the local K rotated (when positions are given) and zeros past P + L."""
    H, P, D = prefix_k.shape
    L = local_k.shape[1]
    if P + L > kv_cap:
        raise ValueError('Condition exceeds the slot capacity')
    k = torch.zeros(H, kv_cap, D, dtype=local_k.dtype)
    v = torch.zeros(H, kv_cap, D, dtype=local_v.dtype)
    lk = local_k if positions is None else axial_rope(local_k[None], positions[None], frequencies)[0]
    k[:, :P], v[:, :P] = prefix_k, prefix_v
    k[:, P:P + L], v[:, P:P + L] = lk, local_v
    return k, v


def quantize_e4m3(x, keys):
    """Per-head e4m3 of x [H, kv_cap, D] over its first `keys` keys: (codes uint8 [H, kv_cap, D], scale fp32 [H])."""
    amax = x[:, :keys].float().abs().amax(dim=(1, 2)) if keys else torch.zeros(x.shape[0])
    scale = torch.clamp(amax / 448.0, min=1e-12)
    codes = (x.float() / scale[:, None, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    return codes, scale
