"""Oracle restatement of the cross-attention core over packed, variable-length cached K/V.

Test infrastructure only (see oracle/__init__.py).

Reference forms restated:
  * `SlotCrossAttention.forward` (stream/engine.py:28-47) and `cross_sdpa` (stream/fast_ops.py:111-115): SDPA with a
    boolean key mask `[B,1,1,K]`, default scale 1/sqrt(D);
  * `cross_flex` + `PackedKeys` (stream/fast_ops.py:104-108, 122-159): FlexAttention over keys `k < lengths[b]`.
Both compute O[b,h,q] = sum_{k < L_b} softmax_k(Q[b,h,q] . K[b,h,k] * scale) V[b,h,k].
"""
from __future__ import annotations

import math

import torch


def cross_attention(q, k, v, lengths, scale=None, dtype=torch.float64):
    """Per-slot exact attention over the first `lengths[b]` keys, computed in `dtype` on the CPU.

    q [B,H,Q,D]; k, v [B,H,Kcap,D] (padded, valid keys first); lengths int [B]. Returns [B,H,Q,D] in `dtype`.
    A slot of length 0 yields zeros (there is nothing to attend to; the HIP kernel writes zeros too)."""
    B, H, Q, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.zeros((B, H, Q, D), dtype=dtype)
    for b in range(B):
        n = int(lengths[b])
        if n == 0:
            continue
        qb = q[b].to(dtype)
        kb = k[b, :, :n].to(dtype)
        vb = v[b, :, :n].to(dtype)
        s = torch.matmul(qb, kb.transpose(-1, -2).contiguous()) * scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p, vb)
    return out


def cross_attention_packed(q, k_packed, v_packed, cu_seqlens, scale=None, dtype=torch.float64):
    """The same over a packed key layout: k/v [H, sum L, D] with slot b at rows cu_seqlens[b]:cu_seqlens[b+1]."""
    B = len(cu_seqlens) - 1
    lengths = [int(cu_seqlens[b + 1]) - int(cu_seqlens[b]) for b in range(B)]
    kcap = max(lengths + [1])
    H, _, D = k_packed.shape
    k = torch.zeros((B, H, kcap, D), dtype=k_packed.dtype)
    v = torch.zeros((B, H, kcap, D), dtype=v_packed.dtype)
    for b in range(B):
        lo, hi = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        k[b, :, :hi - lo] = k_packed[:, lo:hi]
        v[b, :, :hi - lo] = v_packed[:, lo:hi]
    return cross_attention(q, k, v, lengths, scale, dtype)


def masked_sdpa(q, k, v, lengths, scale=None):
    """The reference's masked SDPA call itself (stream/engine.py:46), fp32 on the CPU: the CPU baseline's timed op."""
    B, H, Q, D = q.shape
    kcap = k.shape[2]
    valid = torch.arange(kcap)[None, :] < torch.as_tensor(lengths).reshape(-1, 1)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=valid[:, None, None, :], dropout_p=0.,
                                                            scale=scale)


def masked_sdpa_mask(q, k, v, valid, scale=None):
    """The reference's masked SDPA with any boolean key mask `valid` [B, K] (stream/fast_ops.py:111-115,
    stream/engine.py:46), on the CPU in the inputs' dtype."""
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=valid[:, None, None, :], dropout_p=0.,
                                                            scale=scale)


def cross_attention_bruteforce(q, k, v, lengths, scale=None):
    """Scalar loops (tiny inputs only): the independent check of `cross_attention`."""
    B, H, Q, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.zeros((B, H, Q, D), dtype=torch.float64)
    for b in range(B):
        n = int(lengths[b])
        for h in range(H):
            for i in range(Q):
                logits = [sum(float(q[b, h, i, d]) * float(k[b, h, j, d]) for d in range(D)) * scale for j in range(n)]
                if not logits:
                    continue
                m = max(logits)
                w = [math.exp(x - m) for x in logits]
                t = sum(w)
                for d in range(D):
                    out[b, h, i, d] = sum(w[j] * float(v[b, h, j, d]) for j in range(n)) / t
    return out


def dequant_e4m3(codes, scale):
    """OCP e4m3fn byte codes (uint8 tensor) -> float64 values times `scale` (decoded from the format definition:
    1 sign, 4 exponent (bias 7), 3 mantissa bits; exponent field 15 with mantissa 7 is NaN; no infinities)."""
    c = codes.to(torch.int64)
    sign = torch.where((c >> 7) & 1 == 1, -1.0, 1.0).to(torch.float64)
    e = (c >> 3) & 0xF
    m = (c & 0x7).to(torch.float64)
    normal = (1.0 + m / 8.0) * torch.pow(2.0, (e - 7).to(torch.float64))
    sub = (m / 8.0) * (2.0 ** -6)
    val = torch.where(e == 0, sub, normal) * sign
    val = torch.where((e == 15) & ((c & 7) == 7), torch.tensor(float('nan'), dtype=torch.float64), val)
    return val * torch.as_tensor(scale, dtype=torch.float64)
