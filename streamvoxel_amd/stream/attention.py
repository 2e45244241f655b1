"""Cross attention over packed, variable-length cached K/V on the GPU.

Replaces the attention core of `cross_flex` (`flex_attention()(query, key, val, block_mask=...)`,
streamvoxel/stream/fast_ops.py:104-108) and of the masked SDPA forms (streamvoxel/stream/engine.py:28-47,
streamvoxel/stream/fast_ops.py:111-115): per window b only the first L_b keys are attended.
"""
from __future__ import annotations

import math

import torch

from streamvoxel_amd import _lib

FP8_DTYPES = tuple(getattr(torch, n) for n in ('float8_e4m3fn',) if hasattr(torch, n))


def _kv_code(t):
    if t.dtype == torch.bfloat16:
        return _lib.SVHIP_BF16
    if t.dtype in FP8_DTYPES or t.dtype == torch.uint8:
        return _lib.SVHIP_FP8_E4M3
    raise TypeError(f'K/V dtype {t.dtype} unsupported (bfloat16, float8_e4m3fn or uint8 e4m3 codes)')


def attention(query, key, val, lengths=None, cu_seqlens=None, scale=None, k_scale=None, v_scale=None, out=None,
              key_mask=None, p_dtype='bf16'):
    """softmax(scale * Q K^T) V over the first L_b keys of every window b.

    `key_mask` (optional, bf16 K/V): bool [B, Kcap] (padded) or [B, max L] (packed); key j of window b is attended
    only where it is True (any pattern; a query with no attended key gets zeros). `lengths` / `cu_seqlens` may then
    be omitted (every key up to the capacity, the mask decides).

    query [B,H,Q,D] bf16 (head_dim contiguous; any other strides). key, val: padded [B,H,Kcap,D] with
    lengths int32 [B] (device), or packed [H, sum L, D] with cu_seqlens int32 [B+1] (device). `val` may be a
    transposed view (keys contiguous, e.g. `vt.transpose(-1, -2)` of a [B,H,D,Kcap] buffer), which the kernel
    stages fastest. K/V in float8_e4m3fn (or uint8 codes) need k_scale / v_scale fp32 [B,H] (device); with them
    `p_dtype` 'bf16' (default) keeps the softmax weights in bf16 (the reference's in-kernel dequantisation, within
    5e-2 of fp32 attention over the unquantised K/V), 'e4m3' takes P . V on the fp8 matrix cores with the weights
    rounded to e4m3 (an opt-in outside that bar: every weight carries a 2^-4 relative rounding).
    `out` (optional) [B,H,Q,D] bf16 with head_dim contiguous, e.g. a [B,Q,H,D] buffer's transpose(1, 2) view.
    fp32 query, key and val (head_dim 16, 32, 48 or 64, rows 16-byte aligned) take fp32 arithmetic throughout and
    return fp32 (`svhip_xattn_fwd_f32`, or `svhip_xattn_fwd_f32_masked` with a key mask: the reference's fp32 SDPA).
    Returns out."""
    _lib.require_gpu(query, key, val, lengths, cu_seqlens, k_scale, v_scale, out)
    if query.dtype == torch.float32:
        if k_scale is not None or v_scale is not None:
            raise TypeError('fp32 attention takes no fp8 scales')
        return _attention_f32(query, key, val, lengths, cu_seqlens, scale, out, key_mask)
    if query.dtype != torch.bfloat16:
        raise TypeError('query must be bfloat16 (or float32 with float32 K/V)')
    B, H, Q, D = query.shape
    if lengths is not None and cu_seqlens is not None:
        raise ValueError('pass at most one of lengths / cu_seqlens')
    if lengths is None and cu_seqlens is None and key_mask is None:
        raise ValueError('pass lengths, cu_seqlens or key_mask')
    if key_mask is not None:
        _lib.require_gpu(key_mask)
        if key_mask.dtype != torch.bool or key_mask.dim() != 2 or key_mask.shape[0] != B or key_mask.stride(1) != 1:
            raise ValueError('key_mask must be bool [B, keys] with contiguous keys')
    code = _kv_code(key)
    if _kv_code(val) != code:
        raise TypeError('key and val must share a dtype')
    if code == _lib.SVHIP_FP8_E4M3 and (k_scale is None or v_scale is None):
        raise ValueError('fp8 K/V need k_scale and v_scale')
    if p_dtype not in ('e4m3', 'bf16'):
        raise ValueError("p_dtype is 'e4m3' or 'bf16'")
    fp8 = code == _lib.SVHIP_FP8_E4M3
    if fp8 and p_dtype == 'e4m3':
        code = _lib.SVHIP_FP8_E4M3_PFP8
    if query.stride(-1) != 1 or key.stride(-1) != 1:
        raise ValueError('query and key need a contiguous head_dim')
    if out is None:
        out = torch.empty((B, H, Q, D), dtype=torch.bfloat16, device=query.device)
    if out.shape != (B, H, Q, D) or out.stride(-1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError('out must be bf16 [B,H,Q,D] with a contiguous head_dim')
    if cu_seqlens is not None:
        if key.dim() != 3 or val.dim() != 3:
            raise ValueError('packed K/V are [H, sum L, D]')
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() != B + 1:
            raise ValueError('cu_seqlens must be int32 [B+1]')
        kcap = key.shape[1]
        sk = (0, key.stride(0), key.stride(1))
        sv = (0, val.stride(0), val.stride(1), val.stride(2))
    else:
        if key.dim() != 4 or key.shape[:2] != (B, H) or val.shape != key.shape:
            raise ValueError('padded K/V are [B,H,Kcap,D] like the query')
        if lengths is not None and (lengths.dtype != torch.int32 or lengths.numel() != B):
            raise ValueError('lengths must be int32 [B]')
        kcap = key.shape[2]
        sk = (key.stride(0), key.stride(1), key.stride(2))
        sv = (val.stride(0), val.stride(1), val.stride(2), val.stride(3))
    if key.shape[-1] != D or val.shape[-1] != D:
        raise ValueError('head_dim mismatch')
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    lib = _lib.load()
    if key_mask is not None:
        if fp8:
            raise TypeError('the key mask takes bf16 K/V')
        if cu_seqlens is None and key_mask.shape[1] < kcap:
            raise ValueError(f'key_mask holds {key_mask.shape[1]} keys per window, the cache {kcap}')
        mask_cap = kcap if cu_seqlens is None else key_mask.shape[1]
        if cu_seqlens is None:
            # The windows' lengths cut at their last attended keys (the same output): the kernel ranks the
            # windows by them, which balances the CUs when the mask, not `lengths`, holds the window lengths.
            cut = torch.empty(B, dtype=torch.int32, device=query.device)
            _lib.check(lib.svhip_mask_lengths(_lib.ptr(key_mask.view(torch.uint8)), key_mask.stride(0),
                                              _lib.ptr(lengths), B, mask_cap, _lib.ptr(cut), _lib.stream_of(query)),
                       'svhip_mask_lengths')
            lengths = cut
        _lib.check(lib.svhip_xattn_fwd_masked(
            _lib.ptr(query), _lib.ptr(key), _lib.ptr(val), _lib.ptr(out), _lib.ptr(key_mask.view(torch.uint8)),
            key_mask.stride(0), _lib.ptr(lengths), _lib.ptr(cu_seqlens), B, H, Q, D, mask_cap,
            query.stride(0), query.stride(1), query.stride(2),
            *sk, *sv, out.stride(0), out.stride(1), out.stride(2), scale, _lib.stream_of(query)),
            'svhip_xattn_fwd_masked')
        return out
    kp = key.view(torch.uint8) if fp8 else key
    vp = val.view(torch.uint8) if fp8 else val
    _lib.check(lib.svhip_xattn_fwd(
        _lib.ptr(query), _lib.ptr(kp), _lib.ptr(vp), _lib.ptr(out), code, _lib.ptr(lengths), _lib.ptr(cu_seqlens),
        _lib.ptr(k_scale), _lib.ptr(v_scale), B, H, Q, D, kcap, query.stride(0), query.stride(1), query.stride(2),
        *sk, *sv, out.stride(0), out.stride(1), out.stride(2), scale, _lib.stream_of(query)), 'svhip_xattn_fwd')
    return out


def _attention_f32(query, key, val, lengths, cu_seqlens, scale, out, key_mask=None):
    """fp32 Q/K/V -> fp32 O with fp32 arithmetic throughout (svhip_xattn_fwd_f32; with a key mask
    svhip_xattn_fwd_f32_masked, SlotCrossAttention.forward's masked SDPA, streamvoxel/stream/engine.py:28-47)."""
    if key.dtype != torch.float32 or val.dtype != torch.float32:
        raise TypeError('fp32 query takes fp32 key and val')
    B, H, Q, D = query.shape
    if lengths is not None and cu_seqlens is not None:
        raise ValueError('pass at most one of lengths / cu_seqlens')
    if key_mask is None and lengths is None and cu_seqlens is None:
        raise ValueError('pass lengths, cu_seqlens or key_mask')
    if key_mask is not None:
        _lib.require_gpu(key_mask)
        if key_mask.dtype != torch.bool or key_mask.dim() != 2 or key_mask.shape[0] != B or key_mask.stride(1) != 1:
            raise ValueError('key_mask must be bool [B, keys] with contiguous keys')
    if query.stride(-1) != 1 or key.stride(-1) != 1:
        raise ValueError('query and key need a contiguous head_dim')
    if out is None:
        out = torch.empty((B, H, Q, D), dtype=torch.float32, device=query.device)
    if out.shape != (B, H, Q, D) or out.dtype != torch.float32 or out.stride(-1) != 1:
        raise ValueError('out must be fp32 [B,H,Q,D] with a contiguous head_dim')
    if cu_seqlens is not None:
        if key.dim() != 3 or val.dim() != 3:
            raise ValueError('packed K/V are [H, sum L, D]')
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() != B + 1:
            raise ValueError('cu_seqlens must be int32 [B+1]')
        kcap = key.shape[1]
        sk = (0, key.stride(0), key.stride(1))
        sv = (0, val.stride(0), val.stride(1), val.stride(2))
    else:
        if key.dim() != 4 or key.shape[:2] != (B, H) or val.shape != key.shape:
            raise ValueError('padded K/V are [B,H,Kcap,D] like the query')
        if lengths is not None and (lengths.dtype != torch.int32 or lengths.numel() != B):
            raise ValueError('lengths must be int32 [B]')
        kcap = key.shape[2]
        sk = (key.stride(0), key.stride(1), key.stride(2))
        sv = (val.stride(0), val.stride(1), val.stride(2), val.stride(3))
    if key.shape[-1] != D or val.shape[-1] != D:
        raise ValueError('head_dim mismatch')
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    lib = _lib.load()
    if key_mask is not None:
        if cu_seqlens is None and key_mask.shape[1] < kcap:
            raise ValueError(f'key_mask holds {key_mask.shape[1]} keys per window, the cache {kcap}')
        mask_cap = kcap if cu_seqlens is None else key_mask.shape[1]
        _lib.check(lib.svhip_xattn_fwd_f32_masked(
            _lib.ptr(query), _lib.ptr(key), _lib.ptr(val), _lib.ptr(out), _lib.ptr(key_mask.view(torch.uint8)),
            key_mask.stride(0), _lib.ptr(lengths), _lib.ptr(cu_seqlens), B, H, Q, D, mask_cap,
            query.stride(0), query.stride(1), query.stride(2), *sk, *sv, out.stride(0), out.stride(1), out.stride(2),
            scale, _lib.stream_of(query)), 'svhip_xattn_fwd_f32_masked')
        return out
    _lib.check(lib.svhip_xattn_fwd_f32(
        _lib.ptr(query), _lib.ptr(key), _lib.ptr(val), _lib.ptr(out), _lib.ptr(lengths), _lib.ptr(cu_seqlens),
        B, H, Q, D, kcap, query.stride(0), query.stride(1), query.stride(2), *sk, *sv,
        out.stride(0), out.stride(1), out.stride(2), scale, _lib.stream_of(query)), 'svhip_xattn_fwd_f32')
    return out


def quantize_e4m3(x, dim_b=0, dim_h=1):
    """Per-(window, head) e4m3 quantisation of cached K or V [B,H,L,D] (or a transposed view): scale = amax / 448
    (the reference's e4m3 convention, scripts/bench_ops.py:506-522). Returns (codes float8_e4m3fn, scale fp32 [B,H]).
    Runs once per window at load time with torch ops; not on the per-step path."""
    amax = x.detach().abs().float().amax(dim=(2, 3))
    scale = torch.clamp(amax / 448.0, min=1e-12)
    codes = (x.float() / scale[:, :, None, None]).to(torch.float8_e4m3fn)
    return codes, scale.contiguous()
