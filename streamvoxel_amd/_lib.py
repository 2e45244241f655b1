"""ctypes binding of libsvhip.so (the C ABI declared in include/svhip.h).

The library is built in-tree by `streamvoxel_amd.build`. There is no fallback: if the library is missing or a
call fails, a RuntimeError is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libsvhip.so')

SVHIP_F32, SVHIP_BF16, SVHIP_FP8_E4M3, SVHIP_FP8_E4M3_PFP8 = 0, 1, 3, 5
SVHIP_LEL_LAYER, SVHIP_LEL_BAND, SVHIP_LEL_COLUMN = 0, 1, 2

_c_i64, _c_i32, _c_p, _c_sz, _c_f, _c_d = (ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t,
                                             ctypes.c_float, ctypes.c_double)

# name -> (restype, argtypes); mirrors include/svhip.h
SIGNATURES = {
    'svhip_version': (ctypes.c_int, []),
    'svhip_last_error': (ctypes.c_char_p, []),
    'svhip_entropy': (ctypes.c_int, [_c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    'svhip_air_prob': (ctypes.c_int, [_c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i32,
                                      _c_p, _c_p]),
    'svhip_entropy_patches': (ctypes.c_int, [_c_p, ctypes.c_int] + [_c_i64] * 8 + [_c_p, _c_p]),
    'svhip_air_prob_patches': (ctypes.c_int, [_c_p, ctypes.c_int] + [_c_i64] * 8 + [_c_p, _c_i32, _c_p, _c_p]),
    'svhip_lel_update': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_d, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    'svhip_top_mask': (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p]),
    'svhip_quota_select_workspace_bytes': (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    'svhip_quota_select': (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p,
                                          _c_p, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    'svhip_ease_select_workspace_bytes': (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    'svhip_ease_select': (ctypes.c_int, [_c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p,
                                         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                         _c_p, _c_p, _c_p, _c_sz, _c_p]),
    'svhip_ease_select_noalloc': (ctypes.c_int, [_c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                                 _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p,
                                                 _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    'svhip_ease_select_patches': (ctypes.c_int, [_c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                                 _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p,
                                                 _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    'svhip_xattn_fwd': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, ctypes.c_int, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
                                       _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_f, _c_p]),
    'svhip_mask_lengths': (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    'svhip_xattn_fwd_masked': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p] + [_c_i64] * 18
                               + [_c_f, _c_p]),
    'svhip_xattn_fwd_f32': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p] + [_c_i64] * 18 + [_c_f, _c_p]),
    'svhip_xattn_fwd_f32_masked': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p] + [_c_i64] * 18
                                   + [_c_f, _c_p]),
    'svhip_axial_rope': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p] + [_c_i64] * 12 + [_c_p]),
    'svhip_kv_write_workspace_bytes': (_c_sz, [_c_i64, _c_i64]),
    'svhip_kv_write': (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64,
                                      _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p, _c_p, _c_p,
                                      _c_sz, _c_p]),
    'svhip_qkv_rope': (ctypes.c_int, [_c_p, _c_p, _c_p] + [_c_i64] * 8 + [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                                                       _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                                                       _c_p]),
    'svhip_layer_norm': (ctypes.c_int, [_c_p] * 6 + [_c_i64] * 8 + [_c_f, _c_p]),
    'svhip_residual_norm': (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]
                            + [_c_i64] * 12 + [_c_f, _c_p]),
    'svhip_patch_embed': (ctypes.c_int, [_c_p] * 5 + [_c_i64] * 10 + [_c_p]),
    'svhip_sample_chosen': (ctypes.c_int, [_c_p, ctypes.c_int] + [_c_i64] * 5 + [_c_p] * 6 + [_c_i64] * 4 + [_c_p]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load libsvhip.so (once) and declare the C signatures. Raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f'{LIB_PATH} is not built; run `python -m streamvoxel_amd.build` '
                                   '(or __graft_entry__.build()) first')
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc, what):
    if rc != 0:
        msg = load().svhip_last_error().decode(errors='replace')
        raise RuntimeError(f'{what} failed ({rc}): {msg}')


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    """The current HIP stream of the tensor's device, as the C ABI takes it."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors):
    """The product path runs on the GPU only; refuse host tensors instead of silently computing elsewhere."""
    for t in tensors:
        if t is not None and (not torch.is_tensor(t) or not t.is_cuda):
            raise RuntimeError('streamvoxel_amd kernels take GPU tensors (got %s); there is no CPU path'
                               % (t.device if torch.is_tensor(t) else type(t).__name__))


def dtype_code(dtype):
    if dtype == torch.float32:
        return SVHIP_F32
    if dtype == torch.bfloat16:
        return SVHIP_BF16
    raise TypeError(f'unsupported logits dtype {dtype} (float32 or bfloat16)')


def byte_span(t):
    """[first, last) device byte addresses a tensor's elements occupy (its strides taken into account)."""
    if t.numel() == 0:
        return (t.data_ptr(), t.data_ptr())
    extent = sum((n - 1) * abs(s) for n, s in zip(t.shape, t.stride())) + 1
    low = t.data_ptr() + sum((n - 1) * s for n, s in zip(t.shape, t.stride()) if s < 0) * t.element_size()
    return (low, low + extent * t.element_size())


def overlaps(a, b):
    """True when the elements of two tensors may share memory (their byte spans intersect)."""
    if a is None or b is None:
        return False
    (a0, a1), (b0, b1) = byte_span(a), byte_span(b)
    return a0 < b1 and b0 < a1
