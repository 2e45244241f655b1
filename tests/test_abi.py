"""CPU checks of the C ABI: the library builds/loads and exports every function include/svhip.h declares, and the
host-side argument checks reject bad input without touching a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'svhip.h')


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(svhip_[a-z0-9_]+)\s*\(', text)))


@pytest.fixture(scope='module')
def lib():
    from streamvoxel_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from streamvoxel_amd.build import build
        build()
    return _lib.load()


def test_header_declares_the_hot_path_entry_points():
    names = declared_functions()
    for expected in ('svhip_entropy', 'svhip_air_prob', 'svhip_lel_update', 'svhip_top_mask', 'svhip_quota_select',
                     'svhip_quota_select_workspace_bytes', 'svhip_ease_select', 'svhip_ease_select_workspace_bytes',
                     'svhip_xattn_fwd', 'svhip_last_error', 'svhip_version'):
        assert expected in names


def test_library_exports_every_declared_symbol(lib):
    from streamvoxel_amd import _lib
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert lib.svhip_version() >= 100


def test_workspace_queries_and_argument_errors(lib):
    n = lib.svhip_quota_select_workspace_bytes(8, 256, 16, 16, 4)
    assert n >= 8 * 1024 * 16 + 8 * 8
    assert lib.svhip_ease_select_workspace_bytes(8, 256, 16, 16, 4) >= 8 * 65536 * 4   # at least the voxel keys
    assert lib.svhip_quota_select_workspace_bytes(1, 256, 16, 16, 3) == 0          # unsupported block size
    assert b'unsupported' in lib.svhip_last_error()
    assert lib.svhip_quota_select_workspace_bytes(1, 256, 16, 12, 8) == 0          # 12 not divisible by 8
    assert b'divisible' in lib.svhip_last_error()
    # null pointers are rejected on the host (no launch happens)
    rc = lib.svhip_entropy(None, 0, 1, 256, 65536, 0, 65536, 1, None, None)
    assert rc == -1 and b'null' in lib.svhip_last_error()
    rc = lib.svhip_xattn_fwd(*([None] * 4), 1, None, None, None, None, 1, 1, 1, 64, 64, *([0] * 13), 0.125, None)
    assert rc == -1
    rc = lib.svhip_top_mask(None, None, 1, 16, None, 3, None, None)
    assert rc == -1


def test_noalloc_select_rejects_on_the_host(lib):
    # 200 windows of 65 536 voxels need about 104 MiB of scratch, more than the library's fixed 48 MiB array
    assert lib.svhip_ease_select_workspace_bytes(200, 256, 16, 16, 4) > (48 << 20)
    none = [None] * 9
    rc = lib.svhip_ease_select_noalloc(None, 0, 256, 0, 1, 256, None, 256, None, 200, 256, 16, 16, 4, *none)
    assert rc == -1 and b'scratch' in lib.svhip_last_error(), lib.svhip_last_error()
    # a geometry that fits, with null pointers: refused before the device is touched
    rc = lib.svhip_ease_select_noalloc(None, 0, 256, 0, 1, 256, None, 256, None, 8, 256, 16, 16, 4, *none)
    assert rc == -1 and b'null pointer' in lib.svhip_last_error(), lib.svhip_last_error()
    rc = lib.svhip_ease_select_noalloc(None, 0, 256, 0, 1, 256, None, 256, None, 8, 256, 16, 16, 3, *none)
    assert rc == -1 and b'unsupported' in lib.svhip_last_error()


def test_product_refuses_host_tensors():
    import torch
    from streamvoxel_amd.sampling.entropy import entropy_scores
    from streamvoxel_amd.sampling.block_quota import top_mask
    with pytest.raises(RuntimeError, match='GPU'):
        entropy_scores(torch.zeros(4, 2, 2, 2))
    with pytest.raises(RuntimeError, match='GPU'):
        top_mask(torch.zeros(8), torch.ones(8, dtype=torch.bool), 3)


def test_block_path_refuses_host_tensors():
    import torch
    from streamvoxel_amd.stream.backbone import layer_norm, qkv_rope, residual_norm
    from streamvoxel_amd.stream.forward import GatherPatch
    x = torch.zeros(1, 4, 48, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='GPU'):
        layer_norm(x, torch.nn.LayerNorm(48))
    with pytest.raises(RuntimeError, match='GPU'):
        residual_norm(x, x)
    with pytest.raises(RuntimeError, match='GPU'):
        qkv_rope(torch.zeros(1, 4, 144, dtype=torch.bfloat16), torch.zeros(1, 4, 3), torch.ones(8), 1)
    with pytest.raises(RuntimeError, match='GPU'):
        GatherPatch(torch.nn.Conv3d(3, 16, 4, stride=4))(torch.zeros(1, 4, 4, 4, dtype=torch.int64))


def test_argument_errors_of_the_newer_entry_points(lib):
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails its host checks first
    # patch order: non-power-of-two window or patch larger than the window
    rc = lib.svhip_entropy_patches(fake, 0, 1, 256, 256, 16, 12, 4, 0, 256, fake, None)
    assert rc == -1 and b'power-of-two' in lib.svhip_last_error()
    rc = lib.svhip_air_prob_patches(fake, 0, 1, 256, 256, 16, 16, 32, 0, 256, fake, 1, fake, None)
    assert rc == -1 and b'larger than the window' in lib.svhip_last_error()
    rc = lib.svhip_ease_select_patches(fake, 0, 256, 3, 0, 256, fake, 256, fake, 1, 256, 16, 16, 4, fake, fake, fake,
                                       fake, fake, fake, fake, None, fake, 1 << 30, None)
    assert rc == -1 and b'power-of-two' in lib.svhip_last_error()
    # attention: head_dim above 128 / not a multiple of 8, unknown K/V dtype, non-positive scale
    base = [fake, fake, fake, fake]

    def xattn(kv_dtype, D, scale):
        sizes = [1, 1, 128, D, 64]                                # B, H, Q, D, kv_cap
        strides = [128 * 64, 128 * 64, 64,                        # Q: b, h, q
                   64 * 64, 64 * 64, 64,                          # K: b, h, key
                   64 * 64, 64 * 64, 64, 1,                       # V: b, h, key, d
                   128 * 64, 128 * 64, 64]                        # O: b, h, q
        return lib.svhip_xattn_fwd(*base, kv_dtype, fake, None, None, None, *sizes, *strides, scale, None)

    assert xattn(1, 136, 0.125) == -1 and b'head_dim' in lib.svhip_last_error()
    assert xattn(1, 60, 0.125) == -1 and b'head_dim' in lib.svhip_last_error()
    assert xattn(7, 64, 0.125) == -1 and b'dtype' in lib.svhip_last_error()
    assert xattn(1, 64, -1.0) == -1 and b'scale' in lib.svhip_last_error()
    assert xattn(3, 64, 0.125) == -1 and b'k_scale' in lib.svhip_last_error()
    # block operands: head_dim not a multiple of 24, width not a multiple of 8, shift without scale, no residual
    rc = lib.svhip_qkv_rope(fake, fake, fake, 1, 64, 8, 64, 3 * 512 * 64, 3 * 512, 0, 3, fake, 0, 64, 3 * 512, fake,
                            0, 64, 3 * 512, fake, 8 * 64 * 64, 64 * 64, 64, None)
    assert rc == -1 and b'head_dim' in lib.svhip_last_error()
    rc = lib.svhip_layer_norm(fake, fake, None, None, None, None, 1, 4, 12, 48, 12, 48, 12, 0, 1e-6, None)
    assert rc == -1 and b'width' in lib.svhip_last_error()
    rc = lib.svhip_layer_norm(fake, fake, None, None, fake, None, 1, 4, 16, 64, 16, 64, 16, 16, 1e-6, None)
    assert rc == -1 and b'together' in lib.svhip_last_error()
    rc = lib.svhip_residual_norm(fake, None, None, 0, fake, None, None, None, None, None, 0, 1, 4, 16, 64, 16, 64, 16,
                                 64, 16, 64, 16, 1e-6, None)
    assert rc == -1 and b'null' in lib.svhip_last_error()
    # the cache writer's workspace query grows with heads and capacity
    assert lib.svhip_kv_write_workspace_bytes(16, 12672) >= lib.svhip_kv_write_workspace_bytes(8, 9792) > 0
    # mask lengths: null mask or output, negative window count or capacity
    assert lib.svhip_mask_lengths(None, 64, None, 2, 64, fake, None) == -1 and b'null' in lib.svhip_last_error()
    assert lib.svhip_mask_lengths(fake, 64, None, 2, 64, None, None) == -1 and b'null' in lib.svhip_last_error()
    assert lib.svhip_mask_lengths(fake, 64, None, -1, 64, fake, None) == -1 and b'window' in lib.svhip_last_error()
    assert lib.svhip_mask_lengths(fake, 64, None, 2, -5, fake, None) == -1 and b'kv_cap' in lib.svhip_last_error()
    assert lib.svhip_mask_lengths(fake, 64, None, 0, 64, fake, None) == 0      # nothing to do, no launch


def test_argument_errors_of_the_sampling_tail(lib):
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails its host checks first

    def sample(dtype=0, classes=256, patch=0, shape=(16, 16, 16), err=fake, logits=fake, batch=1):
        return lib.svhip_sample_chosen(logits, dtype, classes, patch, 16 ** 3 * classes, 1, classes, fake, fake, fake,
                                       fake, fake, err, batch, *shape, None)

    assert sample(classes=1025) == -1 and b'classes' in lib.svhip_last_error()
    assert sample(classes=0) == -1 and b'classes' in lib.svhip_last_error()
    assert sample(dtype=3) == -1 and b'dtype' in lib.svhip_last_error()
    assert sample(err=None) == -1 and b'null' in lib.svhip_last_error()
    assert sample(logits=None) == -1 and b'null' in lib.svhip_last_error()
    assert sample(patch=4, shape=(16, 12, 16)) == -1 and b'power-of-two' in lib.svhip_last_error()
    assert sample(patch=32) == -1 and b'larger than the window' in lib.svhip_last_error()
    assert sample(batch=-1) == -1 and b'sizes' in lib.svhip_last_error()
    # nothing to draw: returns without launching
    assert sample(batch=0) == 0 and sample(shape=(0, 16, 16)) == 0


def test_sampling_tail_refuses_host_tensors():
    import torch
    from streamvoxel_amd.stream.sampler import sample_chosen
    shape = (4, 4, 4)
    with pytest.raises(RuntimeError, match='GPU'):
        sample_chosen(torch.zeros(8, *shape), torch.zeros(shape, dtype=torch.bool), torch.zeros(1, dtype=torch.int64),
                      torch.zeros(1, dtype=torch.int64), torch.zeros(shape, dtype=torch.int16),
                      torch.zeros(1, dtype=torch.int32))


def test_argument_errors_of_the_fp32_attention(lib):
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails its host checks first
    lengths = ctypes.c_void_p(0x2000)

    def f32(D, scale=0.125, kv_len=lengths, cu=None, q=fake, sk_k=64, sv=(64 * 64, 64 * 64, 64, 1)):
        sizes = [1, 1, 128, D, 64]
        strides = [128 * 64, 128 * 64, 64, 64 * 64, 64 * 64, sk_k, *sv, 128 * 64, 128 * 64, 64]
        return lib.svhip_xattn_fwd_f32(q, fake, fake, fake, kv_len, cu, *sizes, *strides, scale, None)

    assert f32(96) == -1 and b'head_dim' in lib.svhip_last_error()
    assert f32(40) == -1 and b'head_dim' in lib.svhip_last_error()
    assert f32(64, scale=0.0) == -1 and b'scale' in lib.svhip_last_error()
    assert f32(64, kv_len=None) == -1 and b'kv_len or cu_seqlens' in lib.svhip_last_error()
    assert f32(64, cu=lengths) == -1 and b'exclusive' in lib.svhip_last_error()
    assert f32(64, q=None) == -1 and b'null' in lib.svhip_last_error()
    assert f32(64, sk_k=66) == -1 and b'16-byte' in lib.svhip_last_error()
    assert f32(64, sv=(64 * 64, 64 * 64, 2, 3)) == -1 and b'unit stride' in lib.svhip_last_error()

    def f32m(mask=lengths, kv_len=None, D=64):
        sizes = [1, 1, 128, D, 64]
        strides = [128 * 64, 128 * 64, 64, 64 * 64, 64 * 64, 64, 64 * 64, 64 * 64, 64, 1, 128 * 64, 128 * 64, 64]
        return lib.svhip_xattn_fwd_f32_masked(fake, fake, fake, fake, mask, 64, kv_len, None, *sizes, *strides,
                                              0.125, None)

    assert f32m(mask=None) == -1 and b'null key mask' in lib.svhip_last_error()
    assert f32m(D=40) == -1 and b'head_dim' in lib.svhip_last_error()
    assert f32m(kv_len=lengths, D=96) == -1 and b'head_dim' in lib.svhip_last_error()
