"""GPU parity of the cross-attention kernel against the float64 oracle, through the C ABI.

Tolerances (stated per the hot-path contract): bf16 Q/K/V -> max-abs error <= 2e-2 and relative (max error /
max |reference|) <= 1e-2 against float64 on the same bf16 inputs; e4m3 K/V -> <= 5e-2 against float64 on the
dequantised K/V."""
import math

import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu

BF16_ATOL, BF16_RTOL = 2e-2, 1e-2
FP8_ATOL = 5e-2


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def make_qkv(B, H, Q, kcap, D, seed, scale=None):
    g = torch.Generator().manual_seed(seed)
    s = 1 / math.sqrt(D) if scale is None else scale
    q = (torch.randn(B, H, Q, D, generator=g) * s).to(torch.bfloat16)
    k = (torch.randn(B, H, kcap, D, generator=g) * s).to(torch.bfloat16)
    v = (torch.randn(B, H, kcap, D, generator=g) * s).to(torch.bfloat16)
    return q, k, v


def check(got, ref, atol, rtol=None):
    err = (got.double().cpu() - ref).abs().max().item()
    assert err <= atol, err
    if rtol is not None:
        assert err / ref.abs().max().item() <= rtol, (err, ref.abs().max().item())


@pytest.mark.parametrize('D', [64, 48, 96, 128, 72])
def test_padded_variable_lengths(dev, D):
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 4, 3, 200, 700
    lengths = [1, 63, 700, 257]
    _case(f'xattn padded D={D} lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=D)
    ref = A.cross_attention(q, k, v, lengths)
    out = attention(q.to(dev), k.to(dev), v.to(dev), lengths=torch.tensor(lengths, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    check(out, ref, BF16_ATOL, BF16_RTOL)


def test_zero_length_window_gives_zeros_and_padding_is_ignored(dev):
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap, D = 3, 2, 64, 256, 64
    lengths = [0, 100, 256]
    _case('xattn zero length + padding garbage')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=1)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    out1 = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)
    k2, v2 = k.clone(), v.clone()
    k2[1, :, 100:] = 1e4
    v2[1, :, 100:] = float('nan')
    v2[0] = float('nan')
    out2 = attention(q.to(dev), k2.to(dev), v2.to(dev), lengths=lt)
    torch.cuda.synchronize()
    assert torch.all(out1[0] == 0)
    assert torch.equal(out1, out2)


@pytest.mark.parametrize('D', [64, 96])
def test_packed_cu_seqlens_and_transposed_v(dev, D):
    from streamvoxel_amd.stream.attention import attention
    H, Q = 4, 130
    lengths = [1552, 37, 1024 * 3 + 1552, 65]
    B = len(lengths)
    _case(f'xattn packed cu_seqlens D={D} lengths={lengths}')
    g = torch.Generator().manual_seed(4)
    total = sum(lengths)
    kp = (torch.randn(H, total, D, generator=g) / 8).to(torch.bfloat16)
    vp = (torch.randn(H, total, D, generator=g) / 8).to(torch.bfloat16)
    q = (torch.randn(B, H, Q, D, generator=g) / 8).to(torch.bfloat16)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    ref = A.cross_attention_packed(q, kp, vp, cu)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    out = attention(q.to(dev), kp.to(dev), vp.to(dev), cu_seqlens=cu_t)
    # V stored transposed ([H, D, total]) and passed as a [H, total, D] view: the fast staging path.
    vt = vp.transpose(1, 2).contiguous().to(dev)
    out_t = attention(q.to(dev), kp.to(dev), vt.transpose(1, 2), cu_seqlens=cu_t)
    torch.cuda.synchronize()
    check(out, ref, BF16_ATOL, BF16_RTOL)
    assert torch.equal(out, out_t)


def test_strided_query_and_output_layouts(dev):
    """Q produced as [B,Q,H,D] (the projection's layout) and O written straight into [B,Q,H,D]."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap, D = 2, 12, 1024, 2600, 64
    lengths = [2600, 1552]
    _case('xattn strided q/o [B,Q,H,D]')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=7)
    qd = q.transpose(1, 2).contiguous().to(dev).transpose(1, 2)        # [B,H,Q,D] view of [B,Q,H,D]
    out_buf = torch.empty((B, Q, H, D), dtype=torch.bfloat16, device=dev)
    attention(qd, k.to(dev), v.to(dev), lengths=torch.tensor(lengths, dtype=torch.int32, device=dev),
              out=out_buf.transpose(1, 2))
    torch.cuda.synchronize()
    ref = A.cross_attention(q, k, v, lengths)
    check(out_buf.transpose(1, 2), ref, BF16_ATOL, BF16_RTOL)


def test_config_c2_shape_one_layer(dev):
    """8 windows, 12 heads x 64, 1024 queries, L_b = 1552 + 1024 k_b: checked on a subset of heads and queries
    against float64."""
    from streamvoxel_amd.stream.attention import attention
    g = torch.Generator().manual_seed(123)
    kb = torch.randint(0, 9, (8,), generator=g)
    lengths = (1552 + 1024 * kb).tolist()
    B, H, Q, D, kcap = 8, 12, 1024, 64, 9856
    _case(f'xattn C2 lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=99)
    out = attention(q.to(dev), k.to(dev), v.to(dev), lengths=torch.tensor(lengths, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    sel_h = [0, 5, 11]
    ref = A.cross_attention(q[:, sel_h, ::7], k[:, sel_h], v[:, sel_h], lengths)
    check(out.cpu()[:, sel_h, ::7], ref, BF16_ATOL, BF16_RTOL)


def test_768_wide_model_shape_direct_vt(dev):
    """The 768-wide model's cross-attention: 8 windows, 8 heads x 96, 1024 queries, up to 12 576 keys in a
    12 672-key cache with V stored transposed (direct staging at head_dim 96); a subset of heads and queries
    checked against float64."""
    from streamvoxel_amd.stream.attention import attention
    g = torch.Generator().manual_seed(321)
    kb = torch.randint(0, 9, (8,), generator=g)
    lengths = (256 * 16 + 288 + 1024 * kb).tolist()
    B, H, Q, D, kcap = 8, 8, 1024, 96, 12672
    _case(f'xattn 768-wide D=96 lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=77)
    vt = v.transpose(2, 3).contiguous().to(dev)
    out = attention(q.to(dev), k.to(dev), vt.transpose(2, 3),
                    lengths=torch.tensor(lengths, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    sel_h = [0, 7]
    ref = A.cross_attention(q[:, sel_h, ::9], k[:, sel_h], v[:, sel_h], lengths)
    check(out.cpu()[:, sel_h, ::9], ref, BF16_ATOL, BF16_RTOL)


@pytest.mark.parametrize('p_dtype', ['e4m3', 'bf16'])
@pytest.mark.parametrize('D', [64, 96, 128])
def test_fp8_e4m3_cached_kv(dev, D, p_dtype):
    from streamvoxel_amd.stream.attention import attention, quantize_e4m3
    if not hasattr(torch, 'float8_e4m3fn'):
        pytest.skip('torch without float8_e4m3fn')
    B, H, Q, kcap = 3, 4, 256, 1100
    lengths = [1100, 517, 64]
    _case(f'xattn fp8 e4m3 K/V D={D} P={p_dtype}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=5)
    kc, ks = quantize_e4m3(k.float())
    vc, vs = quantize_e4m3(v.float())
    kd = A.dequant_e4m3(kc.view(torch.uint8), ks[:, :, None, None])
    vd = A.dequant_e4m3(vc.view(torch.uint8), vs[:, :, None, None])
    ref = A.cross_attention(q, kd, vd, lengths)
    out = attention(q.to(dev), kc.to(dev), vc.to(dev), lengths=torch.tensor(lengths, dtype=torch.int32, device=dev),
                    k_scale=ks.to(dev), v_scale=vs.to(dev), p_dtype=p_dtype)
    vt = vc.view(torch.uint8).transpose(2, 3).contiguous().to(dev).transpose(2, 3).view(torch.float8_e4m3fn)
    out_t = attention(q.to(dev), kc.to(dev), vt, lengths=torch.tensor(lengths, dtype=torch.int32, device=dev),
                      k_scale=ks.to(dev), v_scale=vs.to(dev), p_dtype=p_dtype)
    torch.cuda.synchronize()
    # V here is small (std 1/sqrt(D)): the bar is also held relative to the output's scale
    check(out, ref, FP8_ATOL, FP8_ATOL)
    assert torch.equal(out, out_t)
    # and against the unquantised inputs, the contract's looser bound
    check(out, A.cross_attention(q, k, v, lengths), FP8_ATOL)


def test_fp8_decode_is_exact_for_every_code(dev):
    """One key per window and K = 0: the output is the dequantised V row itself, so every finite e4m3 code must
    come out as its exact value (all e4m3 values are bf16 values), pinned by the format table of the oracle."""
    from streamvoxel_amd.stream.attention import attention
    if not hasattr(torch, 'float8_e4m3fn'):
        pytest.skip('torch without float8_e4m3fn')
    codes = torch.tensor([c for c in range(256) if c not in (0x7f, 0xff)], dtype=torch.uint8)
    B, H, Q, D, kcap = 4, 1, 8, 64, 64
    _case('xattn fp8 decode table')
    v = torch.zeros(B, H, kcap, D, dtype=torch.uint8)
    # window b, key 0, head_dim d holds code index 64 b + d
    flat = torch.zeros(B * D, dtype=torch.uint8)
    flat[:codes.numel()] = codes
    v[:, 0, 0, :] = flat.reshape(B, D)
    k = torch.zeros(B, H, kcap, D, dtype=torch.uint8)
    q = torch.zeros(B, H, Q, D, dtype=torch.bfloat16)
    ones = torch.ones(B, H, dtype=torch.float32, device=dev)
    out = attention(q.to(dev), k.to(dev), v.to(dev), lengths=torch.ones(B, dtype=torch.int32, device=dev),
                    k_scale=ones, v_scale=ones)
    torch.cuda.synchronize()
    expect = A.dequant_e4m3(v[:, :, 0, :], 1.0)                      # [B, H, D] float64
    got = out.cpu().double()[:, :, 0, :]
    assert torch.equal(got, expect), (got - expect).abs().max()


@pytest.mark.parametrize('D', [64, 48, 96, 128, 88, 112])
def test_transposed_v_padded_layout_fast_path(dev, D):
    """V stored transposed in a padded [B,H,D,Kcap] buffer (the cached-context layout) takes the direct-to-LDS
    staging: full blocks, a partial last block, a window shorter than one block; NaN in the padding must not
    leak, and the result must equal the row-major-V path (V rows in LDS, read transposed) bit for bit."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 4, 3, 160, 448
    lengths = [448, 100, 64, 7]
    _case(f'xattn direct V^T D={D} lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=11 + D)
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    vt = v.transpose(2, 3).contiguous()
    kg = k.clone()
    for b, n in enumerate(lengths):
        vt[b, :, :, n:] = float('nan')
        kg[b, :, n:] = float('nan')
    vt_dev = vt.to(dev)
    out_direct = attention(q.to(dev), kg.to(dev), vt_dev.transpose(2, 3), lengths=lt)
    out_rows = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)
    torch.cuda.synchronize()
    check(out_direct, ref, BF16_ATOL, BF16_RTOL)
    assert torch.equal(out_direct, out_rows)


@pytest.mark.parametrize('D', [64, 48, 32, 8])
def test_direct_staging_every_block_count(dev, D):
    """Direct staging alternates two LDS tile pairs and peels the last full block and the partial one: windows of
    0..10 full blocks, with and without a partial last block, cover every entry into and exit from its unrolled
    loop and both tile parities at the end. The result must match the float64 oracle and equal the row-major-V
    path (also direct, V rows read transposed) bit for bit; every key block carries its own score scale and value
    offset, so a block read from the wrong tile changes the result."""
    from streamvoxel_amd.stream.attention import attention
    lengths = [64 * n + t for n in range(11) for t in (0, 29) if 64 * n + t > 0]
    B, H, Q, kcap = len(lengths), 2, 96, 704
    _case(f'xattn direct block counts D={D} lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=101 + D)
    block = torch.arange(kcap) // 64
    k = (k.float() * (1 + 0.37 * (block % 5)).view(1, 1, -1, 1)).to(torch.bfloat16)
    v = (v.float() + 0.05 * block.view(1, 1, -1, 1)).to(torch.bfloat16)
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    vt = v.transpose(2, 3).contiguous().to(dev)
    out_direct = attention(q.to(dev), k.to(dev), vt.transpose(2, 3), lengths=lt)
    out_rows = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)
    torch.cuda.synchronize()
    check(out_direct, ref, BF16_ATOL, BF16_RTOL)
    assert torch.equal(out_direct, out_rows)


@pytest.mark.parametrize('transposed,D', [(True, 64), (False, 64), (True, 96)])
def test_score_scale_jumps_between_key_halves(dev, transposed, D):
    """Score magnitudes that jump up and down between 32-key halves (K rows scaled by 1 .. 90 and down to 1e-3):
    the running max must be raised mid-window (after lower halves) and hold through much lower halves, on the
    direct (V^T) and the register-staged path; the windows end inside a half, on a half and inside a block."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 3, 2, 96, 640
    lengths = [640, 333, 47]
    _case(f'xattn score jumps transposed={transposed} D={D} lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=29)
    factors = torch.tensor([1.0, 30.0, 0.01, 90.0, 2.0, 0.3, 60.0, 0.001])
    half = torch.arange(kcap) // 32
    k = (k.float() * factors[half % 8][None, None, :, None]).to(torch.bfloat16)
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    vv = v.transpose(2, 3).contiguous().to(dev).transpose(2, 3) if transposed else v.to(dev)
    out = attention(q.to(dev), k.to(dev), vv, lengths=lt)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    check(out, ref, BF16_ATOL, BF16_RTOL)


@pytest.mark.parametrize('jump', [12.0, 30.0, 100.0, 1000.0])
def test_second_product_taken_back_on_score_jumps(dev, jump):
    """Scores (in nats) that jump by `jump`, 2 `jump`, ... above the window's earlier ones at keys past the first
    half, so that a half's second product was issued against a running max that no longer bounds it: from a few
    clamped weights (12) to weights far beyond the fp32 range against the stale max (1000). Within the bf16 bar
    of float64, and the same bits on every staging at head_dim 64: V^T direct, V rows, the packed layout, and a
    prefix key mask."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap, D = 2, 2, 64, 640, 64
    lengths = [640, 333]
    _case(f'xattn score jumps of {jump} nats after the first half, every staging')
    g = torch.Generator().manual_seed(int(jump))
    logits = torch.randn(B, H, kcap, generator=g)
    for i, key in enumerate([40, 100, 170, 300, 600]):
        logits[:, :, key] += jump * (i + 1)
    q = torch.zeros(B, H, Q, D)
    q[..., 0] = 1.0
    q[..., 1:] = torch.randn(B, H, Q, D - 1, generator=g) * 0.1
    k = torch.randn(B, H, kcap, D, generator=g) * 0.1
    k[..., 0] = logits * math.sqrt(D)          # the score of key j is logits[j] plus a little per query
    v = torch.randn(B, H, kcap, D, generator=g)
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    qd, kd = q.to(dev), k.to(dev)
    vt = v.transpose(2, 3).contiguous().to(dev).transpose(2, 3)
    direct = attention(qd, kd, vt, lengths=lt)
    rows = attention(qd, kd, v.to(dev), lengths=lt)
    masked = attention(qd, kd, vt, key_mask=torch.arange(kcap, device=dev)[None] < lt[:, None])
    cu = torch.tensor([0, lengths[0], sum(lengths)], dtype=torch.int32, device=dev)
    kp = torch.cat([k[i, :, :lengths[i]] for i in range(B)], 1).to(dev)
    vpt = torch.cat([v[i, :, :lengths[i]] for i in range(B)], 1).transpose(1, 2).contiguous().to(dev)
    packed = attention(qd, kp, vpt.transpose(1, 2), cu_seqlens=cu)
    torch.cuda.synchronize()
    assert torch.isfinite(direct.float()).all()
    check(direct, ref, BF16_ATOL, BF16_RTOL)
    assert torch.equal(direct, rows)
    assert torch.equal(direct, masked)
    assert torch.equal(direct, packed)


@pytest.mark.parametrize('p_dtype', ['e4m3', 'bf16'])
@pytest.mark.parametrize('transposed,D', [(True, 64), (False, 64), (True, 48), (True, 96)])
def test_e4m3_score_jumps_between_key_halves(dev, transposed, D, p_dtype):
    """The score jumps above with an e4m3 cache: the running max rises inside a block's second half after the first
    half's P is already packed for the fp8 second product (which must then take half 0 down by the rise), and
    holds through much lower halves; with the ones row (D=48) and without."""
    from streamvoxel_amd.stream.attention import attention, quantize_e4m3
    B, H, Q, kcap = 3, 2, 96, 640
    lengths = [640, 333, 47]
    _case(f'xattn e4m3 score jumps transposed={transposed} D={D} lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=31)
    factors = torch.tensor([1.0, 30.0, 0.01, 90.0, 2.0, 0.3, 60.0, 0.001])
    half = torch.arange(kcap) // 32
    kc, ks = quantize_e4m3(k.float() * factors[half % 8][None, None, :, None])
    vc, vs = quantize_e4m3(v.float())
    kd = A.dequant_e4m3(kc.view(torch.uint8), ks[:, :, None, None])
    vd = A.dequant_e4m3(vc.view(torch.uint8), vs[:, :, None, None])
    ref = A.cross_attention(q, kd, vd, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    if transposed:
        vv = vc.view(torch.uint8).transpose(2, 3).contiguous().to(dev).transpose(2, 3).view(torch.float8_e4m3fn)
    else:
        vv = vc.to(dev)
    out = attention(q.to(dev), kc.to(dev), vv, lengths=lt, k_scale=ks.to(dev), v_scale=vs.to(dev), p_dtype=p_dtype)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    check(out, ref, FP8_ATOL)


@pytest.mark.parametrize('kv', ['bf16', 'e4m3', 'e4m3-pbf16'])
@pytest.mark.parametrize('L', [64, 100, 128])
def test_single_hot_key_returns_its_value_row(dev, kv, L):
    """Window b has one key (b mod L) whose score dwarfs the others and V rows that name their key (V[k, d] = 1 iff
    d = k mod 64): the output of every window must be exactly its hot key's row, so any mismatch between the order
    of the scores and the order of the V^T columns in the second product shows up as the wrong row."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, D = L, 1, 4, 64
    _case(f'xattn single hot key kv={kv} L={L}')
    hot = torch.arange(B) % L
    q = torch.zeros(B, H, Q, D)
    q[..., 0] = 1.0
    k = torch.zeros(B, H, L, D)
    k[torch.arange(B), 0, hot, 0] = 448.0
    v = torch.zeros(B, H, L, D)
    keys = torch.arange(L)
    v[:, 0, keys, keys % D] = 1.0
    lt = torch.full((B,), L, dtype=torch.int32, device=dev)
    qd = q.to(torch.bfloat16).to(dev)
    vt = v.transpose(2, 3).contiguous().transpose(2, 3)
    if kv == 'bf16':
        out = attention(qd, k.to(torch.bfloat16).to(dev), vt.to(torch.bfloat16).to(dev), lengths=lt)
    else:
        ones = torch.ones(B, H, device=dev)
        vt8 = vt.to(torch.float8_e4m3fn).view(torch.uint8).to(dev).view(torch.float8_e4m3fn)
        out = attention(qd, k.to(torch.float8_e4m3fn).to(dev), vt8, lengths=lt, k_scale=ones, v_scale=ones,
                        p_dtype='bf16' if kv == 'e4m3-pbf16' else 'e4m3')
    torch.cuda.synchronize()
    got = out.float().cpu()[:, 0, 0].argmax(-1)
    expect = hot % D
    # A window whose hot key is k >= 64 holds the same row as window k - 64: the key is told apart by its window.
    bad = (got != expect).nonzero().flatten().tolist()
    print(f'[gpu-case] hot-key mismatches (window: got, expected): '
          f'{[(b, int(got[b]), int(expect[b])) for b in bad[:16]]}', flush=True)
    worst = (out.float().cpu()[:, 0] - torch.nn.functional.one_hot(expect, D).float()[:, None]).abs().amax((1, 2))
    print(f'[gpu-case] hot-key windows off by more than 1e-3: {(worst > 1e-3).nonzero().flatten().tolist()[:32]}',
          flush=True)
    assert not bad
    want = torch.nn.functional.one_hot(expect, D).float()[:, None].expand(B, Q, D)
    assert (out.float().cpu()[:, 0] - want).abs().max().item() <= 1e-3


# The default e4m3 form (bf16 softmax weights) holds the fp8 bar at every logit scale. The opt-in fp8 second
# product (p_dtype='e4m3', SVHIP_FP8_E4M3_PFP8) rounds every softmax weight to e4m3 (relative 2^-4); the row sum is
# taken over the rounded weights, so a single dominant key cancels and the error grows with the weight shared by a
# few keys: within the bar up to logit standard deviation 2, 7.6e-2 measured at 4, which is why it is not the
# default. Its documented accuracy there:
PFP8_OPT_IN_STD4 = 1e-1


@pytest.mark.parametrize('p_dtype', ['bf16', 'e4m3'])
@pytest.mark.parametrize('D', [64, 48])
def test_e4m3_sharp_softmax_rows(dev, D, p_dtype):
    """Logit standard deviations 1, 2 and 4 over an e4m3 cache, against float64 on the dequantised cache: the
    default form within the fp8 bar throughout."""
    from streamvoxel_amd.stream.attention import attention, quantize_e4m3
    B, H, Q, kcap = 2, 2, 256, 2048
    lengths = [2048, 1500]
    g = torch.Generator().manual_seed(37)
    for std in (1.0, 2.0, 4.0):
        _case(f'xattn e4m3 sharp rows D={D} P={p_dtype} logit std={std}')
        q = torch.randn(B, H, Q, D, generator=g).to(torch.bfloat16)
        k = torch.randn(B, H, kcap, D, generator=g) * std
        v = torch.randn(B, H, kcap, D, generator=g)
        kc, ks = quantize_e4m3(k)
        vc, vs = quantize_e4m3(v)
        kd = A.dequant_e4m3(kc.view(torch.uint8), ks[:, :, None, None])
        vd = A.dequant_e4m3(vc.view(torch.uint8), vs[:, :, None, None])
        ref = A.cross_attention(q, kd, vd, lengths)
        vt = vc.view(torch.uint8).transpose(2, 3).contiguous().to(dev).transpose(2, 3).view(torch.float8_e4m3fn)
        out = attention(q.to(dev), kc.to(dev), vt, lengths=torch.tensor(lengths, dtype=torch.int32, device=dev),
                        k_scale=ks.to(dev), v_scale=vs.to(dev), p_dtype=p_dtype)
        torch.cuda.synchronize()
        err = (out.double().cpu() - ref).abs().max().item()
        print(f'[gpu-case] e4m3 D={D} P={p_dtype} logit std={std}: |kernel - f64| {err:.2e}', flush=True)
        opt_in_outside_bar = p_dtype == 'e4m3' and std > 2.0
        assert err <= (PFP8_OPT_IN_STD4 if opt_in_outside_bar else FP8_ATOL), (std, err)


@pytest.mark.parametrize('B,H', [(300, 1), (256, 3)])
def test_many_windows(dev, B, H):
    """More windows than the kernel ranks by length (300: natural order), exactly as many (256), and a window x head
    count that is not a multiple of the 8 XCDs (300 x 1) or is (256 x 3)."""
    from streamvoxel_amd.stream.attention import attention
    Q, kcap, D = 40, 200, 32
    g = torch.Generator().manual_seed(B)
    lengths = torch.randint(0, kcap + 1, (B,), generator=g).tolist()
    _case(f'xattn many windows B={B} H={H}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=B + H)
    ref = A.cross_attention(q, k, v, lengths)
    out = attention(q.to(dev), k.to(dev), v.to(dev), lengths=torch.tensor(lengths, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    check(out, ref, BF16_ATOL, BF16_RTOL)


def _masked_reference(q, k, v, mask, lengths=None):
    """float64 attention of every window over exactly its attended keys (mask True, below the length): the
    oracle's attention over the gathered keys; a window-query with no attended key gets zeros."""
    B, H, Q, D = q.shape
    out = torch.zeros((B, H, Q, D), dtype=torch.float64)
    for b in range(B):
        keep = mask[b].clone()
        if lengths is not None:
            keep[int(lengths[b]):] = False
        idx = keep.nonzero().squeeze(1)
        if len(idx) == 0:
            continue
        out[b:b + 1] = A.cross_attention(q[b:b + 1], k[b:b + 1, :, idx], v[b:b + 1, :, idx], [len(idx)])
    return out


@pytest.mark.parametrize('D', [64, 48, 96, 128])
@pytest.mark.parametrize('transposed', [False, True])
def test_key_mask_any_pattern(dev, D, transposed):
    """svhip_xattn_fwd_masked: random masks, a first block wholly masked, a window wholly masked (zeros), with and
    without lengths, V row-major and transposed."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 4, 3, 200, 300
    _case(f'xattn key mask D={D} transposed={transposed}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=100 + D)
    g = torch.Generator().manual_seed(D)
    mask = torch.rand(B, kcap, generator=g) < 0.5
    mask[1, :70] = False                     # the first block and a half without an attended key
    mask[2] = False                          # nothing attended: zeros
    mask[3, :] = False
    mask[3, 299] = True                      # one key, in the partial last block
    vd = v.to(dev)
    if transposed:
        vd = vd.transpose(2, 3).contiguous().transpose(2, 3)
    for lengths in (None, [300, 250, 10, 300]):
        lt = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=dev)
        out = attention(q.to(dev), k.to(dev), vd, lengths=lt, key_mask=mask.to(dev))
        torch.cuda.synchronize()
        ref = _masked_reference(q, k, v, mask, lengths)
        check(out, ref, BF16_ATOL, BF16_RTOL)
        assert torch.all(out[2] == 0)



@pytest.mark.parametrize('D', [64, 48])
def test_key_mask_first_attended_keys_far_below_zero(dev, D):
    """A wave whose queries see no attended key in the first blocks, then only keys whose scores lie far below 0
    (about -150 in natural units, -217 in log2 units, where exp2 of the score underflows against a running max of
    0): the first attended key must set the running max, so that the output is the softmax over those keys and not
    zeros. Row sums from the matrix cores (D = 64) and from the ones row (D = 48)."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 2, 2, 96, 400
    _case(f'xattn key mask, far negative scores after masked blocks D={D}')
    g = torch.Generator().manual_seed(7 + D)
    q = (4.0 * torch.ones(B, H, Q, D) + 0.05 * torch.randn(B, H, Q, D, generator=g)).to(torch.bfloat16)
    # scale 1/sqrt(D): q . k = -4 D (4.7 + 0.2 n) / sqrt(D), about -150 at D = 64 with a spread of a few units
    depth = (4.7 * 8 / math.sqrt(D) + 0.2 * torch.randn(B, H, kcap, 1, generator=g))
    k = (-depth * torch.ones(B, H, kcap, D)).to(torch.bfloat16)
    v = torch.randn(B, H, kcap, D, generator=g).to(torch.bfloat16)
    mask = torch.rand(B, kcap, generator=g) < 0.6
    mask[0, :150] = False                    # two whole blocks and more without an attended key
    mask[1, :64] = False                     # exactly the first block
    out = attention(q.to(dev), k.to(dev), v.to(dev), key_mask=mask.to(dev))
    torch.cuda.synchronize()
    ref = _masked_reference(q, k, v, mask)
    scores = (q[0, 0, 0].double() @ k[0, 0, 150:160].double().t()) / math.sqrt(D)
    assert float(scores.max()) < -100, scores
    assert ref.abs().amax((2, 3)).min() > 0.1        # the reference is not zeros
    check(out, ref, BF16_ATOL, BF16_RTOL)

def test_key_mask_prefix_equals_lengths_and_packed(dev):
    """A prefix mask gives the bits of the length form; the packed cu_seqlens layout takes the mask per window."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap, D = 3, 4, 130, 520, 64
    lengths = [520, 77, 1]
    _case('xattn key mask prefix == lengths; packed + mask')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=7)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    prefix = torch.arange(kcap, device=dev)[None] < lt[:, None]
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    a = attention(qd, kd, vd, lengths=lt)
    b = attention(qd, kd, vd, key_mask=prefix)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # packed: window b's keys at rows cu[b] .. cu[b + 1], a random mask per window
    cu = torch.tensor([0, 520, 597, 598], dtype=torch.int32)
    kp = torch.cat([k[i, :, :lengths[i]] for i in range(B)], 1)
    vp = torch.cat([v[i, :, :lengths[i]] for i in range(B)], 1)
    mask = torch.rand(B, kcap, generator=torch.Generator().manual_seed(3)) < 0.7
    mask[2, 0] = True
    out = attention(qd, kp.to(dev), vp.to(dev), cu_seqlens=cu.to(dev), key_mask=mask.to(dev))
    torch.cuda.synchronize()
    check(out, _masked_reference(q, k, v, mask, lengths), BF16_ATOL, BF16_RTOL)


@pytest.mark.parametrize('D', [64, 48, 96, 128, 32])
def test_row_major_v_every_block_count_padded_packed_and_registers(dev, D):
    """Row-major V stays one key a row in LDS and the second product reads it transposed (ds_read_b64_tr_b16):
    direct loads in the padded and in the packed cu_seqlens layout, and in the key-mask kernel (an all-true mask). Windows of
    0..10 full blocks with and without a partial one (every key block its own score scale and value offset, NaN in
    the padding past each window); all three forms must match the float64 oracle and give the bits of the V^T
    layout."""
    from streamvoxel_amd.stream.attention import attention
    lengths = [64 * n + t for n in range(11) for t in (0, 37) if 64 * n + t > 0]
    B, H, Q, kcap = len(lengths), 2, 96, 704
    _case(f'xattn row-major V (direct, packed, key mask) D={D} lengths={lengths}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=301 + D)
    block = torch.arange(kcap) // 64
    k = (k.float() * (1 + 0.29 * (block % 7)).view(1, 1, -1, 1)).to(torch.bfloat16)
    v = (v.float() + 0.04 * (block % 5).view(1, 1, -1, 1)).to(torch.bfloat16)
    ref = A.cross_attention(q, k, v, lengths)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    vt = v.transpose(2, 3).contiguous().to(dev)
    qd, kd = q.to(dev), k.to(dev)
    out_vt = attention(qd, kd, vt.transpose(2, 3), lengths=lt)
    vn = v.clone()
    for b, n in enumerate(lengths):
        vn[b, :, n:] = float('nan')
    out_rows = attention(qd, kd, vn.to(dev), lengths=lt)
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(lengths).cumsum(0)
    kp = torch.cat([k[b, :, :lengths[b]] for b in range(B)], 1).to(dev)
    vp = torch.cat([v[b, :, :lengths[b]] for b in range(B)], 1).to(dev)
    out_packed = attention(qd, kp, vp, cu_seqlens=cu.to(dev))
    every = torch.ones(B, kcap, dtype=torch.bool, device=dev)
    out_mask = attention(qd, kd, v.to(dev), lengths=lt, key_mask=every)
    torch.cuda.synchronize()
    check(out_rows, ref, BF16_ATOL, BF16_RTOL)
    assert torch.equal(out_rows, out_vt)
    assert torch.equal(out_packed, out_vt)
    assert torch.equal(out_mask, out_vt)


@pytest.mark.parametrize('D', [64, 48])
def test_kv_as_views_of_the_projection_output(dev, D):
    """K and V as the views `local_kv` returns (streamvoxel/stream/fast_ops.py:90-95): [B, L, 2, H, D] projection
    output, K = [:, :, 0] and V = [:, :, 1] transposed to [B, H, L, D], so consecutive keys lie 2 H D elements apart
    and the heads D apart. Row-major V from such a view takes the direct loads; the result must match float64 and
    give the bits of the same K/V made contiguous."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, L = 3, 4, 100, 333
    lengths = [333, 200, 64]
    _case(f'xattn K/V as projection views D={D}')
    g = torch.Generator().manual_seed(77 + D)
    kv = (torch.randn(B, L, 2, H, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    q = (torch.randn(B, H, Q, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    kvd = kv.to(dev)
    k_view, v_view = kvd[:, :, 0].transpose(1, 2), kvd[:, :, 1].transpose(1, 2)    # [B, H, L, D] views
    assert k_view.stride(2) == 2 * H * D and v_view.stride(1) == D
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    out_view = attention(q.to(dev), k_view, v_view, lengths=lt)
    out_dense = attention(q.to(dev), k_view.contiguous(), v_view.contiguous(), lengths=lt)
    torch.cuda.synchronize()
    k = kv[:, :, 0].transpose(1, 2).contiguous()
    v = kv[:, :, 1].transpose(1, 2).contiguous()
    check(out_view, A.cross_attention(q, k, v, lengths), BF16_ATOL, BF16_RTOL)
    assert torch.equal(out_view, out_dense)

@pytest.mark.parametrize('D', [64, 48, 96])
def test_key_mask_row_major_v_whole_blocks(dev, D):
    """A key mask over row-major V skips the blocks it wholly masks and computes the blocks it wholly attends as
    without a mask: masks that alternate whole masked, whole attended and mixed blocks (and a window that starts
    with masked blocks) must match the float64 oracle and give the bits of the same mask over V^T, which masks
    every block's scores."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 4, 3, 130, 640
    _case(f'xattn key mask over row-major V, whole blocks D={D}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=401 + D)
    g = torch.Generator().manual_seed(9 + D)
    blk = torch.arange(kcap) // 64
    mixed = torch.rand(B, kcap, generator=g) < 0.6
    mask = torch.where((blk % 3 == 0)[None], torch.zeros(B, kcap, dtype=torch.bool),
                       torch.where((blk % 3 == 1)[None], torch.ones(B, kcap, dtype=torch.bool), mixed))
    mask[1, :200] = False                   # three whole blocks and more before the first attended key
    mask[2] = True                          # every key attended
    mask[3, 320:] = False                   # a masked tail of whole blocks
    lengths = [640, 600, 411, 640]
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    qd, kd = q.to(dev), k.to(dev)
    md = mask.to(dev)
    out_rows = attention(qd, kd, v.to(dev), lengths=lt, key_mask=md)
    out_vt = attention(qd, kd, v.transpose(2, 3).contiguous().to(dev).transpose(2, 3), lengths=lt, key_mask=md)
    torch.cuda.synchronize()
    check(out_rows, _masked_reference(q, k, v, mask, lengths), BF16_ATOL, BF16_RTOL)
    assert torch.equal(out_rows, out_vt)


@pytest.mark.parametrize('D', [64, 48, 96, 80, 128, 112])
def test_key_mask_register_staging_gives_the_direct_bits(dev, D):
    """The key-mask kernels that stage K/V through registers (V^T of the packed cu_seqlens layout; padded V^T whose
    rows of keys are an odd number of elements apart, read without vectors) against the direct-loaded padded V^T
    under the same mask: whole masked, whole attended and mixed blocks; the same bits, within the bf16 bar of
    float64."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 3, 2, 100, 600
    lengths = [600, 333, 130]
    _case(f'xattn key mask through registers D={D}')
    q, k, v = make_qkv(B, H, Q, kcap, D, seed=501 + D)
    g = torch.Generator().manual_seed(13 + D)
    blk = torch.arange(kcap) // 64
    mixed = torch.rand(B, kcap, generator=g) < 0.5
    mask = torch.where((blk % 3 == 0)[None], torch.zeros(B, kcap, dtype=torch.bool),
                       torch.where((blk % 3 == 1)[None], torch.ones(B, kcap, dtype=torch.bool), mixed))
    mask[2, 100] = True
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    qd, kd, md = q.to(dev), k.to(dev), mask.to(dev)
    out_vt = attention(qd, kd, v.transpose(2, 3).contiguous().to(dev).transpose(2, 3), lengths=lt, key_mask=md)
    wide = torch.zeros(B, H, D, kcap + 3, dtype=torch.bfloat16)
    wide[..., :kcap] = v.transpose(2, 3)
    vt_odd = wide.to(dev)[..., :kcap].transpose(2, 3)  # V^T rows kcap + 3 elements apart: no 16-byte runs
    assert vt_odd.stride(3) % 2 == 1
    out_odd = attention(qd, kd, vt_odd, lengths=lt, key_mask=md)
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(lengths).cumsum(0)
    kp = torch.cat([k[b, :, :lengths[b]] for b in range(B)], 1).to(dev)
    vpt = torch.cat([v[b, :, :lengths[b]] for b in range(B)], 1).transpose(1, 2).contiguous().to(dev)
    out_packed_vt = attention(qd, kp, vpt.transpose(1, 2), cu_seqlens=cu.to(dev), key_mask=md)
    torch.cuda.synchronize()
    check(out_vt, _masked_reference(q, k, v, mask, lengths), BF16_ATOL, BF16_RTOL)
    assert torch.equal(out_odd, out_vt)
    assert torch.equal(out_packed_vt, out_vt)


def test_row_major_v_past_32_bit_offsets(dev):
    """Row-major V whose keys lie 16 MiB apart, so that a (window, head)'s keys span more than 4 GiB: past the 32-bit
    offsets of the direct loads, it is staged through registers (64-bit addresses). Head widths 48-128 (one to
    four output tiles, with and without the ones column), with and without a key mask: the bits of the same V made
    contiguous (direct loads), within the bf16 bar of float64."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap, Dmax = 2, 2, 64, 300, 128
    key_stride = 1 << 23                               # elements: 299 keys span 5.0 GB
    lengths = [300, 171]
    _case(f'xattn row-major V, keys {2 * key_stride} bytes apart, kv_cap {kcap}')
    storage = torch.empty((kcap - 1) * key_stride + B * H * Dmax, dtype=torch.bfloat16, device=dev)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(12)
    mask = torch.rand(B, kcap, generator=g) < 0.6
    mask[:, 64:128] = True
    mask[:, 192:256] = False
    md = mask.to(dev)
    try:
        for D in (48, 64, 80, 96, 112, 128):
            q, k, v = make_qkv(B, H, Q, kcap, D, seed=700 + D)
            v_far = storage.as_strided((B, H, kcap, D), (H * Dmax, Dmax, key_stride, 1))
            v_far.copy_(v.to(dev))
            assert (kcap - 1) * v_far.stride(2) * 2 >= 1 << 32
            qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
            out_far = attention(qd, kd, v_far, lengths=lt)
            out_near = attention(qd, kd, vd, lengths=lt)
            mask_far = attention(qd, kd, v_far, lengths=lt, key_mask=md)
            mask_near = attention(qd, kd, vd, lengths=lt, key_mask=md)
            torch.cuda.synchronize()
            check(out_far, A.cross_attention(q, k, v, lengths), BF16_ATOL, BF16_RTOL)
            check(mask_far, _masked_reference(q, k, v, mask, lengths), BF16_ATOL, BF16_RTOL)
            assert torch.equal(out_far, out_near), D
            assert torch.equal(mask_far, mask_near), D
    finally:
        del storage
        torch.cuda.empty_cache()


def test_mask_lengths_cut_windows_at_their_last_attended_key(dev):
    """svhip_mask_lengths: 1 + the last attended key of each window among its first min(kv_len, kv_cap) keys, 0
    when none; aligned rows (16-byte vector reads) and unaligned ones (a slice of a wider mask: byte reads), with
    and without kv_len, 300 windows, attended keys only in a row's last 16-byte chunk, only in its tail bytes,
    only at key 0, none."""
    import ctypes
    from streamvoxel_amd import _lib
    lib = _lib.load()
    _case('svhip_mask_lengths')
    B, kcap = 300, 1000
    g = torch.Generator().manual_seed(5)
    base = torch.rand(B, kcap + 8, generator=g) < 0.01
    base[0] = False                                    # nothing attended
    base[1] = False
    base[1, 0] = True                                  # only key 0
    base[2] = False
    base[2, 990] = True                                # in the last whole 16-byte chunk of an aligned row
    base[3] = False
    base[3, 998] = True                                # in the tail past the last whole chunk
    kv_len = torch.randint(0, kcap + 40, (B,), generator=g, dtype=torch.int32)
    for mask in (base[:, :kcap].contiguous(), base[:, 3:kcap + 3]):      # aligned rows; rows 3 bytes in, stride 1008
        md = mask.to(dev) if mask.is_contiguous() else base.to(dev)[:, 3:kcap + 3]
        for lens in (None, kv_len):
            out = torch.empty(B, dtype=torch.int32, device=dev)
            lp = None if lens is None else lens.to(dev)
            rc = lib.svhip_mask_lengths(ctypes.c_void_p(md.data_ptr()), md.stride(0), _lib.ptr(lp), B, kcap,
                                        ctypes.c_void_p(out.data_ptr()), None)
            assert rc == 0, lib.svhip_last_error()
            torch.cuda.synchronize()
            n = torch.full((B,), kcap) if lens is None else lens.clamp(0, kcap)
            want = torch.zeros(B, dtype=torch.int32)
            for b in range(B):
                hit = mask[b, :int(n[b])].nonzero()
                want[b] = int(hit[-1]) + 1 if len(hit) else 0
            assert torch.equal(out.cpu(), want), (out.cpu() - want).abs().max()


@pytest.mark.parametrize('D', [64, 48])
def test_sharp_softmax_rows_take_no_extra_query_rounding(dev, D):
    """Sharp softmax rows (attention logits of standard deviation 4 and 8): the kernel stays within the bf16 bar of
    the float64 attention of its bf16 inputs, and much closer to it than the float64 attention of a query rounded
    once more after scaling by scale * log2(e) is (a scaled-query pre-rounding, which the scores would inherit,
    moves the output by that gap on these rows: measured 1.9e-2 / 5.3e-2 at head_dim 64)."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 2, 4, 128, 1000
    lengths = [1000, 517]
    for std in (4.0, 8.0):
        _case(f'xattn sharp rows D={D} logit std={std}')
        g = torch.Generator().manual_seed(61 + D)
        q = torch.randn(B, H, Q, D, generator=g).to(torch.bfloat16)
        k = (torch.randn(B, H, kcap, D, generator=g) * std).to(torch.bfloat16)
        v = torch.randn(B, H, kcap, D, generator=g).to(torch.bfloat16)
        sl2 = torch.tensor((1 / math.sqrt(D)) * 1.4426950408889634, dtype=torch.float32)
        q_pre = (q.float() * sl2).to(torch.bfloat16).double() / sl2.double()
        ref = A.cross_attention(q, k, v, lengths)
        gap = (A.cross_attention(q_pre, k, v, lengths) - ref).abs().max().item()
        out = attention(q.to(dev), k.to(dev), v.to(dev),
                        lengths=torch.tensor(lengths, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        err = (out.double().cpu() - ref).abs().max().item()
        print(f'[gpu-case] D={D} std={std}: |kernel - f64| {err:.2e}, pre-rounded query gap {gap:.2e}', flush=True)
        assert err <= BF16_ATOL, (std, err)
        if std == 8.0:
            assert err <= 0.5 * gap, (err, gap)
