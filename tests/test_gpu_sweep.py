"""GPU parameter sweeps: every kernel instantiation the library compiles, run against the oracle.

The kernels are templates over lanes per row, vectors per lane, layouts and storage forms, chosen at launch from the
class count, the head width, the row width and the alignment of the arguments. The workload tests exercise the
shapes the reference and the configurations use; these sweeps pick one case for every other instantiation, with the
same bars as the workload tests: entropy and air probability within 1e-5 / 2e-6 of float64 (and bit-identical
across layouts wherever one per-voxel order applies), selections bit-exact to the oracle given the kernel's scores,
attention within 2e-2 max-abs and 1e-2 relative (bf16) or 5e-2 (e4m3) of float64, LayerNorm within bf16 rounding of
float64, the gather patchify bit for bit torch's embedding bag, the K/V writer and AxialRoPE bit-exact."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import backbone as O
from oracle import producer as P
from oracle import sampling as S

pytestmark = pytest.mark.gpu

ENTROPY_ATOL, AIR_ATOL = 1e-5, 2e-6
BF16_ATOL, BF16_RTOL, FP8_ATOL = 2e-2, 1e-2, 5e-2


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def _logits(n, classes, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, classes), generator=g) * 1.5
    hot = torch.rand(n, generator=g) < 0.6
    cls = torch.randint(classes, (n,), generator=g)
    x[torch.arange(n)[hot], cls[hot]] += 9.0
    return x.to(dtype)


def _row_plans(elems):
    """One class count per (lanes per voxel, 16-byte vectors per lane) the voxel-row pass instantiates: the plan
    picks 8 lanes when they leave fewer vector slots idle than 16, for 1..128 vectors of `elems` classes."""
    seen = {}
    for vecs in range(1, 129):
        eight = math.ceil(vecs / 8) <= 8 and math.ceil(vecs / 8) * 8 - vecs < math.ceil(vecs / 16) * 16 - vecs
        lpv = 8 if eight else 16
        seen.setdefault((lpv, math.ceil(vecs / lpv)), vecs * elems)
    return sorted(seen.values())


STATS_CASES = ([(torch.float32, c) for c in _row_plans(4)] + [(torch.bfloat16, c) for c in _row_plans(8)]
               + [(torch.float32, 37), (torch.bfloat16, 13), (torch.float32, 640), (torch.bfloat16, 1000)])


# ------------------------------------------------------------------------------ entropy and air probability

@pytest.mark.parametrize('dtype,classes', STATS_CASES)
def test_stats_every_row_plan_and_layout(dev, dtype, classes):
    """Entropy and air probability from voxel rows, contiguous class planes and class planes whose rows are not
    16-byte aligned: within float64's bar, and the planes equal the rows bit for bit wherever the class count takes
    the per-voxel canonical order (a multiple of 16 bytes of classes, at most 384)."""
    from streamvoxel_amd.sampling.entropy import air_prob, entropy_batched
    B, N = 2, 1000
    _case(f'stats sweep {dtype} C={classes}')
    rows = torch.stack([_logits(N, classes, seed=classes + b, dtype=dtype) for b in range(B)])   # [B, N, C]
    planes = rows.transpose(1, 2).contiguous()
    odd = torch.zeros(B, classes, N + 1, dtype=dtype)
    odd[:, :, :N] = planes
    rd, pd, od = rows.to(dev), planes.to(dev), odd.to(dev)[:, :, :N]
    e_rows = entropy_batched(rd, layout='voxel_major')
    e_planes = entropy_batched(pd, layout='class_major')
    e_odd = entropy_batched(od, layout='class_major')
    air = torch.tensor([0, classes // 2, classes - 1], dtype=torch.int32, device=dev)
    shape = (10, 10, 10)
    a_rows = torch.stack([air_prob(rd[b].t().reshape(classes, *shape), air) for b in range(B)]).reshape(B, N)
    a_planes = torch.stack([air_prob(pd[b].reshape(classes, *shape), air) for b in range(B)]).reshape(B, N)
    a_odd = torch.stack([air_prob(od[b].reshape(classes, *shape), air) for b in range(B)]).reshape(B, N)
    torch.cuda.synchronize()
    canonical = (classes * rows.element_size()) % 16 == 0 and classes <= 384
    if canonical:
        assert torch.equal(e_planes, e_rows) and torch.equal(e_odd, e_rows)
        assert torch.equal(a_planes, a_rows) and torch.equal(a_odd, a_rows)
    for b in range(B):
        x64 = rows[b].double().numpy()
        want = S.entropy_scores_f64(x64.T)
        for got in (e_rows, e_planes, e_odd):
            assert np.abs(got[b].cpu().numpy() - want).max() < ENTROPY_ATOL
        p = np.exp(x64 - x64.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        a_want = p[:, [0, classes // 2, classes - 1]].sum(1)
        for got in (a_rows, a_planes, a_odd):
            assert np.abs(got[b].cpu().numpy() - a_want).max() < AIR_ATOL


# -------------------------------------------------------------------------------------------- fused selection

def _select_state(B, shape, b, seed):
    g = np.random.default_rng(seed)
    N = int(np.prod(shape))
    nb = N // b ** 3
    state = []
    for i in range(B):
        tops = g.integers(shape[0] // 2, shape[0] + 1, (shape[1], shape[2]))
        last = (np.arange(shape[0])[:, None, None] >= tops[None]).reshape(-1)
        done = (~last) & (g.random(N) < 0.25)
        k = int(max(1, ((~last) & ~done).sum() // 7))
        committed = int(done.sum())
        frac = (committed + k) / int((~last).sum())
        pos = S.order_to_pos(g.permutation(nb))
        state.append((last, done, k, committed, frac, pos))
    return state


SELECT_CASES = (STATS_CASES + [(torch.float32, c) for c in (300, 384)] + [(torch.bfloat16, c) for c in (272, 304, 384)])


@pytest.mark.parametrize('dtype,classes', SELECT_CASES)
def test_fused_selection_every_layout(dev, dtype, classes):
    """The fused EASE selection from voxel rows, contiguous class planes and unaligned class planes (4^3 blocks,
    mid-window state with deferred voxels and committed tokens): the chosen voxels bit-exact to the oracle's
    selection over the kernel's own scores, the scores within float64's bar, and layouts that share the per-voxel
    order giving the same scores and the same voxels."""
    from streamvoxel_amd.stream.step import EaseSelect
    B, shape, b = 2, (16, 8, 8), 4
    N = int(np.prod(shape))
    _case(f'fused select sweep {dtype} C={classes}')
    rows = torch.stack([_logits(N, classes, seed=3 * classes + i, dtype=dtype) for i in range(B)])
    planes = rows.transpose(1, 2).contiguous()
    odd = torch.zeros(B, classes, N + 1, dtype=dtype)
    odd[:, :, :N] = planes
    inputs = {'rows': rows.to(dev), 'planes': planes.to(dev), 'odd': odd.to(dev)[:, :, :N]}
    state = _select_state(B, shape, b, seed=classes)
    results = {}
    for name, x in inputs.items():
        sel = EaseSelect(B, shape, classes, b, dev)
        for i, (last, done, k, committed, frac, pos) in enumerate(state):
            sel.last[i].copy_(torch.from_numpy(last).to(dev))
            sel.tokens[i][torch.from_numpy(done).to(dev)] = 0
            sel.bind_window(i, torch.from_numpy(np.argsort(pos)).to(dev))
            sel.set_step(i, k, committed, frac)
        sel.run(x, keep_scores=True)
        torch.cuda.synchronize()
        results[name] = (sel.scores.clone(), sel.chosen.clone(), sel.bad.clone())
    canonical = (classes * rows.element_size()) % 16 == 0 and classes <= 384
    for name, (scores, chosen, bad) in results.items():
        assert not bool(bad.any()), name
        hs = scores.cpu().numpy()
        for i, (last, done, k, committed, frac, pos) in enumerate(state):
            assert np.abs(hs[i] - S.entropy_scores_f64(rows[i].double().numpy().T)).max() < ENTROPY_ATOL, name
            selectable = ~done & ~last
            nt = S.block_view((~last).reshape(shape), b).sum(1)
            want = S.quota_select_nosync(hs[i].reshape(shape), selectable.reshape(shape), k, b, pos, frac, nt,
                                         committed)
            assert np.array_equal(chosen[i].cpu().numpy().reshape(shape), want), (name, i)
        if canonical:
            assert torch.equal(scores.view(torch.int32), results['rows'][0].view(torch.int32)), name
            assert torch.equal(chosen, results['rows'][1]), name


@pytest.mark.parametrize('b', [1, 2])
def test_fused_selection_small_blocks(dev, b):
    """The fused selection at 1^3 and 2^3 blocks (the in-block pass over keys the entropy pass left)."""
    from streamvoxel_amd.stream.step import EaseSelect
    B, shape, classes = 2, (8, 8, 8), 64
    N = int(np.prod(shape))
    _case(f'fused select b={b}')
    rows = torch.stack([_logits(N, classes, seed=90 + i, dtype=torch.float32) for i in range(B)])
    state = _select_state(B, shape, b, seed=b)
    sel = EaseSelect(B, shape, classes, b, dev)
    for i, (last, done, k, committed, frac, pos) in enumerate(state):
        sel.last[i].copy_(torch.from_numpy(last).to(dev))
        sel.tokens[i][torch.from_numpy(done).to(dev)] = 0
        sel.bind_window(i, torch.from_numpy(np.argsort(pos)).to(dev))
        sel.set_step(i, k, committed, frac)
    sel.run(rows.to(dev), keep_scores=True)
    torch.cuda.synchronize()
    assert not bool(sel.bad.any())
    hs = sel.scores.cpu().numpy()
    for i, (last, done, k, committed, frac, pos) in enumerate(state):
        nt = S.block_view((~last).reshape(shape), b).sum(1)
        want = S.quota_select_nosync(hs[i].reshape(shape), (~done & ~last).reshape(shape), k, b, pos, frac, nt,
                                     committed)
        assert np.array_equal(sel.chosen[i].cpu().numpy().reshape(shape), want), i


# ------------------------------------------------------------------------------------------------- attention

ATTN_D = [16, 40, 48, 72, 80, 104, 112, 120, 128]


def _qkv(B, H, Q, kcap, D, seed):
    """Logits of standard deviation 1 (Q and K unit normal, the 1/sqrt(D) scale), V of scale 1/sqrt(D)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Q, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, kcap, D, generator=g).to(torch.bfloat16)
    v = (torch.randn(B, H, kcap, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    return q, k, v


def _check(got, ref, atol, rtol=None):
    err = (got.double().cpu() - ref).abs().max().item()
    assert err <= atol, err
    if rtol is not None:
        assert err / ref.abs().max().item() <= rtol, (err, ref.abs().max().item())


@pytest.mark.parametrize('D', ATTN_D)
@pytest.mark.parametrize('kv', ['bf16', 'e4m3', 'e4m3-pbf16'])
def test_attention_every_width_form_and_layout(dev, D, kv):
    """Every head width band (one to four 32-wide output tiles, with and without the padding row that carries the
    row sum), every cache form, and the four K/V layouts: padded with V rows, padded with V^T, packed cu_seqlens
    with V rows and with V^T. All layouts of one form give the same bits."""
    from streamvoxel_amd.stream.attention import attention, quantize_e4m3
    if kv != 'bf16' and not hasattr(torch, 'float8_e4m3fn'):
        pytest.skip('torch without float8_e4m3fn')
    B, H, Q, kcap = 2, 2, 96, 192
    lengths = [150, 61]
    _case(f'attention sweep D={D} kv={kv}')
    q, k, v = _qkv(B, H, Q, kcap, D, seed=D)
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    cu = torch.tensor([0, lengths[0], sum(lengths)], dtype=torch.int32, device=dev)
    kwargs = {}
    if kv == 'bf16':
        kc, vc = k, v
        ref = A.cross_attention(q, k, v, lengths)
        atol, rtol = BF16_ATOL, BF16_RTOL
    else:
        kc, ks = quantize_e4m3(k.float())
        vc, vs = quantize_e4m3(v.float())
        kd = A.dequant_e4m3(kc.view(torch.uint8), ks[:, :, None, None])
        vd = A.dequant_e4m3(vc.view(torch.uint8), vs[:, :, None, None])
        ref = A.cross_attention(q, kd, vd, lengths)
        atol, rtol = FP8_ATOL, None
        kwargs = dict(k_scale=ks.to(dev), v_scale=vs.to(dev), p_dtype='bf16' if kv == 'e4m3-pbf16' else 'e4m3')

    def t(x):
        return x.to(dev)

    def transposed(x):       # V stored [.., D, keys], passed as a [.., keys, D] view
        raw = x.view(torch.uint8) if x.dtype != torch.bfloat16 else x
        vt = raw.transpose(-1, -2).contiguous().transpose(-1, -2)
        return vt.view(x.dtype) if x.dtype != torch.bfloat16 else vt

    def packed(x):           # [H, sum L, D], window b at rows cu[b] .. cu[b + 1] (one scale per window and head)
        raw = x.view(torch.uint8) if x.dtype != torch.bfloat16 else x
        cat = torch.cat([raw[b, :, :lengths[b]] for b in range(B)], dim=1).contiguous()
        return cat.view(x.dtype) if x.dtype != torch.bfloat16 else cat

    kp, vp = packed(kc), packed(vc)
    outs = {
        'padded rows': attention(t(q), t(kc), t(vc), lengths=lt, **kwargs),
        'padded vt': attention(t(q), t(kc), transposed(t(vc)), lengths=lt, **kwargs),
        'packed rows': attention(t(q), t(kp), t(vp), cu_seqlens=cu, **kwargs),
        'packed vt': attention(t(q), t(kp), transposed(t(vp)), cu_seqlens=cu, **kwargs),
    }
    torch.cuda.synchronize()
    for name, out in outs.items():
        _check(out, ref, atol, rtol)
        assert torch.equal(out, outs['padded rows']), name


@pytest.mark.parametrize('D', [72, 96, 104, 128])
def test_key_mask_wide_heads(dev, D):
    """The key-mask path at three and four output tiles, V rows and V^T, with and without lengths."""
    from streamvoxel_amd.stream.attention import attention
    B, H, Q, kcap = 2, 2, 96, 200
    _case(f'attention key mask D={D}')
    q, k, v = _qkv(B, H, Q, kcap, D, seed=7 * D)
    g = torch.Generator().manual_seed(D)
    mask = torch.rand(B, kcap, generator=g) < 0.6
    mask[1, :80] = False
    for lengths in (None, [200, 130]):
        lt = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=dev)
        ref = torch.zeros(B, H, Q, D, dtype=torch.float64)
        for b in range(B):
            keep = mask[b].clone()
            if lengths is not None:
                keep[lengths[b]:] = False
            idx = keep.nonzero().squeeze(1)
            ref[b:b + 1] = A.cross_attention(q[b:b + 1], k[b:b + 1, :, idx], v[b:b + 1, :, idx], [len(idx)])
        for vt in (False, True):
            vd = v.to(dev)
            if vt:
                vd = vd.transpose(2, 3).contiguous().transpose(2, 3)
            out = attention(q.to(dev), k.to(dev), vd, lengths=lt, key_mask=mask.to(dev))
            torch.cuda.synchronize()
            _check(out, ref, BF16_ATOL, BF16_RTOL)


# ------------------------------------------------------------------------------------------------- LayerNorm

NORM_WIDTHS = [64, 200, 256, 320, 448, 512, 640, 768, 1000, 1024, 1280, 2048]


def _norm_reference(x, shift=None, scale=None):
    ref = O.layer_norm(x, 1e-6)
    bound = 2.0 ** -8 * ref.abs()
    if shift is not None:
        onep = (1 + scale.double()).to(torch.bfloat16).double()
        ref = ref * onep[:, None] + shift.double()[:, None]
        bound = 2.0 ** -8 * ref.abs() + 2.0 ** -8 * (ref - shift.double()[:, None]).abs()
    return ref, bound


@pytest.mark.parametrize('W', NORM_WIDTHS)
def test_layer_norm_every_width(dev, W):
    """LayerNorm + modulation at every row plan (16, 32 or 64 lanes per row and 1-8 chunks per lane), with the
    shift / scale rows 16-byte aligned (vector reads) and not, and unmodulated; the gated residual form with and
    without the norm, the gate aligned and not."""
    from streamvoxel_amd.stream.backbone import layer_norm, residual_norm
    B, N = 2, 67
    _case(f'layer norm sweep W={W}')
    g = torch.Generator().manual_seed(W)
    x = (torch.randn(B, N, W, generator=g) * 2 + 0.3).to(torch.bfloat16)
    ada = (torch.randn(B, 3 * W + 8, generator=g) * 0.3).to(torch.bfloat16)
    norm = torch.nn.LayerNorm(W, elementwise_affine=False, eps=1e-6)
    xd, ad = x.to(dev), ada.to(dev)
    forms = {'none': (None, None), 'aligned': (ad[:, :W], ad[:, W:2 * W]),
             'unaligned': (ad[:, 1:W + 1], ad[:, W + 1:2 * W + 1])}
    for name, (sh, sc) in forms.items():
        y = layer_norm(xd, norm.to(dev), sh, sc)
        torch.cuda.synchronize()
        ref, bound = _norm_reference(x, None if sh is None else sh.cpu(), None if sc is None else sc.cpu())
        err = (y.cpu().double() - ref).abs()
        assert bool((err <= bound + 1e-5).all()), (name, float((err - bound).max()))
    a = (torch.randn(B, N, W, generator=g) * 2).to(torch.bfloat16).to(dev)
    for gate in (ad[:, 2 * W:3 * W], ad[:, 2 * W + 1:3 * W + 1]):
        r, y = residual_norm(xd, a, gate, norm.to(dev), ad[:, :W], ad[:, W:2 * W])
        r_only = residual_norm(xd, a, gate)
        want = xd + gate[:, None] * a
        torch.cuda.synchronize()
        assert torch.equal(r, want) and torch.equal(r_only, want)
        ref, bound = _norm_reference(r.cpu(), ada[:, :W], ada[:, W:2 * W])
        err = (y.cpu().double() - ref).abs()
        assert bool((err <= bound + 1e-5).all()), float((err - bound).max())


# --------------------------------------------------------------------------------- patchify, K/V writer, RoPE

@pytest.mark.parametrize('W', [1024, 1536])
def test_gather_patch_wide_rows(dev, W):
    """The gather patchify with four and eight 16-byte column chunks per lane: bit for bit torch's embedding bag
    (the reference's form) plus the bias."""
    from streamvoxel_amd.stream.forward import GatherPatch
    B, shape, C, p = 2, (8, 8, 8), 6, 4
    _case(f'gather patch W={W}')
    g = torch.Generator().manual_seed(W)
    conv = torch.nn.Conv3d(C + 1, W, p, stride=p)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) * 0.3)
        conv.bias.copy_(torch.randn(W, generator=g))
    conv = conv.to(torch.bfloat16)
    tokens = torch.randint(0, C + 1, (B, *shape), generator=g)
    gp = GatherPatch(conv.to(dev))
    out = gp(tokens.to(dev))
    Y, Z, X = shape
    cells = tokens.reshape(B, Y // p, p, Z // p, p, X // p, p).permute(0, 1, 3, 5, 2, 4, 6).reshape(-1, p ** 3)
    index = (cells * p ** 3 + torch.arange(p ** 3)).to(dev)
    ref = (torch.nn.functional.embedding_bag(index, gp.table, mode='sum') + gp.bias).reshape(B, -1, W)
    torch.cuda.synchronize()
    assert int(gp.bad.item()) == 0
    assert torch.equal(out, ref)


def test_kv_write_bf16_value_rows(dev):
    """svhip_kv_write into a bf16 cache with V rows (not transposed): the oracle's window layout bit for bit."""
    from streamvoxel_amd import _lib
    H, D, L, kcap = 3, 48, 150, 256
    _case('kv_write bf16 V rows')
    g = torch.Generator().manual_seed(11)
    k = torch.randn(H, L, D, generator=g).to(torch.bfloat16)
    v = torch.randn(H, L, D, generator=g).to(torch.bfloat16)
    lib = _lib.load()
    nbytes = int(lib.svhip_kv_write_workspace_bytes(H, kcap))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    ck = torch.full((H, kcap, D), 7.0, dtype=torch.bfloat16, device=dev)
    cv = torch.full((H, kcap, D), 7.0, dtype=torch.bfloat16, device=dev)
    kd, vd = k.to(dev), v.to(dev)
    _lib.check(lib.svhip_kv_write(
        None, None, 0, 0, 0, 0, 0, _lib.ptr(kd), _lib.ptr(vd), L, kd.stride(0), kd.stride(1), vd.stride(0),
        vd.stride(1), None, 0, None, H, D, _lib.ptr(ck), ck.stride(0), ck.stride(1), _lib.ptr(cv), cv.stride(0),
        cv.stride(1), cv.stride(2), kcap, _lib.SVHIP_BF16, None, None, _lib.ptr(ws), nbytes, _lib.stream_of(kd)),
        'svhip_kv_write')
    torch.cuda.synchronize()
    wk, wv = P.window_kv(torch.zeros(H, 0, D, dtype=torch.bfloat16), torch.zeros(H, 0, D, dtype=torch.bfloat16),
                         k, v, None, None, kcap)
    assert torch.equal(ck.cpu(), wk) and torch.equal(cv.cpu(), wv)


@pytest.mark.parametrize('D', [48, 18])
def test_axial_rope_one_pair_items(dev, D):
    """AxialRoPE on rows that start on 4- but not 16-byte boundaries, and at a head width that is not a multiple of
    8 (one pair per item): equal to the four-pair launch on the same values where that applies, and to the oracle."""
    from streamvoxel_amd.stream.producer import axial_rope, rope_frequencies
    B, H, N = 2, 3, 70
    _case(f'axial rope one pair per item D={D}')
    g = torch.Generator().manual_seed(D)
    x = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    pos = (torch.rand(B, N, 3, generator=g) * 40).floor()
    freq = rope_frequencies(D, device=dev)
    wide = torch.zeros(B, H, N, D + 2, dtype=torch.bfloat16, device=dev)
    wide[..., 2:] = x.to(dev)
    got = axial_rope(wide[..., 2:], pos.to(dev), freq)          # rows 4 bytes past a 16-byte boundary
    if D % 8 == 0:
        assert torch.equal(got, axial_rope(x.to(dev), pos.to(dev), freq))
    torch.cuda.synchronize()
    # device and host fp32 sin / cos may differ at a bf16 rounding boundary: at most one ulp on 0.1 % of elements
    want = P.axial_rope(x, pos, freq.cpu())
    d = (got.cpu().view(torch.int16).int() - want.view(torch.int16).int()).abs()
    assert int(d.max()) <= 1 and float((d != 0).float().mean()) <= 1e-3
