"""GPU parity of the selection kernels (entropy, air probability, low-entropy-last, top_mask, block-quota select,
fused EASE select) against the oracle, through the C ABI. Bit-exact for every mask given identical scores; entropy
and air probability within the stated float tolerance of float64."""
import math

import numpy as np
import pytest
import torch

import _golden
from oracle import sampling as S

pytestmark = pytest.mark.gpu

ENTROPY_ATOL = 1e-5   # fp32 arithmetic over <= 1000 classes vs float64 (the reference's own fp32 form errs ~2e-6)
AIR_ATOL = 2e-6


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def bimodal_logits(n, classes, seed, peaked=0.7, gap=12.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, classes), generator=g)
    hot = torch.rand(n, generator=g) < peaked
    cls = torch.randint(classes, (n,), generator=g)
    x[torch.arange(n)[hot], cls[hot]] += gap
    return x.to(dtype)


# ---------------------------------------------------------------------------------------------------- entropy

@pytest.mark.parametrize('layout', ['class_major', 'voxel_major'])
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('classes,n', [(256, 65536), (304, 4096), (6, 1024), (1000, 640), (37, 777)])
def test_entropy_matches_f64(dev, layout, dtype, classes, n):
    from streamvoxel_amd.sampling.entropy import entropy_batched
    _case(f'entropy {layout} {dtype} C={classes} N={n}')
    B = 2
    x = torch.stack([bimodal_logits(n, classes, seed=s, dtype=dtype) for s in range(B)])  # [B, N, C]
    expect = np.stack([S.entropy_scores_f64(x[b].float().numpy().T) for b in range(B)])
    if layout == 'class_major':
        xd = x.transpose(1, 2).contiguous().to(dev)
    else:
        xd = x.contiguous().to(dev)
    got = entropy_batched(xd, layout=layout)
    torch.cuda.synchronize()
    err = np.abs(got.cpu().numpy() - expect).max()
    assert err < ENTROPY_ATOL, err


def test_entropy_scores_reference_signature_and_closed_forms(dev):
    from streamvoxel_amd.sampling.entropy import entropy_scores
    _case('entropy_scores [C,Y,Z,X]')
    x = torch.zeros((256, 4, 4, 4), device=dev)
    assert torch.allclose(entropy_scores(x), torch.full((4, 4, 4), -math.log(256), device=dev), atol=2e-6)
    x[7] = 200.
    assert torch.all(entropy_scores(x) == 0)
    logits = bimodal_logits(16 * 8 * 8, 6, seed=3).T.reshape(6, 16, 8, 8)
    got = entropy_scores(logits.to(dev)).cpu().numpy()
    assert np.abs(got - S.entropy_scores_f64(logits.numpy())).max() < ENTROPY_ATOL
    with pytest.raises(RuntimeError):
        entropy_scores(logits)   # host tensors are refused: there is no CPU path


def test_air_prob_matches_f64(dev):
    from streamvoxel_amd.sampling.entropy import air_prob
    for dtype in (torch.float32, torch.bfloat16):
        _case(f'air_prob {dtype}')
        logits = bimodal_logits(64 * 16 * 16, 304, seed=5, dtype=dtype).T.reshape(304, 64, 16, 16)
        air = (0, 1, 303)
        got = air_prob(logits.to(dev), air).cpu().numpy()
        expect = S.air_prob_f64(logits.float().numpy(), air)
        assert np.abs(got - expect).max() < AIR_ATOL


# ------------------------------------------------------------------------------------------- low-entropy-last

def test_lel_update_golden_bit_exact(dev):
    from streamvoxel_amd.sampling.low_entropy_last import low_entropy_last_update
    for c in _golden.lel_cases():
        _case('lel golden ' + c['name'])
        t = {k: torch.from_numpy(np.ascontiguousarray(c[k])).to(dev) for k in ('air', 'mask', 'solid', 'last0')}
        got = low_entropy_last_update(t['last0'], t['mask'], t['air'], t['solid'], c['eps'], c['band'], c['col'])
        assert np.array_equal(got.cpu().numpy(), c['out']), c['name']


def test_lel_update_random_full_window(dev):
    from streamvoxel_amd.sampling.low_entropy_last import low_entropy_last_update
    g = np.random.default_rng(9)
    shape = (256, 16, 16)
    for col, band in ((True, False), (False, False), (False, True)):
        _case(f'lel random col={col} band={band}')
        height = g.integers(0, 256, (16, 16))
        air = np.where(np.arange(256)[:, None, None] > height[None], 1.0, g.random(shape)).astype(np.float32)
        air[g.random(shape) < 0.01] = np.float32(1 - 1e-4)
        mask = g.random(shape) < 0.97
        solid = g.random(shape) < 0.001
        last0 = np.zeros(shape if col else (256,), bool)
        expect = S.low_entropy_last_update(last0, mask, air, solid, 1e-4, band, col)
        got = low_entropy_last_update(torch.from_numpy(last0).to(dev), torch.from_numpy(mask).to(dev),
                                      torch.from_numpy(air).to(dev), torch.from_numpy(solid).to(dev), 1e-4, band, col)
        assert np.array_equal(got.cpu().numpy(), expect)


# ---------------------------------------------------------------------------------------------------- top_mask

@pytest.mark.parametrize('seed', range(4))
def test_top_mask_bit_exact_with_ties(dev, seed):
    from streamvoxel_amd.sampling.block_quota import top_mask
    g = np.random.default_rng(seed)
    for shape in ((8, 8, 8), (256, 16, 16)):
        scores = g.integers(-6, 1, shape).astype(np.float32) / 2
        scores[g.random(shape) < 0.05] = -0.0
        eligible = g.random(shape) < g.random()
        for count in (-3, 0, 1, 7, 40, 500, int(eligible.sum()), int(eligible.sum()) + 5):
            _case(f'top_mask seed={seed} shape={shape} count={count}')
            expect = S.top_mask(scores, eligible, count)
            sd, ed = torch.from_numpy(scores).to(dev), torch.from_numpy(eligible).to(dev)
            assert np.array_equal(top_mask(sd, ed, count).cpu().numpy(), expect)
            dcount = torch.tensor(count, dtype=torch.int64, device=dev)
            assert np.array_equal(top_mask(sd, ed, dcount).cpu().numpy(), expect)


# ------------------------------------------------------------------------------------------------- block quota

def test_quota_select_golden_bit_exact(dev):
    from streamvoxel_amd.sampling.block_quota import block_quota_select, quota_select
    n = 0
    for c in _golden.quota_cases():
        _case('quota golden ' + c['name'])
        b = c['b']
        n_total = S.block_view(c['non_last'], b).sum(1)
        pos = S.order_to_pos(c['order'])
        score = torch.from_numpy(c['score']).to(dev)
        mask = torch.from_numpy(c['selectable']).to(dev)
        got = quota_select(score, mask, c['k'], b, torch.from_numpy(pos).to(dev), c['frac'],
                           torch.from_numpy(n_total).to(dev), c['committed'])
        assert np.array_equal(got.cpu().numpy(), c['chosen']), c['name']
        got2 = block_quota_select(score, mask, c['k'], b, torch.from_numpy(c['order']).to(dev), c['frac'],
                                  torch.from_numpy(n_total).to(dev))
        assert np.array_equal(got2.cpu().numpy(), c['chosen']), c['name']
        n += 1
    assert n == 36


def _lel_state(seed, shape, b, g):
    """A mid-window state: ragged deferred tops, partial commits, real-valued scores with some exact ties."""
    Y, Z, X = shape
    tops = g.integers(Y // 2, Y + 1, (Z, X))
    last = np.arange(Y)[:, None, None] >= tops[None]
    non_last = ~last
    committed_mask = non_last & (g.random(shape) < g.random() * 0.8)
    selectable = non_last & ~committed_mask
    k = int(g.integers(1, max(2, selectable.sum())))
    committed = int(committed_mask.sum())
    frac = (committed + k) / int(non_last.sum())
    score = -g.random(shape).astype(np.float32) * 5
    score[g.random(shape) < 0.2] = -1.5
    pos = S.order_to_pos(g.permutation(Y * Z * X // b ** 3))
    n_total = S.block_view(non_last, b).sum(1)
    return score, selectable, k, pos, frac, n_total, committed


@pytest.mark.parametrize('b', [1, 2, 4, 8, 16])
def test_quota_select_random_states_bit_exact(dev, b):
    from streamvoxel_amd.sampling.block_quota import quota_select
    g = np.random.default_rng(100 + b)
    for trial in range(4):
        shape = (256, 16, 16) if trial < 2 else (64, 16, 16)
        _case(f'quota random b={b} trial={trial} shape={shape}')
        score, selectable, k, pos, frac, n_total, committed = _lel_state(trial, shape, b, g)
        expect = S.quota_select_nosync(score, selectable, k, b, pos, frac, n_total, committed)
        got = quota_select(torch.from_numpy(score).to(dev), torch.from_numpy(selectable).to(dev), k, b,
                           torch.from_numpy(pos).to(dev), frac, torch.from_numpy(n_total).to(dev), committed)
        assert np.array_equal(got.cpu().numpy(), expect)


def test_quota_select_batched_and_bad_flag(dev):
    from streamvoxel_amd.sampling.block_quota import QuotaWorkspace, quota_select_into
    g = np.random.default_rng(7)
    shape, b, B = (256, 16, 16), 4, 5
    states = [_lel_state(s, shape, b, g) for s in range(B)]
    # window 3 asks for more voxels than it has selectable: exactly-k cannot hold -> bad
    sc, sel, k, pos, frac, nt, com = states[3]
    states[3] = (sc, sel, int(sel.sum()) + 3, pos, frac, nt, com)
    _case('quota batched B=5 with one infeasible window')
    t = lambda a, dt=None: torch.as_tensor(np.asarray(a), dtype=dt).to(dev)
    score = t(np.stack([s[0] for s in states]))
    mask = t(np.stack([s[1] for s in states]))
    k = t([s[2] for s in states], torch.int64)
    pos = t(np.stack([s[3] for s in states]), torch.int64)
    frac = t([s[4] for s in states], torch.float64)
    n_total = t(np.stack([s[5] for s in states]), torch.int64)
    committed = t([s[6] for s in states], torch.int64)
    chosen = torch.empty((B, *shape), dtype=torch.bool, device=dev)
    bad = torch.empty(B, dtype=torch.bool, device=dev)
    ws = QuotaWorkspace(B, shape, b, dev)
    quota_select_into(score, mask, k, b, pos, frac, n_total, committed, chosen, bad, ws)
    for i, (sc, sel, kk, ps, fr, nt, com) in enumerate(states):
        expect = S.quota_select_nosync(sc, sel, kk, b, ps, fr, nt, com)
        assert np.array_equal(chosen[i].cpu().numpy(), expect), i
        assert bool(bad[i]) == S.select_bad(expect, sel, kk), i
    assert bool(bad[3]) and not bool(bad[0])


def test_ease_select_fused_equals_split_contract(dev):
    """Fused entropy + selectable + quota select: bit-exact to the oracle given the kernel's own scores, and the
    scores within tolerance of float64."""
    from streamvoxel_amd.sampling.block_quota import QuotaWorkspace
    from streamvoxel_amd import _lib
    g = np.random.default_rng(11)
    shape, b, B, C = (256, 16, 16), 4, 3, 256
    N = int(np.prod(shape))
    _case('ease_select fused B=3 voxel-major fp32')
    logits = torch.stack([bimodal_logits(N, C, seed=20 + i) for i in range(B)])   # [B, N, C]
    tokens = np.full((B, N), C, np.int64)
    last = np.zeros((B, N), bool)
    ks, poss, fracs, nts, coms = [], [], [], [], []
    for i in range(B):
        tops = g.integers(128, 257, (16, 16))
        lm = (np.arange(256)[:, None, None] >= tops[None]).reshape(-1)
        last[i] = lm
        done = (~lm) & (g.random(N) < 0.3 * i)
        tokens[i][done] = g.integers(0, C, done.sum())
        k = 2621 - 500 * i
        ks.append(k)
        coms.append(int(done.sum()))
        fracs.append((coms[-1] + k) / int((~lm).sum()))
        poss.append(S.order_to_pos(g.permutation(1024)))
        nts.append(S.block_view((~lm).reshape(shape), b).sum(1))
    d = lambda a, dt: torch.as_tensor(np.asarray(a), dtype=dt).to(dev)
    xd = logits.contiguous().to(dev)
    tk, ls = d(tokens, torch.int64), d(last, torch.bool)
    k_t, pos_t, frac_t = d(ks, torch.int64), d(np.stack(poss), torch.int64), d(fracs, torch.float64)
    nt_t, com_t = d(np.stack(nts), torch.int64), d(coms, torch.int64)
    chosen = torch.empty((B, N), dtype=torch.bool, device=dev)
    bad = torch.empty(B, dtype=torch.bool, device=dev)
    scores = torch.empty((B, N), dtype=torch.float32, device=dev)
    ws = QuotaWorkspace(B, shape, b, dev, fused=True)
    lib = _lib.load()
    _lib.check(lib.svhip_ease_select(
        _lib.ptr(xd), _lib.SVHIP_F32, C, xd.stride(0), xd.stride(2), xd.stride(1), _lib.ptr(tk), C,
        _lib.ptr(ls.view(torch.uint8)), B, *shape, b, _lib.ptr(k_t), _lib.ptr(pos_t), _lib.ptr(frac_t),
        _lib.ptr(nt_t), _lib.ptr(com_t), _lib.ptr(chosen.view(torch.uint8)), _lib.ptr(bad.view(torch.uint8)),
        _lib.ptr(scores), _lib.ptr(ws.buffer), ws.buffer.numel(), _lib.stream_of(xd)), 'svhip_ease_select')
    torch.cuda.synchronize()
    hs = scores.cpu().numpy()
    for i in range(B):
        e64 = S.entropy_scores_f64(logits[i].numpy().T)
        assert np.abs(hs[i] - e64).max() < ENTROPY_ATOL
        selectable = (tokens[i] == C) & ~last[i]
        expect = S.quota_select_nosync(hs[i].reshape(shape), selectable.reshape(shape), ks[i], b, poss[i], fracs[i],
                                       nts[i], coms[i])
        assert np.array_equal(chosen[i].cpu().numpy().reshape(shape), expect), i
        assert not bool(bad[i])
        # End to end from the logits: the oracle's own fp32 scores give the same mask unless a near-tie straddles
        # a quota boundary.
        ref = S.quota_select_nosync(S.entropy_scores(logits[i].T.contiguous()).numpy().reshape(shape),
                                    selectable.reshape(shape), ks[i], b, poss[i], fracs[i], nts[i], coms[i])
        agree = (ref == expect).mean()
        assert agree > 0.999, agree


def _trajectory_states(seed, steps=25):
    """The selection states of one window walked by the oracle: a low-entropy-last deferred top per column, then
    25 quarter-cosine quotas, each step committing the oracle's own choice over fresh bimodal scores. The clamped
    block quotas leave small trims and top-ups, the common case of a real window."""
    g = np.random.default_rng(seed)
    shape, b = (256, 16, 16), 4
    tops = g.integers(96, 200, (16, 16))
    last = np.arange(256)[:, None, None] >= tops[None]
    n_last = int(last.sum())
    quotas = S.low_entropy_last_quotas(last.size, steps, n_last)
    pos = S.order_to_pos(g.permutation(1024))
    n_total = S.block_view(~last, b).sum(1)
    committed = np.zeros(shape, bool)
    done = 0
    for k in quotas:
        score = np.where(g.random(shape) < 0.7, -g.random(shape) * 1e-2, -1 - 4 * g.random(shape)).astype(np.float32)
        selectable = ~last & ~committed
        frac = (done + k) / int((~last).sum())
        yield score, selectable, k, pos, frac, n_total, done
        chosen = S.quota_select_nosync(score, selectable, k, b, pos, frac, n_total, done)
        committed |= chosen
        done += k


def test_quota_select_window_trajectories_trim_and_top_up(dev):
    """Bit-exact along whole windows, and the small trim / top-up corrections (up to 16 voxels, resolved from the
    per-block boundary candidates) as well as larger ones all occur. A committed count below the true one makes the
    block quotas fall short of k, which is how the top-up cases are made."""
    from streamvoxel_amd.sampling.block_quota import quota_select
    seen = {'trim_small': 0, 'topup_small': 0, 'large': 0, 'exact': 0}
    b = 4
    cases = []
    for seed in range(3):
        for step, (score, selectable, k, pos, frac, n_total, done) in enumerate(_trajectory_states(seed)):
            for shortfall in (0, 5, 40):
                cases.append((seed, step, score, selectable, k, pos, frac, n_total, max(done - shortfall, 0)))
    for seed, step, score, selectable, k, pos, frac, n_total, done in cases:
        quota, *_ = S.apportion(selectable, n_total, pos, frac, done + k, b)
        d = int(S.in_block_select(score, selectable, quota, b).sum()) - k
        seen['exact' if d == 0 else ('large' if abs(d) > 16 else ('trim_small' if d > 0 else 'topup_small'))] += 1
        _case(f'quota trajectory seed={seed} step={step} k={k} committed={done} got-k={d}')
        expect = S.quota_select_nosync(score, selectable, k, b, pos, frac, n_total, done)
        res = quota_select(torch.from_numpy(score).to(dev), torch.from_numpy(selectable).to(dev), k, b,
                           torch.from_numpy(pos).to(dev), frac, torch.from_numpy(n_total).to(dev), done)
        assert np.array_equal(res.cpu().numpy(), expect), (seed, step, d)
    print('trajectory correction cases', seen, flush=True)
    assert seen['trim_small'] > 0 and seen['topup_small'] > 0 and seen['large'] > 0, seen


@pytest.mark.parametrize('dtype,classes', [(torch.float32, 256), (torch.bfloat16, 304), (torch.float32, 64),
                                           (torch.bfloat16, 48), (torch.float32, 384)])
def test_scores_are_bit_identical_in_every_layout(dev, dtype, classes):
    """Entropy and air probability of the same logits from voxel rows, contiguous class planes (what the reference's
    permute leaves), a voxel-row view, a strided class-plane view and the class head's patch order: one per-voxel
    order, the same bits."""
    from streamvoxel_amd.sampling.entropy import air_prob, entropy_batched, entropy_scores
    from streamvoxel_amd.stream.patches import PatchLogits
    B, shape = 2, (32, 16, 16)
    N = 32 * 16 * 16
    _case(f'layout-independent scores {dtype} C={classes}')
    rows = torch.stack([bimodal_logits(N, classes, seed=40 + i, dtype=dtype) for i in range(B)]).to(dev)  # [B,N,C]
    planes = rows.transpose(1, 2).contiguous()                                                  # [B,C,N]
    view = rows.transpose(1, 2)                                                                 # class stride 1
    wide = torch.zeros(B, classes, N + 64, dtype=dtype, device=dev)
    wide[:, :, :N] = planes
    strided = wide[:, :, :N]                                                                    # row stride N + 64
    odd = torch.zeros(B, classes, N + 1, dtype=dtype, device=dev)
    odd[:, :, :N] = planes
    unaligned = odd[:, :, :N]                               # class rows not 16-byte aligned: scalar tile loads
    want = entropy_batched(rows, layout='voxel_major')
    for x in (planes, view, strided, unaligned):
        assert torch.equal(entropy_batched(x, layout='class_major'), want)
    pl = PatchLogits(torch.empty(B, N // 64, 64 * classes, dtype=dtype, device=dev), shape, 4, classes)
    pl.rows[:, pl.row_index(torch.arange(N, device=dev))] = rows
    assert torch.equal(entropy_scores(pl).reshape(B, N), want)
    air = torch.tensor([0, 3, classes - 1], dtype=torch.int32, device=dev)
    a_rows = torch.stack([air_prob(rows[i].t().reshape(classes, *shape), air) for i in range(B)])
    a_planes = torch.stack([air_prob(planes[i].reshape(classes, *shape), air) for i in range(B)])
    torch.cuda.synchronize()
    assert torch.equal(a_rows, a_planes)
    err = (want.double().cpu() - torch.as_tensor(np.stack([S.entropy_scores_f64(rows[i].float().cpu().numpy().T)
                                                             for i in range(B)]))).abs().max().item()
    assert err < ENTROPY_ATOL, err


def test_ease_select_bit_identical_from_class_planes_and_voxel_rows(dev):
    """The fused selection from contiguous class planes and from voxel rows of the same logits: the same scores,
    the same chosen voxels (mid-window state with deferred voxels and committed tokens)."""
    from streamvoxel_amd import _lib
    from streamvoxel_amd.stream.step import EaseSelect
    g = np.random.default_rng(5)
    B, shape, C = 3, (256, 16, 16), 256
    N = 256 * 16 * 16
    _case('ease_select class planes vs voxel rows')
    rows = torch.stack([bimodal_logits(N, C, seed=70 + i) for i in range(B)]).to(dev)
    planes = rows.transpose(1, 2).contiguous()
    sels = []
    for x in (rows, planes):
        sel = EaseSelect(B, shape, C, 4, dev)
        for i in range(B):
            rng = np.random.default_rng(i)
            tops = rng.integers(128, 257, (16, 16))
            last = torch.from_numpy((np.arange(256)[:, None, None] >= tops[None]).reshape(-1)).to(dev)
            sel.last[i].copy_(last)
            done = torch.from_numpy(rng.random(N) < 0.2).to(dev) & ~last
            sel.tokens[i][done] = 1
            sel.bind_window(i, torch.from_numpy(rng.permutation(1024)).to(dev))
            k = 2000 - 300 * i
            committed = int(done.sum())
            sel.set_step(i, k, committed, (committed + k) / int((~last).sum()))
        sel.run(x, keep_scores=True)
        sels.append(sel)
    torch.cuda.synchronize()
    assert torch.equal(sels[0].scores.view(torch.int32), sels[1].scores.view(torch.int32))
    assert torch.equal(sels[0].chosen, sels[1].chosen)
    assert not bool(sels[0].bad.any())
