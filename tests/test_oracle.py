"""Pins the CPU oracle (oracle/) before anything is compared with it: golden vectors written by the reference,
closed forms, brute force and defining properties. CPU only."""
import itertools
import math

import numpy as np
import pytest
import torch

import _golden
from oracle import attention as A
from oracle import sampling as S
from oracle.slot import ForwardBudget, LowEntropyLastSlot

# ------------------------------------------------------------------------------------------------------ entropy


def test_entropy_uniform_is_minus_log_c():
    for c in (2, 6, 256, 304):
        logits = torch.full((c, 3, 2, 2), 1.7)
        np.testing.assert_allclose(S.entropy_scores_f64(logits.numpy()), -math.log(c), rtol=0, atol=1e-14)
        np.testing.assert_allclose(S.entropy_scores(logits).numpy(), -math.log(c), rtol=0, atol=2e-6)
    assert abs(-math.log(256) - (-5.545177444479562)) < 1e-15


def test_entropy_one_hot_is_zero_and_two_class_closed_form():
    logits = torch.zeros(5, 4)
    logits[2] = 200.
    assert np.all(np.abs(S.entropy_scores_f64(logits.numpy())) < 1e-80)
    assert torch.all(S.entropy_scores(logits) == 0)
    a = np.linspace(-8, 8, 33)
    two = np.stack([a, np.zeros_like(a)])
    p = 1 / (1 + np.exp(-a))
    expect = p * np.log(p) + (1 - p) * np.log1p(-p)
    np.testing.assert_allclose(S.entropy_scores_f64(two), expect, rtol=0, atol=1e-12)


def test_entropy_shift_invariance_and_fp32_form_agree():
    g = torch.Generator().manual_seed(0)
    x = torch.randn((256, 4096), generator=g) * 3
    x[:, :2000] += 12 * torch.nn.functional.one_hot(torch.randint(256, (2000,), generator=g), 256).T
    e64 = S.entropy_scores_f64(x.numpy())
    np.testing.assert_allclose(S.entropy_scores_f64(x.double().numpy() + 100), e64, rtol=0, atol=1e-12)
    # The reference's own fp32 form sits within a few e-6 of float64 at these logit spreads.
    assert np.abs(S.entropy_scores(x).numpy() - e64).max() < 5e-6
    assert np.all(e64 <= 1e-12) and np.all(e64 >= -math.log(256) - 1e-12)


def test_air_prob_closed_form():
    x = torch.zeros(4, 3)
    x[1] = math.log(3.)     # p = [1, 3, 1, 1] / 6
    np.testing.assert_allclose(S.air_prob_f64(x.numpy(), (0, 1)), 4 / 6, atol=1e-15)
    np.testing.assert_allclose(S.air_prob(x, (0, 1)).numpy(), 4 / 6, atol=1e-6)

# ----------------------------------------------------------------------------------------------------- top_mask


def _is_top(selected, scores, eligible, count):
    """Defining property: |S| = min(count, #eligible), S within eligible, and every chosen voxel precedes every
    unchosen eligible one in (score desc, index asc)."""
    s = np.flatnonzero(selected.reshape(-1))
    e = np.flatnonzero(eligible.reshape(-1))
    rest = np.setdiff1d(e, s)
    flat = scores.reshape(-1)
    if len(s) != max(0, min(count, len(e))) or not np.isin(s, e).all():
        return False
    for i in s:
        for j in rest:
            if not (flat[i] > flat[j] or (flat[i] == flat[j] and i < j)):
                return False
    return True


@pytest.mark.parametrize('seed', range(6))
def test_top_mask_defining_property_with_ties(seed):
    g = np.random.default_rng(seed)
    for count in (-1, 0, 1, 3, 7, 40, 500):
        scores = g.integers(-4, 1, (4, 4, 4)).astype(np.float32)
        scores[g.random(scores.shape) < .1] = -0.0
        eligible = g.random((4, 4, 4)) < .4
        got = S.top_mask(scores, eligible, count)
        assert _is_top(got, scores, eligible, count)
        assert np.array_equal(S.top_mask_nosync(scores, eligible, count), got)


def test_top_mask_exhaustive_tiny():
    """All score patterns over {0,1} on 5 voxels, every eligibility and count."""
    for bits in itertools.product([0., 1.], repeat=5):
        scores = np.array(bits, np.float32)
        for el in itertools.product([False, True], repeat=5):
            eligible = np.array(el)
            for count in range(0, 6):
                assert _is_top(S.top_mask(scores, eligible, count), scores, eligible, count)

# --------------------------------------------------------------------------------------------------- block view


@pytest.mark.parametrize('shape,b', [((16, 8, 8), 4), ((8, 8, 8), 2), ((256, 16, 16), 16), ((4, 4, 4), 1)])
def test_block_view_closed_form(shape, b):
    Y, Z, X = shape
    flat = np.arange(Y * Z * X).reshape(shape)
    view = S.block_view(flat, b)
    nz, nx = Z // b, X // b
    for j in range(0, view.shape[0], max(1, view.shape[0] // 17)):
        by, bz, bx = j // (nz * nx), (j // nx) % nz, j % nx
        for i in range(0, b ** 3, max(1, b ** 3 // 13)):
            dy, dz, dx = i // (b * b), (i // b) % b, i % b
            assert view[j, i] == ((by * b + dy) * Z + bz * b + dz) * X + bx * b + dx
    assert np.array_equal(S.block_unview(view, b, shape), flat)
    assert np.all(np.diff(view, axis=1) > 0)        # in-block order is monotone in flat index

# ------------------------------------------------------------------------------------------------ block quota


def test_block_quota_select_matches_reference_golden_vectors():
    n = 0
    for case in _golden.quota_cases():
        pos = S.order_to_pos(case['order'])
        n_total = S.block_view(case['non_last'], case['b']).sum(1)
        got = S.block_quota_select(case['score'], case['selectable'], case['k'], case['b'], case['order'],
                                   case['frac'], n_total)
        assert np.array_equal(got, case['chosen']), case['name']
        nosync = S.quota_select_nosync(case['score'], case['selectable'], case['k'], case['b'], pos, case['frac'],
                                       n_total, case['committed'])
        assert np.array_equal(nosync, case['chosen']), case['name']
        assert int(got.sum()) == case['k'] and not (got & ~case['selectable']).any()
        n += 1
    assert n == 36


def test_fresh_4cube_closed_form():
    """Fresh 65 536-voxel window, k = 2621: every 4^3 block takes 2, and the 573 blocks earliest in the seeded order
    take a third; inside a block the highest scores win."""
    g = np.random.default_rng(3)
    shape, b, k = (256, 16, 16), 4, 2621
    score = g.standard_normal(shape).astype(np.float32)
    mask = np.ones(shape, bool)
    order = g.permutation(1024)
    pos = S.order_to_pos(order)
    n_total = np.full(1024, 64)
    sel = S.quota_select_nosync(score, mask, k, b, pos, k / 65536, n_total, 0)
    per_block = S.block_view(sel, b).sum(1)
    assert int(sel.sum()) == k
    assert np.array_equal(per_block, 2 + (pos < 573))
    bs, bm = S.block_view(score, b), S.block_view(sel, b)
    for j in range(0, 1024, 97):
        chosen, rest = bs[j][bm[j]], bs[j][~bm[j]]
        assert chosen.min() > rest.max()


def test_block_balance_within_one_in_fresh_state():
    g = np.random.default_rng(5)
    shape, b = (16, 8, 8), 2
    order = g.permutation(128)
    pos = S.order_to_pos(order)
    tokens = np.ones(shape, bool)
    committed = 0
    for k in S.counts(1024, dict(steps=8, schedule='linear', rounding='positive')):
        score = g.standard_normal(shape).astype(np.float32)
        sel = S.quota_select_nosync(score, tokens, k, b, pos, (committed + k) / 1024, np.full(128, 8), committed)
        assert int(sel.sum()) == k and not (sel & ~tokens).any()
        tokens &= ~sel
        committed += k
        done = S.block_view(~tokens, b).sum(1)
        assert done.max() - done.min() <= 1

# ------------------------------------------------------------------------------------------- low-entropy-last


def _lel_bruteforce(last, mask, air, solid, eps, band, col):
    thr = np.float32(1 - eps)
    Y = air.shape[0]
    bad = np.zeros(air.shape, bool)
    for idx in np.ndindex(air.shape):
        bad[idx] = (mask[idx] and air[idx] <= thr) or solid[idx]
    out = last.copy()
    if col:
        for z in range(air.shape[1]):
            for x in range(air.shape[2]):
                y = Y - 1
                while y >= 0 and not bad[y, z, x]:
                    out[y, z, x] = True
                    y -= 1
        return out
    clean = [not bad[y].any() for y in range(Y)]
    if band:
        clean = [all(clean[(y // 8) * 8:(y // 8) * 8 + 8]) for y in range(Y)]
    y = Y - 1
    while y >= 0 and clean[y]:
        out[y] = True
        y -= 1
    return out


def test_lel_update_matches_golden_and_bruteforce():
    n = 0
    for c in _golden.lel_cases():
        got = S.low_entropy_last_update(c['last0'], c['mask'], c['air'], c['solid'], c['eps'], c['band'], c['col'])
        assert np.array_equal(got, c['out']), c['name']
        brute = _lel_bruteforce(c['last0'], c['mask'], c['air'], c['solid'], c['eps'], c['band'], c['col'])
        assert np.array_equal(brute, c['out']), c['name']
        n += 1
    assert n == 18

# ---------------------------------------------------------------------------------------------------- schedule


def test_schedule_matches_golden_and_invariants():
    gold = _golden.schedule()
    for row in gold['counts']:
        got = S.counts(row['total'], row['spec'])
        assert got == row['counts'], row
        assert sum(got) == row['total']
        if row['spec']['rounding'] == 'positive':
            assert min(got) >= 1
    for row in gold['quotas']:
        got = S.low_entropy_last_quotas(row['total'], row['steps'], row['n_last'])
        assert got == row['quotas'], row
        assert sum(got) == row['total'] - row['n_last'] and all(q > 0 for q in got)
    for row in gold['actual_time']:
        assert S.actual_time(row['f']) == row['t']
    assert S.actual_time(1.) == 1. and S.actual_time(0.) == 0.

# -------------------------------------------------------------------------------------------------------- slot


def test_forward_budget_example():
    slots = [ForwardBudget() for _ in range(4)]
    jobs = iter([20, 21, 22, 20, 21, 21])

    def fill():
        for slot in slots:
            if slot.phase == 'idle':
                slot.arm(next(jobs))
    fill()
    for _ in range(20):
        [slot.forward() for slot in slots]
    assert [slot.phase for slot in slots] == ['idle', 'solid', 'solid', 'idle']
    fill()
    assert [slot.forward() for slot in slots] == [False, True, False, False]


def test_oracle_slot_reproduces_reference_trajectories():
    for c in _golden.slot_cases():
        shape = tuple(c['shape'])
        slot = LowEntropyLastSlot(shape, c['classes'], air_ids=(0,), air_token=0, last_eps=c['eps'],
                                  block_size=c['block'], device='cpu')
        tokens = torch.full(shape, c['classes'], dtype=torch.long)
        slot.arm(c['seed'], c['cap'], (c['index'], 0))
        step, record, commits = 0, None, []
        while record is None:
            logits = _golden.tiny_logits(step + 31 * c['index'], shape, c['classes'], c['ground'])
            record, commit = slot.consume(logits, tokens)
            if commit is not None:
                commits.append(dict(step=commit['step'], n=len(commit['positions'])))
            step += 1
        assert step == c['forwards'] and commits == c['commits'], c['name']
        assert record['nfe'] == c['nfe'] and record['last_count'] == c['last_count']
        assert np.array_equal(record['step_map'].numpy(), c['step_map']), c['name']
        assert np.array_equal(record['values'].numpy(), c['values']), c['name']
        assert np.array_equal(tokens.numpy().astype(np.int16), c['tokens']), c['name']

# --------------------------------------------------------------------------------------------------- attention


def test_attention_matches_bruteforce_and_ignores_padding():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 2, 3, 4, generator=g)
    k = torch.randn(2, 2, 6, 4, generator=g)
    v = torch.randn(2, 2, 6, 4, generator=g)
    lengths = [5, 2]
    ref = A.cross_attention(q, k, v, lengths)
    torch.testing.assert_close(ref, A.cross_attention_bruteforce(q, k, v, lengths), rtol=0, atol=1e-12)
    k2, v2 = k.clone(), v.clone()
    k2[0, :, 5:] = 1e3
    v2[1, :, 2:] = -7
    assert torch.equal(A.cross_attention(q, k2, v2, lengths), ref)
    sdpa = A.masked_sdpa(q, k, v, lengths)
    torch.testing.assert_close(sdpa.double(), ref, rtol=0, atol=1e-5)
    zero = A.cross_attention(q, k, v, [0, 2])
    assert torch.all(zero[0] == 0)


def test_masked_sdpa_with_any_mask_is_attention_over_the_kept_keys():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 2, 3, 4, generator=g, dtype=torch.float64)
    k = torch.randn(2, 2, 9, 4, generator=g, dtype=torch.float64)
    v = torch.randn(2, 2, 9, 4, generator=g, dtype=torch.float64)
    valid = torch.tensor([[1, 0, 1, 1, 0, 0, 1, 0, 1], [0, 0, 0, 0, 1, 0, 0, 0, 0]], dtype=torch.bool)
    got = A.masked_sdpa_mask(q, k, v, valid)
    for b in range(2):
        idx = valid[b].nonzero().squeeze(1)
        want = A.cross_attention_bruteforce(q[b:b + 1], k[b:b + 1, :, idx], v[b:b + 1, :, idx], [len(idx)])
        torch.testing.assert_close(got[b:b + 1], want, rtol=0, atol=1e-12)


def test_attention_packed_equals_padded():
    g = torch.Generator().manual_seed(3)
    lengths = [7, 1, 12]
    H, D = 2, 8
    kp = torch.randn(H, sum(lengths), D, generator=g)
    vp = torch.randn(H, sum(lengths), D, generator=g)
    q = torch.randn(3, H, 4, D, generator=g)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    k = torch.zeros(3, H, 12, D)
    v = torch.zeros(3, H, 12, D)
    for b in range(3):
        k[b, :, :lengths[b]] = kp[:, cu[b]:cu[b + 1]]
        v[b, :, :lengths[b]] = vp[:, cu[b]:cu[b + 1]]
    assert torch.equal(A.cross_attention_packed(q, kp, vp, cu), A.cross_attention(q, k, v, lengths))


def test_e4m3_decode_matches_format_table():
    codes = torch.arange(256, dtype=torch.uint8)
    ours = A.dequant_e4m3(codes, 1.0)
    assert ours[0x7E] == 448 and ours[0x38] == 1 and ours[0xB8] == -1 and ours[0x08] == 2 ** -6
    assert ours[0x01] == 2 ** -9 and math.isnan(ours[0x7F]) and math.isnan(ours[0xFF])
    if hasattr(torch, 'float8_e4m3fn'):
        theirs = codes.view(torch.float8_e4m3fn).to(torch.float64)
        finite = ~torch.isnan(theirs)
        assert torch.equal(torch.isnan(ours), ~finite)
        assert torch.equal(ours[finite], theirs[finite])
