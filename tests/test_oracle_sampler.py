"""Pins of the counter-based sampler's oracle (oracle/sampler.py): Philox4x64-10 against numpy's own Philox
generator, the uniforms' format, and the inverse-CDF draw against closed forms and frequencies."""
import numpy as np
import pytest

from oracle import sampler as S


@pytest.mark.parametrize('counter,key', [
    ((1, 0, 0, 0), (1, 2)),
    ((12345, 77, 0, 0), (2 ** 64 - 1, S.SAMPLE_STREAM)),
    ((2 ** 64 - 1, 5, 0, 0), (987654321, 0)),      # numpy's counter before it is 2^64 - 2 (no carry)
    ((0, 6, 0, 0), (987654321, 0)),                 # and here it carries out of the first word
    ((3, 2 ** 63, 2 ** 40, 9), (0, 0)),
])
def test_philox_equals_numpy_philox(counter, key):
    """numpy.random.Philox is Philox4x64-10; it advances its 256-bit counter before each block, so its first four
    words from counter c - 1 are the block at c."""
    c = list(counter)
    prev = c.copy()
    for i in range(4):          # 256-bit decrement
        if prev[i] > 0:
            prev[i] -= 1
            break
        prev[i] = 2 ** 64 - 1
    bg = np.random.Philox(counter=np.array(prev, dtype=np.uint64), key=np.array(key, dtype=np.uint64))
    want = bg.random_raw(4)
    got = S.philox4x64(np.array(c, dtype=np.uint64), np.array(key, dtype=np.uint64))
    assert [int(v) for v in got] == [int(v) for v in want]


def test_philox_vectorised_equals_scalar():
    voxels = np.arange(37, dtype=np.uint64) * np.uint64(1000003)
    counter = np.zeros((37, 4), dtype=np.uint64)
    counter[:, 0] = voxels
    counter[:, 1] = 11
    key = np.array([5, S.SAMPLE_STREAM], dtype=np.uint64)
    many = S.philox4x64(counter, key)
    for i in range(37):
        assert np.array_equal(many[i], S.philox4x64(counter[i], key))


def test_uniforms_format_and_spread():
    u = S.uniforms(seed=42, step=3, voxels=np.arange(200_000))
    assert np.all((u > 0) & (u < 1))
    assert np.array_equal(u.astype(np.float32).astype(np.float64), u)          # exact fp32 numbers
    assert np.array_equal(np.floor(u * 2 ** 23), np.floor(u * 2 ** 23 - 0.25))  # odd multiples of 2^-24
    # Uniform on (0, 1): mean, variance and the deciles within a few standard errors of 200 000 draws.
    assert abs(u.mean() - 0.5) < 4 * np.sqrt(1 / 12 / len(u))
    assert abs(u.var() - 1 / 12) < 0.002
    counts = np.histogram(u, bins=10, range=(0, 1))[0]
    assert np.all(np.abs(counts - 20_000) < 5 * np.sqrt(20_000))
    # Each coordinate of the counter and the key changes the stream.
    base = S.uniforms(1, 0, np.arange(64))
    for other in (S.uniforms(2, 0, np.arange(64)), S.uniforms(1, 1, np.arange(64)), S.uniforms(1, 0, np.arange(64) + 64)):
        assert np.mean(base == other) < 0.05


def test_inverse_cdf_closed_forms():
    # Equal logits: CDF(c) = (c + 1) / C, so the draw is floor(u C).
    C = 7
    u = np.array([0.01, 1 / 7 - 1e-9, 1 / 7 + 1e-9, 0.5, 0.999])
    cdf = S.softmax_cdf(np.zeros((5, C)))
    assert np.array_equal(S.invert(cdf, u), np.floor(u * C).astype(np.int64))
    # Two classes with p = (1/4, 3/4).
    cdf = S.softmax_cdf(np.tile([0.0, np.log(3.0)], (4, 1)))
    assert np.array_equal(S.invert(cdf, np.array([0.1, 0.2499, 0.2501, 0.9])), [0, 0, 1, 1])
    # A dominant class takes every draw; a -inf class never.
    rows = np.array([[0.0, 60.0, 0.0], [-np.inf, 0.0, 0.0]])
    cdf = S.softmax_cdf(rows)
    assert np.array_equal(S.invert(cdf, np.array([1e-6, 1e-6])), [1, 1])
    assert np.array_equal(S.invert(cdf, np.array([0.999999, 0.4])), [1, 1])
    # u above the whole row (rounding) keeps the last class.
    assert S.invert(np.array([[0.3, 0.999999]]), np.array([0.9999995]))[0] == 1


def test_sample_chosen_frequencies_follow_softmax():
    """20 000 voxels sharing one row of 6 logits: class frequencies within 5 standard errors of softmax."""
    logits = np.array([0.0, 1.0, -1.0, 2.0, 0.5, -3.0])
    p = np.exp(logits) / np.exp(logits).sum()
    n = 20_000
    rows = np.tile(logits, (n, 1))
    chosen = np.zeros(n, dtype=bool)
    chosen[::1] = True
    values, idx, u, cdf = S.sample_chosen(rows, chosen, seed=3, step=1)
    assert np.array_equal(idx, np.arange(n))
    freq = np.bincount(values, minlength=6) / n
    assert np.all(np.abs(freq - p) < 5 * np.sqrt(p * (1 - p) / n)), (freq, p)


def test_sample_chosen_leaves_others_and_orders_ascending():
    rng = np.random.default_rng(0)
    rows = rng.standard_normal((500, 9))
    chosen = rng.random(500) < 0.1
    values, idx, u, cdf = S.sample_chosen(rows, chosen, seed=9, step=4)
    assert np.array_equal(idx, np.flatnonzero(chosen))
    assert np.all(values[~chosen] == -1)
    assert np.all((values[chosen] >= 0) & (values[chosen] < 9))
    # The draw sits where its uniform falls in the row's CDF.
    lo = np.where(values[idx] > 0, cdf[np.arange(len(idx)), np.maximum(values[idx] - 1, 0)], 0.0)
    hi = cdf[np.arange(len(idx)), values[idx]]
    assert np.all((lo <= u) & (u < hi))
