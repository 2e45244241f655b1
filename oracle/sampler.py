"""Counter-based categorical sampling of the chosen voxels — TEST INFRASTRUCTURE ONLY (part of the oracle).

The reference samples a solid step's chosen voxels with `torch.multinomial` over `softmax(logits.float())` on the
slot's generator (stream/fast_ops.py:548-553): the draws depend on the generator's position, so the tail cannot run
at a fixed size inside a captured graph. The counter-based form restated here draws voxel v of step `step` of the
window seeded `seed` from its own uniform

    u(seed, step, v) = (floor(w0 / 2^41) + 1/2) / 2^23,   (w0, w1, w2, w3) = Philox4x64-10(counter = (v, step, 0, 0),
                                                                                     key = (seed, SAMPLE_STREAM))

and takes the class by inversion of the row's softmax CDF: the first class c with sum_{j <= c} p_j > u. Philox4x64-10
is the counter-based generator of Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3"
(SC 2011): ten rounds of two 64 x 64 -> 128-bit products with the published multipliers, the key bumped by the
published Weyl constants between rounds. The restatement is pinned by numpy's own Philox (numpy.random.Philox, the
same generator: its first block for counter c - 1 is this function at c) and the sampler by closed forms and
frequency checks (tests/test_oracle_sampler.py).
"""
from __future__ import annotations

import numpy as np

PHILOX_M0 = 0xD2E7470EE14C6C93
PHILOX_M1 = 0xCA5A826395121157
PHILOX_W0 = 0x9E3779B97F4A7C15
PHILOX_W1 = 0xBB67AE8584CAA73B
SAMPLE_STREAM = 0x53414D504C455631  # the key's second word: "SAMPLEV1"

_M32 = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)


def _mulhilo(a, b):
    """(high, low) 64-bit halves of the 128-bit products a * b (uint64 arrays)."""
    a_lo, a_hi = a & _M32, a >> _S32
    b_lo, b_hi = b & _M32, b >> _S32
    ll, lh, hl, hh = a_lo * b_lo, a_lo * b_hi, a_hi * b_lo, a_hi * b_hi
    mid = (ll >> _S32) + (lh & _M32) + (hl & _M32)
    hi = hh + (lh >> _S32) + (hl >> _S32) + (mid >> _S32)
    return hi, a * b


def philox4x64(counter, key):
    """Philox4x64-10 of counters [..., 4] under keys [..., 2] (uint64, broadcast) -> [..., 4] uint64."""
    with np.errstate(over='ignore'):
        c = np.asarray(counter, dtype=np.uint64)
        k = np.asarray(key, dtype=np.uint64)
        c0, c1, c2, c3 = (c[..., i].copy() for i in range(4))
        k0, k1 = k[..., 0].copy(), k[..., 1].copy()
        m0, m1 = np.uint64(PHILOX_M0), np.uint64(PHILOX_M1)
        w0, w1 = np.uint64(PHILOX_W0), np.uint64(PHILOX_W1)
        for r in range(10):
            if r:
                k0, k1 = k0 + w0, k1 + w1
            hi0, lo0 = _mulhilo(m0, c0)
            hi1, lo1 = _mulhilo(m1, c2)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        return np.stack(np.broadcast_arrays(c0, c1, c2, c3), -1)


def uniforms(seed, step, voxels):
    """u(seed, step, v) for the voxel indices `voxels` (float64 values, each exactly an fp32 number in (0, 1))."""
    v = np.asarray(voxels, dtype=np.uint64)
    counter = np.zeros(v.shape + (4,), dtype=np.uint64)
    counter[..., 0] = v
    counter[..., 1] = np.uint64(int(step) & (2 ** 64 - 1))
    key = np.array([int(seed) & (2 ** 64 - 1), SAMPLE_STREAM], dtype=np.uint64)
    w0 = philox4x64(counter, key)[..., 0]
    return ((w0 >> np.uint64(41)).astype(np.float64) + 0.5) / 2.0 ** 23


def softmax_cdf(rows):
    """Inclusive softmax CDF of logit rows [k, C] in float64."""
    x = np.asarray(rows, dtype=np.float64)
    e = np.exp(x - x.max(-1, keepdims=True))
    return np.cumsum(e, -1) / e.sum(-1, keepdims=True)


def invert(cdf, u):
    """First class c with cdf[c] > u, per row (the last class when rounding leaves u above the whole row)."""
    c = (cdf <= np.asarray(u)[:, None]).sum(-1)
    return np.minimum(c, cdf.shape[-1] - 1)


def sample_chosen(rows, chosen, seed, step):
    """The sampled class of every chosen voxel: rows [N, C] logits in (y, z, x) voxel order, chosen [N] bool ->
    values [N] int64 (-1 where not chosen), with the uniforms and the CDFs of the chosen voxels (ascending)."""
    chosen = np.asarray(chosen, dtype=bool).reshape(-1)
    idx = np.flatnonzero(chosen)
    values = np.full(chosen.shape, -1, dtype=np.int64)
    u = uniforms(seed, step, idx)
    cdf = softmax_cdf(np.asarray(rows)[idx]) if len(idx) else np.zeros((0, np.asarray(rows).shape[-1]))
    values[idx] = invert(cdf, u)
    return values, idx, u, cdf
