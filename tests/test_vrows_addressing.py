"""The row-major V operand reads of the cross-attention kernel (csrc/xattn.hip, VROWS), on the CPU: V rows stored
as the kernel stores them (K's sub-tile layout, 16-byte chunk c of row r at chunk swzv(r, c) = c ^ 4 ((r / 2) % 2)),
the per-lane byte offsets of output tile j (`rvt` in the kernel) and two reads a k-step (keys + 0..3, + 4..7), run
through the lane layout of ds_read_b64_tr_b16 measured on the GPU (within each 16-lane group lane i receives, as
its value n, element i % 4 of the 8-byte read of lane 4 n + i / 4; streamvoxel_amd/microbench/tr16_probe.hip).
Every lane must hold the A operand of the second product, keys 8 (l / 32) + 0..7 of head_dim column 32 j + l % 32,
and the 32 lanes one LDS cycle serves must touch 64 distinct banks (4-byte banks, 64 of them)."""
import numpy as np
import pytest

ROW = 64  # bf16 elements per LDS row (128 bytes)


def swzv(r, c):
    return c ^ (((r >> 1) & 1) << 2)


def rvt(lane, j):
    """The kernel's per-lane byte offset of output tile j's first read (relative to the V tile)."""
    row_lane = 8 * (lane >> 5) + ((lane & 15) >> 2)
    flip = (row_lane >> 1) & 1
    c_lane = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)
    return ((j >> 1) * 64 * ROW + row_lane * ROW) * 2 + 16 * (4 * ((j & 1) ^ flip) + c_lane) + 8 * (lane & 1)


def tr16_b64(lds, byte_addrs):
    """ds_read_b64_tr_b16 of 64 lanes (byte addresses) over a uint16 LDS image -> [64, 4]."""
    reads = np.stack([lds[a // 2: a // 2 + 4] for a in byte_addrs])
    out = np.empty((64, 4), dtype=lds.dtype)
    for lane in range(64):
        g, i = divmod(lane, 16)
        for n in range(4):
            out[lane, n] = reads[16 * g + 4 * n + i // 4, i % 4]
    return out


@pytest.mark.parametrize('DT', [2, 3, 4])
def test_row_major_v_operands_and_banks(DT):
    sub = (DT + 1) // 2
    rng = np.random.default_rng(DT)
    v = rng.integers(0, 65535, size=(64, 64 * sub), dtype=np.int64)   # one block: [key, head_dim]
    lds = np.full(sub * 64 * ROW, -1, dtype=np.int64)
    for u in range(sub):
        for r in range(64):
            for c in range(8):
                p = u * 64 * ROW + r * ROW + swzv(r, c) * 8
                lds[p:p + 8] = v[r, 64 * u + 8 * c: 64 * u + 8 * c + 8]
    assert (lds >= 0).all()
    lanes = np.arange(64)
    for j in range(DT):
        off = np.array([rvt(int(l), j) for l in lanes])
        assert (off % 8 == 0).all()
        for t in range(2):
            for ks in range(2):
                base = off + (32 * t + 16 * ks) * ROW * 2
                assert base.min() >= 0 and (base + 4 * ROW * 2).max() + 8 <= lds.size * 2
                a = np.concatenate([tr16_b64(lds, base), tr16_b64(lds, base + 4 * ROW * 2)], axis=1)
                for l in range(64):
                    keys = 32 * t + 16 * ks + 8 * (l >> 5) + np.arange(8)
                    assert (a[l] == v[keys, 32 * j + (l & 31)]).all(), (DT, j, t, ks, l)
        for h in range(2):
            addr = off + 4 * h * ROW * 2
            for half in range(2):
                banks = {((int(addr[l]) + 4 * w) // 4) % 64 for l in range(32 * half, 32 * half + 32) for w in range(2)}
                assert len(banks) == 64, (DT, j, h, half, len(banks))


def test_swizzle_is_an_involution_and_spreads_bank_sharing_rows():
    for r in range(64):
        assert sorted(swzv(r, c) for c in range(8)) == list(range(8))
        assert all(swzv(r, swzv(r, c)) == c for c in range(8))
    # rows r and r + 2 (same banks: 256-byte period) take the chunks of a 64-byte half on different halves
    for r in range(0, 64, 4):
        for c in range(4):
            assert (swzv(r, c) >> 2) != (swzv(r + 2, c) >> 2)
