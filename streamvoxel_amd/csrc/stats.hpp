// Per-voxel softmax statistics over the class axis (negative entropy sum p log p, air probability), as device
// passes that a kernel runs over its share of the voxels and hands to an output functor.
//
// HBM-bound: every logit is read exactly once; all arithmetic is fp32.
//
// The canonical per-voxel order. When C is a multiple of E = 16 / sizeof(T) elements and C / E <= 128, a voxel's
// statistics are one fixed function of its C values (and of the element type), whatever the layout: LPV lanes
// (8 or 16, `row_plan`), lane g holding the classes (g + LPV j) E + e for j < NV, e < E; the row max; per-lane
// sums of p = exp(x - max) and of fma(p, x - max, .) (or of the air classes' p) in (j, e) order; then a balanced
// tree over the lanes (DPP). The passes that follow it:
//  * voxel-major rows ([B,N,C], stride_c == 1, 16-byte aligned): the LPV lanes load the voxel's row as NV 16-byte
//    vectors each (coalesced segments per row) and keep it in registers;
//  * any other layout with C <= kCanonMaxC (class-major planes [B,C,N] as the reference's permute leaves them,
//    views, odd strides): a workgroup stages 32 voxels x C classes into LDS (16-byte loads along the voxels when
//    stride_n == 1), transposed to voxel rows, and runs the same per-voxel function on them.
// So the scores (and the selections ranked by them) of the same logits are bit-identical in every layout.
// Other class counts: a class-major pass with an online (running max) softmax, each lane owning a 16-byte run of
// voxels (stride_n == 1) or one voxel (scalar loads), streaming the classes.
// Loads are issued unconditionally with clamped indices and masked afterwards: a load inside a branch is waited
// for before the branch ends, which would serialise them.
//
// An output functor `out` provides `auto pre = out.prefetch(voxel)` (issued at the top of a voxel's iteration,
// so its own loads overlap the logits) and `out.store(voxel, value, pre)`; voxel = b * n + i.
#pragma once

#include <algorithm>

#include "common.hpp"

namespace svhip {

enum StatMode { kEntropy = 0, kAirProb = 1 };

constexpr int kMaxAirClasses = 4096;

// Air class membership bitmap in LDS, built from the device id list.
__device__ __forceinline__ void load_air_bits(uint32_t* bits, const int32_t* air_ids, int n_air, int64_t C) {
  int words = static_cast<int>((C + 31) / 32);
  for (int w = threadIdx.x; w < words; w += blockDim.x) bits[w] = 0u;
  __syncthreads();
  for (int a = threadIdx.x; a < n_air; a += blockDim.x) {
    int c = air_ids[a];
    if (c >= 0 && c < C) atomicOr(&bits[c >> 5], 1u << (c & 31));
  }
  __syncthreads();
}

__device__ __forceinline__ bool is_air(const uint32_t* bits, int c) { return (bits[c >> 5] >> (c & 31)) & 1u; }

template <typename T>
struct Vec16 {
  static constexpr int kElems = 16 / sizeof(T);
};

template <typename T>
__device__ __forceinline__ void unpack16(const uint4& raw, float* dst) {
  if constexpr (sizeof(T) == 4) {
    dst[0] = __uint_as_float(raw.x);
    dst[1] = __uint_as_float(raw.y);
    dst[2] = __uint_as_float(raw.z);
    dst[3] = __uint_as_float(raw.w);
  } else {
    uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dst[2 * i] = __uint_as_float(w[i] << 16);
      dst[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

template <typename T>
__device__ __forceinline__ void load16(const T* p, float* dst) {
  unpack16<T>(*reinterpret_cast<const uint4*>(p), dst);
}

// One logit of the canonical order into a lane's sums (the same instructions in every pass), in log2 units:
// t = x log2(e) - mL with mL = max log2(e) rounded (one FMA; the row's max gets t = delta, the rounding of mL, the
// same for every voxel element equal to the max), p = 2^t, s += p, w += p t (entropy) or w += p (air classes). A
// common shift of t leaves the statistic unchanged; finish_stat turns (s, w) into it.
template <int MODE>
__device__ __forceinline__ void accumulate(float x, float mL, int c, const uint32_t* air_bits, float& s, float& w) {
  const float t = __builtin_fmaf(x, kLog2e, -mL);
  const float p = __builtin_amdgcn_exp2f(t);
  s += p;
  if constexpr (MODE == kEntropy) {
    w = __builtin_fmaf(p, t, w);
  } else {
    if (is_air(air_bits, c)) w += p;
  }
}

// Lanes per voxel and 16-byte vectors per lane of the canonical order for C classes of T, or false when C has no
// canonical order (not a multiple of the vector, or more than 128 vectors). Eight lanes when that leaves fewer
// vector slots idle (e.g. 304 bf16 classes: 38 vectors, 5 per lane with 8 lanes, 3 with 16) and fits in eight
// vectors per lane.
struct RowPlan {
  int lpv, nv;
};

template <typename T>
__host__ __device__ inline bool row_plan(int64_t C, RowPlan* rp) {
  constexpr int E = Vec16<T>::kElems;
  if (C < E || C % E != 0) return false;
  const int64_t vecs = C / E;
  if (cdiv(vecs, 16) > 8) return false;
  // 8 lanes leave fewer vector slots idle than 16 exactly when ceil(vecs / 8) is odd (for an even count both leave
  // the same): 8 lanes therefore always come with an odd vector count per lane, and the launchers build only those.
  const bool eight = cdiv(vecs, 8) <= 8 && cdiv(vecs, 8) * 8 - vecs < cdiv(vecs, 16) * 16 - vecs;
  rp->lpv = eight ? 8 : 16;
  rp->nv = static_cast<int>(cdiv(vecs, rp->lpv));
  return true;
}

constexpr int64_t kCanonMaxC = 384;  // classes the LDS-staged canonical pass takes: 32 x (C + 1) floats, under 64 KB with
                                     // the selection kernel's own LDS
constexpr int kCanonTile = 32;       // voxels per LDS tile

__host__ inline size_t canon_lds_bytes(int64_t C) { return sizeof(float) * kCanonTile * (C + 1); }

// sum p log p / sum p - log sum p with p = 2^t: (w / s - log2 s) ln 2 (entropy, w = sum p t in log2 units), or the
// air classes' share w / s. pm = the max's own p (max_p): a sum that is exactly that is a row whose other p vanish
// beside it (a one-hot row), whose statistic is 0 (within 1e-6 of it whenever the sum takes nothing else).
template <int MODE>
__device__ __forceinline__ float max_p(float m, float mL) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(m, kLog2e, -mL));
}

template <int MODE>
__device__ __forceinline__ float finish_stat(float s, float w, float pm) {
  if constexpr (MODE == kEntropy) {
    if (s == pm) return 0.f;
    return (w / s - __builtin_amdgcn_logf(s)) * kLn2;
  } else {
    return w / s;
  }
}

// Row of voxel i (flat (y, z, x) index of a [Y, Z, X] window) in voxel-major logits: i itself (YZX order), or the
// row the class head writes it to (patch order): patches of p^3 voxels in (y / p, z / p, x / p) order, the voxels of
// a patch in (y % p, z % p, x % p) order. Patch order needs power-of-two p, Z and X (log2 in p_log, z_log, x_log).
// The pass walks voxels in (y, z, x) order and gathers their rows: the per-voxel side arrays (tokens, deferred
// flags, keys, scores) stay contiguous, which measured faster than walking the rows in storage order.
struct VoxelRows {
  int p_log;  // -1: YZX order
  int z_log, x_log;
  __device__ __forceinline__ int64_t operator()(int64_t i) const {
    if (p_log < 0) return i;
    const uint64_t u = static_cast<uint64_t>(i);
    const uint64_t pm = (1ull << p_log) - 1;
    const uint64_t x = u & ((1ull << x_log) - 1);
    const uint64_t t = u >> x_log;
    const uint64_t z = t & ((1ull << z_log) - 1);
    const uint64_t y = t >> z_log;
    const uint64_t patch = ((((y >> p_log) << (z_log - p_log)) | (z >> p_log)) << (x_log - p_log)) | (x >> p_log);
    return static_cast<int64_t>((((((patch << p_log) | (y & pm)) << p_log) | (z & pm)) << p_log) | (x & pm));
  }
};

constexpr VoxelRows kYzxRows{-1, 0, 0};

// Voxel-major pass: LPV (8 or 16) lanes own a voxel; workgroup `blk` of `nblk` takes voxels
// blk * (256 / LPV) + (tid / LPV), stepping by nblk * (256 / LPV). Each lane loads NV 16-byte vectors of the row.
// Requires 256-thread workgroups, C % (16 / sizeof(T)) == 0 and 16-byte aligned rows.
// C / E vectors per row: the first `vfull` vectors of every lane are inside the row; a lane's later ones may lie
// past it (only when C / E is not a multiple of LPV) and are loaded from vector 0, set to -inf for the max and
// skipped by the sums (a divergent branch: no per-element selects). (window, voxel) advance by the stride without
// a division.
template <typename T, int NV, int MODE, typename Out, int LPV = 16>
__device__ __forceinline__ void voxel_major_pass(const T* __restrict__ x, int64_t total, int64_t n, int64_t C,
                                                 int64_t sb, int64_t sn, const uint32_t* air_bits, Out& out,
                                                 int64_t blk, int64_t nblk, VoxelRows rows = kYzxRows) {
  constexpr int E = Vec16<T>::kElems;
  const int g = threadIdx.x & (LPV - 1);
  constexpr int64_t kRowsPerBlock = 256 / LPV;
  const int64_t stride = nblk * kRowsPerBlock;
  const int vecs = static_cast<int>(C / E);
  const int vfull = vecs / LPV;
  int64_t voxel = blk * kRowsPerBlock + (threadIdx.x / LPV);
  int64_t b = voxel / n;
  int64_t i = voxel - b * n;
  const int64_t sdiv = stride / n, smod = stride - sdiv * n;
  // One voxel's row: load, the canonical arithmetic, the output.
  auto one = [&](int64_t vox, const T* row) __attribute__((always_inline)) {
    const auto pre = out.prefetch(vox);
    uint4 raw[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vj = g + LPV * j;
      raw[j] = *reinterpret_cast<const uint4*>(row + (vj < vecs ? vj : 0) * E);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (j >= vfull && g + LPV * j >= vecs) {
        const uint32_t ninf = sizeof(T) == 4 ? 0xff800000u : 0xff80ff80u;
        raw[j] = make_uint4(ninf, ninf, ninf, ninf);
      }
    }
    float v[NV * E];
#pragma unroll
    for (int j = 0; j < NV; ++j) unpack16<T>(raw[j], v + j * E);
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < NV * E; ++e) m = fmaxf(m, v[e]);
    m = group_max<LPV>(m);
    const float mL = m * kLog2e;
    float s = 0.f, w = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (j < vfull || g + LPV * j < vecs) {
#pragma unroll
        for (int e = 0; e < E; ++e) accumulate<MODE>(v[j * E + e], mL, (g + LPV * j) * E + e, air_bits, s, w);
      }
    }
    s = group_sum<LPV>(s);
    w = group_sum<LPV>(w);
    if (g == 0) out.store(vox, finish_stat<MODE>(s, w, max_p<MODE>(m, mL)), pre);
  };
  // Element offsets of the lane's window and of its voxel's row in it. A stride of whole windows (smod == 0, e.g.
  // 24 workgroups a CU over 65536-voxel windows) leaves a lane's voxel index, so its row offset, unchanged: the
  // (uniform) branch that steps them is then skipped and an iteration only steps the window offset.
  int64_t boff = b * sb;
  const int64_t bstep = sdiv * sb;
  int64_t roff = rows(i) * sn;
  for (; voxel < total; voxel += stride) {
    one(voxel, x + boff + roff);
    boff += bstep;
    if (smod != 0) {
      i += smod;
      if (i >= n) {
        i -= n;
        boff += sb;
      }
      roff = rows(i) * sn;
    }
  }
}

// The canonical order over any layout, staged through LDS: workgroup `blk` of `nblk` takes tiles of kCanonTile
// voxels of one window, loads their C x kCanonTile logits into `tile` (kCanonTile rows of C + 1 floats, the odd
// row length keeps the transposed writes conflict-free), then LPV lanes per voxel run the canonical per-voxel
// function over the rows. VEC: stride_n == 1 with 16-byte aligned class rows (16-byte loads along the voxels).
// Requires 256-thread workgroups and row_plan<T>(C) = (LPV, nv).
// CMAX: a bound on C (256 or kCanonMaxC) that fixes the number of loads per thread and tile.
template <typename T, int LPV, bool VEC, int MODE, int CMAX, typename Out>
__device__ __forceinline__ void canonical_tile_pass(const T* __restrict__ x, int64_t batch, int64_t n, int64_t C,
                                                    int64_t sb, int64_t sc, int64_t sn, int nv,
                                                    const uint32_t* air_bits, Out& out, int64_t blk, int64_t nblk,
                                                    float* tile) {
  constexpr int E = Vec16<T>::kElems;
  constexpr int TV = kCanonTile;
  constexpr int VPR = 256 / LPV;  // voxels per round of the workgroup
  static_assert(TV % VPR == 0 && TV % E == 0, "tile shape");
  constexpr int CPV = TV / E;                              // 16-byte chunks per class row of a tile
  constexpr int CLS = 256 / CPV;                           // classes per 16-byte load of the workgroup
  constexpr int kLoads = (CMAX + CLS - 1) / CLS;           // a thread's loads per tile
  const int64_t ld = C + 1;
  const int64_t tiles = cdiv(n, TV);
  const int64_t total = batch * tiles;
  const int g = threadIdx.x & (LPV - 1);
  const int v0 = (threadIdx.x % CPV) * E;
  const int crow = threadIdx.x / CPV;
  // VEC: the next tile's logits are loaded into registers while the current one is computed (n is a multiple of
  // E, so a chunk lies wholly inside or outside the window; outside ones load a valid chunk and are not written).
  float pf[VEC ? kLoads : 1][E];
  auto issue = [&](int64_t id) __attribute__((always_inline)) {
    const int64_t b = id / tiles;
    const int64_t i0 = (id - b * tiles) * TV;
    const int64_t iv = i0 + v0 < n ? i0 + v0 : n - E;
    const T* base = x + b * sb + iv;
    // Every load is issued unconditionally (class index clamped; the repeats of row C - 1 are served by the
    // cache): a load under a branch would be waited for at the branch's end.
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int64_t c = u * CLS + crow;
      load16<T>(base + (c < C ? c : C - 1) * sc, pf[u]);
    }
  };
  if constexpr (VEC) {
    if (blk < total) issue(blk);
  }
  for (int64_t id = blk; id < total; id += nblk) {
    const int64_t b = id / tiles;
    const int64_t i0 = (id - b * tiles) * TV;
    decltype(out.prefetch(0)) pre[TV / VPR];
#pragma unroll
    for (int r = 0; r < TV / VPR; ++r) {
      const int64_t i = i0 + r * VPR + threadIdx.x / LPV;
      pre[r] = out.prefetch(b * n + (i < n ? i : n - 1));
    }
    __syncthreads();  // the previous tile's rows have been read
    if constexpr (VEC) {
      // Unconditional writes too: classes past C land in the row's padding column C, which is never read, and
      // voxels past the window in rows that are not stored.
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int64_t c = u * CLS + crow < C ? u * CLS + crow : C;
#pragma unroll
        for (int e = 0; e < E; ++e) tile[(v0 + e) * ld + c] = pf[u][e];
      }
    } else {
      const T* base = x + b * sb;
      for (int64_t idx = threadIdx.x; idx < C * TV; idx += 256) {
        const int64_t c = idx / TV;
        const int v = static_cast<int>(idx - c * TV);
        const int64_t i = i0 + v < n ? i0 + v : n - 1;
        tile[v * ld + c] = to_float<T>(base[c * sc + i * sn]);
      }
    }
    __syncthreads();
    // Issued after the barrier (which waits for outstanding loads): they land while this tile is computed.
    if constexpr (VEC) {
      if (id + nblk < total) issue(id + nblk);
    }
#pragma unroll
    for (int r = 0; r < TV / VPR; ++r) {
      const int vi = r * VPR + threadIdx.x / LPV;
      const float* row = tile + vi * ld;
      // The lane's classes in registers (at most 8 vectors), -inf past C, then the canonical arithmetic.
      float v[8 * E];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int c = (g + LPV * j) * E + e;
          v[j * E + e] = (j < nv && c < C) ? row[c] : -INFINITY;
        }
      }
      float m = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8 * E; ++e) m = fmaxf(m, v[e]);
      m = group_max<LPV>(m);
      const float mL = m * kLog2e;
      float s = 0.f, w = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int c = (g + LPV * j) * E + e;
          if (j < nv && c < C) accumulate<MODE>(v[j * E + e], mL, c, air_bits, s, w);
        }
      }
      s = group_sum<LPV>(s);
      w = group_sum<LPV>(w);
      const int64_t i = i0 + vi;
      if (g == 0 && i < n) out.store(b * n + i, finish_stat<MODE>(s, w, max_p<MODE>(m, mL)), pre[r]);
    }
  }
}

// Class-major pass: thread `blk * 256 + tid` of `nblk * 256` owns VPL consecutive voxels (one 16-byte vector when
// VEC, else one voxel) and streams all classes.
template <typename T, bool VEC, int MODE, typename Out>
__device__ __forceinline__ void class_major_pass(const T* __restrict__ x, int64_t batch, int64_t n, int64_t C,
                                                 int64_t sb, int64_t sc, int64_t sn, const uint32_t* air_bits,
                                                 Out& out, int64_t blk, int64_t nblk) {
  constexpr int VPL = VEC ? Vec16<T>::kElems : 1;
  constexpr int CH = (sizeof(T) == 4) ? 8 : 4;
  const int64_t runs_per_window = cdiv(n, VPL);
  const int64_t total = batch * runs_per_window;
  for (int64_t run = blk * 256 + threadIdx.x; run < total; run += nblk * 256) {
    const int64_t b = run / runs_per_window;
    const int64_t i0 = (run - b * runs_per_window) * VPL;
    decltype(out.prefetch(0)) pre[VPL];
#pragma unroll
    for (int u = 0; u < VPL; ++u) pre[u] = out.prefetch(b * n + (i0 + u < n ? i0 + u : n - 1));
    const T* base = x + b * sb + i0 * sn;
    float m[VPL], mL[VPL], s[VPL], w[VPL];
#pragma unroll
    for (int u = 0; u < VPL; ++u) {
      m[u] = -INFINITY;
      mL[u] = -INFINITY;
      s[u] = 0.f;
      w[u] = 0.f;
    }
    for (int64_t c0 = 0; c0 < C; c0 += CH) {
      float v[CH][VPL];
#pragma unroll
      for (int r = 0; r < CH; ++r) {
        const int64_t c = c0 + r < C ? c0 + r : C - 1;
        if constexpr (VEC) {
          load16<T>(base + c * sc, v[r]);
        } else {
          v[r][0] = to_float<T>(base[c * sc]);
        }
      }
#pragma unroll
      for (int r = 0; r < CH; ++r) {
        if (c0 + r >= C) {
#pragma unroll
          for (int u = 0; u < VPL; ++u) v[r][u] = -INFINITY;
        }
      }
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        float cm = v[0][u];
#pragma unroll
        for (int r = 1; r < CH; ++r) cm = fmaxf(cm, v[r][u]);
        const float mn = fmaxf(m[u], cm);
        if (mn > m[u]) {
          const float mLn = mn * kLog2e;
          const float d = mL[u] - mLn;   // the shift of t, log2 units like w
          const float rs = __builtin_amdgcn_exp2f(d);
          if constexpr (MODE == kEntropy) {
            w[u] = (s[u] == 0.f) ? 0.f : (w[u] + s[u] * d) * rs;
          } else {
            w[u] *= rs;
          }
          s[u] *= rs;
          m[u] = mn;
          mL[u] = mLn;
        }
#pragma unroll
        for (int r = 0; r < CH; ++r) {
          if (c0 + r < C) accumulate<MODE>(v[r][u], mL[u], static_cast<int>(c0 + r), air_bits, s[u], w[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < VPL; ++u) {
      if (i0 + u < n) out.store(b * n + i0 + u, finish_stat<MODE>(s[u], w[u], max_p<MODE>(m[u], mL[u])), pre[u]);
    }
  }
}

// How a logits tensor is walked: 0 voxel-major vectors, 1 class-major vectors, 2 class-major scalars (both
// online), 3 / 4 the canonical order through LDS tiles (16-byte loads along the voxels / scalar loads).
enum StatsLayout {
  kVoxelMajor = 0,
  kClassMajorVec = 1,
  kClassMajorScalar = 2,
  kCanonVec = 3,
  kCanonScalar = 4
};

struct StatsPlan {
  int layout;
  int nv;        // canonical order: 16-byte vectors per lane
  int lpv;       // canonical order: lanes per voxel (8 or 16)
  int64_t grid;  // workgroups of 256 threads
  size_t lds;    // dynamic LDS bytes (the canonical tile passes)
};

__host__ inline int64_t stats_grid(int64_t work_items) {
  int64_t g = cdiv(work_items, 256);
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return g;
}

constexpr int64_t kShortRowWorkgroups = 24 * 256;  // 24 per CU of MI355X

// Picks the pass for a [batch, C, n] logits tensor with element strides (sb, sc, sn).
template <typename T>
__host__ inline StatsPlan plan_stats(const T* x, int64_t batch, int64_t C, int64_t n, int64_t sb, int64_t sc,
                                     int64_t sn) {
  constexpr int E = Vec16<T>::kElems;
  const bool aligned_base = (reinterpret_cast<uintptr_t>(x) % 16) == 0;
  const int64_t bytes = sizeof(T);
  RowPlan rp;
  const bool canon = row_plan<T>(C, &rp);
  if (canon && sc == 1 && aligned_base && ((sn * bytes) % 16) == 0 && ((sb * bytes) % 16) == 0) {
    // Short rows run faster from a grid of 24 workgroups per CU that loops over the voxels (304 bf16 classes in
    // patch order, per 8-window selection: 74.5 us at 8 per CU, 69.5 at 16, 68.0 at 24, 71 with one pass of
    // workgroups over all voxels; with the loop that keeps a whole-window stride's row offset, 8, 16 and 32 per CU
    // measured 1-5 % slower than 24); long rows from one pass of workgroups (256 fp32 classes: 100 us, 113 us with
    // a capped grid).
    const int64_t grid = rp.lpv == 8 ? std::min<int64_t>(stats_grid(batch * n * rp.lpv), kShortRowWorkgroups)
                                     : stats_grid(batch * n * rp.lpv);
    return StatsPlan{kVoxelMajor, rp.nv, rp.lpv, grid, 0};
  }
  const bool vec = sn == 1 && aligned_base && (n % E) == 0 && ((sc * bytes) % 16) == 0 && ((sb * bytes) % 16) == 0;
  if (canon && C <= kCanonMaxC) {
    // A resident grid (the tile pass prefetches each workgroup's next tile): 4 workgroups per CU.
    const int64_t tiles = batch * cdiv(n, kCanonTile);
    return StatsPlan{vec ? kCanonVec : kCanonScalar, rp.nv, rp.lpv, std::min<int64_t>(std::max<int64_t>(tiles, 1), 1024),
                     canon_lds_bytes(C)};
  }
  if (vec) return StatsPlan{kClassMajorVec, 0, 0, stats_grid(batch * (n / E)), 0};
  return StatsPlan{kClassMajorScalar, 0, 0, stats_grid(batch * n), 0};
}

// VoxelRows of a [Y, Z, X] window whose logits are in the class head's patch order with patch size `patch`
// (0: YZX order). Patch order needs power-of-two patch, Y, Z and X with patch <= each.
__host__ inline int make_rows(int64_t Y, int64_t Z, int64_t X, int64_t patch, VoxelRows* rows, const char* name) {
  *rows = kYzxRows;
  if (patch == 0) return SVHIP_OK;
  auto log2_exact = [](int64_t v) {
    int l = 0;
    while ((int64_t{1} << l) < v && l < 62) ++l;
    return (v > 0 && (int64_t{1} << l) == v) ? l : -1;
  };
  const int pl = log2_exact(patch), yl = log2_exact(Y), zl = log2_exact(Z), xl = log2_exact(X);
  SVHIP_REQUIRE(pl >= 0 && yl >= 0 && zl >= 0 && xl >= 0,
                "%s: patch order needs power-of-two patch and window extents (patch %lld, window %lldx%lldx%lld)",
                name, (long long)patch, (long long)Y, (long long)Z, (long long)X);
  SVHIP_REQUIRE(pl <= yl && pl <= zl && pl <= xl, "%s: patch %lld larger than the window %lldx%lldx%lld", name,
                (long long)patch, (long long)Y, (long long)Z, (long long)X);
  *rows = VoxelRows{pl, zl, xl};
  return SVHIP_OK;
}

}  // namespace svhip
