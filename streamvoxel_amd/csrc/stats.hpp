// Per-voxel softmax statistics over the class axis (negative entropy sum p log p, air probability), as device
// passes that a kernel runs over its share of the voxels and hands to an output functor.
//
// HBM-bound: every logit is read exactly once; all arithmetic is fp32.
//  * voxel-major rows ([B,N,C], stride_c == 1): a 16-lane DPP row owns one voxel. Each lane loads NV 16-byte
//    vectors of the voxel's row (coalesced 256-byte segments per row), keeps them in registers, and the row does
//    an exact two-pass softmax (max, then sum e and sum e*(x-max)) with 16-lane DPP all-reduces.
//  * class-major planes ([B,C,N], stride_n == 1, the layout the class head produces): each lane owns a 16-byte
//    run of consecutive voxels and streams the classes in chunks of CH rows with an online (running max)
//    softmax, so the plane is also read once and fully coalesced across the wave.
//  * anything else: the class-major pass with scalar loads.
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

template <int MODE>
__device__ __forceinline__ float finish_stat(float s, float w) {
  if constexpr (MODE == kEntropy) {
    return w / s - __builtin_amdgcn_logf(s) * kLn2;
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
template <typename T, int NV, int MODE, typename Out, int LPV = 16>
__device__ __forceinline__ void voxel_major_pass(const T* __restrict__ x, int64_t total, int64_t n, int64_t C,
                                                 int64_t sb, int64_t sn, const uint32_t* air_bits, Out& out,
                                                 int64_t blk, int64_t nblk, VoxelRows rows = kYzxRows) {
  constexpr int E = Vec16<T>::kElems;
  const int g = threadIdx.x & (LPV - 1);
  constexpr int64_t kRowsPerBlock = 256 / LPV;
  const int64_t stride = nblk * kRowsPerBlock;
  for (int64_t voxel = blk * kRowsPerBlock + (threadIdx.x / LPV); voxel < total; voxel += stride) {
    const auto pre = out.prefetch(voxel);
    const int64_t b = voxel / n;
    const int64_t i = voxel - b * n;
    const T* row = x + b * sb + rows(i) * sn;
    float v[NV * E];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t c0 = static_cast<int64_t>(g + LPV * j) * E;
      load16<T>(row + (c0 < C ? c0 : 0), v + j * E);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (static_cast<int64_t>(g + LPV * j) * E >= C) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[j * E + e] = -INFINITY;
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < NV * E; ++e) m = fmaxf(m, v[e]);
    m = group_max<LPV>(m);
    float s = 0.f, w = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int c = (g + LPV * j) * E + e;
        if (c < C) {
          const float t = v[j * E + e] - m;
          const float p = fast_exp(t);
          s += p;
          if constexpr (MODE == kEntropy) {
            w += p * t;
          } else {
            if (is_air(air_bits, c)) w += p;
          }
        }
      }
    }
    s = group_sum<LPV>(s);
    w = group_sum<LPV>(w);
    if (g == 0) out.store(voxel, finish_stat<MODE>(s, w), pre);
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
    float m[VPL], s[VPL], w[VPL];
#pragma unroll
    for (int u = 0; u < VPL; ++u) {
      m[u] = -INFINITY;
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
          const float d = m[u] - mn;
          const float rs = fast_exp(d);
          if constexpr (MODE == kEntropy) {
            w[u] = (s[u] == 0.f) ? 0.f : (w[u] + s[u] * d) * rs;
          } else {
            w[u] *= rs;
          }
          s[u] *= rs;
          m[u] = mn;
        }
#pragma unroll
        for (int r = 0; r < CH; ++r) {
          if (c0 + r < C) {
            const float t = v[r][u] - m[u];
            const float p = fast_exp(t);
            s[u] += p;
            if constexpr (MODE == kEntropy) {
              w[u] += p * t;
            } else {
              if (is_air(air_bits, static_cast<int>(c0 + r))) w[u] += p;
            }
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < VPL; ++u) {
      if (i0 + u < n) out.store(b * n + i0 + u, finish_stat<MODE>(s[u], w[u]), pre[u]);
    }
  }
}

// How a logits tensor is walked: 0 voxel-major vectors, 1 class-major vectors, 2 class-major scalars.
enum StatsLayout { kVoxelMajor = 0, kClassMajorVec = 1, kClassMajorScalar = 2 };

struct StatsPlan {
  int layout;
  int nv;        // voxel-major: 16-byte vectors per lane
  int lpv;       // voxel-major: lanes per voxel (8 when a row fits in 8 vectors per lane, else 16)
  int64_t grid;  // workgroups of 256 threads
};

__host__ inline int64_t stats_grid(int64_t work_items) {
  int64_t g = cdiv(work_items, 256);
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return g;
}

constexpr int64_t kShortRowWorkgroups = 8 * 256;  // 8 per CU of MI355X

// Picks the pass for a [batch, C, n] logits tensor with element strides (sb, sc, sn).
template <typename T>
__host__ inline StatsPlan plan_stats(const T* x, int64_t batch, int64_t C, int64_t n, int64_t sb, int64_t sc,
                                     int64_t sn) {
  constexpr int E = Vec16<T>::kElems;
  const bool aligned_base = (reinterpret_cast<uintptr_t>(x) % 16) == 0;
  const int64_t bytes = sizeof(T);
  if (sc == 1 && aligned_base && (C % E) == 0 && ((sn * bytes) % 16) == 0 && ((sb * bytes) % 16) == 0 &&
      cdiv(C / E, 16) <= 8) {
    // Eight lanes per row when that leaves fewer vector slots idle (e.g. 304 bf16 classes: 38 vectors, 5 per lane
    // with 8 lanes, 3 with 16) and the row fits in eight vectors per lane.
    const int64_t vecs = C / E;
    const bool eight = cdiv(vecs, 8) <= 8 && cdiv(vecs, 8) * 8 - vecs < cdiv(vecs, 16) * 16 - vecs;
    const int lpv = eight ? 8 : 16;
    // Short rows run faster from a grid of 8 workgroups per CU that loops over the voxels (measured: 304 bf16
    // classes 99 -> 93 us per 8-window selection); long rows from one pass of workgroups over all voxels (256 fp32
    // classes: 100 us, 113 us with the capped grid).
    const int64_t grid = eight ? std::min<int64_t>(stats_grid(batch * n * lpv), kShortRowWorkgroups)
                               : stats_grid(batch * n * lpv);
    return StatsPlan{kVoxelMajor, static_cast<int>(cdiv(C / E, lpv)), lpv, grid};
  }
  if (sn == 1 && aligned_base && (n % E) == 0 && ((sc * bytes) % 16) == 0 && ((sb * bytes) % 16) == 0) {
    return StatsPlan{kClassMajorVec, 0, 0, stats_grid(batch * (n / E))};
  }
  return StatsPlan{kClassMajorScalar, 0, 0, stats_grid(batch * n)};
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
