// Per-voxel softmax statistics over the class axis: negative entropy (sum p log p) and air probability.
//
// HBM-bound: every logit is read exactly once; all arithmetic is fp32.
//  * voxel-major rows ([B,N,C], stride_c == 1): a 16-lane DPP row owns one voxel. Each lane loads NV 16-byte
//    vectors of the voxel's row (coalesced 256-byte segments per row), keeps them in registers, and the row does
//    an exact two-pass softmax (max, then sum e and sum e*(x-max)) with 16-lane DPP all-reduces.
//  * class-major planes ([B,C,N], stride_n == 1, the layout the class head produces): each lane owns a 16-byte
//    run of consecutive voxels and streams the classes in chunks of CH rows with an online (running max)
//    softmax, so the plane is also read once and fully coalesced across the wave.
//  * anything else: the class-major kernel with scalar loads.
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
__device__ __forceinline__ void load16(const T* p, float* dst) {
  uint4 raw = *reinterpret_cast<const uint4*>(p);
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

// ------------------------------------------------------------------------------------------------ voxel-major

template <typename T, int NV, int MODE>
__global__ __launch_bounds__(256) void stats_voxel_major(const T* __restrict__ x, int64_t total, int64_t n, int64_t C,
                                                         int64_t sb, int64_t sn, const int32_t* __restrict__ air_ids,
                                                         int n_air, float* __restrict__ out) {
  constexpr int E = Vec16<T>::kElems;
  __shared__ uint32_t air_bits[MODE == kAirProb ? kMaxAirClasses / 32 : 1];
  if constexpr (MODE == kAirProb) load_air_bits(air_bits, air_ids, n_air, C);
  const int g = threadIdx.x & 15;
  const int64_t rows_per_block = blockDim.x >> 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * rows_per_block;
  for (int64_t voxel = blockIdx.x * rows_per_block + (threadIdx.x >> 4); voxel < total; voxel += stride) {
    const int64_t b = voxel / n;
    const int64_t i = voxel - b * n;
    const T* row = x + b * sb + i * sn;
    float v[NV * E];
    // All NV loads are issued before any is used: the index is clamped instead of branched on (a load inside a
    // branch is waited for before the branch ends), and the lanes past the row are masked afterwards.
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t c0 = static_cast<int64_t>(g + 16 * j) * E;
      load16<T>(row + (c0 < C ? c0 : 0), v + j * E);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (static_cast<int64_t>(g + 16 * j) * E >= C) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[j * E + e] = -INFINITY;
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < NV * E; ++e) m = fmaxf(m, v[e]);
    m = row16_max(m);
    float s = 0.f, w = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int c = (g + 16 * j) * E + e;
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
    s = row16_sum(s);
    w = row16_sum(w);
    if (g == 0) {
      if constexpr (MODE == kEntropy) {
        out[voxel] = w / s - __builtin_amdgcn_logf(s) * kLn2;
      } else {
        out[voxel] = w / s;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------ class-major

// Each thread owns VPL consecutive voxels (one 16-byte vector when VEC, else one voxel) and streams all classes.
template <typename T, bool VEC, int MODE>
__global__ __launch_bounds__(256) void stats_class_major(const T* __restrict__ x, int64_t batch, int64_t n, int64_t C,
                                                         int64_t sb, int64_t sc, int64_t sn,
                                                         const int32_t* __restrict__ air_ids, int n_air,
                                                         float* __restrict__ out) {
  constexpr int VPL = VEC ? Vec16<T>::kElems : 1;
  constexpr int CH = (sizeof(T) == 4) ? 8 : 4;
  __shared__ uint32_t air_bits[MODE == kAirProb ? kMaxAirClasses / 32 : 1];
  if constexpr (MODE == kAirProb) load_air_bits(air_bits, air_ids, n_air, C);
  const int64_t runs_per_window = cdiv(n, VPL);
  const int64_t total = batch * runs_per_window;
  for (int64_t run = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; run < total;
       run += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t b = run / runs_per_window;
    const int64_t i0 = (run - b * runs_per_window) * VPL;
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
        const int64_t c = c0 + r;
        if (c < C) {
          if constexpr (VEC) {
            load16<T>(base + c * sc, v[r]);
          } else {
            v[r][0] = to_float<T>(base[c * sc]);
          }
        } else {
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
      if (i0 + u < n) {
        float r;
        if constexpr (MODE == kEntropy) {
          r = w[u] / s[u] - __builtin_amdgcn_logf(s[u]) * kLn2;
        } else {
          r = w[u] / s[u];
        }
        out[b * n + i0 + u] = r;
      }
    }
  }
}

// ----------------------------------------------------------------------------------------------------- launch

static int grid_for(int64_t work_items, int threads) {
  int64_t g = cdiv(work_items, threads);
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

template <typename T, int MODE>
static int launch_stats(const T* x, int64_t batch, int64_t C, int64_t n, int64_t sb, int64_t sc, int64_t sn,
                        const int32_t* air_ids, int n_air, float* out, hipStream_t stream) {
  constexpr int E = Vec16<T>::kElems;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(x);
  const bool aligned_base = (addr % 16) == 0;
  const int64_t bytes = sizeof(T);
  // Voxel-major vector path.
  if (sc == 1 && aligned_base && (C % E) == 0 && ((sn * bytes) % 16) == 0 && ((sb * bytes) % 16) == 0) {
    const int64_t nvec = C / E;
    const int nv = static_cast<int>(cdiv(nvec, 16));
    const int64_t total = batch * n;
    const int grid = grid_for(total * 16, 256);
#define SVHIP_VM(NVV)                                                                                        \
  case NVV:                                                                                                  \
    stats_voxel_major<T, NVV, MODE><<<grid, 256, 0, stream>>>(x, total, n, C, sb, sn, air_ids, n_air, out); \
    return SVHIP_OK;
    switch (nv) {
      SVHIP_VM(1)
      SVHIP_VM(2)
      SVHIP_VM(3)
      SVHIP_VM(4)
      SVHIP_VM(5)
      SVHIP_VM(6)
      SVHIP_VM(7)
      SVHIP_VM(8)
      default:
        break;
    }
#undef SVHIP_VM
  }
  // Class-major vector path.
  if (sn == 1 && aligned_base && (n % E) == 0 && ((sc * bytes) % 16) == 0 && ((sb * bytes) % 16) == 0) {
    const int grid = grid_for(batch * (n / E), 256);
    stats_class_major<T, true, MODE><<<grid, 256, 0, stream>>>(x, batch, n, C, sb, sc, sn, air_ids, n_air, out);
    return SVHIP_OK;
  }
  const int grid = grid_for(batch * n, 256);
  stats_class_major<T, false, MODE><<<grid, 256, 0, stream>>>(x, batch, n, C, sb, sc, sn, air_ids, n_air, out);
  return SVHIP_OK;
}

template <int MODE>
static int stats_entry(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n, int64_t sb,
                       int64_t sc, int64_t sn, const int32_t* air_ids, int n_air, float* out, void* stream,
                       const char* name) {
  clear_error();
  SVHIP_REQUIRE(logits != nullptr && out != nullptr, "%s: null pointer", name);
  SVHIP_REQUIRE(batch >= 0 && n >= 0 && classes >= 1, "%s: bad sizes batch=%lld n=%lld classes=%lld", name,
                (long long)batch, (long long)n, (long long)classes);
  SVHIP_REQUIRE(dtype == SVHIP_F32 || dtype == SVHIP_BF16, "%s: dtype %d not supported (fp32 or bf16)", name, dtype);
  if (MODE == kAirProb) {
    SVHIP_REQUIRE(air_ids != nullptr && n_air >= 1, "%s: need at least one air class id", name);
    SVHIP_REQUIRE(classes <= kMaxAirClasses, "%s: at most %d classes", name, kMaxAirClasses);
  }
  if (batch == 0 || n == 0) return SVHIP_OK;
  hipStream_t s = as_stream(stream);
  int rc;
  if (dtype == SVHIP_F32) {
    rc = launch_stats<float, MODE>(static_cast<const float*>(logits), batch, classes, n, sb, sc, sn, air_ids, n_air,
                                   out, s);
  } else {
    rc = launch_stats<uint16_t, MODE>(static_cast<const uint16_t*>(logits), batch, classes, n, sb, sc, sn, air_ids,
                                      n_air, out, s);
  }
  if (rc != SVHIP_OK) return rc;
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

}  // namespace svhip

extern "C" int svhip_entropy(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n,
                             int64_t stride_b, int64_t stride_c, int64_t stride_n, float* out, void* stream) {
  return svhip::stats_entry<svhip::kEntropy>(logits, dtype, batch, classes, n, stride_b, stride_c, stride_n, nullptr,
                                             0, out, stream, "svhip_entropy");
}

extern "C" int svhip_air_prob(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n,
                              int64_t stride_b, int64_t stride_c, int64_t stride_n, const int32_t* air_ids,
                              int32_t n_air, float* out, void* stream) {
  return svhip::stats_entry<svhip::kAirProb>(logits, dtype, batch, classes, n, stride_b, stride_c, stride_n, air_ids,
                                             n_air, out, stream, "svhip_air_prob");
}
