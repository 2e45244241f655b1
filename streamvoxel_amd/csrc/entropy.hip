// Per-voxel softmax statistics over the class axis as plain outputs: negative entropy (sum p log p) and air
// probability, fp32 [batch, n]. The passes themselves live in stats.hpp.
#include "stats.hpp"

namespace svhip {

struct StoreF32 {
  float* out;
  struct None {};
  __device__ __forceinline__ None prefetch(int64_t) const { return None{}; }
  __device__ __forceinline__ void store(int64_t voxel, float value, None) const { out[voxel] = value; }
};

template <typename T, int NV, int MODE, int LPV>
__global__ __launch_bounds__(256) void stats_voxel_major(const T* __restrict__ x, int64_t total, int64_t n, int64_t C,
                                                         int64_t sb, int64_t sn, const int32_t* __restrict__ air_ids,
                                                         int n_air, float* __restrict__ out, VoxelRows rows) {
  __shared__ uint32_t air_bits[MODE == kAirProb ? kMaxAirClasses / 32 : 1];
  if constexpr (MODE == kAirProb) load_air_bits(air_bits, air_ids, n_air, C);
  StoreF32 o{out};
  voxel_major_pass<T, NV, MODE, StoreF32, LPV>(x, total, n, C, sb, sn, air_bits, o, blockIdx.x, gridDim.x, rows);
}

template <typename T, bool VEC, int MODE>
__global__ __launch_bounds__(256) void stats_class_major(const T* __restrict__ x, int64_t batch, int64_t n, int64_t C,
                                                         int64_t sb, int64_t sc, int64_t sn,
                                                         const int32_t* __restrict__ air_ids, int n_air,
                                                         float* __restrict__ out) {
  __shared__ uint32_t air_bits[MODE == kAirProb ? kMaxAirClasses / 32 : 1];
  if constexpr (MODE == kAirProb) load_air_bits(air_bits, air_ids, n_air, C);
  StoreF32 o{out};
  class_major_pass<T, VEC, MODE>(x, batch, n, C, sb, sc, sn, air_bits, o, blockIdx.x, gridDim.x);
}

template <typename T, int LPV, bool VEC, int MODE, int CMAX>
__global__ __launch_bounds__(256) void stats_canonical(const T* __restrict__ x, int64_t batch, int64_t n, int64_t C,
                                                       int64_t sb, int64_t sc, int64_t sn, int nv,
                                                       const int32_t* __restrict__ air_ids, int n_air,
                                                       float* __restrict__ out) {
  extern __shared__ float tile[];
  __shared__ uint32_t air_bits[MODE == kAirProb ? kMaxAirClasses / 32 : 1];
  if constexpr (MODE == kAirProb) load_air_bits(air_bits, air_ids, n_air, C);
  StoreF32 o{out};
  canonical_tile_pass<T, LPV, VEC, MODE, CMAX>(x, batch, n, C, sb, sc, sn, nv, air_bits, o, blockIdx.x, gridDim.x,
                                               tile);
}

template <typename T, int MODE>
static int launch_stats(const T* x, int64_t batch, int64_t C, int64_t n, int64_t sb, int64_t sc, int64_t sn,
                        const int32_t* air_ids, int n_air, float* out, hipStream_t stream, VoxelRows rows,
                        const char* name) {
  const StatsPlan plan = plan_stats<T>(x, batch, C, n, sb, sc, sn);
  SVHIP_REQUIRE(rows.p_log < 0 || plan.layout == kVoxelMajor,
                "%s: patch-order logits must be voxel-major rows (stride_c 1, 16-byte aligned rows, classes a "
                "multiple of %d, at most %d)",
                name, Vec16<T>::kElems, 128 * Vec16<T>::kElems);
  const unsigned grid = static_cast<unsigned>(plan.grid);
  if (plan.layout == kVoxelMajor) {
    const int64_t total = batch * n;
    // The row plan takes 8 lanes per voxel only with an odd vector count (row_plan), so only those are built.
#define SVHIP_VM(NVV)                                                                                            \
  case NVV:                                                                                                      \
    if constexpr (NVV % 2 == 1) {                                                                                \
      if (plan.lpv == 8) {                                                                                       \
        stats_voxel_major<T, NVV, MODE, 8><<<grid, 256, 0, stream>>>(x, total, n, C, sb, sn, air_ids, n_air, out, \
                                                                     rows);                                      \
        return SVHIP_OK;                                                                                         \
      }                                                                                                          \
    }                                                                                                            \
    stats_voxel_major<T, NVV, MODE, 16><<<grid, 256, 0, stream>>>(x, total, n, C, sb, sn, air_ids, n_air, out,    \
                                                                  rows);                                         \
    return SVHIP_OK;
    switch (plan.nv) {
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
  if (plan.layout == kCanonVec || plan.layout == kCanonScalar) {
    const bool vec = plan.layout == kCanonVec;
    const size_t lds = plan.lds;
#define SVHIP_CANON(LPVV, VECV, CM)                                                                         \
  stats_canonical<T, LPVV, VECV, MODE, CM><<<grid, 256, lds, stream>>>(x, batch, n, C, sb, sc, sn, plan.nv,    \
                                                                       air_ids, n_air, out)
    if (C <= 256) {
      if (plan.lpv == 8) {
        if (vec) SVHIP_CANON(8, true, 256); else SVHIP_CANON(8, false, 256);
      } else {
        if (vec) SVHIP_CANON(16, true, 256); else SVHIP_CANON(16, false, 256);
      }
    } else {
      // Above 256 classes 8 lanes per voxel occur only for bf16 rows (fp32 rows then have more than 8 vectors per
      // lane of 8), so the fp32 form of that case is not built.
      if constexpr (sizeof(T) == 2) {
        if (plan.lpv == 8) {
          if (vec) SVHIP_CANON(8, true, kCanonMaxC); else SVHIP_CANON(8, false, kCanonMaxC);
          return SVHIP_OK;
        }
      }
      if (vec) SVHIP_CANON(16, true, kCanonMaxC); else SVHIP_CANON(16, false, kCanonMaxC);
    }
#undef SVHIP_CANON
    return SVHIP_OK;
  }
  if (plan.layout == kClassMajorVec) {
    stats_class_major<T, true, MODE><<<grid, 256, 0, stream>>>(x, batch, n, C, sb, sc, sn, air_ids, n_air, out);
    return SVHIP_OK;
  }
  stats_class_major<T, false, MODE><<<grid, 256, 0, stream>>>(x, batch, n, C, sb, sc, sn, air_ids, n_air, out);
  return SVHIP_OK;
}

template <int MODE>
static int stats_entry(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n, int64_t sb,
                       int64_t sc, int64_t sn, const int32_t* air_ids, int n_air, float* out, void* stream,
                       const char* name, VoxelRows rows = kYzxRows) {
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
                                   out, s, rows, name);
  } else {
    rc = launch_stats<uint16_t, MODE>(static_cast<const uint16_t*>(logits), batch, classes, n, sb, sc, sn, air_ids,
                                      n_air, out, s, rows, name);
  }
  if (rc != SVHIP_OK) return rc;
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

}  // namespace svhip

extern "C" int svhip_entropy(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n,
                             int64_t stride_b, int64_t stride_c, int64_t stride_n, float* out, void* stream) {
  svhip::clear_error();
  return svhip::stats_entry<svhip::kEntropy>(logits, dtype, batch, classes, n, stride_b, stride_c, stride_n, nullptr,
                                             0, out, stream, "svhip_entropy");
}

extern "C" int svhip_air_prob(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n,
                              int64_t stride_b, int64_t stride_c, int64_t stride_n, const int32_t* air_ids,
                              int32_t n_air, float* out, void* stream) {
  svhip::clear_error();
  return svhip::stats_entry<svhip::kAirProb>(logits, dtype, batch, classes, n, stride_b, stride_c, stride_n, air_ids,
                                             n_air, out, stream, "svhip_air_prob");
}

extern "C" int svhip_entropy_patches(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t Y,
                                     int64_t Z, int64_t X, int64_t patch, int64_t stride_b, int64_t stride_n,
                                     float* out, void* stream) {
  const char* name = "svhip_entropy_patches";
  svhip::clear_error();
  SVHIP_REQUIRE(Y >= 0 && Z >= 0 && X >= 0 && patch >= 1, "%s: bad window or patch", name);
  svhip::VoxelRows rows;
  const int rc = svhip::make_rows(Y, Z, X, patch, &rows, name);
  if (rc != SVHIP_OK) return rc;
  return svhip::stats_entry<svhip::kEntropy>(logits, dtype, batch, classes, Y * Z * X, stride_b, 1, stride_n,
                                             nullptr, 0, out, stream, name, rows);
}

extern "C" int svhip_air_prob_patches(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t Y,
                                      int64_t Z, int64_t X, int64_t patch, int64_t stride_b, int64_t stride_n,
                                      const int32_t* air_ids, int32_t n_air, float* out, void* stream) {
  const char* name = "svhip_air_prob_patches";
  svhip::clear_error();
  SVHIP_REQUIRE(Y >= 0 && Z >= 0 && X >= 0 && patch >= 1, "%s: bad window or patch", name);
  svhip::VoxelRows rows;
  const int rc = svhip::make_rows(Y, Z, X, patch, &rows, name);
  if (rc != SVHIP_OK) return rc;
  return svhip::stats_entry<svhip::kAirProb>(logits, dtype, batch, classes, Y * Z * X, stride_b, 1, stride_n,
                                             air_ids, n_air, out, stream, name, rows);
}
