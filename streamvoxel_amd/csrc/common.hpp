// Shared device/host helpers for the gfx950 kernels of libsvhip.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/svhip.h"

namespace svhip {

// ------------------------------------------------------------------------------------------ host error handling

void set_error(const char* fmt, ...);
void clear_error();

#define SVHIP_REQUIRE(cond, ...)             \
  do {                                       \
    if (!(cond)) {                           \
      ::svhip::set_error(__VA_ARGS__);       \
      return SVHIP_EINVAL;                   \
    }                                        \
  } while (0)

#define SVHIP_LAUNCHED(what)                                                            \
  do {                                                                                  \
    hipError_t _e = hipGetLastError();                                                  \
    if (_e != hipSuccess) {                                                             \
      ::svhip::set_error("%s: launch failed: %s", what, hipGetErrorString(_e));         \
      return SVHIP_ELAUNCH;                                                             \
    }                                                                                   \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ----------------------------------------------------------------------------------------------- device helpers

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ float bf16_bits_to_float(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even bf16 in hardware (v_cvt_pk_bf16_f32, two values per instruction). Equal to the integer
// rounding (u + 0x7fff + lsb) >> 16 for every non-NaN value; a NaN comes out as the quiet NaN.
typedef __bf16 svhip_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float svhip_f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t bf16_pack2(float a, float b) {
  const svhip_f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, svhip_bf16x2_t));
}

__device__ __forceinline__ uint16_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

// Both values rounded to bf16 and back to fp32.
__device__ __forceinline__ void bf16_round2(float& a, float& b) {
  const uint32_t p = bf16_pack2(a, b);
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

__device__ __forceinline__ float bf16_round1(float f) { return __uint_as_float(static_cast<uint32_t>(bf16_bits(f)) << 16); }

template <typename T>
__device__ __forceinline__ float to_float(T v);
template <>
__device__ __forceinline__ float to_float<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_float<uint16_t>(uint16_t v) { return bf16_bits_to_float(v); }

// DPP row-local (16-lane) all-reduce: after the four steps every lane of a 16-lane row holds the row result.
// quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}

// The same over groups of LPV (8 or 16) lanes: quad xor 1, quad xor 2, half-row mirror (8 lanes), row mirror (16).
// A max step moves the neighbour with bound control (every lane of these patterns reads a lane of its own row, so
// no old value is needed and none is materialised).
template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
  return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true)));
}

template <int LPV>
__device__ __forceinline__ float group_max(float v) {
  v = dpp_max_step<0xB1>(v);
  v = dpp_max_step<0x4E>(v);
  v = dpp_max_step<0x141>(v);
  if constexpr (LPV == 16) v = dpp_max_step<0x140>(v);
  return v;
}

template <int LPV>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  if constexpr (LPV == 16) v += dpp_f<0x140>(v);
  return v;
}

// Order-preserving fp32 -> u32 map (ascending float -> ascending key); -0.0 is folded onto +0.0 first so that the
// two compare equal, as IEEE comparisons (and torch's sort) treat them.
__device__ __forceinline__ uint32_t ordered_u32(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Key that sorts descending scores first: smaller key = larger score.
__device__ __forceinline__ uint32_t desc_key(float f) { return ~ordered_u32(f); }

__device__ __forceinline__ uint64_t ordered_u64(double d) {
  uint64_t u = static_cast<uint64_t>(__double_as_longlong(d));
  if ((u & 0x7fffffffffffffffull) == 0ull) u = 0ull;
  return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace svhip
