// LayerNorm of the transformer blocks' residual stream, with the AdaLN modulation fused in:
//   y = LN(x) * (1 + scale[b]) + shift[b],   LN(x) = (x - mean) / sqrt(var + eps) [* weight + bias]
// (models/unconditional_md4_timefree.py:12-13,60-63: modulate(norm(x), shift, scale); models/unconditional_md4.py:
// 44-56 for the affine form without modulation, fp32 weight and bias). x and y bf16 [B, N, W] (y may be x); mean
// and the biased variance in fp32 over the row held in registers (two passes over registers, one HBM read);
// 1 + scale is rounded to bf16 as the reference's bf16 tensors compute it, the rest is fp32 and y is rounded once.
//
// HBM-bound: one wave per row, 16-byte loads and stores, four rows per workgroup.
#include "common.hpp"

namespace svhip {

constexpr int kNormThreads = 256;
constexpr int kNormRowsPerBlock = kNormThreads / 64;
constexpr int kNormMaxChunks = 4;  // 16-byte chunks per lane: rows up to 64 * 4 * 8 = 2048 elements

__device__ __forceinline__ uint16_t norm_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

struct NormArgs {
  const uint16_t* x;
  uint16_t* y;
  const float *weight, *bias;     // [W] fp32 or null
  const uint16_t *shift, *scale;  // [B, W] bf16 (rows s_mod apart) or null
  int64_t B, N, W;
  int64_t sxb, sxn, syb, syn, s_mod;
  float eps;
};

template <int CH>
__global__ __launch_bounds__(kNormThreads) void layer_norm_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.B * a.N) return;
  const int64_t b = row / a.N, n = row - b * a.N;
  const uint16_t* xr = a.x + b * a.sxb + n * a.sxn;
  const int chunks = static_cast<int>(a.W / 8);
  float v[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + 64 * c;
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (ch < chunks) w = *reinterpret_cast<const uint4*>(xr + 8 * ch);
    const uint32_t e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = bf16_bits_to_float(static_cast<uint16_t>(e[j >> 1] >> (16 * (j & 1))));
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[c][j];
  }
  const float inv_w = 1.0f / static_cast<float>(a.W);
  const float mean = wave_sum(sum) * inv_w;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (lane + 64 * c < chunks) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = v[c][j] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) * inv_w + a.eps);
  uint16_t* yr = a.y + b * a.syb + n * a.syn;
  const uint16_t* sh = a.shift ? a.shift + b * a.s_mod : nullptr;
  const uint16_t* sc = a.scale ? a.scale + b * a.s_mod : nullptr;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= chunks) continue;
    uint32_t out[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float r[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int col = 8 * ch + j + e;
        float t = (v[c][j + e] - mean) * rstd;
        if (a.weight) t = t * a.weight[col] + (a.bias ? a.bias[col] : 0.f);
        if (sc) {
          const float one_plus = bf16_bits_to_float(norm_bf16_rne(1.0f + bf16_bits_to_float(sc[col])));
          t = t * one_plus + bf16_bits_to_float(sh[col]);
        }
        r[e] = t;
      }
      out[j / 2] = static_cast<uint32_t>(norm_bf16_rne(r[0])) | (static_cast<uint32_t>(norm_bf16_rne(r[1])) << 16);
    }
    *reinterpret_cast<uint4*>(yr + 8 * ch) = make_uint4(out[0], out[1], out[2], out[3]);
  }
}

}  // namespace svhip

using namespace svhip;

extern "C" int svhip_layer_norm(const void* x, void* y, const float* weight, const float* bias, const void* shift,
                                const void* scale, int64_t B, int64_t N, int64_t W, int64_t sx_b, int64_t sx_n,
                                int64_t sy_b, int64_t sy_n, int64_t s_mod, float eps, void* stream) {
  const char* name = "svhip_layer_norm";
  clear_error();
  SVHIP_REQUIRE(x && y, "%s: null pointer", name);
  SVHIP_REQUIRE(B >= 0 && N >= 0, "%s: bad sizes", name);
  SVHIP_REQUIRE(W >= 8 && W % 8 == 0 && W <= 64 * 8 * kNormMaxChunks,
                "%s: width %lld unsupported (a multiple of 8 up to %d)", name, (long long)W, 64 * 8 * kNormMaxChunks);
  SVHIP_REQUIRE(!bias || weight, "%s: bias without weight", name);
  SVHIP_REQUIRE((shift == nullptr) == (scale == nullptr), "%s: shift and scale come together", name);
  SVHIP_REQUIRE(eps >= 0.f, "%s: eps must be non-negative", name);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                    sx_b % 8 == 0 && sx_n % 8 == 0 && sy_b % 8 == 0 && sy_n % 8 == 0,
                "%s: rows must start on 16-byte boundaries", name);
  if (B == 0 || N == 0) return SVHIP_OK;
  NormArgs a{static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), weight, bias,
             static_cast<const uint16_t*>(shift), static_cast<const uint16_t*>(scale), B, N, W, sx_b, sx_n, sy_b,
             sy_n, s_mod, eps};
  const int64_t grid = cdiv(B * N, kNormRowsPerBlock);
  SVHIP_REQUIRE(grid < (1ll << 31), "%s: grid too large", name);
  const int ch = static_cast<int>(cdiv(W / 8, 64));
  hipStream_t s = as_stream(stream);
  const unsigned g = static_cast<unsigned>(grid);
  if (ch == 1) {
    layer_norm_kernel<1><<<g, kNormThreads, 0, s>>>(a);
  } else if (ch == 2) {
    layer_norm_kernel<2><<<g, kNormThreads, 0, s>>>(a);
  } else {
    layer_norm_kernel<4><<<g, kNormThreads, 0, s>>>(a);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}
