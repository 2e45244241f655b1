// LayerNorm of the transformer blocks' residual stream, with the AdaLN modulation and the gated residual fused in:
//   r = x + g[b] * a            (optional; each product and the sum rounded to bf16, as the reference's bf16
//                                tensors compute `x + g1[:, None] * attn(...)`; without g: r = x + a)
//   y = LN(r) * (1 + scale[b]) + shift[b],   LN(r) = (r - mean) / sqrt(var + eps) [* weight + bias]
// (models/unconditional_md4_timefree.py:12-13,60-63; models/unconditional_md4.py:44-56 for the affine form without
// modulation, fp32 weight and bias). x, a, r, y bf16 [B, N, W] (r may be x, y may be x); mean and the biased
// variance in fp32 over the row held in registers (one HBM read of each input); 1 + scale is rounded to bf16 as
// the reference's bf16 tensors compute it, the rest is fp32 and y is rounded once.
//
// HBM-bound: rows of 256 to 1024 in multiples of 256 take 32 lanes each (2 rows per wave), other rows up to 1024
// wide 16 lanes (4 rows per wave, sums over DPP within the 16-lane row), wider rows a whole wave; 16-byte loads and stores of the rows and of the per-window gate / shift / scale rows
// when those are 16-byte aligned.
#include "common.hpp"

namespace svhip {

constexpr int kNormThreads = 256;
constexpr int kNormMaxWidth = 2048;  // 64 lanes x 4 chunks x 8 elements



// Sum over the LPR lanes of a row (16: one DPP row; 32: two DPP rows joined by a lane swap across 16; 64: the
// whole wave, the four DPP rows read back by readlane).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
  v = row16_sum(v);
  if constexpr (LPR == 32) {
    v += __shfl_xor(v, 16, 64);  // the other 16-lane row of the pair
  } else if constexpr (LPR == 64) {
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  }
  return v;
}

// 8 bf16 of a 16-byte chunk -> fp32.
__device__ __forceinline__ void unpack8(const uint4& w, float* v) {
  const uint32_t e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = bf16_bits_to_float(static_cast<uint16_t>(e[j >> 1] >> (16 * (j & 1))));
}

// 8 elements of a per-window row: one 16-byte load when VEC, else 8 two-byte loads.
template <bool VEC>
__device__ __forceinline__ void load_row8(const uint16_t* p, float* v) {
  if constexpr (VEC) {
    unpack8(*reinterpret_cast<const uint4*>(p), v);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = bf16_bits_to_float(p[j]);
  }
}

struct NormArgs {
  const uint16_t* x;
  const uint16_t* a;     // residual branch [B, N, W] or null
  const uint16_t* gate;  // [B, W] (rows s_gate apart) or null
  uint16_t* r;           // residual output or null
  uint16_t* y;           // normalised output or null
  const float *weight, *bias;     // [W] fp32 or null
  const uint16_t *shift, *scale;  // [B, W] bf16 (rows s_mod apart) or null
  int64_t B, N, W;
  int64_t sxb, sxn, sab, san, srb, srn, syb, syn, s_gate, s_mod;
  float eps;
};

// LPR lanes per row, CH 16-byte chunks per lane (chunk lane + LPR c). RES: a residual branch is added (gated when
// gate is set). VEC: gate / shift / scale rows take 16-byte loads.
template <int LPR, int CH, bool RES, bool VEC>
__global__ __launch_bounds__(kNormThreads) void layer_norm_kernel(NormArgs a) {
  constexpr int kRowsPerBlock = kNormThreads / LPR;
  const int lane = threadIdx.x % LPR;
  int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / LPR;
  // Rows past the end repeat the last row's loads and reductions (the DPP sums need the whole row group) and
  // store nothing.
  const bool live = row < a.B * a.N;
  if (!live) row = a.B * a.N - 1;
  const int64_t b = row / a.N, n = row - b * a.N;
  const uint16_t* xr = a.x + b * a.sxb + n * a.sxn;
  const int chunks = static_cast<int>(a.W / 8);
  float v[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + LPR * c;
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (ch < chunks) w = *reinterpret_cast<const uint4*>(xr + 8 * ch);
    unpack8(w, v[c]);
  }
  if constexpr (RES) {
    const uint16_t* ar = a.a + b * a.sab + n * a.san;
    uint16_t* rr = a.r + b * a.srb + n * a.srn;
    const uint16_t* gr = a.gate ? a.gate + b * a.s_gate : nullptr;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = lane + LPR * c;
      if (ch >= chunks) continue;
      float br[8];
      unpack8(*reinterpret_cast<const uint4*>(ar + 8 * ch), br);
      if (gr) {
        float g[8];
        load_row8<VEC>(gr + 8 * ch, g);
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          br[j] *= g[j];
          br[j + 1] *= g[j + 1];
          bf16_round2(br[j], br[j + 1]);
        }
      }
      uint32_t out[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        out[j / 2] = bf16_pack2(v[c][j] + br[j], v[c][j + 1] + br[j + 1]);
        v[c][j] = __uint_as_float(out[j / 2] << 16);
        v[c][j + 1] = __uint_as_float(out[j / 2] & 0xffff0000u);
      }
      if (live) *reinterpret_cast<uint4*>(rr + 8 * ch) = make_uint4(out[0], out[1], out[2], out[3]);
    }
    if (!a.y) return;
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += (lane + LPR * c < chunks) ? v[c][j] : 0.f;
  }
  const float inv_w = 1.0f / static_cast<float>(a.W);
  const float mean = row_sum<LPR>(sum) * inv_w;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (lane + LPR * c < chunks) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = v[c][j] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(row_sum<LPR>(sq) * inv_w + a.eps);
  if (!live) return;
  uint16_t* yr = a.y + b * a.syb + n * a.syn;
  const uint16_t* sh = a.shift ? a.shift + b * a.s_mod : nullptr;
  const uint16_t* sc = a.scale ? a.scale + b * a.s_mod : nullptr;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + LPR * c;
    if (ch >= chunks) continue;
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = (v[c][j] - mean) * rstd;
    if (a.weight) {
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] = t[j] * a.weight[8 * ch + j] + (a.bias ? a.bias[8 * ch + j] : 0.f);
    }
    if (sc) {
      float s8[8], h8[8];
      load_row8<VEC>(sc + 8 * ch, s8);
      load_row8<VEC>(sh + 8 * ch, h8);
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float o0 = 1.0f + s8[j], o1 = 1.0f + s8[j + 1];
        bf16_round2(o0, o1);
        t[j] = t[j] * o0 + h8[j];
        t[j + 1] = t[j + 1] * o1 + h8[j + 1];
      }
    }
    uint32_t out[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      out[j / 2] = bf16_pack2(t[j], t[j + 1]);
    }
    *reinterpret_cast<uint4*>(yr + 8 * ch) = make_uint4(out[0], out[1], out[2], out[3]);
  }
}

template <bool RES, bool VEC>
void launch_norm(const NormArgs& a, hipStream_t s) {
  const int64_t rows = a.B * a.N;
  const int64_t chunks = a.W / 8;
  if (chunks % 32 == 0 && chunks <= 32 * 4) {
    // Rows of 256, 512, 768 or 1024: 32 lanes per row, two rows per wave (twice the waves of 16 lanes per row).
    const unsigned g = static_cast<unsigned>(cdiv(rows, kNormThreads / 32));
    switch (chunks / 32) {
      case 1: layer_norm_kernel<32, 1, RES, VEC><<<g, kNormThreads, 0, s>>>(a); break;
      case 2: layer_norm_kernel<32, 2, RES, VEC><<<g, kNormThreads, 0, s>>>(a); break;
      case 3: layer_norm_kernel<32, 3, RES, VEC><<<g, kNormThreads, 0, s>>>(a); break;
      default: layer_norm_kernel<32, 4, RES, VEC><<<g, kNormThreads, 0, s>>>(a); break;
    }
  } else if (chunks <= 16 * 8) {
    const unsigned g = static_cast<unsigned>(cdiv(rows, kNormThreads / 16));
    if (chunks <= 16 * 2) {
      layer_norm_kernel<16, 2, RES, VEC><<<g, kNormThreads, 0, s>>>(a);
    } else if (chunks <= 16 * 3) {
      layer_norm_kernel<16, 3, RES, VEC><<<g, kNormThreads, 0, s>>>(a);
    } else if (chunks <= 16 * 4) {
      layer_norm_kernel<16, 4, RES, VEC><<<g, kNormThreads, 0, s>>>(a);
    } else if (chunks <= 16 * 6) {
      layer_norm_kernel<16, 6, RES, VEC><<<g, kNormThreads, 0, s>>>(a);
    } else {
      layer_norm_kernel<16, 8, RES, VEC><<<g, kNormThreads, 0, s>>>(a);
    }
  } else {
    const unsigned g = static_cast<unsigned>(cdiv(rows, kNormThreads / 64));
    layer_norm_kernel<64, 4, RES, VEC><<<g, kNormThreads, 0, s>>>(a);
  }
}

static bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

static int norm_entry(const char* name, NormArgs a, hipStream_t stream) {
  SVHIP_REQUIRE(a.B >= 0 && a.N >= 0, "%s: bad sizes", name);
  SVHIP_REQUIRE(a.W >= 8 && a.W % 8 == 0 && a.W <= kNormMaxWidth,
                "%s: width %lld unsupported (a multiple of 8 up to %d)", name, (long long)a.W, kNormMaxWidth);
  SVHIP_REQUIRE(!a.bias || a.weight, "%s: bias without weight", name);
  SVHIP_REQUIRE((a.shift == nullptr) == (a.scale == nullptr), "%s: shift and scale come together", name);
  SVHIP_REQUIRE(a.eps >= 0.f, "%s: eps must be non-negative", name);
  SVHIP_REQUIRE(aligned16(a.x) && a.sxb % 8 == 0 && a.sxn % 8 == 0, "%s: x rows must start on 16-byte boundaries",
                name);
  SVHIP_REQUIRE(!a.y || (aligned16(a.y) && a.syb % 8 == 0 && a.syn % 8 == 0),
                "%s: y rows must start on 16-byte boundaries", name);
  SVHIP_REQUIRE(!a.a || (aligned16(a.a) && a.sab % 8 == 0 && a.san % 8 == 0 && aligned16(a.r) && a.srb % 8 == 0 &&
                         a.srn % 8 == 0),
                "%s: residual rows must start on 16-byte boundaries", name);
  if (a.B == 0 || a.N == 0) return SVHIP_OK;
  SVHIP_REQUIRE(cdiv(a.B * a.N, kNormThreads / 16) < (1ll << 31), "%s: grid too large", name);
  const bool vec = (!a.gate || (aligned16(a.gate) && a.s_gate % 8 == 0)) &&
                   (!a.shift || (aligned16(a.shift) && aligned16(a.scale) && a.s_mod % 8 == 0));
  if (a.a) {
    if (vec) {
      launch_norm<true, true>(a, stream);
    } else {
      launch_norm<true, false>(a, stream);
    }
  } else if (vec) {
    launch_norm<false, true>(a, stream);
  } else {
    launch_norm<false, false>(a, stream);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

}  // namespace svhip

using namespace svhip;

extern "C" int svhip_layer_norm(const void* x, void* y, const float* weight, const float* bias, const void* shift,
                                const void* scale, int64_t B, int64_t N, int64_t W, int64_t sx_b, int64_t sx_n,
                                int64_t sy_b, int64_t sy_n, int64_t s_mod, float eps, void* stream) {
  const char* name = "svhip_layer_norm";
  clear_error();
  SVHIP_REQUIRE(x && y, "%s: null pointer", name);
  NormArgs a{static_cast<const uint16_t*>(x), nullptr, nullptr, nullptr, static_cast<uint16_t*>(y), weight, bias,
             static_cast<const uint16_t*>(shift), static_cast<const uint16_t*>(scale), B, N, W, sx_b, sx_n, 0, 0, 0,
             0, sy_b, sy_n, 0, s_mod, eps};
  return norm_entry(name, a, as_stream(stream));
}

extern "C" int svhip_residual_norm(const void* x, const void* branch, const void* gate, int64_t s_gate, void* r,
                                   void* y, const float* weight, const float* bias, const void* shift,
                                   const void* scale, int64_t s_mod, int64_t B, int64_t N, int64_t W, int64_t sx_b,
                                   int64_t sx_n, int64_t sa_b, int64_t sa_n, int64_t sr_b, int64_t sr_n,
                                   int64_t sy_b, int64_t sy_n, float eps, void* stream) {
  const char* name = "svhip_residual_norm";
  clear_error();
  SVHIP_REQUIRE(x && branch && r, "%s: null pointer", name);
  NormArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(branch),
             static_cast<const uint16_t*>(gate), static_cast<uint16_t*>(r), static_cast<uint16_t*>(y), weight, bias,
             static_cast<const uint16_t*>(shift), static_cast<const uint16_t*>(scale), B, N, W, sx_b, sx_n, sa_b,
             sa_n, sr_b, sr_n, sy_b, sy_n, s_gate, s_mod, eps};
  return norm_entry(name, a, as_stream(stream));
}
