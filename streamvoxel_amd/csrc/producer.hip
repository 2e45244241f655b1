// Producers of the cross-attention operands.
//
//  * svhip_axial_rope: AxialRoPE (models/unconditional_md4.py:10-24) on bf16 activations. head_dim D splits into
//    three axes of D/3; inside an axis the adjacent pairs (a, b) = (x[2i], x[2i+1]) turn by the phase
//    pos[axis] * freq[i]. The arithmetic follows the reference under bf16 autocast step by step: the phase is one
//    fp32 product, sin and cos are fp32 and rounded to bf16, and each product and each sum of
//    (a cos - b sin, a sin + b cos) is rounded to bf16 (fp32 operation, then round to nearest even).
//  * svhip_kv_write: one window of the cached context (stream/fast_ops.py:228-250): keys [0, P) from the prefix
//    bank (already rotated), keys [P, P + L) from the local projection (K rotated at the local positions when
//    positions are given), zeros up to the capacity; K as rows [H, Kcap, D], V as rows or transposed
//    [H, D, Kcap]. bf16, or OCP e4m3fn with per-head scales amax / 448 (clamped below at 1e-12) over the window's
//    keys and codes round-to-nearest-even of x / scale.
//  * svhip_qkv_rope: the self-attention operands of RotaryAttention.forward (models/unconditional_md4_timefree.py:
//    41-47) from the fused qkv projection's rows [3, H, D]: Q and K rotated as svhip_axial_rope does (in place or
//    to their own strides), V written transposed [H, D, N] so the attention kernel stages it straight to LDS.
//
// HBM-bound, once per window (K/V) or once per layer and step (Q); one thread per bf16 pair.
#include "common.hpp"

namespace svhip {

constexpr int kTileKeys = 64;
constexpr int kProducerThreads = 256;
constexpr int kMaxHeadDim = 128;

__device__ __forceinline__ uint16_t bf16_rne(float f) { return bf16_bits(f); }

__device__ __forceinline__ float bf16_round(float f) { return bf16_round1(f); }

// OCP e4m3fn (bias 7, 3 mantissa bits, no infinities, S.1111.111 = NaN, largest finite 448, quantum 2^-9 below
// 2^-6), round to nearest even. Magnitudes above 464 (half way between 448 and the NaN code's 480) and NaN give
// the NaN code.
__device__ __forceinline__ uint8_t e4m3fn_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint8_t sign = static_cast<uint8_t>((u >> 24) & 0x80u);
  const float a = __uint_as_float(u & 0x7fffffffu);
  if (!(a <= 464.0f)) return sign | 0x7fu;
  if (a < 0.015625f) {
    // Subnormal range (and the rounding up into 2^-6): m * 2^-9, m = rne(a * 512) in 0..8; m = 8 is the smallest
    // normal, whose code (exponent 1, mantissa 0) is 8 as well.
    return sign | static_cast<uint8_t>(__builtin_rintf(a * 512.0f));
  }
  const uint32_t au = u & 0x7fffffffu;
  int e = static_cast<int>(au >> 23) - 127;  // -6 .. 8
  const uint32_t mant = au & 0x7fffffu;
  uint32_t m = mant >> 20;
  const uint32_t rest = mant & 0xfffffu;
  if (rest > 0x80000u || (rest == 0x80000u && (m & 1u))) ++m;
  if (m == 8u) {
    m = 0u;
    ++e;
  }
  return sign | static_cast<uint8_t>(((e + 7) << 3) | static_cast<int>(m));
}

// One rotated pair (a, b) by sin s and cos c (already rounded to bf16): every product and both sums rounded to
// bf16, two roundings per instruction.
__device__ __forceinline__ void rope_rot(float a, float b, float s, float c, float& ra, float& rb) {
  float ac = a * c, bs = b * s, as = a * s, bc = b * c;
  bf16_round2(ac, bs);
  bf16_round2(as, bc);
  ra = ac - bs;
  rb = as + bc;
  bf16_round2(ra, rb);
}

// One rotated pair: (a, b) at phase p.
__device__ __forceinline__ void rope_pair(float a, float b, float p, float& ra, float& rb) {
  rope_rot(a, b, bf16_round(sinf(p)), bf16_round(cosf(p)), ra, rb);
}

__device__ __forceinline__ void unpack2(uint32_t w, float& a, float& b) {
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) { return bf16_pack2(a, b); }

struct RopeArgs {
  const uint16_t* x;
  uint16_t* out;
  const float* pos;
  const float* freq;
  int64_t B, H, N, D;
  int64_t sxb, sxh, sxn;
  int64_t sob, soh, son;
  int64_t spb, spn;
};

constexpr int kRopeTokens = 8;  // tokens per workgroup of the rotation kernel

// Workgroup = (b, 8 tokens), all heads: the tile's sin / cos (rounded to bf16) of every (token, pair) go to LDS once
// (the phase depends on the token and the pair, not on the head), then every (token, head) row is rotated, 4 pairs
// (16 bytes) per item when VEC (rows 16-byte aligned), else one pair.
template <bool VEC>
__global__ __launch_bounds__(kProducerThreads) void axial_rope_kernel(RopeArgs a) {
  __shared__ float2 sc[kRopeTokens * kMaxHeadDim / 2];
  const int64_t tiles = cdiv(a.N, kRopeTokens);
  const int64_t b = blockIdx.x / tiles, n0 = (blockIdx.x % tiles) * kRopeTokens;
  const int tokens = static_cast<int>(a.N - n0 < kRopeTokens ? a.N - n0 : kRopeTokens);
  const int pairs = static_cast<int>(a.D / 2);
  const int per_axis = static_cast<int>(a.D / 6);  // pairs per axis = number of frequencies
  for (int i = threadIdx.x; i < tokens * pairs; i += kProducerThreads) {
    const int t = i / pairs, pr = i - t * pairs;
    const int axis = pr / per_axis, fi = pr - axis * per_axis;
    const float phase = a.pos[b * a.spb + (n0 + t) * a.spn + axis] * a.freq[fi];
    sc[i] = make_float2(bf16_round(sinf(phase)), bf16_round(cosf(phase)));
  }
  __syncthreads();
  constexpr int kPer = VEC ? 4 : 1;  // pairs per item
  const int groups = pairs / kPer;
  const int items = tokens * static_cast<int>(a.H) * groups;
  for (int i = threadIdx.x; i < items; i += kProducerThreads) {
    const int g = i % groups;
    const int th = i / groups;
    const int h = th % static_cast<int>(a.H), t = th / static_cast<int>(a.H);
    const int64_t n = n0 + t;
    const uint16_t* src = a.x + b * a.sxb + h * a.sxh + n * a.sxn + 2 * kPer * g;
    uint16_t* dst = a.out + b * a.sob + h * a.soh + n * a.son + 2 * kPer * g;
    uint32_t in[kPer], out[kPer];
    if constexpr (VEC) {
      const uint4 w = *reinterpret_cast<const uint4*>(src);
      in[0] = w.x;
      in[1] = w.y;
      in[2] = w.z;
      in[3] = w.w;
    } else {
      in[0] = *reinterpret_cast<const uint32_t*>(src);
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const float2 r = sc[t * pairs + kPer * g + j];
      float x0, x1, r0, r1;
      unpack2(in[j], x0, x1);
      rope_rot(x0, x1, r.x, r.y, r0, r1);
      out[j] = pack2(r0, r1);
    }
    if constexpr (VEC) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(out[0], out[1], out[2], out[3]);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = out[0];
    }
  }
}

struct KvArgs {
  const uint16_t *pk, *pv;  // prefix [H, P, D]
  int64_t P, spk_h, spk_l, spv_h, spv_l;
  const uint16_t *lk, *lv;  // local [H, L, D]
  int64_t L, slk_h, slk_l, slv_h, slv_l;
  const float* pos;  // [L, 3] or null
  int64_t sp_l;
  const float* freq;
  int64_t H, D, kcap;
  void* ck;
  int64_t sck_h, sck_k;
  void* cv;
  int64_t scv_h, scv_k, scv_d;
  float *k_scale, *v_scale;  // [H] (e4m3)
  float* partial;            // [H, tiles, 2] (e4m3)
  int64_t tiles;
};

// K and V pair `pr` of key j of head h (zeros past the window's keys; local K rotated when positions are given).
__device__ __forceinline__ void load_pair(const KvArgs& a, int64_t h, int64_t j, int64_t pr, float& k0, float& k1,
                                          float& v0, float& v1) {
  k0 = k1 = v0 = v1 = 0.f;
  if (j < a.P) {
    unpack2(*reinterpret_cast<const uint32_t*>(a.pk + h * a.spk_h + j * a.spk_l + 2 * pr), k0, k1);
    unpack2(*reinterpret_cast<const uint32_t*>(a.pv + h * a.spv_h + j * a.spv_l + 2 * pr), v0, v1);
  } else if (j < a.P + a.L) {
    const int64_t l = j - a.P;
    unpack2(*reinterpret_cast<const uint32_t*>(a.lk + h * a.slk_h + l * a.slk_l + 2 * pr), k0, k1);
    unpack2(*reinterpret_cast<const uint32_t*>(a.lv + h * a.slv_h + l * a.slv_l + 2 * pr), v0, v1);
    if (a.pos) {
      const int64_t per_axis = a.D / 6;
      const int64_t axis = pr / per_axis, i = pr - axis * per_axis;
      float r0, r1;
      rope_pair(k0, k1, a.pos[l * a.sp_l + axis] * a.freq[i], r0, r1);
      k0 = r0;
      k1 = r1;
    }
  }
}

__device__ __forceinline__ float block_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kProducerThreads / 64; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

// e4m3 only: per (head, 64-key tile) max |K| and max |V| of the window's keys.
__global__ __launch_bounds__(kProducerThreads) void kv_stats_kernel(KvArgs a) {
  __shared__ float red[kProducerThreads / 64];
  const int64_t h = blockIdx.y, tile = blockIdx.x;
  const int64_t pairs = a.D / 2;
  float mk = 0.f, mv = 0.f;
  for (int64_t e = threadIdx.x; e < kTileKeys * pairs; e += kProducerThreads) {
    const int64_t j = tile * kTileKeys + e / pairs;
    if (j >= a.P + a.L) continue;
    float k0, k1, v0, v1;
    load_pair(a, h, j, e % pairs, k0, k1, v0, v1);
    mk = fmaxf(mk, fmaxf(fabsf(k0), fabsf(k1)));
    mv = fmaxf(mv, fmaxf(fabsf(v0), fabsf(v1)));
  }
  mk = block_max(mk, red);
  mv = block_max(mv, red);
  if (threadIdx.x == 0) {
    a.partial[(h * a.tiles + tile) * 2] = mk;
    a.partial[(h * a.tiles + tile) * 2 + 1] = mv;
  }
}

template <bool FP8, bool VT>
__global__ __launch_bounds__(kProducerThreads) void kv_write_kernel(KvArgs a) {
  __shared__ float red[kProducerThreads / 64];
  // V^T staging: [d][key] of one tile, in output element bytes.
  __shared__ __attribute__((aligned(16))) uint8_t sv[kMaxHeadDim * kTileKeys * (FP8 ? 1 : 2)];
  const int64_t h = blockIdx.y, tile = blockIdx.x;
  const int64_t pairs = a.D / 2;
  float sk = 1.f, svs = 1.f;  // e4m3 scales of K and V
  if constexpr (FP8) {
    float mk = 0.f, mv = 0.f;
    for (int64_t t = threadIdx.x; t < a.tiles; t += kProducerThreads) {
      mk = fmaxf(mk, a.partial[(h * a.tiles + t) * 2]);
      mv = fmaxf(mv, a.partial[(h * a.tiles + t) * 2 + 1]);
    }
    mk = block_max(mk, red);
    mv = block_max(mv, red);
    sk = fmaxf(__fdiv_rn(mk, 448.0f), 1e-12f);
    svs = fmaxf(__fdiv_rn(mv, 448.0f), 1e-12f);
    if (tile == 0 && threadIdx.x == 0) {
      a.k_scale[h] = sk;
      a.v_scale[h] = svs;
    }
  }
  for (int64_t e = threadIdx.x; e < kTileKeys * pairs; e += kProducerThreads) {
    const int64_t key = e / pairs, pr = e % pairs;
    const int64_t j = tile * kTileKeys + key;
    if (j >= a.kcap) continue;
    float k0, k1, v0, v1;
    load_pair(a, h, j, pr, k0, k1, v0, v1);
    const int64_t kofs = h * a.sck_h + j * a.sck_k + 2 * pr;
    if constexpr (FP8) {
      const uint16_t kc = static_cast<uint16_t>(e4m3fn_rne(__fdiv_rn(k0, sk))) |
                          static_cast<uint16_t>(static_cast<uint16_t>(e4m3fn_rne(__fdiv_rn(k1, sk))) << 8);
      *reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(a.ck) + kofs) = kc;
      const uint8_t c0 = e4m3fn_rne(__fdiv_rn(v0, svs)), c1 = e4m3fn_rne(__fdiv_rn(v1, svs));
      if constexpr (VT) {
        sv[(2 * pr) * kTileKeys + key] = c0;
        sv[(2 * pr + 1) * kTileKeys + key] = c1;
      } else {
        *reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(a.cv) + h * a.scv_h + j * a.scv_k + 2 * pr) =
            static_cast<uint16_t>(c0) | static_cast<uint16_t>(static_cast<uint16_t>(c1) << 8);
      }
    } else {
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.ck) + kofs) = pack2(k0, k1);
      if constexpr (VT) {
        uint16_t* s16 = reinterpret_cast<uint16_t*>(sv);
        s16[(2 * pr) * kTileKeys + key] = bf16_rne(v0);
        s16[(2 * pr + 1) * kTileKeys + key] = bf16_rne(v1);
      } else {
        *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.cv) + h * a.scv_h + j * a.scv_k + 2 * pr) =
            pack2(v0, v1);
      }
    }
  }
  if constexpr (VT) {
    __syncthreads();
    // Rows of the transposed tile: consecutive threads write consecutive keys of one head_dim element.
    for (int64_t e = threadIdx.x; e < a.D * kTileKeys; e += kProducerThreads) {
      const int64_t d = e / kTileKeys, key = e % kTileKeys;
      const int64_t j = tile * kTileKeys + key;
      if (j >= a.kcap) continue;
      const int64_t vofs = h * a.scv_h + d * a.scv_d + j;
      if constexpr (FP8) {
        static_cast<uint8_t*>(a.cv)[vofs] = sv[d * kTileKeys + key];
      } else {
        static_cast<uint16_t*>(a.cv)[vofs] = reinterpret_cast<const uint16_t*>(sv)[d * kTileKeys + key];
      }
    }
  }
}


// Self-attention operands from the qkv projection, in one launch of two kinds of workgroup:
//  * rotation, (window b, 8-token tile): the tile's sin / cos (rounded to bf16) of every (token, pair) go to LDS
//    once and serve Q and K of all heads (the phase depends on the token and the pair only); the Q | K part of a
//    token's row (2 H D contiguous elements) is then rotated 16 bytes (4 pairs) per thread, four loads in flight;
//  * layout, (window b, head h, 64-token tile): V rows [64 tokens, D] in through LDS, V^T rows [D, 64 tokens] out,
//    16 bytes per store.
struct QkvArgs {
  const uint16_t* x;   // element (b, n, s, h, d) at b*sxb + n*sxn + (s*H + h)*D + d
  const float* pos;    // (b, n, axis) at b*spb + n*spn + axis
  const float* freq;   // [D/6]
  uint16_t *q, *k, *vt;
  int64_t B, N, H, D;
  int64_t sxb, sxn, spb, spn;
  int64_t sqb, sqh, sqn, skb, skh, skn;
  int64_t svb, svh, svd;  // V^T element (b, h, d, n) at b*svb + h*svh + d*svd + n
  int64_t rot_tiles;      // 8-token tiles per window
  int64_t v_tiles;        // 64-token tiles per window
};

constexpr int kRotTokens = 8;
constexpr int kQkvBatch = 4;  // 16-byte loads a thread issues before it uses the first
constexpr int kQkvTokens = 64;
constexpr int kQkvRow = kQkvTokens + 2;  // LDS V^T row stride (bf16 elements), padded against bank conflicts

__device__ __forceinline__ void qkv_rotate(const QkvArgs& a, int64_t b, int64_t tile, float2* sc) {
  const int64_t n0 = tile * kRotTokens;
  const int tokens = static_cast<int>(a.N - n0 < kRotTokens ? a.N - n0 : kRotTokens);
  const int pairs = static_cast<int>(a.D / 2);
  const int per_axis = static_cast<int>(a.D / 6);
  for (int i = threadIdx.x; i < tokens * pairs; i += kProducerThreads) {
    const int t = i / pairs, pr = i - t * pairs;
    const int axis = pr / per_axis, fi = pr - axis * per_axis;
    const float phase = a.pos[b * a.spb + (n0 + t) * a.spn + axis] * a.freq[fi];
    sc[i] = make_float2(bf16_round(sinf(phase)), bf16_round(cosf(phase)));
  }
  __syncthreads();
  const int D = static_cast<int>(a.D);
  const int W = static_cast<int>(a.H) * D;
  const int row_chunks = 2 * W / 8;  // Q | K of one token in 16-byte chunks
  const int total = tokens * row_chunks;
  for (int base = 0; base < total; base += kQkvBatch * kProducerThreads) {
    uint4 w[kQkvBatch];
#pragma unroll
    for (int u = 0; u < kQkvBatch; ++u) {
      const int i = base + u * kProducerThreads + static_cast<int>(threadIdx.x);
      if (i < total) {
        const int t = i / row_chunks, e = 8 * (i - t * row_chunks);
        w[u] = *reinterpret_cast<const uint4*>(a.x + b * a.sxb + (n0 + t) * a.sxn + e);
      }
    }
#pragma unroll
    for (int u = 0; u < kQkvBatch; ++u) {
      const int i = base + u * kProducerThreads + static_cast<int>(threadIdx.x);
      if (i >= total) continue;
      const int t = i / row_chunks, e = 8 * (i - t * row_chunks);
      const int s = e / W, h = (e - s * W) / D, d = e - s * W - h * D;
      const int64_t n = n0 + t;
      const uint32_t in[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
      uint32_t out[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float2 r = sc[t * pairs + d / 2 + j];
        float x0, x1, r0, r1;
        unpack2(in[j], x0, x1);
        rope_rot(x0, x1, r.x, r.y, r0, r1);
        out[j] = pack2(r0, r1);
      }
      uint16_t* dst = s == 0 ? a.q + b * a.sqb + h * a.sqh + n * a.sqn : a.k + b * a.skb + h * a.skh + n * a.skn;
      *reinterpret_cast<uint4*>(dst + d) = make_uint4(out[0], out[1], out[2], out[3]);
    }
  }
}

__device__ __forceinline__ void qkv_layout_v(const QkvArgs& a, int64_t b, int64_t h, int64_t tile, uint16_t* sv) {
  const int64_t n0 = tile * kQkvTokens;
  const int tokens = static_cast<int>(a.N - n0 < kQkvTokens ? a.N - n0 : kQkvTokens);
  const int D = static_cast<int>(a.D);
  const uint16_t* xb = a.x + b * a.sxb + n0 * a.sxn + (2 * a.H + h) * a.D;
  // V rows -> LDS, transposed: sv[d][token].
  const int total = tokens * (D / 8);
  for (int base = 0; base < total; base += kQkvBatch * kProducerThreads) {
    uint4 w[kQkvBatch];
#pragma unroll
    for (int u = 0; u < kQkvBatch; ++u) {
      const int c = base + u * kProducerThreads + static_cast<int>(threadIdx.x);
      if (c < total) w[u] = *reinterpret_cast<const uint4*>(xb + (c / (D / 8)) * a.sxn + 8 * (c % (D / 8)));
    }
#pragma unroll
    for (int u = 0; u < kQkvBatch; ++u) {
      const int c = base + u * kProducerThreads + static_cast<int>(threadIdx.x);
      if (c >= total) continue;
      const int t = c / (D / 8), dc = c % (D / 8);
      const uint32_t e[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sv[(8 * dc + j) * kQkvRow + t] = static_cast<uint16_t>(e[j >> 1] >> (16 * (j & 1)));
      }
    }
  }
  __syncthreads();
  // V^T rows: d-th row of the tile = tokens n0 .. n0 + tokens - 1, 8 per 16-byte store.
  uint16_t* vt = a.vt + b * a.svb + h * a.svh + n0;
  const int tchunks = (tokens + 7) / 8;
  for (int c = threadIdx.x; c < D * tchunks; c += kProducerThreads) {
    const int d = c / tchunks, tc = c % tchunks;
    const uint16_t* src = sv + d * kQkvRow + 8 * tc;
    if (8 * tc + 8 <= tokens) {
      uint4 w;
      w.x = src[0] | (static_cast<uint32_t>(src[1]) << 16);
      w.y = src[2] | (static_cast<uint32_t>(src[3]) << 16);
      w.z = src[4] | (static_cast<uint32_t>(src[5]) << 16);
      w.w = src[6] | (static_cast<uint32_t>(src[7]) << 16);
      *reinterpret_cast<uint4*>(vt + d * a.svd + 8 * tc) = w;
    } else {
      for (int j = 0; 8 * tc + j < tokens; ++j) vt[d * a.svd + 8 * tc + j] = src[j];
    }
  }
}

__global__ __launch_bounds__(kProducerThreads) void qkv_rope_kernel(QkvArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kMaxHeadDim * kQkvRow * 2];
  const int64_t rot_blocks = a.B * a.rot_tiles;
  const int64_t id = blockIdx.x;
  if (id < rot_blocks) {
    qkv_rotate(a, id / a.rot_tiles, id % a.rot_tiles, reinterpret_cast<float2*>(smem));
  } else {
    const int64_t v = id - rot_blocks;
    const int64_t tile = v % a.v_tiles, bh = v / a.v_tiles;
    qkv_layout_v(a, bh / a.H, bh % a.H, tile, reinterpret_cast<uint16_t*>(smem));
  }
}

}  // namespace svhip

using namespace svhip;

extern "C" int svhip_axial_rope(const void* x, void* out, const float* positions, const float* freq, int64_t B,
                                int64_t H, int64_t N, int64_t D, int64_t sx_b, int64_t sx_h, int64_t sx_n,
                                int64_t so_b, int64_t so_h, int64_t so_n, int64_t sp_b, int64_t sp_n, void* stream) {
  const char* name = "svhip_axial_rope";
  clear_error();
  SVHIP_REQUIRE(x && out && positions && freq, "%s: null pointer", name);
  SVHIP_REQUIRE(B >= 0 && H >= 0 && N >= 0, "%s: bad sizes", name);
  SVHIP_REQUIRE(D >= 6 && D % 6 == 0, "%s: head_dim %lld must be a positive multiple of 6 (three even axes)", name,
                (long long)D);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(x) % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 4 == 0 &&
                    sx_b % 2 == 0 && sx_h % 2 == 0 && sx_n % 2 == 0 && so_b % 2 == 0 && so_h % 2 == 0 &&
                    so_n % 2 == 0,
                "%s: rows must start on 4-byte boundaries (head_dim contiguous)", name);
  SVHIP_REQUIRE(D <= kMaxHeadDim, "%s: head_dim %lld above %d", name, (long long)D, kMaxHeadDim);
  const int64_t total = B * H * N * (D / 2);
  if (total == 0) return SVHIP_OK;
  RopeArgs a{static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), positions, freq, B, H, N, D,
             sx_b, sx_h, sx_n, so_b, so_h, so_n, sp_b, sp_n};
  const int64_t grid = B * cdiv(N, kRopeTokens);
  SVHIP_REQUIRE(grid < (1ll << 31), "%s: grid too large", name);
  // Four pairs per item when every row of x and out starts on a 16-byte boundary (head_dim a multiple of 8).
  const bool vec = D % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0 && sx_b % 8 == 0 && sx_h % 8 == 0 && sx_n % 8 == 0 &&
                   so_b % 8 == 0 && so_h % 8 == 0 && so_n % 8 == 0;
  if (vec) {
    axial_rope_kernel<true><<<static_cast<unsigned>(grid), kProducerThreads, 0, as_stream(stream)>>>(a);
  } else {
    axial_rope_kernel<false><<<static_cast<unsigned>(grid), kProducerThreads, 0, as_stream(stream)>>>(a);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

extern "C" size_t svhip_kv_write_workspace_bytes(int64_t H, int64_t kv_cap) {
  if (H <= 0 || kv_cap < 0) return 0;
  return static_cast<size_t>(H * cdiv(kv_cap, kTileKeys) * 2) * sizeof(float);
}

extern "C" int svhip_kv_write(const void* prefix_k, const void* prefix_v, int64_t P, int64_t spk_h, int64_t spk_l,
                              int64_t spv_h, int64_t spv_l, const void* local_k, const void* local_v, int64_t L,
                              int64_t slk_h, int64_t slk_l, int64_t slv_h, int64_t slv_l, const float* positions,
                              int64_t sp_l, const float* freq, int64_t H, int64_t D, void* cache_k, int64_t sck_h,
                              int64_t sck_k, void* cache_v, int64_t scv_h, int64_t scv_k, int64_t scv_d,
                              int64_t kv_cap, int kv_dtype, float* k_scale, float* v_scale, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const char* name = "svhip_kv_write";
  clear_error();
  SVHIP_REQUIRE(cache_k && cache_v, "%s: null cache pointer", name);
  SVHIP_REQUIRE(H >= 1 && D >= 2 && D % 2 == 0 && D <= kMaxHeadDim, "%s: head_dim %lld unsupported (even, <= %d)",
                name, (long long)D, kMaxHeadDim);
  SVHIP_REQUIRE(P >= 0 && L >= 0 && kv_cap >= 0 && P + L <= kv_cap, "%s: %lld + %lld keys exceed the capacity %lld",
                name, (long long)P, (long long)L, (long long)kv_cap);
  SVHIP_REQUIRE(P == 0 || (prefix_k && prefix_v), "%s: null prefix pointer", name);
  SVHIP_REQUIRE(L == 0 || (local_k && local_v), "%s: null local pointer", name);
  SVHIP_REQUIRE(!positions || (freq && D % 6 == 0), "%s: rotation needs frequencies and head_dim a multiple of 6",
                name);
  SVHIP_REQUIRE(kv_dtype == SVHIP_BF16 || kv_dtype == SVHIP_FP8_E4M3, "%s: kv dtype %d unsupported", name, kv_dtype);
  const bool fp8 = kv_dtype == SVHIP_FP8_E4M3;
  SVHIP_REQUIRE(scv_d == 1 || scv_k == 1, "%s: V needs a unit stride along head_dim or keys", name);
  const bool vt = scv_k == 1 && scv_d != 1;
  // 4-byte (bf16) / 2-byte (e4m3) pair accesses.
  auto even = [](const void* p, int64_t a, int64_t b) {
    return reinterpret_cast<uintptr_t>(p) % 4 == 0 && a % 2 == 0 && b % 2 == 0;
  };
  SVHIP_REQUIRE(P == 0 || (even(prefix_k, spk_h, spk_l) && even(prefix_v, spv_h, spv_l)),
                "%s: prefix rows must start on 4-byte boundaries", name);
  SVHIP_REQUIRE(L == 0 || (even(local_k, slk_h, slk_l) && even(local_v, slv_h, slv_l)),
                "%s: local rows must start on 4-byte boundaries", name);
  SVHIP_REQUIRE(even(cache_k, sck_h, sck_k) && (vt || even(cache_v, scv_h, scv_k)),
                "%s: cache rows must start on pair boundaries", name);
  const int64_t tiles = cdiv(kv_cap, kTileKeys);
  if (tiles == 0) return SVHIP_OK;
  if (fp8) {
    SVHIP_REQUIRE(k_scale && v_scale, "%s: e4m3 needs k_scale and v_scale outputs", name);
    SVHIP_REQUIRE(workspace && workspace_bytes >= svhip_kv_write_workspace_bytes(H, kv_cap),
                  "%s: workspace too small (%zu < %zu bytes)", name, workspace_bytes,
                  svhip_kv_write_workspace_bytes(H, kv_cap));
  }
  KvArgs a{static_cast<const uint16_t*>(prefix_k), static_cast<const uint16_t*>(prefix_v), P, spk_h, spk_l, spv_h,
           spv_l, static_cast<const uint16_t*>(local_k), static_cast<const uint16_t*>(local_v), L, slk_h, slk_l,
           slv_h, slv_l, positions, sp_l, freq, H, D, kv_cap, cache_k, sck_h, sck_k, cache_v, scv_h, scv_k, scv_d,
           k_scale, v_scale, static_cast<float*>(workspace), tiles};
  SVHIP_REQUIRE(tiles < 65536 && H < 65536, "%s: grid too large", name);
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(H));
  hipStream_t s = as_stream(stream);
  if (fp8) {
    kv_stats_kernel<<<grid, kProducerThreads, 0, s>>>(a);
    if (vt) {
      kv_write_kernel<true, true><<<grid, kProducerThreads, 0, s>>>(a);
    } else {
      kv_write_kernel<true, false><<<grid, kProducerThreads, 0, s>>>(a);
    }
  } else if (vt) {
    kv_write_kernel<false, true><<<grid, kProducerThreads, 0, s>>>(a);
  } else {
    kv_write_kernel<false, false><<<grid, kProducerThreads, 0, s>>>(a);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

extern "C" int svhip_qkv_rope(const void* qkv, const float* positions, const float* freq, int64_t B, int64_t N,
                              int64_t H, int64_t D, int64_t sx_b, int64_t sx_n, int64_t sp_b, int64_t sp_n, void* q,
                              int64_t sq_b, int64_t sq_h, int64_t sq_n, void* k, int64_t sk_b, int64_t sk_h,
                              int64_t sk_n, void* vt, int64_t svt_b, int64_t svt_h, int64_t svt_d, void* stream) {
  const char* name = "svhip_qkv_rope";
  clear_error();
  SVHIP_REQUIRE(qkv && positions && freq && q && k && vt, "%s: null pointer", name);
  SVHIP_REQUIRE(B >= 0 && N >= 0 && H >= 1, "%s: bad sizes", name);
  SVHIP_REQUIRE(D >= 24 && D <= kMaxHeadDim && D % 24 == 0,
                "%s: head_dim %lld unsupported (a multiple of 24 up to %d: three even axes, 16-byte rows)", name,
                (long long)D, kMaxHeadDim);
  auto aligned16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  SVHIP_REQUIRE(aligned16(qkv) && sx_b % 8 == 0 && sx_n % 8 == 0, "%s: qkv rows must start on 16-byte boundaries",
                name);
  SVHIP_REQUIRE(aligned16(q) && aligned16(k) && sq_b % 8 == 0 && sq_h % 8 == 0 && sq_n % 8 == 0 && sk_b % 8 == 0 &&
                    sk_h % 8 == 0 && sk_n % 8 == 0,
                "%s: Q/K rows must start on 16-byte boundaries (head_dim contiguous)", name);
  SVHIP_REQUIRE(aligned16(vt) && svt_b % 8 == 0 && svt_h % 8 == 0 && svt_d % 8 == 0,
                "%s: V^T rows must start on 16-byte boundaries", name);
  if (B == 0 || N == 0) return SVHIP_OK;
  QkvArgs a{static_cast<const uint16_t*>(qkv), positions, freq, static_cast<uint16_t*>(q), static_cast<uint16_t*>(k),
            static_cast<uint16_t*>(vt), B, N, H, D, sx_b, sx_n, sp_b, sp_n, sq_b, sq_h, sq_n, sk_b, sk_h, sk_n,
            svt_b, svt_h, svt_d, cdiv(N, kRotTokens), cdiv(N, kQkvTokens)};
  const int64_t grid = B * a.rot_tiles + B * H * a.v_tiles;
  SVHIP_REQUIRE(grid < (1ll << 31), "%s: grid too large", name);
  qkv_rope_kernel<<<static_cast<unsigned>(grid), kProducerThreads, 0, as_stream(stream)>>>(a);
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}
