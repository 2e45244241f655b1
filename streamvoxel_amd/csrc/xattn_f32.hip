// Cross attention in fp32 arithmetic: fp32 Q/K/V/O, every product, sum and exponential in fp32 on the VALU.
//
// The single-column configuration runs the reference's cross attention in fp32 (the masked SDPA of
// SlotCrossAttention.forward, streamvoxel/stream/engine.py:28-47, on fp32 tensors). The bf16 kernel rounds its
// operands to bf16 for the matrix cores; this one keeps the reference's arithmetic width, for callers that hand
// over fp32 tensors and want fp32 results (it runs on the VALU at the fp32 FMA rate, well below the bf16 kernel's
// throughput).
//
// Work item: one workgroup = (window b, head h, 64-query tile), 8 waves; lane l of every wave holds query l of the
// tile (q and the running O in registers). Wave w takes the window's 16-key blocks w, w + 8, w + 16, ...: it
// stages a block's K and V rows in its own LDS area (16-byte loads, the next block's loads in flight while the
// current one is computed, keys >= L as zeros), reads each row back with one address for all lanes (an LDS
// broadcast), forms the 16 scores, raises its running max m (log2 units) to the block's, rescales O and l once and
// adds the 16 weighted V rows. The eight partial (m, l, O) are merged pairwise through LDS in three rounds.
//
// KMASK: a key mask on top of the window length (the reference's `prefix_valid ++ local_valid`): key j of window b
// is attended only where kv_mask[b * sm_b + j] != 0. A block's 16 mask bytes are read one per lane and gathered
// by a ballot; a block (and every block before it) may then hold no attended key, so the running max may stay
// -inf, against which nothing is added.
#include "common.hpp"

namespace svhip {

constexpr int kF32Waves = 8;
constexpr int kF32Threads = 64 * kF32Waves;
constexpr int kF32Keys = 16;  // keys per block
constexpr int kF32MaxD = 64;

struct XattnF32Params {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  const int32_t* kv_len;
  const int32_t* cu_seqlens;
  const uint8_t* kv_mask;  // KMASK: [B, kv_cap] bytes, rows sm_b apart
  int64_t sm_b;
  int64_t B, H, Q, kv_cap;
  int64_t sq_b, sq_h, sq_q;
  int64_t sk_b, sk_h, sk_k;
  int64_t sv_b, sv_h, sv_k, sv_d;
  int64_t so_b, so_h, so_q;
  float scale_log2;  // softmax scale * log2(e)
  int q_tiles;
};

// VT: V given as V^T rows (keys contiguous, element (key, d) at d * sv_d + key), else V rows (head_dim
// contiguous). Rows start 16-byte aligned (checked by the entry point).
template <int D, bool VT, bool KMASK>
__global__ __launch_bounds__(kF32Threads) void xattn_f32_kernel(XattnF32Params p) {
  constexpr int kBlock = kF32Keys * D;   // floats of one staged K (or V) block
  constexpr int kPer = kBlock / 256;     // float4 per lane and block
  static_assert(kBlock % 256 == 0, "head_dim a multiple of 16");
  // Staging (8 waves x K, V blocks, [key][d]) during the loop; the merge area ([wave][D + 2][lane] for four
  // waves) afterwards.
  constexpr int kStage = kF32Waves * 2 * kF32Keys * kF32MaxD;
  constexpr int kMerge = 4 * (kF32MaxD + 2) * 64;
  __shared__ __attribute__((aligned(16))) float s_buf[kStage > kMerge ? kStage : kMerge];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t unit = blockIdx.x / p.q_tiles;
  const int qt = static_cast<int>(blockIdx.x % p.q_tiles);
  const int64_t b = unit / p.H, h = unit % p.H;
  int64_t L, off = 0;
  if (p.cu_seqlens) {
    off = p.cu_seqlens[b];
    L = static_cast<int64_t>(p.cu_seqlens[b + 1]) - off;
    if (KMASK && L > p.kv_cap) L = p.kv_cap;  // the mask rows hold kv_cap keys
  } else {
    L = p.kv_len ? p.kv_len[b] : p.kv_cap;    // no kv_len (key mask only): every key of the row
    if (L > p.kv_cap) L = p.kv_cap;
  }
  if (L < 0) L = 0;
  const uint8_t* mrow = KMASK ? p.kv_mask + b * p.sm_b : nullptr;
  const int64_t q = static_cast<int64_t>(qt) * 64 + lane;
  const bool q_ok = q < p.Q;
  const float* K = p.k + (p.cu_seqlens ? 0 : b * p.sk_b) + h * p.sk_h + off * p.sk_k;
  const float* V = p.v + (p.cu_seqlens ? 0 : b * p.sv_b) + h * p.sv_h + off * p.sv_k;
  float* sK = s_buf + w * 2 * kBlock;
  float* sV = sK + kBlock;

  float qv[D], o[D];
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q_ok) x = *reinterpret_cast<const float4*>(p.q + b * p.sq_b + h * p.sq_h + q * p.sq_q + d);
    qv[d] = x.x;
    qv[d + 1] = x.y;
    qv[d + 2] = x.z;
    qv[d + 3] = x.w;
  }
#pragma unroll
  for (int d = 0; d < D; ++d) o[d] = 0.f;
  const float sl2 = p.scale_log2;
  float m = -INFINITY, l = 0.f;

  // Block loads: float4 r of this lane is element 4 (lane + 64 r) of the block: K row / V row (key, d) with
  // d = e % D, or V^T row d = e / 16 at keys 4 ((e % 16) / 4) .. + 3 (4 consecutive keys of one head_dim element).
  // Every load is issued (keys >= L read row L - 1, in bounds) and a select puts zeros there: no branch in the loop,
  // so the compiler keeps each row's reads next to its products.
  float4 nk[kPer], nv[kPer];
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
  auto load_block = [&](int64_t kv0) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int e = 4 * (lane + 64 * r);
      const int64_t key = kv0 + e / D;
      const int64_t kc = key < L ? key : L - 1;
      const int d = e % D;
      const float4 xk = *reinterpret_cast<const float4*>(K + kc * p.sk_k + d);
      nk[r] = key < L ? xk : zero4;
      if constexpr (VT) {
        const int dv = e / kF32Keys;
        const int64_t k4 = kv0 + (e % kF32Keys);
        const float* row = V + dv * p.sv_d;
        float xv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t kj = k4 + j < L ? k4 + j : L - 1;
          const float x = row[kj];
          xv[j] = k4 + j < L ? x : 0.f;
        }
        nv[r] = make_float4(xv[0], xv[1], xv[2], xv[3]);
      } else {
        const float4 xv = *reinterpret_cast<const float4*>(V + kc * p.sv_k + d);
        nv[r] = key < L ? xv : zero4;
      }
    }
  };
  auto store_block = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int e = 4 * (lane + 64 * r);
      *reinterpret_cast<float4*>(sK + e) = nk[r];
      if constexpr (VT) {
        const int dv = e / kF32Keys, kk = e % kF32Keys;
        sV[kk * D + dv] = nv[r].x;
        sV[(kk + 1) * D + dv] = nv[r].y;
        sV[(kk + 2) * D + dv] = nv[r].z;
        sV[(kk + 3) * D + dv] = nv[r].w;
      } else {
        *reinterpret_cast<float4*>(sV + e) = nv[r];
      }
    }
  };

  int64_t kv0 = static_cast<int64_t>(w) * kF32Keys;
  if (kv0 < L) {
    load_block(kv0);
    store_block();
  }
  for (; kv0 < L; kv0 += kF32Waves * kF32Keys) {
    // KMASK: bit i of `attended` = key kv0 + i below L and attended (lane i reads its byte; lanes 16-63 repeat
    // lanes 0-15); wave-uniform.
    uint32_t attended = 0xffffu;
    if constexpr (KMASK) {
      const int left = static_cast<int>(L - kv0);  // keys of the window from kv0 on (>= 1; L < 2^31)
      const int kk = min(lane & (kF32Keys - 1), left - 1);
      attended = static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(mrow[kv0 + kk] != 0)) & 0xffffu;
      if (left < kF32Keys) attended &= (1u << left) - 1u;
    }
    const int64_t next = kv0 + kF32Waves * kF32Keys;
    load_block(next);  // in flight while this block is computed (zeros past the window)
    float t[kF32Keys];
    float mb = -INFINITY;
#pragma unroll
    for (int i = 0; i < kF32Keys; ++i) {
      const float* kr = sK + i * D;
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 x = *reinterpret_cast<const float4*>(kr + d);
        acc = __builtin_fmaf(qv[d], x.x, acc);
        acc = __builtin_fmaf(qv[d + 1], x.y, acc);
        acc = __builtin_fmaf(qv[d + 2], x.z, acc);
        acc = __builtin_fmaf(qv[d + 3], x.w, acc);
      }
      // Branch-free: keys >= L (zero rows, acc = 0) take the bias -inf. A select on acc would let the compiler put
      // each row's products under a branch and hoist every row's LDS reads above all of them.
      const float bias = (KMASK ? ((attended >> i) & 1u) != 0u : kv0 + i < L) ? 0.f : -INFINITY;
      t[i] = __builtin_fmaf(acc, sl2, bias);
      mb = fmaxf(mb, t[i]);
    }
    const float mn = fmaxf(m, mb);  // finite without a key mask: the block holds at least one key
    // With a key mask mn is -inf while no attended key has come: the exponentials are then taken against 0, which
    // gives 0 for every weight and for alpha (O and l hold nothing yet).
    const float mref = (KMASK && mn == -INFINITY) ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - mref);  // 0 on the wave's first block
    m = mn;
    l *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] *= alpha;
#pragma unroll
    for (int i = 0; i < kF32Keys; ++i) {
      const float pw = __builtin_amdgcn_exp2f(t[i] - mref);  // 0 for keys >= L and keys not attended
      l += pw;
      const float* vr = sV + i * D;
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 x = *reinterpret_cast<const float4*>(vr + d);
        o[d] = __builtin_fmaf(pw, x.x, o[d]);
        o[d + 1] = __builtin_fmaf(pw, x.y, o[d + 1]);
        o[d + 2] = __builtin_fmaf(pw, x.z, o[d + 2]);
        o[d + 3] = __builtin_fmaf(pw, x.w, o[d + 3]);
      }
    }
    store_block();
  }

  // Merge: round r, waves [n/2, n) hand their (O, m, l) to waves [0, n/2) (n = 8, 4, 2).
  float* part = s_buf;
  for (int n = kF32Waves; n > 1; n >>= 1) {
    const int half = n >> 1;
    __syncthreads();
    if (w >= half && w < n) {
      float* dst = part + (w - half) * (kF32MaxD + 2) * 64 + lane;
#pragma unroll
      for (int d = 0; d < D; ++d) dst[d * 64] = o[d];
      dst[D * 64] = m;
      dst[(D + 1) * 64] = l;
    }
    __syncthreads();
    if (w < half) {
      const float* src = part + w * (kF32MaxD + 2) * 64 + lane;
      const float m2 = src[D * 64], l2 = src[(D + 1) * 64];
      const float mm = fmaxf(m, m2);
      // A wave that saw no key keeps m = -inf, l = 0 and O = 0: its factor is exp2(-inf) = 0; with both at -inf
      // (no key at all) both factors are 0.
      const float a1 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mm);
      const float a2 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - mm);
#pragma unroll
      for (int d = 0; d < D; ++d) o[d] = o[d] * a1 + src[d * 64] * a2;
      l = l * a1 + l2 * a2;
      m = mm;
    }
  }
  if (w == 0 && q_ok) {
    // No key at all (L = 0, or no attended key): zeros, as the bf16 kernel writes.
    const float inv = l > 0.f ? 1.f / l : 0.f;
    float* out = p.o + b * p.so_b + h * p.so_h + q * p.so_q;
#pragma unroll
    for (int d = 0; d < D; ++d) out[d] = o[d] * inv;
  }
}

template <int D, bool KMASK>
static void launch_f32(const XattnF32Params& p, unsigned grid, hipStream_t s, bool vt) {
  if (vt) {
    xattn_f32_kernel<D, true, KMASK><<<grid, kF32Threads, 0, s>>>(p);
  } else {
    xattn_f32_kernel<D, false, KMASK><<<grid, kF32Threads, 0, s>>>(p);
  }
}

template <int D>
static void launch_f32(const XattnF32Params& p, unsigned grid, hipStream_t s, bool vt) {
  if (p.kv_mask) {
    launch_f32<D, true>(p, grid, s, vt);
  } else {
    launch_f32<D, false>(p, grid, s, vt);
  }
}

}  // namespace svhip

using namespace svhip;

static int xattn_f32_impl(const float* q, const float* k, const float* v, float* o, const uint8_t* kv_mask,
                          int64_t sm_b, const int32_t* kv_len, const int32_t* cu_seqlens, int64_t B, int64_t H,
                          int64_t Q, int64_t D, int64_t kv_cap, int64_t sq_b, int64_t sq_h, int64_t sq_q,
                          int64_t sk_b, int64_t sk_h, int64_t sk_k, int64_t sv_b, int64_t sv_h, int64_t sv_k,
                          int64_t sv_d, int64_t so_b, int64_t so_h, int64_t so_q, float scale, void* stream,
                          const char* name) {
  clear_error();
  SVHIP_REQUIRE(q && k && v && o, "%s: null pointer", name);
  if (kv_mask) {
    SVHIP_REQUIRE(sm_b >= 0, "%s: negative mask row stride", name);
  } else {
    SVHIP_REQUIRE(kv_len || cu_seqlens, "%s: need kv_len or cu_seqlens", name);
  }
  SVHIP_REQUIRE(!(kv_len && cu_seqlens), "%s: kv_len and cu_seqlens are exclusive", name);
  SVHIP_REQUIRE(B >= 0 && H >= 1 && Q >= 0, "%s: bad sizes", name);
  SVHIP_REQUIRE(D == 16 || D == 32 || D == 48 || D == 64, "%s: head_dim %lld unsupported (16, 32, 48 or 64)", name,
                (long long)D);
  SVHIP_REQUIRE(scale > 0.f && scale < 3.0e38f, "%s: softmax scale must be positive and finite", name);
  SVHIP_REQUIRE(kv_cap >= 0 && kv_cap < (1ll << 31), "%s: kv_cap out of range", name);
  SVHIP_REQUIRE(sv_k == 1 || sv_d == 1, "%s: V needs a unit stride along keys or head_dim", name);
  const bool vt = sv_k == 1 && sv_d != 1;
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && sq_q % 4 == 0 && sq_h % 4 == 0 && sq_b % 4 == 0,
                "%s: Q rows must be 16-byte aligned", name);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(k) % 16 == 0 && sk_k % 4 == 0 && sk_h % 4 == 0 && sk_b % 4 == 0,
                "%s: K rows must be 16-byte aligned", name);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(v) % 16 == 0 && (vt ? sv_d : sv_k) % 4 == 0 && sv_h % 4 == 0 &&
                    sv_b % 4 == 0,
                "%s: V rows must be 16-byte aligned", name);
  if (B == 0 || Q == 0) return SVHIP_OK;
  XattnF32Params p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.kv_len = kv_len;
  p.cu_seqlens = cu_seqlens;
  p.kv_mask = kv_mask;
  p.sm_b = sm_b;
  p.B = B;
  p.H = H;
  p.Q = Q;
  p.kv_cap = kv_cap;
  p.sq_b = sq_b;
  p.sq_h = sq_h;
  p.sq_q = sq_q;
  p.sk_b = sk_b;
  p.sk_h = sk_h;
  p.sk_k = sk_k;
  p.sv_b = sv_b;
  p.sv_h = sv_h;
  p.sv_k = sv_k;
  p.sv_d = sv_d;
  p.so_b = so_b;
  p.so_h = so_h;
  p.so_q = so_q;
  p.scale_log2 = scale * kLog2e;
  p.q_tiles = static_cast<int>(cdiv(Q, 64));
  const int64_t grid = static_cast<int64_t>(p.q_tiles) * H * B;
  SVHIP_REQUIRE(grid < (1ll << 31), "%s: grid too large", name);
  hipStream_t s = as_stream(stream);
  const unsigned g = static_cast<unsigned>(grid);
  switch (D) {
    case 16:
      launch_f32<16>(p, g, s, vt);
      break;
    case 32:
      launch_f32<32>(p, g, s, vt);
      break;
    case 48:
      launch_f32<48>(p, g, s, vt);
      break;
    default:
      launch_f32<64>(p, g, s, vt);
      break;
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

extern "C" int svhip_xattn_fwd_f32(const float* q, const float* k, const float* v, float* o, const int32_t* kv_len,
                                   const int32_t* cu_seqlens, int64_t B, int64_t H, int64_t Q, int64_t D,
                                   int64_t kv_cap, int64_t sq_b, int64_t sq_h, int64_t sq_q, int64_t sk_b,
                                   int64_t sk_h, int64_t sk_k, int64_t sv_b, int64_t sv_h, int64_t sv_k, int64_t sv_d,
                                   int64_t so_b, int64_t so_h, int64_t so_q, float scale, void* stream) {
  return xattn_f32_impl(q, k, v, o, nullptr, 0, kv_len, cu_seqlens, B, H, Q, D, kv_cap, sq_b, sq_h, sq_q, sk_b, sk_h,
                        sk_k, sv_b, sv_h, sv_k, sv_d, so_b, so_h, so_q, scale, stream, "svhip_xattn_fwd_f32");
}

extern "C" int svhip_xattn_fwd_f32_masked(const float* q, const float* k, const float* v, float* o,
                                          const uint8_t* kv_mask, int64_t sm_b, const int32_t* kv_len,
                                          const int32_t* cu_seqlens, int64_t B, int64_t H, int64_t Q, int64_t D,
                                          int64_t kv_cap, int64_t sq_b, int64_t sq_h, int64_t sq_q, int64_t sk_b,
                                          int64_t sk_h, int64_t sk_k, int64_t sv_b, int64_t sv_h, int64_t sv_k,
                                          int64_t sv_d, int64_t so_b, int64_t so_h, int64_t so_q, float scale,
                                          void* stream) {
  const char* name = "svhip_xattn_fwd_f32_masked";
  clear_error();
  SVHIP_REQUIRE(kv_mask, "%s: null key mask", name);
  return xattn_f32_impl(q, k, v, o, kv_mask, sm_b, kv_len, cu_seqlens, B, H, Q, D, kv_cap, sq_b, sq_h, sq_q, sk_b,
                        sk_h, sk_k, sv_b, sv_h, sv_k, sv_d, so_b, so_h, so_q, scale, stream, name);
}
