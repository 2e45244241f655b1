// Counter-based categorical sampling of a solid step's chosen voxels, in place, at a fixed launch size.
//
// The reference's tail after the selection (stream/fast_ops.py:548-553) gathers the k chosen rows
// (nonzero_static with the step's k), takes softmax and torch.multinomial on the slot's generator and writes the
// draws with index_copy_: its sizes and its random stream depend on k and on the calls before it. This kernel
// draws every chosen voxel from its own counter instead, so one launch over the whole window does the tail and
// a captured step replays it:
//   u = (floor(w0 / 2^41) + 1/2) / 2^23,  w = Philox4x64-10(counter = (voxel, step, 0, 0), key = (seed, stream)),
//   class = the first c with sum_{j <= c} softmax(row)_j > u.
// Philox4x64-10 is the counter-based generator of Salmon, Moraes, Dror and Shaw ("Parallel random numbers: as
// easy as 1, 2, 3", SC 2011): ten rounds of two 64 x 64 -> 128-bit products with the published multipliers, the
// key bumped by the published Weyl constants between rounds. u is an fp32 number in (0, 1).
//
// One workgroup per 512 voxels of a window: every thread reads the chosen flags of 2 voxels and writes -1 (not
// chosen) to `values`; the chosen voxels are compacted into a list in LDS (ballots and prefix counts, in voxel
// order) and only they are hashed (the 64-bit products of Philox are the kernel's costliest arithmetic), while the
// first rows' loads are in flight. The four waves take the listed rows G at a time each, one group of 64 / G lanes
// per row, so that the rows' loads and reductions overlap (a row's chain of load, max, scan and pick is
// latency-bound). For a chosen row each lane of its group holds ceil(C / lanes) consecutive classes; the group
// takes the row max, the exponentials exp(x - max) and their per-lane sums, an inclusive scan of the sums over
// the group gives the CDF at each lane's last class, the first lane whose prefix passes u * total holds the class,
// walks its own classes and writes the draw. Rows whose max is not finite (NaN, all -inf) set `err`.
#include "common.hpp"
#include "stats.hpp"

namespace svhip {

constexpr int kSampleThreads = 256;
constexpr int kSampleVoxels = 512;  // voxels per workgroup, 2 per thread
constexpr int kSampleMaxClasses = 1024;
constexpr int kSampleMaxPerLane = kSampleMaxClasses / 64;
constexpr uint64_t kPhiloxM0 = 0xD2E7470EE14C6C93ull;
constexpr uint64_t kPhiloxM1 = 0xCA5A826395121157ull;
constexpr uint64_t kPhiloxW0 = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kPhiloxW1 = 0xBB67AE8584CAA73Bull;
constexpr uint64_t kSampleStream = 0x53414D504C455631ull;  // "SAMPLEV1"

struct SampleArgs {
  const void* x;        // logit (b, c, voxel v) at b*sb + c*sc + row(v)*sn
  int dtype;
  int64_t C, sb, sc, sn;
  VoxelRows rows;
  const uint8_t* chosen;  // [B, N]
  int64_t* tokens;        // [B, N] or null: chosen voxels get their class
  int16_t* values;        // [B, N]: the class of a chosen voxel, -1 elsewhere
  const int64_t* seed;    // [B]
  const int64_t* step;    // [B]
  int* err;               // set when a chosen row has no finite max
  int64_t N;
};

// First output word of Philox4x64-10 at counter (c0, c1, 0, 0) under key (k0, k1).
__device__ __forceinline__ uint64_t philox_w0(uint64_t c0, uint64_t c1, uint64_t k0, uint64_t k1) {
  uint64_t c2 = 0, c3 = 0;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += kPhiloxW0;
      k1 += kPhiloxW1;
    }
    const uint64_t hi0 = __umul64hi(kPhiloxM0, c0), lo0 = kPhiloxM0 * c0;
    const uint64_t hi1 = __umul64hi(kPhiloxM1, c2), lo1 = kPhiloxM1 * c2;
    const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c1 = lo1;
    c3 = lo0;
    c0 = n0;
    c2 = n2;
  }
  return c0;
}

__device__ __forceinline__ float load_logit(const void* x, int dtype, int64_t off) {
  if (dtype == SVHIP_BF16) return bf16_bits_to_float(static_cast<const uint16_t*>(x)[off]);
  return static_cast<const float*>(x)[off];
}

// LPR lanes per row (16 or 32: four or two rows per wave at a time, or 64), PL classes per lane held in registers
// (LPR * PL >= C; a launch has about two waves per SIMD, so registers do not bound its residency). VEC: rows are
// contiguous (class stride 1) and 16-byte aligned: a lane whose classes all lie inside the row and fill whole
// 16-byte loads reads them so.
template <int LPR, int PL, bool VEC>
__global__ __launch_bounds__(kSampleThreads) void sample_chosen_kernel(SampleArgs a) {
  constexpr int G = 64 / LPR;              // rows per wave at a time
  constexpr int kPerPass = 4 * G;          // rows per pass of the workgroup
  constexpr int kPerThread = kSampleVoxels / kSampleThreads;
  __shared__ uint16_t s_list[kSampleVoxels];  // chosen voxels (offsets in the workgroup's range), voxel order
  __shared__ float s_u[kSampleVoxels];        // their draws
  __shared__ int s_count[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  const int64_t b = blockIdx.y;
  const int64_t wg0 = static_cast<int64_t>(blockIdx.x) * kSampleVoxels;
  // Flags of voxels wg0 + kPerThread tid + k.
  bool f[kPerThread];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t v = wg0 + kPerThread * tid + k;
    f[k] = v < a.N && a.chosen[b * a.N + v] != 0;
    if (v < a.N && !f[k]) a.values[b * a.N + v] = -1;
  }
  // Rank of each chosen voxel: chosen voxels of lower lanes (all k), then this lane's earlier k.
  int below = 0, own = 0;
  int rank[kPerThread];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const uint64_t m = __ballot(f[k]);
    below += __builtin_popcountll(m & ((1ull << lane) - 1));
  }
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    rank[k] = below + own;
    own += f[k] ? 1 : 0;
  }
  if (lane == 63) s_count[w] = below + own;
  __syncthreads();
  int wave_off = 0, total = 0;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    wave_off += x < w ? s_count[x] : 0;
    total += s_count[x];
  }
  if (total == 0) return;  // workgroup-uniform
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    if (f[k]) s_list[wave_off + rank[k]] = static_cast<uint16_t>(kPerThread * tid + k);
  }
  __syncthreads();

  const int c0 = sub * PL;
  const char* xb = static_cast<const char*>(a.x) + b * a.sb * (a.dtype == SVHIP_BF16 ? 2 : 4);
  float e[PL];
  float m = -INFINITY;
  // The row of the pass starting at list entry r0 into e (and its max into m); lanes without a row read nothing.
  auto load_row = [&](int r0) __attribute__((always_inline)) {
    const int r = r0 + w * G + grp;
    const bool active = r < total;
    const int64_t vox = wg0 + s_list[active ? r : r0 + w * G];
    const int64_t row = a.rows(vox) * a.sn;
    m = -INFINITY;
    // (the lane's classes must fill whole 16-byte loads: PL % 8 == 0 for bf16, PL % 4 == 0 for fp32)
    const bool whole = a.dtype == SVHIP_BF16 ? PL % 8 == 0 : PL % 4 == 0;
    if (VEC && whole && active && c0 + PL <= a.C) {
      if (a.dtype == SVHIP_BF16) {
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(static_cast<const void*>(xb)) +
                                                          row + c0);
#pragma unroll
        for (int q = 0; q < PL / 8; ++q) {
          const uint4 x = src[q];
          const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            e[8 * q + 2 * t] = __uint_as_float(xs[t] << 16);
            e[8 * q + 2 * t + 1] = __uint_as_float(xs[t] & 0xffff0000u);
          }
        }
      } else {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(static_cast<const void*>(xb)) +
                                                            row + c0);
#pragma unroll
        for (int q = 0; q < PL / 4; ++q) {
          const float4 x = src[q];
          e[4 * q] = x.x;
          e[4 * q + 1] = x.y;
          e[4 * q + 2] = x.z;
          e[4 * q + 3] = x.w;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < PL; ++j) {
        const int c = c0 + j;
        e[j] = (active && c < a.C) ? load_logit(xb, a.dtype, row + c * a.sc) : -INFINITY;
      }
    }
  };
  // The rest of the pass: the categorical draw of the row each group holds.
  auto finish_row = [&](int r0) __attribute__((always_inline)) {
    const int r = r0 + w * G + grp;
    const bool active = r < total;
    const int64_t vox = wg0 + s_list[active ? r : r0 + w * G];
    const float u = active ? s_u[r] : 0.f;
#pragma unroll
    for (int j = 0; j < PL; ++j) m = fmaxf(m, e[j]);
    // The row max over the group (a NaN logit makes fmaxf skip it; it is caught by the sum below).
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      e[j] = fast_exp(e[j] - m);
      s += e[j];
    }
    // Inclusive scan of the lane sums over the group (class order) and the exclusive prefix of this lane.
    float incl = s;
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) {
      const float t = __shfl_up(incl, o, 64);
      if (sub >= o) incl += t;
    }
    float excl = __shfl_up(incl, 1, 64);
    if (sub == 0) excl = 0.f;
    const float tot = __shfl(incl, grp * LPR + LPR - 1, 64);
    const bool ok = m > -INFINITY && m < INFINITY && tot > 0.f && tot < INFINITY;
    const float target = u * tot;
    const uint64_t gmask = (LPR == 64) ? ~0ull : (((1ull << LPR) - 1) << (grp * LPR));
    const uint64_t past = __ballot(incl > target) & gmask;
    // Rounding can leave u * total at the very top: the last lane with mass then holds the class.
    const uint64_t mass = __ballot(s > 0.f) & gmask;
    const int owner = past ? __builtin_ctzll(past) : (mass ? 63 - __builtin_clzll(mass) : grp * LPR);
    if (active && !ok && sub == 0) {
      // No class is drawn (the reference's multinomial raises here): the voxel keeps its token and reads -1.
      atomicOr(a.err, 1);
      a.values[b * a.N + vox] = -1;
    }
    if (active && ok && lane == owner) {
      int found = -1, last = -1;
      float run = excl;
#pragma unroll
      for (int j = 0; j < PL; ++j) {
        if (e[j] > 0.f) last = c0 + j;
        run += e[j];
        if (found < 0 && run > target && e[j] > 0.f) found = c0 + j;
      }
      if (found < 0) found = last;
      a.values[b * a.N + vox] = static_cast<int16_t>(found);
      if (a.tokens) a.tokens[b * a.N + vox] = found;
    }
  };

  // The first pass's rows are in flight while the listed voxels' draws are hashed:
  // u = (floor(w0 / 2^41) + 1/2) / 2^23.
  const bool first_pass = w * G < total;  // wave-uniform
  if (first_pass) load_row(0);
  const uint64_t seed = static_cast<uint64_t>(a.seed[b]), step = static_cast<uint64_t>(a.step[b]);
  for (int t = tid; t < total; t += kSampleThreads) {
    const uint64_t w0 = philox_w0(static_cast<uint64_t>(wg0 + s_list[t]), step, seed, kSampleStream);
    s_u[t] = (static_cast<float>(w0 >> 41) + 0.5f) * (1.0f / 8388608.0f);
  }
  __syncthreads();
  if (!first_pass) return;  // wave-uniform: no barrier follows
  finish_row(0);
  for (int r0 = kPerPass; r0 < total; r0 += kPerPass) {
    if (r0 + w * G >= total) break;  // wave-uniform: this wave has no row left
    load_row(r0);
    finish_row(r0);
  }
}

}  // namespace svhip

using namespace svhip;

extern "C" int svhip_sample_chosen(const void* logits, int dtype, int64_t classes, int64_t patch, int64_t stride_b,
                                   int64_t stride_c, int64_t stride_n, const uint8_t* chosen, int64_t* tokens,
                                   int16_t* values, const int64_t* seed, const int64_t* step, int* err,
                                   int64_t batch, int64_t Y, int64_t Z, int64_t X, void* stream) {
  const char* name = "svhip_sample_chosen";
  clear_error();
  SVHIP_REQUIRE(logits && chosen && values && seed && step && err, "%s: null pointer", name);
  SVHIP_REQUIRE(dtype == SVHIP_F32 || dtype == SVHIP_BF16, "%s: dtype %d unsupported", name, dtype);
  SVHIP_REQUIRE(classes >= 1 && classes <= kSampleMaxClasses && classes <= 32767,
                "%s: %lld classes unsupported (1..%d)", name, (long long)classes, kSampleMaxClasses);
  SVHIP_REQUIRE(batch >= 0 && Y >= 0 && Z >= 0 && X >= 0 && patch >= 0, "%s: bad sizes", name);
  SVHIP_REQUIRE(stride_b >= 0 && stride_c >= 0 && stride_n >= 0, "%s: negative stride", name);
  const int64_t N = Y * Z * X;
  if (batch == 0 || N == 0) return SVHIP_OK;
  SVHIP_REQUIRE(N <= (int64_t{1} << 40) && batch <= 65535, "%s: window too large", name);
  SampleArgs a;
  a.rows = kYzxRows;
  if (patch > 0) {
    const int rc = make_rows(Y, Z, X, patch, &a.rows, name);
    if (rc != SVHIP_OK) return rc;
  }
  a.x = logits;
  a.dtype = dtype;
  a.C = classes;
  a.sb = stride_b;
  a.sc = stride_c;
  a.sn = stride_n;
  a.chosen = chosen;
  a.tokens = tokens;
  a.values = values;
  a.seed = seed;
  a.step = step;
  a.err = err;
  a.N = N;
  const dim3 grid(static_cast<unsigned>(cdiv(N, kSampleVoxels)), static_cast<unsigned>(batch));
  hipStream_t st = as_stream(stream);
  const int64_t esize = dtype == SVHIP_BF16 ? 2 : 4;
  // 16-byte loads of contiguous rows: class stride 1, 16-byte aligned base and row and window strides (a lane's
  // PL classes start at a multiple of 16 bytes for every PL below).
  const bool vec = stride_c == 1 && reinterpret_cast<uintptr_t>(logits) % 16 == 0 && (stride_n * esize) % 16 == 0 &&
                   (stride_b * esize) % 16 == 0;
#define SVHIP_SAMPLE(LPR, PL)                                                 \
  do {                                                                        \
    if (vec) {                                                                \
      sample_chosen_kernel<LPR, PL, true><<<grid, kSampleThreads, 0, st>>>(a);  \
    } else {                                                                  \
      sample_chosen_kernel<LPR, PL, false><<<grid, kSampleThreads, 0, st>>>(a); \
    }                                                                         \
  } while (0)
  if (classes <= 64) {
    SVHIP_SAMPLE(16, 4);
  } else if (classes <= 128) {
    SVHIP_SAMPLE(16, 8);
  } else if (classes <= 256) {
    SVHIP_SAMPLE(16, 16);
  } else if (classes <= 384) {
    SVHIP_SAMPLE(16, 24);
  } else if (classes <= 512) {
    SVHIP_SAMPLE(32, 16);
  } else {
    SVHIP_SAMPLE(64, kSampleMaxPerLane);
  }
#undef SVHIP_SAMPLE
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}
