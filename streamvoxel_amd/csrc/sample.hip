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
// One wave per 64 voxels: the lanes read their voxels' chosen flags, write -1 (not chosen) to `values`, and the
// wave then walks its chosen voxels one at a time. For a chosen row each lane holds ceil(C / 64) consecutive
// classes; the wave takes the row max, the exponentials exp(x - max) and their per-lane sums, an inclusive scan of
// the sums over the lanes gives the CDF at each lane's last class, the first lane whose prefix passes u * total
// holds the class and walks its own classes. Rows whose max is not finite (NaN, all -inf) set `err`.
#include "common.hpp"
#include "stats.hpp"

namespace svhip {

constexpr int kSampleThreads = 256;
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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// PL: classes per lane held in registers (4, 8 or 16: up to 256, 512 or 1024 classes), so that short rows keep
// more waves resident.
template <int PL>
__global__ __launch_bounds__(kSampleThreads) void sample_chosen_kernel(SampleArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t b = blockIdx.y;
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * (kSampleThreads / 64) + (threadIdx.x >> 6)) * 64;
  if (base >= a.N) return;  // wave-uniform
  const int64_t v = base + lane;
  const bool in = v < a.N;
  const bool ch = in && a.chosen[b * a.N + v] != 0;
  uint64_t todo = __ballot(ch);
  const int cpl = static_cast<int>((a.C + 63) / 64);
  const int c0 = lane * cpl;
  const uint64_t seed = static_cast<uint64_t>(a.seed[b]);
  const uint64_t step = static_cast<uint64_t>(a.step[b]);
  const char* xb = static_cast<const char*>(a.x) + b * a.sb * (a.dtype == SVHIP_BF16 ? 2 : 4);
  int mine = -1;  // the class of this lane's voxel
  while (todo) {
    const int i = __builtin_ctzll(todo);
    todo &= todo - 1;
    const int64_t vox = base + i;
    const int64_t row = a.rows(vox) * a.sn;
    float e[PL];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int c = c0 + j;
      e[j] = (j < cpl && c < a.C) ? load_logit(xb, a.dtype, row + c * a.sc) : -INFINITY;
      m = fmaxf(m, e[j]);
    }
    // A NaN logit makes fmaxf skip it; it is caught by the sum below.
    const float mx = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      e[j] = fast_exp(e[j] - mx);
      s += e[j];
    }
    // Inclusive scan of the lane sums (class order) and the exclusive prefix of this lane.
    float incl = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float t = __shfl_up(incl, o, 64);
      if (lane >= o) incl += t;
    }
    float excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = 0.f;
    const float total = __shfl(incl, 63, 64);
    const uint64_t w0 = philox_w0(static_cast<uint64_t>(vox), step, seed, kSampleStream);
    const float u = (static_cast<float>(w0 >> 41) + 0.5f) * (1.0f / 8388608.0f);
    int cls;
    if (!(mx > -INFINITY && mx < INFINITY) || !(total > 0.f && total < INFINITY)) {
      // No class is drawn (the reference's multinomial raises here): the voxel keeps its token and reads -1.
      if (lane == 0) atomicOr(a.err, 1);
      cls = -1;
    } else {
      const float target = u * total;
      const uint64_t past = __ballot(incl > target);
      // Rounding can leave u * total at the very top: the last lane with mass then holds the class.
      const uint64_t mass = __ballot(s > 0.f);
      const int owner = past ? __builtin_ctzll(past) : 63 - __builtin_clzll(mass);
      int found = -1, last = -1;
      float run = excl;
#pragma unroll
      for (int j = 0; j < PL; ++j) {
        if (e[j] > 0.f) last = c0 + j;
        run += e[j];
        if (found < 0 && run > target && e[j] > 0.f) found = c0 + j;
      }
      if (found < 0) found = last;
      cls = __shfl(found, owner, 64);
    }
    if (lane == i) mine = cls;
  }
  if (in) {
    a.values[b * a.N + v] = static_cast<int16_t>(ch ? mine : -1);
    if (ch && mine >= 0 && a.tokens) a.tokens[b * a.N + v] = mine;
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
  const int64_t waves = cdiv(N, 64);
  const dim3 grid(static_cast<unsigned>(cdiv(waves, kSampleThreads / 64)), static_cast<unsigned>(batch));
  const int64_t per_lane = cdiv(classes, 64);
  if (per_lane <= 4) {
    sample_chosen_kernel<4><<<grid, kSampleThreads, 0, as_stream(stream)>>>(a);
  } else if (per_lane <= 8) {
    sample_chosen_kernel<8><<<grid, kSampleThreads, 0, as_stream(stream)>>>(a);
  } else {
    sample_chosen_kernel<kSampleMaxPerLane><<<grid, kSampleThreads, 0, as_stream(stream)>>>(a);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}
