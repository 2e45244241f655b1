// EASE selection: block-quota apportionment, in-block top-quota, global trim / top-up, top_mask and the
// low-entropy-last update. Integer / ordering work, bit-exact by construction:
//  * every "largest scores first, ties to the lower index" order is a total order on (key, index) where
//    key = ~ordered(score) (smaller key = larger score, -0.0 folded onto +0.0);
//  * the apportionment keys -(ideal - base) * 1e6 + pos are evaluated in fp64 with contraction disabled, so each
//    operation rounds exactly as the separate tensor ops do; collisions are broken by block index;
//  * selections of "the `count` smallest (key, index)" use one workgroup per problem: an MSB-first 8-bit radix
//    select on the key finds the threshold key T and how many of the T-ties to keep, then ties are taken in index
//    order with a ballot prefix count over index-ordered rounds.
#include "common.hpp"

namespace svhip {

constexpr int kWG = 1024;  // threads of the workgroup-level selection kernels
constexpr int kWaves = kWG / 64;

template <typename K>
struct KeyTraits;
template <>
struct KeyTraits<uint32_t> {
  static constexpr int kBits = 32;
  static constexpr uint32_t kSentinel = 0xffffffffu;
};
template <>
struct KeyTraits<uint64_t> {
  static constexpr int kBits = 64;
  static constexpr uint64_t kSentinel = ~0ull;
};

// Block-wide int64 sum (all threads of a kWG-thread block must call it).
__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* scratch /* >= kWaves */) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  int64_t t = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) t += scratch[i];
  return t;
}

template <typename K>
struct SelectShared {
  uint32_t hist[256];
  int64_t red[kWaves];
  int64_t tie_counts[2][kWaves];
  K prefix;
  int64_t remaining;
};

// Selects the `count` smallest (key, index) among elements whose key is not the sentinel.
// get(i) returns the key of element i in [0, n). Afterwards:
//   mode 0: nothing selected; mode 1: every eligible element selected; mode 2: key < threshold, plus the first
//   `take_ties` elements (in index order) with key == threshold.
template <typename K>
struct SelectPlan {
  int mode;
  K threshold;
  int64_t take_ties;
  int64_t eligible;
};

template <typename K, typename Get>
__device__ SelectPlan<K> wg_select_plan(Get get, int64_t n, int64_t count, SelectShared<K>& sh) {
  constexpr K kSent = KeyTraits<K>::kSentinel;
  int64_t local = 0;
  for (int64_t i = threadIdx.x; i < n; i += kWG) local += (get(i) != kSent) ? 1 : 0;
  const int64_t eligible = block_sum_i64(local, sh.red);
  SelectPlan<K> plan{0, K(0), 0, eligible};
  if (count <= 0 || eligible == 0) return plan;
  if (count >= eligible) {
    plan.mode = 1;
    return plan;
  }
  K prefix = 0, hi_mask = 0;
  int64_t remaining = count;
  for (int shift = KeyTraits<K>::kBits - 8; shift >= 0; shift -= 8) {
    for (int t = threadIdx.x; t < 256; t += kWG) sh.hist[t] = 0u;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += kWG) {
      const K key = get(i);
      if (key != kSent && (key & hi_mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 0xff], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      const uint32_t h0 = sh.hist[4 * l], h1 = sh.hist[4 * l + 1], h2 = sh.hist[4 * l + 2], h3 = sh.hist[4 * l + 3];
      const int64_t mine = static_cast<int64_t>(h0) + h1 + h2 + h3;
      int64_t incl = mine;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int64_t up = __shfl_up(incl, off, 64);
        if (l >= off) incl += up;
      }
      int64_t before = incl - mine;
      const uint32_t hs[4] = {h0, h1, h2, h3};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (before < remaining && remaining <= before + hs[q]) {
          sh.prefix = prefix | (static_cast<K>(4 * l + q) << shift);
          sh.remaining = remaining - before;
        }
        before += hs[q];
      }
    }
    __syncthreads();
    prefix = sh.prefix;
    remaining = sh.remaining;
    hi_mask |= static_cast<K>(0xff) << shift;
    __syncthreads();
  }
  plan.mode = 2;
  plan.threshold = prefix;
  plan.take_ties = remaining;
  return plan;
}

// Applies a plan: apply(i, selected) is called once for every i in [0, n) (every thread walks index-ordered
// rounds of kWG elements so that ties are taken in index order).
template <typename K, typename Get, typename Apply>
__device__ void wg_select_apply(const SelectPlan<K>& plan, Get get, int64_t n, SelectShared<K>& sh, Apply apply) {
  constexpr K kSent = KeyTraits<K>::kSentinel;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int64_t running = 0;
  int parity = 0;
  for (int64_t base = 0; base < n; base += kWG) {
    const int64_t i = base + threadIdx.x;
    const bool inside = i < n;
    const K key = inside ? get(i) : kSent;
    bool sel = false;
    bool tie = false;
    if (plan.mode == 1) {
      sel = key != kSent;
    } else if (plan.mode == 2) {
      sel = key < plan.threshold;
      tie = key == plan.threshold;
    }
    if (plan.mode == 2) {
      const uint64_t ballot = __ballot(tie);
      if (lane == 0) sh.tie_counts[parity][w] = __popcll(ballot);
      __syncthreads();
      int64_t before = running;
      int64_t round_total = 0;
#pragma unroll
      for (int q = 0; q < kWaves; ++q) {
        const int64_t c = sh.tie_counts[parity][q];
        if (q < w) before += c;
        round_total += c;
      }
      before += __popcll(ballot & ((1ull << lane) - 1ull));
      if (tie && before < plan.take_ties) sel = true;
      running += round_total;
      parity ^= 1;
    }
    if (inside) apply(i, sel);
  }
}

// ----------------------------------------------------------------------------------------------- mask sources

// selectable = mask byte
struct MaskBytes {
  const uint8_t* mask;
  int64_t n;
  __device__ __forceinline__ bool operator()(int64_t b, int64_t flat) const { return mask[b * n + flat] != 0; }
};

// selectable = (tokens == mask_token) & ~last
struct MaskTokens {
  const int64_t* tokens;
  const uint8_t* last;
  int64_t mask_token;
  int64_t n;
  __device__ __forceinline__ bool operator()(int64_t b, int64_t flat) const {
    return tokens[b * n + flat] == mask_token && last[b * n + flat] == 0;
  }
};

struct Geometry {
  int64_t Y, Z, X, b, nb, n, nz, nx;  // nz = Z / b, nx = X / b
  __host__ __device__ int64_t flat_of(int64_t j, int64_t i) const {
    const int64_t by = j / (nz * nx);
    const int64_t bz = (j / nx) % nz;
    const int64_t bx = j % nx;
    const int64_t dy = i / (b * b);
    const int64_t dz = (i / b) % b;
    const int64_t dx = i % b;
    return ((by * b + dy) * Z + bz * b + dz) * X + bx * b + dx;
  }
};

// ---------------------------------------------------------------------------------------------- apportionment

// One workgroup per window: target[j] = base[j] + (j among the `extra` smallest apportionment keys).
// Also clears the window's `got` counter for the in-block pass that follows on the same stream.
__global__ __launch_bounds__(kWG) void apportion_kernel(const int64_t* __restrict__ n_total,
                                                        const int64_t* __restrict__ pos,
                                                        const double* __restrict__ frac,
                                                        const int64_t* __restrict__ k,
                                                        const int64_t* __restrict__ committed, int64_t nb,
                                                        uint64_t* __restrict__ keys, int64_t* __restrict__ target,
                                                        int64_t* __restrict__ got) {
#pragma clang fp contract(off)
  __shared__ SelectShared<uint64_t> sh;
  const int64_t b = blockIdx.x;
  const double f = frac[b];
  const int64_t* nt = n_total + b * nb;
  const int64_t* ps = pos + b * nb;
  uint64_t* ky = keys + b * nb;
  int64_t* tg = target + b * nb;
  int64_t local = 0;
  for (int64_t j = threadIdx.x; j < nb; j += kWG) {
    const double ideal = f * static_cast<double>(nt[j]);
    const double shifted = ideal + 1e-9;
    const double base = floor(shifted);
    const double neg_frac = -(ideal - base);
    const double scaled = neg_frac * 1e6;
    const double key = scaled + static_cast<double>(ps[j]);
    ky[j] = ordered_u64(key);
    tg[j] = static_cast<int64_t>(base);
    local += static_cast<int64_t>(base);
  }
  const int64_t base_sum = block_sum_i64(local, sh.red);
  int64_t extra = committed[b] + k[b] - base_sum;
  if (extra < 0) extra = 0;
  if (threadIdx.x == 0) got[b] = 0;
  if (extra == 0) return;
  __syncthreads();  // keys written by other threads
  auto get = [&](int64_t j) -> uint64_t { return ky[j]; };
  const SelectPlan<uint64_t> plan = wg_select_plan<uint64_t>(get, nb, extra, sh);
  wg_select_apply<uint64_t>(plan, get, nb, sh, [&](int64_t j, bool sel) {
    if (sel) tg[j] += 1;
  });
}

// ------------------------------------------------------------------------------------------ in-block selection

// Blocks of at most 64 voxels (b in {1, 2, 4}): one wave holds 64 / b^3 whole blocks, lane = in-block index.
template <int B3, typename Mask>
__global__ __launch_bounds__(256) void inblock_wave_kernel(const float* __restrict__ score, Mask mask, Geometry g,
                                                           int64_t batch, const int64_t* __restrict__ n_total,
                                                           const int64_t* __restrict__ target,
                                                           uint8_t* __restrict__ chosen, int64_t* __restrict__ got) {
  const int lane = threadIdx.x & 63;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // block-major element
  const int64_t total = batch * g.n;
  if (e - lane >= total) return;  // whole wave past the end (total is a multiple of 64)
  const int64_t jg = e / B3;
  const int i = static_cast<int>(e % B3);
  const int64_t b = jg / g.nb;
  const int64_t j = jg - b * g.nb;
  const int64_t flat = g.flat_of(j, i);
  const bool masked = mask(b, flat);
  const uint32_t key = masked ? desc_key(score[b * g.n + flat]) : KeyTraits<uint32_t>::kSentinel;
  const int group0 = lane & ~(B3 - 1);
  const uint64_t ballot = __ballot(masked);
  const uint64_t gmask = (B3 == 64) ? ~0ull : (((1ull << B3) - 1ull) << group0);
  const int64_t legal = __popcll(ballot & gmask);
  const int64_t already = n_total[jg] - legal;
  int64_t quota = target[jg] - already;
  if (quota < 0) quota = 0;
  if (quota > legal) quota = legal;
  int rank = 0;
#pragma unroll
  for (int t = 0; t < B3; ++t) {
    const uint32_t other = __shfl(key, group0 + t, 64);
    rank += (other < key || (other == key && t < i)) ? 1 : 0;
  }
  const bool sel = masked && rank < quota;
  chosen[b * g.n + flat] = sel ? 1 : 0;
  // Sum of quotas of this wave's blocks (all in one window since n is a multiple of 64).
  int64_t q = (i == 0) ? quota : 0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) q += __shfl_xor(q, off, 64);
  if (lane == 0) atomicAdd(reinterpret_cast<unsigned long long*>(got + b), static_cast<unsigned long long>(q));
}

// Blocks of more than 64 voxels (b >= 8): one workgroup per block.
template <typename Mask>
__global__ __launch_bounds__(kWG) void inblock_wg_kernel(const float* __restrict__ score, Mask mask, Geometry g,
                                                         const int64_t* __restrict__ n_total,
                                                         const int64_t* __restrict__ target,
                                                         uint8_t* __restrict__ chosen, int64_t* __restrict__ got) {
  __shared__ SelectShared<uint32_t> sh;
  const int64_t jg = blockIdx.x;
  const int64_t b = jg / g.nb;
  const int64_t j = jg - b * g.nb;
  const int64_t b3 = g.b * g.b * g.b;
  const float* sc = score + b * g.n;
  auto get = [&](int64_t i) -> uint32_t {
    const int64_t flat = g.flat_of(j, i);
    return mask(b, flat) ? desc_key(sc[flat]) : KeyTraits<uint32_t>::kSentinel;
  };
  // legal = number of masked voxels (the plan counts eligible keys)
  int64_t local = 0;
  for (int64_t i = threadIdx.x; i < b3; i += kWG) local += mask(b, g.flat_of(j, i)) ? 1 : 0;
  const int64_t legal = block_sum_i64(local, sh.red);
  int64_t quota = target[jg] - (n_total[jg] - legal);
  if (quota < 0) quota = 0;
  if (quota > legal) quota = legal;
  const SelectPlan<uint32_t> plan = wg_select_plan<uint32_t>(get, b3, quota, sh);
  wg_select_apply<uint32_t>(plan, get, b3, sh, [&](int64_t i, bool sel) {
    chosen[b * g.n + g.flat_of(j, i)] = sel ? 1 : 0;
  });
  if (threadIdx.x == 0) atomicAdd(reinterpret_cast<unsigned long long*>(got + b), static_cast<unsigned long long>(quota));
}

// ------------------------------------------------------------------------------------------ trim / top-up / bad

// One workgroup per window: if the clamped quotas gave got != k, keep the top k of `chosen` (trim) or add the top
// (k - got) of mask & ~chosen (top-up), by score; then bad = (final count != k).
template <typename Mask>
__global__ __launch_bounds__(kWG) void fix_kernel(const float* __restrict__ score, Mask mask, int64_t n,
                                                  const int64_t* __restrict__ k, const int64_t* __restrict__ got,
                                                  uint8_t* __restrict__ chosen, uint8_t* __restrict__ bad) {
  __shared__ SelectShared<uint32_t> sh;
  const int64_t b = blockIdx.x;
  const int64_t kk = k[b];
  const int64_t have = got[b];
  const float* sc = score + b * n;
  uint8_t* ch = chosen + b * n;
  if (have == kk) {
    if (threadIdx.x == 0) bad[b] = 0;
    return;
  }
  if (have > kk) {
    auto get = [&](int64_t i) -> uint32_t { return ch[i] ? desc_key(sc[i]) : KeyTraits<uint32_t>::kSentinel; };
    const SelectPlan<uint32_t> plan = wg_select_plan<uint32_t>(get, n, kk, sh);
    __syncthreads();
    wg_select_apply<uint32_t>(plan, get, n, sh, [&](int64_t i, bool sel) {
      if (!sel && ch[i]) ch[i] = 0;
    });
    const int64_t final_count = plan.mode == 0 ? 0 : (plan.mode == 1 ? plan.eligible : kk);
    if (threadIdx.x == 0) bad[b] = (final_count != kk) ? 1 : 0;
  } else {
    auto get = [&](int64_t i) -> uint32_t {
      return (!ch[i] && mask(b, i)) ? desc_key(sc[i]) : KeyTraits<uint32_t>::kSentinel;
    };
    const int64_t need = kk - have;
    const SelectPlan<uint32_t> plan = wg_select_plan<uint32_t>(get, n, need, sh);
    __syncthreads();
    // Each element is read and then (maybe) set by the same thread, so marking in place is race-free.
    wg_select_apply<uint32_t>(plan, get, n, sh, [&](int64_t i, bool sel) {
      if (sel) ch[i] = 1;
    });
    const int64_t added = plan.mode == 0 ? 0 : (plan.mode == 1 ? plan.eligible : need);
    if (threadIdx.x == 0) bad[b] = (have + added != kk) ? 1 : 0;
  }
}

// ------------------------------------------------------------------------------------------------- top_mask

__global__ __launch_bounds__(kWG) void top_mask_kernel(const float* __restrict__ scores,
                                                       const uint8_t* __restrict__ eligible, int64_t n,
                                                       const int64_t* __restrict__ count_dev, int64_t count_host,
                                                       uint8_t* __restrict__ out) {
  __shared__ SelectShared<uint32_t> sh;
  const int64_t b = blockIdx.x;
  const float* sc = scores + b * n;
  const uint8_t* el = eligible + b * n;
  uint8_t* o = out + b * n;
  const int64_t count = count_dev ? count_dev[b] : count_host;
  auto get = [&](int64_t i) -> uint32_t { return el[i] ? desc_key(sc[i]) : KeyTraits<uint32_t>::kSentinel; };
  const SelectPlan<uint32_t> plan = wg_select_plan<uint32_t>(get, n, count, sh);
  __syncthreads();
  wg_select_apply<uint32_t>(plan, get, n, sh, [&](int64_t i, bool sel) { o[i] = sel ? 1 : 0; });
}

// ------------------------------------------------------------------------------------------- low-entropy-last

// Column mode: one thread per (window, z, x) column scans y downward to the first bad voxel.
__global__ __launch_bounds__(256) void lel_column_kernel(uint8_t* __restrict__ last, const uint8_t* __restrict__ mask,
                                                         const float* __restrict__ air,
                                                         const uint8_t* __restrict__ solid, float threshold,
                                                         int64_t batch, int64_t Y, int64_t ZX) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= batch * ZX) return;
  const int64_t b = c / ZX;
  const int64_t col = c - b * ZX;
  const int64_t off = b * Y * ZX + col;
  int64_t y = Y - 1;
  for (; y >= 0; --y) {
    const int64_t idx = off + y * ZX;
    const bool m = mask ? mask[idx] != 0 : true;
    const bool bad = (m && air[idx] <= threshold) || (solid ? solid[idx] != 0 : false);
    if (bad) break;
  }
  // voxels above y (exclusive) are the clean top run
  for (int64_t t = y + 1; t < Y; ++t) last[off + t * ZX] = 1;
}

// Layer / band mode: one workgroup per window; last is [B, Y].
__global__ __launch_bounds__(256) void lel_layer_kernel(uint8_t* __restrict__ last, const uint8_t* __restrict__ mask,
                                                        const float* __restrict__ air,
                                                        const uint8_t* __restrict__ solid, float threshold,
                                                        int64_t Y, int64_t ZX, int band) {
  extern __shared__ uint32_t layer_bad[];
  const int64_t b = blockIdx.x;
  for (int64_t y = threadIdx.x; y < Y; y += blockDim.x) layer_bad[y] = 0u;
  __syncthreads();
  const int64_t off = b * Y * ZX;
  for (int64_t e = threadIdx.x; e < Y * ZX; e += blockDim.x) {
    const int64_t idx = off + e;
    const bool m = mask ? mask[idx] != 0 : true;
    const bool bad = (m && air[idx] <= threshold) || (solid ? solid[idx] != 0 : false);
    if (bad) atomicOr(&layer_bad[e / ZX], 1u);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t y = Y - 1;
    for (; y >= 0; --y) {
      bool clean;
      if (band) {
        const int64_t lo = (y / 8) * 8;
        clean = true;
        for (int64_t t = lo; t < lo + 8 && t < Y; ++t) clean = clean && layer_bad[t] == 0u;
      } else {
        clean = layer_bad[y] == 0u;
      }
      if (!clean) break;
    }
    for (int64_t t = y + 1; t < Y; ++t) last[b * Y + t] = 1;
  }
}

// ------------------------------------------------------------------------------------------------ host side

static int check_geometry(int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const char* name,
                          Geometry* g) {
  SVHIP_REQUIRE(batch >= 1 && Y >= 1 && Z >= 1 && X >= 1, "%s: bad window shape", name);
  SVHIP_REQUIRE(block == 1 || block == 2 || block == 4 || block >= 8,
                "%s: block size %lld unsupported (1, 2, 4 or >= 8)", name, (long long)block);
  SVHIP_REQUIRE(Y % block == 0 && Z % block == 0 && X % block == 0,
                "%s: window [%lld,%lld,%lld] not divisible by block %lld", name, (long long)Y, (long long)Z,
                (long long)X, (long long)block);
  const int64_t n = Y * Z * X;
  SVHIP_REQUIRE(n % 64 == 0, "%s: window voxel count %lld must be a multiple of 64", name, (long long)n);
  SVHIP_REQUIRE(block * block * block <= (1 << 24), "%s: block too large", name);
  g->Y = Y;
  g->Z = Z;
  g->X = X;
  g->b = block;
  g->nb = n / (block * block * block);
  g->n = n;
  g->nz = Z / block;
  g->nx = X / block;
  return SVHIP_OK;
}

static size_t quota_ws_bytes(int64_t batch, const Geometry& g) {
  // keys u64 [B,nb] + target i64 [B,nb] + got i64 [B], each 256-byte aligned
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  return al(sizeof(uint64_t) * batch * g.nb) + al(sizeof(int64_t) * batch * g.nb) + al(sizeof(int64_t) * batch);
}

struct QuotaWs {
  uint64_t* keys;
  int64_t* target;
  int64_t* got;
};

static QuotaWs carve(void* ws, int64_t batch, const Geometry& g) {
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  char* p = static_cast<char*>(ws);
  QuotaWs w;
  w.keys = reinterpret_cast<uint64_t*>(p);
  p += al(sizeof(uint64_t) * batch * g.nb);
  w.target = reinterpret_cast<int64_t*>(p);
  p += al(sizeof(int64_t) * batch * g.nb);
  w.got = reinterpret_cast<int64_t*>(p);
  return w;
}

template <typename Mask>
static int launch_quota(const float* score, Mask mask, int64_t batch, const Geometry& g, const int64_t* k,
                        const int64_t* pos, const double* frac, const int64_t* n_total, const int64_t* committed,
                        uint8_t* chosen, uint8_t* bad, const QuotaWs& w, hipStream_t s, const char* name) {
  apportion_kernel<<<static_cast<unsigned>(batch), kWG, 0, s>>>(n_total, pos, frac, k, committed, g.nb, w.keys,
                                                                 w.target, w.got);
  SVHIP_LAUNCHED(name);
  const int64_t b3 = g.b * g.b * g.b;
  if (b3 <= 64) {
    const int64_t threads = batch * g.n;
    const unsigned grid = static_cast<unsigned>(cdiv(threads, 256));
    switch (b3) {
      case 1:
        inblock_wave_kernel<1, Mask><<<grid, 256, 0, s>>>(score, mask, g, batch, n_total, w.target, chosen, w.got);
        break;
      case 8:
        inblock_wave_kernel<8, Mask><<<grid, 256, 0, s>>>(score, mask, g, batch, n_total, w.target, chosen, w.got);
        break;
      default:
        inblock_wave_kernel<64, Mask><<<grid, 256, 0, s>>>(score, mask, g, batch, n_total, w.target, chosen, w.got);
        break;
    }
  } else {
    inblock_wg_kernel<Mask><<<static_cast<unsigned>(batch * g.nb), kWG, 0, s>>>(score, mask, g, n_total, w.target,
                                                                                chosen, w.got);
  }
  SVHIP_LAUNCHED(name);
  fix_kernel<Mask><<<static_cast<unsigned>(batch), kWG, 0, s>>>(score, mask, g.n, k, w.got, chosen, bad);
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

}  // namespace svhip

using namespace svhip;

extern "C" size_t svhip_quota_select_workspace_bytes(int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block) {
  Geometry g;
  if (check_geometry(batch, Y, Z, X, block, "svhip_quota_select_workspace_bytes", &g) != SVHIP_OK) return 0;
  return quota_ws_bytes(batch, g);
}

extern "C" int svhip_quota_select(const float* score, const uint8_t* mask, int64_t batch, int64_t Y, int64_t Z,
                                  int64_t X, int64_t block, const int64_t* k, const int64_t* pos, const double* frac,
                                  const int64_t* n_total, const int64_t* committed, uint8_t* chosen, uint8_t* bad,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  const char* name = "svhip_quota_select";
  clear_error();
  Geometry g;
  int rc = check_geometry(batch, Y, Z, X, block, name, &g);
  if (rc != SVHIP_OK) return rc;
  SVHIP_REQUIRE(score && mask && k && pos && frac && n_total && committed && chosen && bad, "%s: null pointer", name);
  const size_t need = quota_ws_bytes(batch, g);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need, workspace_bytes);
    return SVHIP_EWORKSPACE;
  }
  return launch_quota(score, MaskBytes{mask, g.n}, batch, g, k, pos, frac, n_total, committed, chosen, bad,
                      carve(workspace, batch, g), as_stream(stream), name);
}

extern "C" size_t svhip_ease_select_workspace_bytes(int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block) {
  Geometry g;
  if (check_geometry(batch, Y, Z, X, block, "svhip_ease_select_workspace_bytes", &g) != SVHIP_OK) return 0;
  return quota_ws_bytes(batch, g) + ((sizeof(float) * batch * g.n + 255) & ~size_t(255));
}

extern "C" int svhip_ease_select(const void* logits, int dtype, int64_t classes, int64_t stride_b, int64_t stride_c,
                                 int64_t stride_n, const int64_t* tokens, int64_t mask_token, const uint8_t* last,
                                 int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const int64_t* k,
                                 const int64_t* pos, const double* frac, const int64_t* n_total,
                                 const int64_t* committed, uint8_t* chosen, uint8_t* bad, float* scores_out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  const char* name = "svhip_ease_select";
  clear_error();
  Geometry g;
  int rc = check_geometry(batch, Y, Z, X, block, name, &g);
  if (rc != SVHIP_OK) return rc;
  SVHIP_REQUIRE(logits && tokens && last && k && pos && frac && n_total && committed && chosen && bad,
                "%s: null pointer", name);
  const size_t qbytes = quota_ws_bytes(batch, g);
  const size_t need = qbytes + ((sizeof(float) * batch * g.n + 255) & ~size_t(255));
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need, workspace_bytes);
    return SVHIP_EWORKSPACE;
  }
  float* scores = scores_out ? scores_out : reinterpret_cast<float*>(static_cast<char*>(workspace) + qbytes);
  rc = svhip_entropy(logits, dtype, batch, classes, g.n, stride_b, stride_c, stride_n, scores, stream);
  if (rc != SVHIP_OK) return rc;
  return launch_quota(scores, MaskTokens{tokens, last, mask_token, g.n}, batch, g, k, pos, frac, n_total, committed,
                      chosen, bad, carve(workspace, batch, g), as_stream(stream), name);
}

extern "C" int svhip_top_mask(const float* scores, const uint8_t* eligible, int64_t batch, int64_t n,
                              const int64_t* count_dev, int64_t count_host, uint8_t* out, void* stream) {
  const char* name = "svhip_top_mask";
  clear_error();
  SVHIP_REQUIRE(scores && eligible && out, "%s: null pointer", name);
  SVHIP_REQUIRE(batch >= 0 && n >= 0, "%s: bad sizes", name);
  if (batch == 0 || n == 0) return SVHIP_OK;
  top_mask_kernel<<<static_cast<unsigned>(batch), kWG, 0, as_stream(stream)>>>(scores, eligible, n, count_dev,
                                                                               count_host, out);
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

extern "C" int svhip_lel_update(uint8_t* last, const uint8_t* mask, const float* air, const uint8_t* solid, double eps,
                                int32_t mode, int64_t batch, int64_t Y, int64_t Z, int64_t X, void* stream) {
  const char* name = "svhip_lel_update";
  clear_error();
  SVHIP_REQUIRE(last && air, "%s: null pointer", name);
  SVHIP_REQUIRE(batch >= 0 && Y >= 1 && Z >= 1 && X >= 1, "%s: bad sizes", name);
  SVHIP_REQUIRE(mode == SVHIP_LEL_LAYER || mode == SVHIP_LEL_BAND || mode == SVHIP_LEL_COLUMN, "%s: bad mode %d", name,
                mode);
  SVHIP_REQUIRE(mode != SVHIP_LEL_BAND || Y % 8 == 0, "%s: band mode needs Y divisible by 8", name);
  if (batch == 0) return SVHIP_OK;
  // The compare is fp32 against the fp32 rounding of the double 1 - eps.
  const float threshold = static_cast<float>(1.0 - eps);
  hipStream_t s = as_stream(stream);
  const int64_t zx = Z * X;
  if (mode == SVHIP_LEL_COLUMN) {
    const unsigned grid = static_cast<unsigned>(cdiv(batch * zx, 256));
    lel_column_kernel<<<grid, 256, 0, s>>>(last, mask, air, solid, threshold, batch, Y, zx);
  } else {
    SVHIP_REQUIRE(Y <= 16384, "%s: at most 16384 layers", name);
    lel_layer_kernel<<<static_cast<unsigned>(batch), 256, sizeof(uint32_t) * Y, s>>>(
        last, mask, air, solid, threshold, Y, zx, mode == SVHIP_LEL_BAND ? 1 : 0);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}
