// EASE selection: block-quota apportionment, in-block top-quota, global trim / top-up, top_mask and the
// low-entropy-last update. Integer / ordering work, bit-exact by construction:
//  * every "largest scores first, ties to the lower index" order is a total order on (key, index) where
//    key = ~ordered(score) (smaller key = larger score, -0.0 folded onto +0.0);
//  * the apportionment keys -(ideal - base) * 1e6 + pos are evaluated in fp64 with contraction disabled, so each
//    operation rounds exactly as the separate tensor ops do; collisions are broken by block index;
//  * selections of "the `count` smallest (key, index)" use one workgroup per problem: an MSB-first 8-bit radix
//    select on the key finds the threshold key T and how many of the T-ties to keep, then ties are taken in index
//    order with a ballot prefix count over index-ordered rounds.
#include <atomic>
#include <mutex>

#include "common.hpp"
#include "stats.hpp"

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

// Radix histogram: kCopies copies per bin (bin d of copy c at hist[kCopies d + c], lane l adds into copy
// l % kCopies). Scores cluster in a few bins, and with a single copy the lanes of a wave would serialise on the
// same LDS counter; 64 copies make every lane's counter its own.
// Block-wide minimum / maximum of one uint64 per thread (all threads of a kWG-thread block must call them).
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, int64_t* scratch /* >= kWaves */) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off, 64);
    v = o < v ? o : v;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = static_cast<int64_t>(v);
  __syncthreads();
  uint64_t r = static_cast<uint64_t>(scratch[0]);
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    const uint64_t o = static_cast<uint64_t>(scratch[i]);
    r = o < r ? o : r;
  }
  return r;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, int64_t* scratch /* >= kWaves */) {
  return ~block_min_u64(~v, scratch);
}

template <typename K, int kCopies = 1>
struct SelectShared {
  static constexpr int copies = kCopies;
  uint32_t hist[256 * kCopies];
  uint32_t bins[256];
  int64_t red[kWaves];
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

constexpr int kUnroll = 8;  // keys each thread has in flight in the streaming passes
// Boundary candidates kept per 4^3 block for the trim / top-up pass: the kBoundary last chosen and the kBoundary
// first unchosen selectable voxels of the block, in (key, flat index) order.
constexpr int kBoundary = 16;

// Calls f(key) for the key of every element i in [0, n); each thread loads kUnroll keys (strided by kWG, so the
// loads of a wave stay coalesced) before it uses any, so the passes are not bound by load latency.
template <typename K, typename Get, typename F>
__device__ __forceinline__ void for_each_key(Get get, int64_t n, F f) {
  for (int64_t base = threadIdx.x; base < n; base += static_cast<int64_t>(kWG) * kUnroll) {
    K keys[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + static_cast<int64_t>(u) * kWG;
      keys[u] = i < n ? get(i) : KeyTraits<K>::kSentinel;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) f(keys[u]);
  }
}

// Block-wide exclusive prefix sum of one int64 per thread (all threads of a kWG-thread block must call it).
__device__ __forceinline__ int64_t block_exclusive_scan_i64(int64_t v, int64_t* scratch /* >= kWaves */) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t up = __shfl_up(incl, off, 64);
    if (lane >= off) incl += up;
  }
  __syncthreads();
  if (lane == 63) scratch[w] = incl;
  __syncthreads();
  int64_t before = 0;
#pragma unroll
  for (int q = 0; q < kWaves; ++q) before += (q < w) ? scratch[q] : 0;
  return before + incl - v;
}

template <typename K, typename Get, typename Shared>
__device__ SelectPlan<K> wg_select_plan(Get get, int64_t n, int64_t count, Shared& sh) {
  constexpr int kCopies = Shared::copies;
  constexpr K kSent = KeyTraits<K>::kSentinel;
  int64_t local = 0;
  for_each_key<K>(get, n, [&](K key) { local += (key != kSent) ? 1 : 0; });
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
    for (int t = threadIdx.x; t < 256 * kCopies; t += kWG) sh.hist[t] = 0u;
    __syncthreads();
    const int copy = threadIdx.x % kCopies;
    for_each_key<K>(get, n, [&](K key) {
      if (key != kSent && (key & hi_mask) == prefix) {
        atomicAdd(&sh.hist[kCopies * static_cast<int>((key >> shift) & 0xff) + copy], 1u);
      }
    });
    __syncthreads();
    // Fold the copies into bins[].
    for (int d = threadIdx.x; d < 256; d += kWG) {
      uint32_t sum = 0;
#pragma unroll 16
      for (int c = 0; c < kCopies; ++c) sum += sh.hist[kCopies * d + ((c + d) % kCopies)];
      sh.bins[d] = sum;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      const uint32_t h0 = sh.bins[4 * l], h1 = sh.bins[4 * l + 1], h2 = sh.bins[4 * l + 2], h3 = sh.bins[4 * l + 3];
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

// Applies a plan: apply(i, selected) is called once for every i in [0, n). Thread t owns the contiguous run
// [t C, t C + C) of the elements (C = ceil(n / kWG)); ties are taken in index order through an exclusive scan of
// the per-thread tie counts. apply(i, .) may write element i: no other thread reads it.
template <typename K, typename Get, typename Shared, typename Apply>
__device__ void wg_select_apply(const SelectPlan<K>& plan, Get get, int64_t n, Shared& sh, Apply apply) {
  constexpr K kSent = KeyTraits<K>::kSentinel;
  const int64_t C = (n + kWG - 1) / kWG;
  const int64_t lo = threadIdx.x * C < n ? threadIdx.x * C : n;
  const int64_t hi = lo + C < n ? lo + C : n;
  int64_t ties_before = 0;
  if (plan.mode == 2) {
    int64_t mine = 0;
    for (int64_t base = lo; base < hi; base += kUnroll) {
      K keys[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) keys[u] = base + u < hi ? get(base + u) : kSent;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) mine += (keys[u] == plan.threshold) ? 1 : 0;
    }
    ties_before = block_exclusive_scan_i64(mine, sh.red);
  }
  for (int64_t base = lo; base < hi; base += kUnroll) {
    K keys[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) keys[u] = base + u < hi ? get(base + u) : kSent;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (base + u < hi) {
        const K key = keys[u];
        bool sel = false;
        if (plan.mode == 1) {
          sel = key != kSent;
        } else if (plan.mode == 2) {
          if (key < plan.threshold) {
            sel = true;
          } else if (key == plan.threshold) {
            sel = ties_before < plan.take_ties;
            ++ties_before;
          }
        }
        apply(base + u, sel);
      }
    }
  }
}

// ----------------------------------------------------------------------------------------------- mask sources

// selectable = mask byte
struct MaskBytes {
  const uint8_t* mask;
  int64_t n;
  __device__ __forceinline__ bool operator()(int64_t b, int64_t flat) const { return mask[b * n + flat] != 0; }
};


// Where the in-block pass gets each voxel's descending-score key (the sentinel for a voxel that is not
// selectable): load() reads it, publish() leaves it in ckey for the trim / top-up pass.
template <typename Mask>
struct KeyFromScore {  // fp32 scores and a selectable mask; the keys are published
  const float* score;
  Mask mask;
  uint32_t* ckey;
  __device__ __forceinline__ uint32_t load(int64_t b, int64_t n, int64_t flat) const {
    const float sv = score[b * n + flat];
    return mask(b, flat) ? desc_key(sv) : KeyTraits<uint32_t>::kSentinel;
  }
  __device__ __forceinline__ void publish(int64_t b, int64_t n, int64_t flat, uint32_t key) const {
    ckey[b * n + flat] = key;
  }
};

struct KeyStored {  // keys already in ckey (the fused entropy pass wrote them)
  const uint32_t* ckey;
  __device__ __forceinline__ uint32_t load(int64_t b, int64_t n, int64_t flat) const { return ckey[b * n + flat]; }
  __device__ __forceinline__ void publish(int64_t, int64_t, int64_t, uint32_t) const {}
};

struct Geometry {
  int64_t Y, Z, X, b, nb, n, nz, nx;  // nz = Z / b, nx = X / b
  // Flat index of in-block entry i of block j for a compile-time block edge BB (32-bit arithmetic: every
  // index of a selection call fits, which the host checks).
  template <int BB>
  __device__ __forceinline__ int flat32(int j, int i) const {
    const int nzx = static_cast<int>(nz * nx), nx32 = static_cast<int>(nx);
    const int by = j / nzx;
    const int rem = j - by * nzx;
    const int bz = rem / nx32;
    const int bx = rem - bz * nx32;
    const int dy = i / (BB * BB), dz = (i / BB) % BB, dx = i % BB;
    return ((by * BB + dy) * static_cast<int>(Z) + bz * BB + dz) * static_cast<int>(X) + bx * BB + dx;
  }
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
__global__ __launch_bounds__(kWG) void apportion_kernel(const int64_t* __restrict__ n_total,
                                                        const int64_t* __restrict__ pos,
                                                        const double* __restrict__ frac,
                                                        const int64_t* __restrict__ k,
                                                        const int64_t* __restrict__ committed, int64_t nb,
                                                        uint64_t* __restrict__ keys, int64_t* __restrict__ target) {
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
  if (extra == 0) return;
  __syncthreads();  // keys written by other threads
  auto get = [&](int64_t j) -> uint64_t { return ky[j]; };
  const SelectPlan<uint64_t> plan = wg_select_plan<uint64_t>(get, nb, extra, sh);
  wg_select_apply<uint64_t>(plan, get, nb, sh, [&](int64_t j, bool sel) {
    if (sel) tg[j] += 1;
  });
}

// The same for one window of at most kWaveBlocks blocks, run by one wave without workgroup barriers: the keys in
// LDS (`skey`, kWaveBlocks entries), an MSB-first 8-bit radix select over the 64-bit keys with the histogram
// (`hist`, 256 entries) in LDS, then the `extra` smallest (key, block index) get one more voxel. Called by lanes
// 0..63 of one wave; block j is handled by lane j % 64 throughout, so its global reads and writes need no fence.
constexpr int kWaveBlocks = 1024;

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct ApportionArgs {
  const int64_t* n_total;
  const int64_t* pos;
  const double* frac;
  const int64_t* k;
  const int64_t* committed;
  int64_t nb;
  int64_t* target;
};

__device__ void apportion_window(const ApportionArgs& a, int64_t b, int lane, uint64_t* skey, uint32_t* hist) {
#pragma clang fp contract(off)
  const int64_t nb = a.nb;
  const double f = a.frac[b];
  const int64_t* nt = a.n_total + b * nb;
  const int64_t* ps = a.pos + b * nb;
  int64_t* tg = a.target + b * nb;
  constexpr int kUnrollBlocks = 4;
  int64_t local = 0;
  for (int64_t j0 = lane; j0 < nb; j0 += 64 * kUnrollBlocks) {
    // Loads are unconditional (clamped index) so that all of them are in flight at once.
    int64_t ntv[kUnrollBlocks], psv[kUnrollBlocks];
#pragma unroll
    for (int u = 0; u < kUnrollBlocks; ++u) {
      const int64_t j = j0 + 64 * u < nb ? j0 + 64 * u : nb - 1;
      ntv[u] = nt[j];
      psv[u] = ps[j];
    }
#pragma unroll
    for (int u = 0; u < kUnrollBlocks; ++u) {
      const int64_t j = j0 + 64 * u;
      if (j < nb) {
        const double ideal = f * static_cast<double>(ntv[u]);
        const double shifted = ideal + 1e-9;
        const double base = floor(shifted);
        const double neg_frac = -(ideal - base);
        const double scaled = neg_frac * 1e6;
        const double key = scaled + static_cast<double>(psv[u]);
        skey[j] = ordered_u64(key);
        tg[j] = static_cast<int64_t>(base);
        local += static_cast<int64_t>(base);
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) local += __shfl_xor(local, off, 64);
  const int64_t extra = a.committed[b] + a.k[b] - local;
  if (extra <= 0) return;
  if (extra >= nb) {
    for (int64_t j = lane; j < nb; j += 64) tg[j] += 1;
    return;
  }
  wave_sync_lds();
  // Threshold key T and how many T-ties to take (remaining) after the last digit.
  uint64_t prefix = 0, hi_mask = 0;
  int64_t remaining = extra;
  for (int shift = 56; shift >= 0; shift -= 8) {
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[4 * lane + q] = 0u;
    wave_sync_lds();
    for (int64_t j = lane; j < nb; j += 64) {
      const uint64_t key = skey[j];
      if ((key & hi_mask) == prefix) atomicAdd(&hist[(key >> shift) & 0xff], 1u);
    }
    wave_sync_lds();
    const uint32_t hs[4] = {hist[4 * lane], hist[4 * lane + 1], hist[4 * lane + 2], hist[4 * lane + 3]};
    const int64_t mine = static_cast<int64_t>(hs[0]) + hs[1] + hs[2] + hs[3];
    int64_t incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t up = __shfl_up(incl, off, 64);
      if (lane >= off) incl += up;
    }
    // The lane whose four bins hold the remaining-th key finds the bin; everyone reads it from that lane.
    const uint64_t who = __ballot(incl - mine < remaining && remaining <= incl);
    const int src = __builtin_ctzll(who);
    int64_t before = incl - mine;
    int bin = 4 * lane + 3;
    bool found = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (!found) {
        if (before + hs[q] < remaining) {
          before += hs[q];
        } else {
          bin = 4 * lane + q;
          found = true;
        }
      }
    }
    prefix |= static_cast<uint64_t>(__shfl(bin, src, 64)) << shift;
    remaining -= __shfl(before, src, 64);
    hi_mask |= static_cast<uint64_t>(0xff) << shift;
    wave_sync_lds();
  }
  // key < T: one more; key == T: the first `remaining` in block order.
  int64_t ties_before = 0;
  for (int64_t j0 = 0; j0 < nb; j0 += 64) {
    const int64_t j = j0 + lane;
    const uint64_t key = j < nb ? skey[j] : ~0ull;
    const bool tie = j < nb && key == prefix;
    const uint64_t tb = __ballot(tie);
    const int64_t rank = ties_before + __popcll(tb & ((1ull << lane) - 1ull));
    if (j < nb && (key < prefix || (tie && rank < remaining))) tg[j] += 1;
    ties_before += __popcll(tb);
  }
}

// Standalone: one wave per window, 4 windows per workgroup.
__global__ __launch_bounds__(256) void apportion_wave_kernel(ApportionArgs a, int64_t batch) {
  __shared__ uint64_t skey[4][kWaveBlocks];
  __shared__ uint32_t hist[4][256];
  const int w = threadIdx.x >> 6;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (b >= batch) return;
  apportion_window(a, b, threadIdx.x & 63, skey[w], hist[w]);
}

// ------------------------------------------------------------------------------------------ in-block selection

// Every in-block kernel also leaves, for the trim / top-up pass: bq[B, nb] the quota each block took, and
// ckey[B, N] (flat order) the descending-score key of every selectable voxel (the sentinel elsewhere).

// Blocks of at most 64 voxels (b in {1, 2, 4}): one wave holds 64 / b^3 whole blocks, lane = in-block index.
template <int BB, typename KeySrc>
__global__ __launch_bounds__(256) void inblock_wave_kernel(KeySrc src, Geometry g, int total,
                                                           const int64_t* __restrict__ n_total,
                                                           const int64_t* __restrict__ target,
                                                           uint8_t* __restrict__ chosen, int32_t* __restrict__ bq,
                                                           uint64_t* __restrict__ bnd) {
  constexpr int B3 = BB * BB * BB;
  const int lane = threadIdx.x & 63;
  const int e = static_cast<int>(blockIdx.x) * blockDim.x + threadIdx.x;  // block-major element
  if (e - lane >= total) return;  // whole wave past the end (total is a multiple of 64)
  const int n = static_cast<int>(g.n), nb = static_cast<int>(g.nb);
  const int jg = e / B3;
  const int i = e % B3;
  const int b = jg / nb;
  const int j = jg - b * nb;
  const int flat = g.flat32<BB>(j, i);
  const uint32_t key = src.load(b, n, flat);
  const bool masked = key != KeyTraits<uint32_t>::kSentinel;
  src.publish(b, n, flat, key);
  const int group0 = lane & ~(B3 - 1);
  const uint64_t ballot = __ballot(masked);
  const uint64_t gmask = (B3 == 64) ? ~0ull : (((1ull << B3) - 1ull) << group0);
  const int64_t legal = __popcll(ballot & gmask);
  const int64_t already = n_total[jg] - legal;
  int64_t quota = target[jg] - already;
  if (quota < 0) quota = 0;
  if (quota > legal) quota = legal;
  int rank = 0;
  if constexpr (B3 == 64) {
    // One block per wave. Only selectable voxels' ranks are used, and every other voxel holds the sentinel, above
    // every selectable key: rank = voxels with a smaller key, plus equal keys at lower in-block indices. Each lane's
    // key is broadcast by readlane (a constant lane, no LDS). The tie pass runs only when there is a tie: without
    // one the smaller-key counts of the legal selectable voxels are 0 .. legal - 1, whose sum is
    // legal (legal - 1) / 2.
#pragma unroll
    for (int t = 0; t < 64; ++t) {
      const uint32_t other = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), t));
      rank += other < key ? 1 : 0;
    }
    int64_t sum = masked ? rank : 0;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (sum != legal * (legal - 1) / 2) {
#pragma unroll
      for (int t = 0; t < 64; ++t) {
        const uint32_t other = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), t));
        rank += (other == key && t < i) ? 1 : 0;
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < B3; ++t) {
      const uint32_t other = __shfl(key, group0 + t, 64);
      rank += (other < key || (other == key && t < i)) ? 1 : 0;
    }
  }
  const bool sel = masked && rank < quota;
  chosen[b * n + flat] = sel ? 1 : 0;
  if (i == 0) bq[jg] = static_cast<int32_t>(quota);
  if constexpr (B3 == 64) {
    // Boundary candidates: slot t holds the voxel of in-block rank quota - kBoundary + t as (key << 32 | flat),
    // the sentinel when that rank does not exist. The wave sorts itself into LDS by rank (ranks of the selectable
    // voxels are 0 .. legal-1, each held by one lane), then lanes 0 .. 2 kBoundary - 1 gather.
    __shared__ uint64_t by_rank[256];
    uint64_t* mine = by_rank + (threadIdx.x & ~63);
    if (masked) mine[rank] = (static_cast<uint64_t>(key) << 32) | static_cast<uint32_t>(flat);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 2 * kBoundary) {
      const int64_t r = quota - kBoundary + lane;
      bnd[static_cast<int64_t>(jg) * 2 * kBoundary + lane] = (r >= 0 && r < legal) ? mine[r] : ~0ull;
    }
  }
}

// Blocks of more than 64 voxels (b >= 8): one workgroup per block.
template <typename KeySrc>
__global__ __launch_bounds__(kWG) void inblock_wg_kernel(KeySrc src, Geometry g, const int64_t* __restrict__ n_total,
                                                         const int64_t* __restrict__ target,
                                                         uint8_t* __restrict__ chosen, int32_t* __restrict__ bq) {
  __shared__ SelectShared<uint32_t> sh;
  const int64_t jg = blockIdx.x;
  const int64_t b = jg / g.nb;
  const int64_t j = jg - b * g.nb;
  const int64_t b3 = g.b * g.b * g.b;
  auto get = [&](int64_t i) -> uint32_t { return src.load(b, g.n, g.flat_of(j, i)); };
  // legal = number of selectable voxels; the keys are also left for the trim / top-up pass
  int64_t local = 0;
  for (int64_t i = threadIdx.x; i < b3; i += kWG) {
    const int64_t flat = g.flat_of(j, i);
    const uint32_t key = get(i);
    src.publish(b, g.n, flat, key);
    local += key != KeyTraits<uint32_t>::kSentinel ? 1 : 0;
  }
  const int64_t legal = block_sum_i64(local, sh.red);
  int64_t quota = target[jg] - (n_total[jg] - legal);
  if (quota < 0) quota = 0;
  if (quota > legal) quota = legal;
  const SelectPlan<uint32_t> plan = wg_select_plan<uint32_t>(get, b3, quota, sh);
  wg_select_apply<uint32_t>(plan, get, b3, sh, [&](int64_t i, bool sel) {
    chosen[b * g.n + g.flat_of(j, i)] = sel ? 1 : 0;
  });
  if (threadIdx.x == 0) bq[jg] = static_cast<int32_t>(quota);
}

// ------------------------------------------------------------------------------------------ trim / top-up / bad

// One workgroup per window: if the clamped quotas gave got != k, keep the top k of `chosen` (trim) or add the top
// (k - got) of selectable & ~chosen (top-up), by score; then bad = (final count != k). Reads only the keys and the
// per-block quotas the in-block pass left (a selectable voxel has a non-sentinel key).
__global__ __launch_bounds__(kWG) void fix_kernel(int64_t n, int64_t nb, const int64_t* __restrict__ k,
                                                  const int32_t* __restrict__ bq, const uint32_t* __restrict__ ckey,
                                                  const uint64_t* __restrict__ bnd, uint8_t* __restrict__ chosen,
                                                  uint8_t* __restrict__ bad) {
  constexpr uint32_t kSent = KeyTraits<uint32_t>::kSentinel;
  __shared__ SelectShared<uint32_t, 64> sh;
  const int64_t b = blockIdx.x;
  const int64_t kk = k[b];
  int64_t local = 0;
  for (int64_t j = threadIdx.x; j < nb; j += kWG) local += bq[b * nb + j];
  const int64_t have = block_sum_i64(local, sh.red);
  const uint32_t* ky = ckey + b * n;
  uint8_t* ch = chosen + b * n;
  if (have == kk) {
    if (threadIdx.x == 0) bad[b] = 0;
    return;
  }
  const int64_t d = have > kk ? have - kk : kk - have;
  if (bnd != nullptr && d <= kBoundary && nb <= kWG) {
    // One block per thread. Its first d candidates (trim: the last d chosen, top-up: the first d unchosen
    // selectable; the sentinel where a rank does not exist) are distinct (key << 32 | flat) values in rank order,
    // so with r = trim ? c : ~c (0 for the sentinel) each thread's list is sorted descending and the d voxels to
    // flip are the d largest r of all lists. Their chosen state needs no read: the in-block pass chose exactly the
    // ranks below the quota and only this pass flips them. Phase 1: every wave takes its own d largest by d
    // wave-wide maxima over its lanes' list heads (no workgroup barrier), into LDS; phase 2: wave 0 merges the
    // waves' sorted lists the same way and flips the winners.
    const bool trim = have > kk;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int64_t j = threadIdx.x;
    auto rank_of = [&](uint64_t c) __attribute__((always_inline)) { return c == ~0ull ? 0ull : (trim ? c : ~c); };
    auto wave_max = [&](uint64_t v) __attribute__((always_inline)) {
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
      }
      return v;
    };
    uint64_t cand[kBoundary];
#pragma unroll
    for (int t = 0; t < kBoundary; ++t) {
      cand[t] = (j < nb && t < d)
                    ? rank_of(bnd[(b * nb + j) * 2 * kBoundary + (trim ? kBoundary - 1 - t : kBoundary + t)])
                    : 0ull;
    }
    uint64_t* wtop = reinterpret_cast<uint64_t*>(sh.hist);  // [wave][kBoundary]; the histogram is unused here
    int head = 0;
    for (int64_t r = 0; r < d; ++r) {
      uint64_t cur = 0ull;
#pragma unroll
      for (int t = 0; t < kBoundary; ++t) cur = (t == head) ? cand[t] : cur;
      const uint64_t best = wave_max(cur);
      if (best != 0ull && cur == best) ++head;  // one lane holds it
      if (lane == 0) wtop[w * kBoundary + r] = best;
    }
    __syncthreads();
    if (w == 0) {
      // Lane l: list l % kWaves, positions 4 (l / kWaves) .. + 3 (sorted descending within the lane).
      static_assert(kWaves * 4 == 64, "phase 2 holds four entries of every wave's list per lane");
      const int list = lane % kWaves, p0 = 4 * (lane / kWaves);
      uint64_t c4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) c4[i] = p0 + i < d ? wtop[list * kBoundary + p0 + i] : 0ull;
      int h2 = 0;
      int64_t done = 0;
      for (int64_t r = 0; r < d; ++r) {
        uint64_t cur = 0ull;
#pragma unroll
        for (int i = 0; i < 4; ++i) cur = (i == h2) ? c4[i] : cur;
        const uint64_t best = wave_max(cur);
        if (best == 0ull) break;  // no candidate left (uniform)
        if (cur == best) {
          ++h2;
          const uint64_t c = trim ? best : ~best;
          ch[static_cast<uint32_t>(c)] = trim ? 0 : 1;
        }
        ++done;
      }
      if (lane == 0) bad[b] = (done != d) ? 1 : 0;
    }
    return;
  }
  if (bnd != nullptr && d <= kBoundary) {
    // The d voxels to drop (trim: the last d chosen in (key, index) order) or to add (top-up: the first d
    // unchosen selectable ones) are among the boundary candidates: such a voxel has fewer than d voxels of its own
    // block on the far side of it. d rounds of a block-wide extremum over the candidates.
    const bool trim = have > kk;
    const uint64_t* cb = bnd + b * nb * 2 * kBoundary;
    int64_t done = 0;
    for (int64_t round = 0; round < d; ++round) {
      // trim: largest candidate (the sentinel is excluded); top-up: smallest.
      uint64_t best = trim ? 0ull : ~0ull;
      for (int64_t j = threadIdx.x; j < nb; j += kWG) {
        for (int64_t t = 0; t < d; ++t) {
          const uint64_t c = cb[j * 2 * kBoundary + (trim ? kBoundary - 1 - t : kBoundary + t)];
          if (c == ~0ull) continue;
          const uint8_t taken = ch[static_cast<uint32_t>(c)];
          if (trim ? (taken && c > best) : (!taken && c < best)) best = c;
        }
      }
      best = trim ? block_max_u64(best, sh.red) : block_min_u64(best, sh.red);
      if (trim ? best == 0ull : best == ~0ull) break;  // no candidate left
      if (threadIdx.x == 0) ch[static_cast<uint32_t>(best)] = trim ? 0 : 1;
      ++done;
      __syncthreads();  // the flip is visible to the next round's reads
    }
    if (threadIdx.x == 0) bad[b] = (done != d) ? 1 : 0;
    return;
  }
  __syncthreads();
  if (have > kk) {
    auto get = [&](int64_t i) -> uint32_t {
      const uint8_t c = ch[i];
      const uint32_t v = ky[i];
      return c ? v : kSent;
    };
    const SelectPlan<uint32_t> plan = wg_select_plan<uint32_t>(get, n, kk, sh);
    __syncthreads();
    wg_select_apply<uint32_t>(plan, get, n, sh, [&](int64_t i, bool sel) {
      if (!sel && ch[i]) ch[i] = 0;
    });
    const int64_t final_count = plan.mode == 0 ? 0 : (plan.mode == 1 ? plan.eligible : kk);
    if (threadIdx.x == 0) bad[b] = (final_count != kk) ? 1 : 0;
  } else {
    auto get = [&](int64_t i) -> uint32_t {
      const uint8_t c = ch[i];
      const uint32_t v = ky[i];
      return c ? kSent : v;
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
  __shared__ SelectShared<uint32_t, 64> sh;
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
  SVHIP_REQUIRE(batch * n < (int64_t(1) << 31), "%s: %lld windows x %lld voxels exceed 2^31 elements", name,
                (long long)batch, (long long)n);
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

// Boundary candidates are kept for 4^3 blocks only (the block size the window schedule uses).
static int64_t boundary_entries(int64_t batch, const Geometry& g) {
  return g.b == 4 ? batch * g.nb * 2 * kBoundary : 0;
}

static size_t quota_ws_bytes(int64_t batch, const Geometry& g) {
  // keys u64 [B,nb] + target i64 [B,nb] + bq i32 [B,nb] + ckey u32 [B,N] + bnd u64 [B,nb,2 kBoundary] (4^3
  // blocks) + derived committed counts i64 [B], each 256-byte aligned
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  return al(sizeof(uint64_t) * batch * g.nb) + al(sizeof(int64_t) * batch * g.nb) + al(sizeof(int32_t) * batch * g.nb) +
         al(sizeof(uint32_t) * batch * g.n) + al(sizeof(uint64_t) * boundary_entries(batch, g)) +
         al(sizeof(int64_t) * batch);
}

struct QuotaWs {
  uint64_t* keys;
  int64_t* target;
  int32_t* bq;
  uint32_t* ckey;
  uint64_t* bnd;  // null unless the blocks are 4^3
  int64_t* committed;  // per-window committed counts derived on the device (svhip_quota_select without them)
};

static QuotaWs carve(void* ws, int64_t batch, const Geometry& g) {
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  char* p = static_cast<char*>(ws);
  QuotaWs w;
  w.keys = reinterpret_cast<uint64_t*>(p);
  p += al(sizeof(uint64_t) * batch * g.nb);
  w.target = reinterpret_cast<int64_t*>(p);
  p += al(sizeof(int64_t) * batch * g.nb);
  w.bq = reinterpret_cast<int32_t*>(p);
  p += al(sizeof(int32_t) * batch * g.nb);
  w.ckey = reinterpret_cast<uint32_t*>(p);
  p += al(sizeof(uint32_t) * batch * g.n);
  w.bnd = boundary_entries(batch, g) ? reinterpret_cast<uint64_t*>(p) : nullptr;
  p += al(sizeof(uint64_t) * boundary_entries(batch, g));
  w.committed = reinterpret_cast<int64_t*>(p);
  return w;
}

// committed[b] = sum of n_total[b, :] - number of non-zero mask bytes of window b (the non-deferred voxels that are
// no longer selectable): block_quota_select's `already.sum()`. One workgroup per window.
__global__ __launch_bounds__(256) void committed_kernel(const uint8_t* __restrict__ mask,
                                                        const int64_t* __restrict__ n_total, int64_t nb, int64_t n,
                                                        int64_t* __restrict__ committed) {
  __shared__ int64_t red[4];
  const int64_t b = blockIdx.x;
  const uint8_t* m = mask + b * n;
  int64_t local = 0;
  for (int64_t j = threadIdx.x; j < nb; j += 256) local += n_total[b * nb + j];
  // n is a multiple of 64: 16-byte loads while 16 bytes remain, single bytes for the rest (unaligned rows).
  const bool vec = (reinterpret_cast<uintptr_t>(m) & 15) == 0;
  const int64_t nv = vec ? n / 16 : 0;
  for (int64_t i = threadIdx.x; i < nv; i += 256) {
    const uint4 v = reinterpret_cast<const uint4*>(m)[i];
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t x = w4[q];
      local -= ((x & 0xffu) != 0) + ((x & 0xff00u) != 0) + ((x & 0xff0000u) != 0) + ((x & 0xff000000u) != 0);
    }
  }
  for (int64_t i = 16 * nv + threadIdx.x; i < n; i += 256) local -= m[i] != 0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) local += __shfl_xor(local, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = local;
  __syncthreads();
  if (threadIdx.x == 0) committed[b] = red[0] + red[1] + red[2] + red[3];
}

// Apportionment alone (the fused entropy pass runs it on the side when the window has at most kWaveBlocks
// blocks).
static int launch_apportion(int64_t batch, const Geometry& g, const int64_t* k, const int64_t* pos,
                            const double* frac, const int64_t* n_total, const int64_t* committed, const QuotaWs& w,
                            hipStream_t s, const char* name) {
  if (g.nb <= kWaveBlocks) {
    const ApportionArgs a{n_total, pos, frac, k, committed, g.nb, w.target};
    apportion_wave_kernel<<<static_cast<unsigned>(cdiv(batch, 4)), 256, 0, s>>>(a, batch);
  } else {
    apportion_kernel<<<static_cast<unsigned>(batch), kWG, 0, s>>>(n_total, pos, frac, k, committed, g.nb, w.keys,
                                                                   w.target);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

// In-block selection and trim / top-up, after the targets exist.
template <typename KeySrc>
static int launch_inblock_fix(KeySrc src, int64_t batch, const Geometry& g, const int64_t* k,
                              const int64_t* n_total, uint8_t* chosen, uint8_t* bad, const QuotaWs& w,
                              hipStream_t s, const char* name) {
  const int64_t b3 = g.b * g.b * g.b;
  if (b3 <= 64) {
    const int total = static_cast<int>(batch * g.n);
    const unsigned grid = static_cast<unsigned>(cdiv(total, 256));
    switch (b3) {
      case 1:
        inblock_wave_kernel<1, KeySrc><<<grid, 256, 0, s>>>(src, g, total, n_total, w.target, chosen, w.bq, nullptr);
        break;
      case 8:
        inblock_wave_kernel<2, KeySrc><<<grid, 256, 0, s>>>(src, g, total, n_total, w.target, chosen, w.bq, nullptr);
        break;
      default:
        inblock_wave_kernel<4, KeySrc><<<grid, 256, 0, s>>>(src, g, total, n_total, w.target, chosen, w.bq, w.bnd);
        break;
    }
  } else {
    inblock_wg_kernel<KeySrc><<<static_cast<unsigned>(batch * g.nb), kWG, 0, s>>>(src, g, n_total, w.target, chosen,
                                                                                  w.bq);
  }
  SVHIP_LAUNCHED(name);
  fix_kernel<<<static_cast<unsigned>(batch), kWG, 0, s>>>(g.n, g.nb, k, w.bq, w.ckey, w.bnd, chosen, bad);
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

// --------------------------------------------------------------------------------------- fused EASE entropy pass

// Output of the fused pass: the voxel's key (descending score if tokens == mask_token and not deferred, else the
// sentinel) into ckey, the fp32 score into `scores` when given.
struct KeyStore {
  const int64_t* tokens;
  const uint8_t* last;
  int64_t mask_token;
  uint32_t* ckey;
  float* scores;
  struct Pre {
    int64_t token;
    uint8_t deferred;
  };
  __device__ __forceinline__ Pre prefetch(int64_t voxel) const { return Pre{tokens[voxel], last[voxel]}; }
  __device__ __forceinline__ void store(int64_t voxel, float value, Pre pre) const {
    const bool selectable = (pre.token == mask_token) & (pre.deferred == 0);
    ckey[voxel] = selectable ? desc_key(value) : KeyTraits<uint32_t>::kSentinel;
    if (scores) scores[voxel] = value;
  }
};

// Workgroups [0, side) apportion window blockIdx.x (one wave); the rest run the entropy pass over the logits and
// write the keys. The apportionment depends only on the selection state, so it runs alongside the HBM-bound pass.
template <typename T, int LAYOUT, int NV, int LPV = 16, int CMAX = 256>
__global__ __launch_bounds__(256) void ease_stats_kernel(const T* __restrict__ x, int64_t batch, int64_t n, int64_t C,
                                                         int64_t sb, int64_t sc, int64_t sn, KeyStore ks,
                                                         ApportionArgs ap, int side, VoxelRows rows, int nv = 0) {
  __shared__ uint64_t skey[kWaveBlocks];
  __shared__ uint32_t hist[256];
  if (static_cast<int>(blockIdx.x) < side) {
    if (threadIdx.x < 64) apportion_window(ap, blockIdx.x, threadIdx.x, skey, hist);
    return;
  }
  const int64_t blk = blockIdx.x - side, nblk = gridDim.x - side;
  if constexpr (LAYOUT == kVoxelMajor) {
    voxel_major_pass<T, NV, kEntropy, KeyStore, LPV>(x, batch * n, n, C, sb, sn, nullptr, ks, blk, nblk, rows);
  } else if constexpr (LAYOUT == kCanonVec || LAYOUT == kCanonScalar) {
    extern __shared__ float tile[];
    canonical_tile_pass<T, LPV, LAYOUT == kCanonVec, kEntropy, CMAX>(x, batch, n, C, sb, sc, sn, nv, nullptr, ks, blk,
                                                                     nblk, tile);
  } else {
    class_major_pass<T, LAYOUT == kClassMajorVec, kEntropy>(x, batch, n, C, sb, sc, sn, nullptr, ks, blk, nblk);
  }
}

template <typename T>
static int launch_ease_stats(const T* x, int64_t batch, int64_t C, int64_t n, int64_t sb, int64_t sc, int64_t sn,
                             const KeyStore& ks, const ApportionArgs& ap, int side, hipStream_t s, VoxelRows rows,
                             const char* name) {
  const StatsPlan plan = plan_stats<T>(x, batch, C, n, sb, sc, sn);
  SVHIP_REQUIRE(rows.p_log < 0 || plan.layout == kVoxelMajor,
                "%s: patch-order logits must be voxel-major rows (stride_c 1, 16-byte aligned rows, classes a "
                "multiple of %d, at most %d)",
                name, Vec16<T>::kElems, 128 * Vec16<T>::kElems);
  const unsigned grid = static_cast<unsigned>(plan.grid + side);
  if (plan.layout == kVoxelMajor) {
    // The row plan takes 8 lanes per voxel only with an odd vector count (row_plan), so only those are built.
#define SVHIP_EVM(NVV)                                                                                        \
  case NVV:                                                                                                   \
    if constexpr (NVV % 2 == 1) {                                                                             \
      if (plan.lpv == 8) {                                                                                    \
        ease_stats_kernel<T, kVoxelMajor, NVV, 8><<<grid, 256, 0, s>>>(x, batch, n, C, sb, sc, sn, ks, ap,     \
                                                                        side, rows);                          \
        return SVHIP_OK;                                                                                      \
      }                                                                                                       \
    }                                                                                                         \
    ease_stats_kernel<T, kVoxelMajor, NVV, 16><<<grid, 256, 0, s>>>(x, batch, n, C, sb, sc, sn, ks, ap, side,  \
                                                                     rows);                                   \
    return SVHIP_OK;
    switch (plan.nv) {
      SVHIP_EVM(1)
      SVHIP_EVM(2)
      SVHIP_EVM(3)
      SVHIP_EVM(4)
      SVHIP_EVM(5)
      SVHIP_EVM(6)
      SVHIP_EVM(7)
      SVHIP_EVM(8)
      default:
        break;
    }
#undef SVHIP_EVM
  }
  if (plan.layout == kCanonVec || plan.layout == kCanonScalar) {
    // NV is passed at run time here (the tile pass loops over it); the template slot carries 0.
    const size_t lds = plan.lds;
    const int nv = plan.nv;
#define SVHIP_ECANON(LAY, LPVV, CM)                                                                          \
  ease_stats_kernel<T, LAY, 0, LPVV, CM><<<grid, 256, lds, s>>>(x, batch, n, C, sb, sc, sn, ks, ap, side, rows, nv)
    // Above 256 classes 8 lanes per voxel occur only for bf16 rows (fp32 rows then have more than 8 vectors per
    // lane of 8), so the fp32 form of that case is not built.
#define SVHIP_ECANON_C(LAY, LPVV)                                 \
  if (C <= 256) {                                                 \
    SVHIP_ECANON(LAY, LPVV, 256);                                 \
  } else if constexpr (LPVV == 16 || sizeof(T) == 2) {            \
    SVHIP_ECANON(LAY, LPVV, kCanonMaxC);                          \
  }
    if (plan.layout == kCanonVec) {
      if (plan.lpv == 8) {
        SVHIP_ECANON_C(kCanonVec, 8)
      } else {
        SVHIP_ECANON_C(kCanonVec, 16)
      }
    } else {
      if (plan.lpv == 8) {
        SVHIP_ECANON_C(kCanonScalar, 8)
      } else {
        SVHIP_ECANON_C(kCanonScalar, 16)
      }
    }
#undef SVHIP_ECANON_C
#undef SVHIP_ECANON
    return SVHIP_OK;
  }
  if (plan.layout == kClassMajorVec) {
    ease_stats_kernel<T, kClassMajorVec, 0><<<grid, 256, 0, s>>>(x, batch, n, C, sb, sc, sn, ks, ap, side, rows);
  } else {
    ease_stats_kernel<T, kClassMajorScalar, 0><<<grid, 256, 0, s>>>(x, batch, n, C, sb, sc, sn, ks, ap, side, rows);
  }
  return SVHIP_OK;
}

// The EASE selection over logits whose voxel rows are found through `rows` (YZX or patch order).
static int ease_select_impl(const void* logits, int dtype, int64_t classes, int64_t stride_b, int64_t stride_c,
                            int64_t stride_n, const int64_t* tokens, int64_t mask_token, const uint8_t* last,
                            int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const int64_t* k,
                            const int64_t* pos, const double* frac, const int64_t* n_total, const int64_t* committed,
                            uint8_t* chosen, uint8_t* bad, float* scores_out, void* workspace, size_t workspace_bytes,
                            void* stream, VoxelRows rows, const char* name) {
  Geometry g;
  int rc = check_geometry(batch, Y, Z, X, block, name, &g);
  if (rc != SVHIP_OK) return rc;
  SVHIP_REQUIRE(logits && tokens && last && k && pos && frac && n_total && committed && chosen && bad,
                "%s: null pointer", name);
  SVHIP_REQUIRE(classes >= 1, "%s: bad class count %lld", name, (long long)classes);
  SVHIP_REQUIRE(dtype == SVHIP_F32 || dtype == SVHIP_BF16, "%s: dtype %d not supported (fp32 or bf16)", name, dtype);
  const size_t need = quota_ws_bytes(batch, g);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need, workspace_bytes);
    return SVHIP_EWORKSPACE;
  }
  const QuotaWs w = carve(workspace, batch, g);
  hipStream_t s = as_stream(stream);
  // Windows of at most kWaveBlocks blocks are apportioned by side workgroups of the entropy pass.
  const int side = g.nb <= kWaveBlocks ? static_cast<int>(batch) : 0;
  if (side == 0) {
    rc = launch_apportion(batch, g, k, pos, frac, n_total, committed, w, s, name);
    if (rc != SVHIP_OK) return rc;
  }
  const KeyStore ks{tokens, last, mask_token, w.ckey, scores_out};
  const ApportionArgs ap{n_total, pos, frac, k, committed, g.nb, w.target};
  if (dtype == SVHIP_F32) {
    rc = launch_ease_stats<float>(static_cast<const float*>(logits), batch, classes, g.n, stride_b, stride_c, stride_n,
                                  ks, ap, side, s, rows, name);
  } else {
    rc = launch_ease_stats<uint16_t>(static_cast<const uint16_t*>(logits), batch, classes, g.n, stride_b, stride_c,
                                     stride_n, ks, ap, side, s, rows, name);
  }
  if (rc != SVHIP_OK) return rc;
  SVHIP_LAUNCHED(name);
  return launch_inblock_fix(KeyStored{w.ckey}, batch, g, k, n_total, chosen, bad, w, s, name);
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
  SVHIP_REQUIRE(score && mask && k && pos && frac && n_total && chosen && bad, "%s: null pointer", name);
  const size_t need = quota_ws_bytes(batch, g);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need, workspace_bytes);
    return SVHIP_EWORKSPACE;
  }
  const QuotaWs w = carve(workspace, batch, g);
  hipStream_t s = as_stream(stream);
  if (committed == nullptr) {
    committed_kernel<<<static_cast<unsigned>(batch), 256, 0, s>>>(mask, n_total, g.nb, g.n, w.committed);
    SVHIP_LAUNCHED(name);
    committed = w.committed;
  }
  rc = launch_apportion(batch, g, k, pos, frac, n_total, committed, w, s, name);
  if (rc != SVHIP_OK) return rc;
  return launch_inblock_fix(KeyFromScore<MaskBytes>{score, MaskBytes{mask, g.n}, w.ckey}, batch, g, k, n_total,
                            chosen, bad, w, s, name);
}

extern "C" size_t svhip_ease_select_workspace_bytes(int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block) {
  Geometry g;
  if (check_geometry(batch, Y, Z, X, block, "svhip_ease_select_workspace_bytes", &g) != SVHIP_OK) return 0;
  return quota_ws_bytes(batch, g);
}

extern "C" int svhip_ease_select(const void* logits, int dtype, int64_t classes, int64_t stride_b, int64_t stride_c,
                                 int64_t stride_n, const int64_t* tokens, int64_t mask_token, const uint8_t* last,
                                 int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const int64_t* k,
                                 const int64_t* pos, const double* frac, const int64_t* n_total,
                                 const int64_t* committed, uint8_t* chosen, uint8_t* bad, float* scores_out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return ease_select_impl(logits, dtype, classes, stride_b, stride_c, stride_n, tokens, mask_token, last, batch, Y, Z,
                          X, block, k, pos, frac, n_total, committed, chosen, bad, scores_out, workspace,
                          workspace_bytes, stream, kYzxRows, "svhip_ease_select");
}

extern "C" int svhip_ease_select_patches(const void* logits, int dtype, int64_t classes, int64_t patch,
                                         int64_t stride_b, int64_t stride_n, const int64_t* tokens,
                                         int64_t mask_token, const uint8_t* last, int64_t batch, int64_t Y,
                                         int64_t Z, int64_t X, int64_t block, const int64_t* k, const int64_t* pos,
                                         const double* frac, const int64_t* n_total, const int64_t* committed,
                                         uint8_t* chosen, uint8_t* bad, float* scores_out, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  const char* name = "svhip_ease_select_patches";
  clear_error();
  SVHIP_REQUIRE(patch >= 1, "%s: bad patch size %lld", name, (long long)patch);
  VoxelRows rows;
  const int rc = make_rows(Y, Z, X, patch, &rows, name);
  if (rc != SVHIP_OK) return rc;
  return ease_select_impl(logits, dtype, classes, stride_b, 1, stride_n, tokens, mask_token, last, batch, Y, Z, X,
                          block, k, pos, frac, n_total, committed, chosen, bad, scores_out, workspace,
                          workspace_bytes, stream, rows, name);
}

// ------------------------------------------------------------------ fixed-scratch selection (allocates nothing)

namespace svhip {

// The selection's scratch (targets, quotas, keys, boundary candidates) for callers that cannot allocate: one
// array per GPU, held until the process ends. 48 MiB covers 92 windows of 65 536 voxels at 4^3 blocks
// (544 768 bytes per window).
constexpr size_t kScratchBytes = size_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's `scratch`, looked up once per device with that device current. The array's
// name is only a host-side handle; kernels get this address.
static int scratch_address(void** out, const char* name) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("%s: hipGetDevice failed: %s", name, hipGetErrorString(e));
    return SVHIP_ELAUNCH;
  }
  SVHIP_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond the %d supported", name, dev, kMaxDevices);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev, hipGetErrorString(e));
        return SVHIP_ELAUNCH;
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SVHIP_OK;
}

}  // namespace svhip

extern "C" int svhip_ease_select_noalloc(const void* logits, int dtype, int64_t classes, int64_t stride_b,
                                         int64_t stride_c, int64_t stride_n, const int64_t* tokens,
                                         int64_t mask_token, const uint8_t* last, int64_t batch, int64_t Y, int64_t Z,
                                         int64_t X, int64_t block, const int64_t* k, const int64_t* pos,
                                         const double* frac, const int64_t* n_total, const int64_t* committed,
                                         uint8_t* chosen, uint8_t* bad, float* scores_out, void* stream) {
  const char* name = "svhip_ease_select_noalloc";
  clear_error();
  Geometry g;
  int rc = check_geometry(batch, Y, Z, X, block, name, &g);
  if (rc != SVHIP_OK) return rc;
  const size_t need = quota_ws_bytes(batch, g);
  SVHIP_REQUIRE(need <= kScratchBytes, "%s: %lld windows of %lld voxels need %zu bytes of scratch, the fixed array "
                "holds %zu", name, (long long)batch, (long long)g.n, need, kScratchBytes);
  SVHIP_REQUIRE(logits && tokens && last && k && pos && frac && n_total && committed && chosen && bad,
                "%s: null pointer", name);
  void* ws = nullptr;
  rc = scratch_address(&ws, name);
  if (rc != SVHIP_OK) return rc;
  // Every scratch word the kernels read is written earlier in the same call, so nothing needs clearing.
  return ease_select_impl(logits, dtype, classes, stride_b, stride_c, stride_n, tokens, mask_token, last, batch, Y, Z,
                          X, block, k, pos, frac, n_total, committed, chosen, bad, scores_out, ws, kScratchBytes,
                          stream, kYzxRows, name);
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
