// Cross attention over per-window variable-length cached K/V, bf16 MFMA (gfx950), fp32 accumulation.
//
// Work item: one workgroup = (window b, head h, 128-query tile), 4 waves x 32 queries. Keys are walked in
// 64-key blocks staged through LDS, double-buffered: the next block is in flight while the current one is
// computed, one workgroup barrier per block.
//
// Per wave and key block (v_mfma_f32_32x32x16_bf16 throughout), in two 32-key halves that each run the whole
// online-softmax step (a half's scores take 16 registers, which leaves room for three waves per SIMD):
//   S^T[key, q] = K . Q^T         A = K rows from LDS, B = the wave's Q (registers, loaded once)
//   P^T = exp2(S^T - m)           online softmax; every lane owns one query column (q = lane % 32) and
//                                       8 of every 16 keys, its partner lane (lane ^ 32) the other 8
//   O^T[d, q] += V^T . P^T        A = V^T rows from LDS, B = P^T straight from the S^T accumulators
// The C layout of a 32x32 MFMA gives lane l the rows 8*(i/4) + 4*(l/32) + i%4 of column l%32. K rows are
// stored in LDS under the involution sigma (swap of the 4-row groups 1 and 2 of every 16 rows), so accumulator
// entries i = 0..7 of lane l hold keys 8*(l/32) + i and i = 8..15 keys 16 + 8*(l/32) + (i-8): exactly the B
// operand slice (k index 8*(l/32) + j) the second product needs, with no cross-lane movement.
// Because O^T's columns are queries too, the per-query rescale and the final 1/l are lane-local.
//
// The softmax is VALU-bound at head_dim 64 (one exp per score against 2 x 64 MACs), so per score it costs one
// FMA, one exp and half a bf16 pack on the VALU, and no max and no add: the row sum comes from the matrix cores
// (two v_mfma_f32_16x16x32_bf16 per 32-key half over the packed P with a ones pattern, a sixteenth of the half's
// matrix-core time, in place of 15 fp32 adds per lane; v_dot2c_f32_bf16 would not co-execute with the matrix
// cores):
//   * Q enters the score product as given (bf16) and the fp32 scores are scaled by sl2 = scale * log2(e) (and the
//     e4m3 K scale) inside the exponent's FMA, P = exp2(fma(S, sl2, -m)) with m the running max in log2 units, so
//     the only roundings of the query are the caller's.
//   * P is formed against the running max m as it stands. The half's row sum (read back from the matrix cores
//     before the second product is issued) tells whether m still bounds the half's scores: only a sum above 2^20
//     (and always the window's first half) makes the wave take the half's max (16 three-input maxes and the
//     partner's over v_permlane32_swap), raise m, rescale O and l and redo P and its sum shifted by the rise. P may thus reach 2^20, harmless in fp32 sums and bf16 P; O and l always share m, so
//     O / l does not depend on where m sits.
//   * With direct staging and head_dim below 32 DT (the shipped 48) V^T row D, a padding row, holds ones: the
//     second product then accumulates the row sum of the bf16 P in O^T row D, and the VALU drops the adds. The
//     trigger becomes the half's own max (8 three-input maxes): a score more than 20 above m.
//   * key masking runs only in the last, partial block; padding keys are staged as zeros.
//
// e4m3 K/V with PV8 (SVHIP_FP8_E4M3_PFP8): the second product runs on the fp8 matrix cores,
// v_mfma_f32_32x32x64_f8f6f4 over a whole 64-key block per output tile (half the bf16 product's matrix-core time).
// V^T stays e4m3 in LDS (its per-head scale applied at the end); P is formed 2^4 above the running max and rounded
// to e4m3 as it is packed, a lane's 32 weights being exactly the B operand's 32 k slots (K rows are placed by
// pv8_row for that); the row sum is taken over the rounded weights (decoded, or from the ones row), so a dominant
// key's rounding cancels in O / l. The score product stays bf16 over the exactly decoded keys. The price is a 2^-4
// relative rounding of every softmax weight, so PV8 is an opt-in (SVHIP_FP8_E4M3_PFP8); SVHIP_FP8_E4M3, the e4m3
// cache's default, keeps P in bf16 (PV8 off): the reference's in-kernel dequantisation.
//
// Staging. An LDS tile holds 64 rows of 128 bytes, the eight 16-byte chunks of row r XOR-swizzled by (r / 2) % 8
// so that the 16-byte operand reads are bank-conflict-free; a K row is one key's head_dim, a V^T row one
// head_dim element's 64 keys. Row-major V with a bf16 second product stays one key a row (in K's tile layout,
// swizzled by swzv) and the second product reads its V^T operand with ds_read_b64_tr_b16, the LDS transpose load
// of gfx950, so V rows are stored as they come. bf16 K and V with 16-byte aligned rows (V^T of the padded
// [B,H,Kcap,*] layout, V rows of the padded or the packed layout) take buffer_load_dwordx4 ... lds, which moves a
// full block straight into LDS without registers, addressed by a per-lane offset fixed for the window plus a
// scalar block offset. Every other form goes through registers, prefetched one block ahead in its storage format
// and converted when it is written to LDS: OCP e4m3fn K/V converted exactly to bf16 (v_cvt_scalef32_pk_bf16_fp8
// with scale 1; the fp8 scales are folded into the softmax scale (k_scale) and the output (v_scale)), V^T of the
// packed cu_seqlens layout, key masks.
// The last, partial block of a window is peeled out of the loop and staged through registers (its loads issued
// before the last full block is computed), keys >= L as zeros.
//
// Workgroup order: windows are ranked by key count (longest first, ties by index; up to kMaxRankWindows windows)
// inside the kernel, so the longest (window, head) pairs start first; consecutive workgroup ids go round robin to
// the 8 XCDs and all query tiles of one (window, head) pair land on the same XCD, which reads that pair's K/V into
// its L2 once.
//
// Head widths: DT = 2, 3 or 4 output tiles of 32 head_dim elements (head_dim <= 64, 96, 128). A K block is DT / 2
// rounded up 64 x 64 sub-tiles (head_dim 0..63 and 64..127 of every key, same layout and swizzle), V^T one tile of
// 32 DT rows (V rows: K's sub-tiles); the score product takes up to 2 DT k-steps, the second product DT
// accumulators. DT = 2 is the
// 384-wide (8 x 48) and the 64-wide heads, DT = 3 the 768-wide model's 8 x 96.
#include <type_traits>

#include "common.hpp"

namespace svhip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kQTile = 128;   // queries per workgroup
constexpr int kKB = 64;       // keys per block
constexpr int kSub = 64;      // head_dim elements per K sub-tile row (smaller head_dim is zero-padded)
constexpr int kMaxD = 128;    // widest head (DT = 4)
constexpr int kRow = 64;      // LDS row stride in bf16 elements (128 bytes, 16-byte chunks XOR-swizzled)
constexpr int kKTile = kKB * kRow;  // bf16 elements of one K sub-tile
constexpr int kThreads = 256;
constexpr float kSumHigh = 1048576.0f;  // 2^20: a half's row sum above it makes the running max be raised
constexpr float kMaxHigh = 20.0f;       // the same bound on a single score above the running max (log2 units)
// The bf16 row-sum form issues a half's second product before it reads the half's row sum back: its stored max
// is the running max plus kSpecBias, so P = exp2(S - m) stays below 2^-20 of the fast path's while m bounds the
// scores, and P is clamped to 1 (the exponential's clamp modifier) so that a stale m cannot overflow O. A row sum
// above kSpecHigh (a score more than about 19 above the running max, every clamped P among them) takes the half
// back out of O and does it again against the raised max.
constexpr float kSpecBias = 20.0f;
constexpr float kSpecHigh = 0.5f;
constexpr float kFltMax = 3.40282347e38f;
// e4m3 second product: P is formed 2^4 above the running max and packed only while it stays below 448, the
// largest e4m3 value: a score more than 4.8 above the running max (2^(4 + 4.8) = 445.7) raises the max first.
constexpr float kPv8Lift = 4.0f;
constexpr float kPv8MaxHigh = 4.8f;
// Windows are ranked by length inside every workgroup (each thread compares its candidates against all windows);
// beyond this many windows that quadratic cost is not worth the balance and the grid keeps the window order.
constexpr int kMaxRankWindows = 256;
constexpr int kCusPerXcd = 32;  // MI355X: 8 XCDs x 32 CUs

// Wave timelines (built only with -DSVHIP_XATTN_TRACE, into the separate trace library that
// streamvoxel_amd/xattn_trace.py loads; the product library compiles every hook below to nothing). Per wave of the
// bf16 direct-staged full-width kernel: the wave's HW_ID / XCC_ID registers, its (window, head, query tile, full
// blocks), s_memtime at the wave's start and end, and for key blocks kTraceBlock0 .. + kTraceBlocks - 1 five stamps
// per 32-key half (before the score product's operand reads; after the score product, read back by a
// compiler-visible VALU op; after the exponentials and packs; after the row-sum readback; after the second product
// is issued) and one after the block's barrier. The stamps are s_memtime (a per-CU counter: compare stamps of one
// CU only); the asm takes the value a stamp must follow as an operand, so it cannot move above it.
#ifdef SVHIP_XATTN_TRACE
__device__ unsigned long long* g_trace = nullptr;
constexpr int kTraceBlock0 = 4, kTraceBlocks = 8, kTraceWords = 4 + kTraceBlocks * 11;
struct WaveTrace {
  unsigned long long* slot = nullptr;
  unsigned long long tt[11];
  bool block_on = false;
  static __device__ __forceinline__ unsigned long long stamp() {
    unsigned long long t;
    asm volatile("s_memtime %0" : "=s"(t));
    return t;
  }
  static __device__ __forceinline__ unsigned long long stamp_after(float dep, float dep2 = 0.f) {
    unsigned long long t;
    asm volatile("s_memtime %0" : "=s"(t) : "v"(dep), "v"(dep2));
    return t;
  }
  static __device__ __forceinline__ unsigned long long stamp_now(float dep) {
    unsigned long long t;
    asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) : "v"(dep));
    return t;
  }
  __device__ __forceinline__ void begin(bool on, int w, int lane, int64_t b, int64_t h, int qt, int nfull) {
    if (!on || g_trace == nullptr) return;
    slot = g_trace + (static_cast<long long>(blockIdx.x) * 4 + w) * kTraceWords;
    if (lane == 0) {
      unsigned int hw, xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      slot[0] = (static_cast<unsigned long long>(xcc) << 32) | hw;
      slot[1] = (static_cast<unsigned long long>(b) << 40) | (static_cast<unsigned long long>(h) << 24) |
                (static_cast<unsigned long long>(qt) << 16) | static_cast<unsigned long long>(nfull);
      slot[2] = stamp_now(0.f);
    }
  }
  __device__ __forceinline__ void block(int blk) {
    block_on = slot != nullptr && blk >= kTraceBlock0 && blk < kTraceBlock0 + kTraceBlocks;
  }
  __device__ __forceinline__ void mark(int i) {
    if (block_on) tt[i] = stamp();
  }
  __device__ __forceinline__ void mark_after(int i, float dep, float dep2 = 0.f) {
    if (block_on) tt[i] = stamp_after(dep, dep2);
  }
  __device__ __forceinline__ void block_end(int blk, int lane) {
    const int k = blk - kTraceBlock0;
    if (slot == nullptr || k < 0 || k >= kTraceBlocks) return;
    tt[10] = stamp();
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 11; ++i) slot[4 + 11 * k + i] = tt[i];
    }
  }
  __device__ __forceinline__ void end(int lane, float dep) {
    if (slot != nullptr && lane == 0) slot[3] = stamp_now(dep);
  }
};
#define SVHIP_TRACE(...) __VA_ARGS__
#else
#define SVHIP_TRACE(...)
#endif

struct XattnParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* kv_len;
  const int32_t* cu_seqlens;
  const float* k_scale;
  const float* v_scale;
  const uint8_t* kv_mask;  // optional key mask: key j of window b is attended iff kv_mask[b * sm_b + j] != 0
  int64_t sm_b;
  int64_t B, H, Q, D, kv_cap;
  int64_t sq_b, sq_h, sq_q;
  int64_t sk_b, sk_h, sk_k;
  int64_t sv_b, sv_h, sv_k, sv_d;
  int64_t so_b, so_h, so_q;
  float scale_log2;  // softmax scale * log2(e), > 0
  int q_tiles;
};

// Physical 16-byte chunk of logical chunk c in LDS row r. The 64 banks span two 128-byte rows and a 16-byte read
// serves 16 lanes per cycle: 16 consecutive rows read at one logical chunk land on 16 different (row parity,
// chunk) bank groups, so the operand reads (lane i of a group on row i) are conflict-free.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// Row of key `key` (0..63) of a block inside the LDS K tile.
__device__ __forceinline__ int sigma_row(int key) {
  const int y = key & 15;
  const int g = y >> 2;
  const int swapped = (g == 1) ? y + 4 : (g == 2 ? y - 4 : y);
  return (key & ~15) | swapped;
}

// e4m3 second product (PV8): row of key `key` (0..63) of a block inside the LDS K tile. Key bits
// [hh t a1 a0 b1 b0] go to row bits [t a1 a0 hh b1 b0], so that score entry i of half t in lane half hh is key
// 32 hh + 16 t + i: a lane's 32 P values are then the 32 consecutive keys that byte j of its B operand of
// v_mfma_f32_32x32x64_f8f6f4 pairs with in the A operand (keys 32 hh + j of a V^T row in natural order).
__device__ __forceinline__ int pv8_row(int key) {
  return (((key >> 4) & 1) << 5) | (((key >> 2) & 3) << 3) | ((key >> 5) << 2) | (key & 3);
}

// The e4m3 V^T tile of PV8: rows of 64 bytes (one head_dim element's 64 keys), the four 16-byte chunks of row r
// XOR-swizzled by (r / 4) % 4, so that 16 consecutive rows read at one logical chunk hit 16 distinct bank groups.
constexpr int kRow8 = 64;
__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 2) & 3); }

// Row-major V with a bf16 second product (VROWS): V stays one key a row in LDS, in K's tile layout (64 keys x 64
// head_dim elements a sub-tile, keys in natural order), and the second product reads its V^T operand transposed
// (ds_read_b64_tr_b16). The eight 16-byte chunks of row r are XOR-swizzled by 4 ((r / 2) % 2): the 32 lanes a
// transposed read serves per cycle touch rows r0 .. r0 + 3 (r0 a multiple of 4), 64 contiguous bytes each, and the
// swizzle puts rows r0 and r0 + 2 (which share banks, as do r0 + 1 and r0 + 3) on different 64-byte halves.
__device__ __forceinline__ int swzv(int r, int c) { return c ^ (((r >> 1) & 1) << 2); }

// 8 OCP e4m3fn bytes (two dwords) -> 8 bf16 packed in a uint4 (exact: every e4m3 value is a bf16 value).
__device__ __forceinline__ uint4 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  return make_uint4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, c),
                    __builtin_bit_cast(uint32_t, d));
}

// v_max3_f32 without the operand canonicalisation the compiler adds around fmaxf (the MFMA results feeding it
// are never signalling NaNs). Inline asm: its operands must not be MFMA results the compiler has not yet waited
// for (it inserts no wait states for inline asm).
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

template <bool FP8>
struct Elem {
  using T = typename std::conditional<FP8, uint8_t, uint16_t>::type;
};

// Staged data stays in its storage format until it is written to LDS (16 bytes of bf16 or 8 bytes of e4m3 per 8
// elements): a conversion right after a load inside a conditional would make the compiler wait for the load before
// the branch closes, exposing its latency once per load.
template <bool FP8>
struct Raw {
  using type = typename std::conditional<FP8, uint2, uint4>::type;
};

template <bool FP8>
__device__ __forceinline__ typename Raw<FP8>::type raw_zero() {
  if constexpr (FP8) {
    return make_uint2(0u, 0u);
  } else {
    return make_uint4(0u, 0u, 0u, 0u);
  }
}

// 8 consecutive elements (bf16 or e4m3) with one vector load (16 / 8 bytes, aligned).
template <bool FP8>
__device__ __forceinline__ typename Raw<FP8>::type load8_vec(const typename Elem<FP8>::T* p) {
  return *reinterpret_cast<const typename Raw<FP8>::type*>(p);
}

// The first `valid` (0..8) of 8 consecutive elements, any alignment; the rest are zero.
template <bool FP8>
__device__ __forceinline__ typename Raw<FP8>::type load8_scalar(const typename Elem<FP8>::T* p, int valid) {
  constexpr int kBits = FP8 ? 8 : 16;
  constexpr int kPerWord = 32 / kBits;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (e < valid) w[e / kPerWord] |= static_cast<uint32_t>(p[e]) << (kBits * (e % kPerWord));
  }
  if constexpr (FP8) {
    return make_uint2(w[0], w[1]);
  } else {
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Storage -> 8 bf16 in a uint4 (e4m3 converted exactly).
template <bool FP8>
__device__ __forceinline__ uint4 to_bf16x8(const typename Raw<FP8>::type& r) {
  if constexpr (FP8) {
    return fp8x8_to_bf16x8(r.x, r.y);
  } else {
    return r;
  }
}

// DT output tiles of 32 head_dim elements: K sub-tiles per block, and the per-thread chunk counts of one block
// (a 64 x 64 K sub-tile is 512 chunks of 8 elements, two per thread; V^T takes 32 rows = 256 chunks per pass).
template <int DT>
struct Width {
  static constexpr int kSubTiles = (DT + 1) / 2;
  static constexpr int kKPasses = 2 * kSubTiles;
};

template <bool FP8, bool VT, int DT>
struct Stage {
  typename Raw<FP8>::type k[Width<DT>::kKPasses];
  typename Raw<FP8>::type v[VT ? DT : Width<DT>::kKPasses];
};

// Global -> registers for the key block starting at kv0. K pass r: sub-tile r / 2, chunk c = thread + 256 (r % 2)
// (key c / 8, head_dim chunk 8 (r / 2) + c % 8); V^T pass r: rows 32 r .. 32 r + 31; row-major V as K.
// TAIL: the block holds keys >= L (they are staged as zeros). vt_vec: V^T rows allow vector loads.
template <bool FP8>
__device__ __forceinline__ typename Raw<FP8>::type raw_one() {
  if constexpr (FP8) {
    return make_uint2(0x38383838u, 0x38383838u);  // e4m3 1.0
  } else {
    return make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);  // bf16 1.0
  }
}

// The same with only the first of the 8 elements 1.0 (head_dim D of a row-major V row, when D % 8 == 0).
template <bool FP8>
__device__ __forceinline__ typename Raw<FP8>::type raw_one_first() {
  if constexpr (FP8) {
    return make_uint2(0x38u, 0u);
  } else {
    return make_uint4(0x3F80u, 0u, 0u, 0u);
  }
}

template <bool FP8>
__device__ __forceinline__ typename Raw<FP8>::type raw_select(bool keep, const typename Raw<FP8>::type& v,
                                                             const typename Raw<FP8>::type& other) {
  if constexpr (FP8) {
    return make_uint2(keep ? v.x : other.x, keep ? v.y : other.y);
  } else {
    return make_uint4(keep ? v.x : other.x, keep ? v.y : other.y, keep ? v.z : other.z, keep ? v.w : other.w);
  }
}

// ONES: V^T row D (the first padding row) is staged as ones, so that the second product forms the row sum.
// A full block (TAIL false) issues every load without a branch, lanes outside head_dim reading the window's first
// row instead: a load under a per-lane condition makes the compiler merge its result with the other arm's value
// right away, which waits for the load and exposes its latency in the prefetch. stage_store then puts zeros (and
// the ones row) where head_dim ends. The partial block masks its loads (keys >= L read nothing).
// VREG false: V^T is staged another way (direct loads) and left alone here.
template <bool FP8, bool VT, int DT, bool TAIL, bool ONES = false, bool VREG = true>
__device__ __forceinline__ void stage_load(Stage<FP8, VT, DT>& st, const XattnParams& p,
                                           const typename Elem<FP8>::T* K, const typename Elem<FP8>::T* V, int L,
                                           int kv0, int dchunks, bool vt_vec) {
#pragma unroll
  for (int r = 0; r < Width<DT>::kKPasses; ++r) {
    const int c = threadIdx.x + kThreads * (r & 1);  // 0..511
    const int key = c >> 3, dc = 8 * (r >> 1) + (c & 7);
    const int kg = kv0 + key;
    if constexpr (TAIL) {
      const bool ok = dc < dchunks && kg < L;
      st.k[r] = ok ? load8_vec<FP8>(K + kg * p.sk_k + dc * 8) : raw_zero<FP8>();
      if constexpr (!VT) st.v[r] = ok ? load8_vec<FP8>(V + kg * p.sv_k + dc * 8) : raw_zero<FP8>();
    } else {
      const bool ok = dc < dchunks;
      st.k[r] = load8_vec<FP8>(K + (ok ? static_cast<int64_t>(kg) * p.sk_k + dc * 8 : 0));
      if constexpr (!VT) st.v[r] = load8_vec<FP8>(V + (ok ? static_cast<int64_t>(kg) * p.sv_k + dc * 8 : 0));
    }
  }
  if constexpr (VT && VREG) {
#pragma unroll
    for (int r = 0; r < DT; ++r) {
      const int c = threadIdx.x + kThreads * r;
      const int d = c >> 3, kc = c & 7;
      const int kg = kv0 + kc * 8;
      if (!TAIL && vt_vec) {
        st.v[r] = load8_vec<FP8>(V + (d < p.D ? d * p.sv_d : 0) + kg);
      } else if (d < p.D && (!TAIL || kg < L)) {
        const int valid = TAIL ? ((L - kg) < 8 ? (L - kg) : 8) : 8;
        const auto* src = V + d * p.sv_d + kg;
        st.v[r] = (vt_vec && valid == 8) ? load8_vec<FP8>(src) : load8_scalar<FP8>(src, valid);
      } else {
        st.v[r] = raw_zero<FP8>();
      }
    }
  }
}

// Registers -> LDS (K rows under sigma in their sub-tile; V^T [d][key] from V^T, row-major V kept as rows in K's
// layout; all swizzled), with zeros past head_dim and, with ONES, the ones row D of V^T (for V rows: the ones
// column D). PV8: K rows under pv8_row, V^T kept in e4m3 in its own tile (keys in natural order), transposed from
// row-major V byte by byte.
template <bool FP8, bool VT, int DT, bool ONES, bool PV8 = false, bool VREG = true>
__device__ __forceinline__ void stage_store(const Stage<FP8, VT, DT>& st, uint16_t* sK, uint16_t* sV, int dchunks,
                                            int D) {
  static_assert(!PV8 || FP8, "the e4m3 second product takes e4m3 V");
  using R8 = typename Raw<FP8>::type;
#pragma unroll
  for (int r = 0; r < Width<DT>::kKPasses; ++r) {
    const int c = threadIdx.x + kThreads * (r & 1);
    const int R = PV8 ? pv8_row(c >> 3) : sigma_row(c >> 3), dc = c & 7;
    const bool ok = 8 * (r >> 1) + dc < dchunks;
    *reinterpret_cast<uint4*>(sK + (r >> 1) * kKTile + R * kRow + swz(R, dc) * 8) =
        to_bf16x8<FP8>(raw_select<FP8>(ok, st.k[r], raw_zero<FP8>()));
    if constexpr (!VT) {
      const R8 pad = (ONES && 8 * (r >> 1) + dc == dchunks) ? raw_one_first<FP8>() : raw_zero<FP8>();
      const R8 vv = raw_select<FP8>(ok, st.v[r], pad);
      const int key = c >> 3;
      if constexpr (PV8) {
        // Row-major V transposed byte by byte: key c / 8, head_dim 64 (r / 2) + 8 dc + e.
        uint8_t* sV8 = reinterpret_cast<uint8_t*>(sV);
        const uint32_t w[2] = {vv.x, vv.y};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = kSub * (r >> 1) + dc * 8 + e;
          if (d < 32 * DT) {
            sV8[d * kRow8 + swz8(d, key >> 4) * 16 + (key & 15)] = static_cast<uint8_t>(w[e >> 2] >> (8 * (e & 3)));
          }
        }
      } else {
        // V rows kept as rows (VROWS): key c / 8, head_dim chunk 8 (r / 2) + dc, swizzled by swzv.
        *reinterpret_cast<uint4*>(sV + (r >> 1) * kKTile + key * kRow + swzv(key, dc) * 8) = to_bf16x8<FP8>(vv);
      }
    }
  }
  if constexpr (VT && VREG) {
#pragma unroll
    for (int r = 0; r < DT; ++r) {
      const int c = threadIdx.x + kThreads * r;
      const int d = c >> 3, kc = c & 7;
      const R8 vv = raw_select<FP8>(d < D, st.v[r], (ONES && d == D) ? raw_one<FP8>() : raw_zero<FP8>());
      if constexpr (PV8) {
        uint8_t* sV8 = reinterpret_cast<uint8_t*>(sV);
        *reinterpret_cast<R8*>(sV8 + d * kRow8 + swz8(d, kc >> 1) * 16 + (kc & 1) * 8) = vv;
      } else {
        *reinterpret_cast<uint4*>(sV + d * kRow + swz(d, kc) * 8) = to_bf16x8<FP8>(vv);
      }
    }
  }
}

__device__ __forceinline__ int window_length(const XattnParams& p, int64_t b) {
  int64_t L;
  if (p.cu_seqlens) {
    L = static_cast<int64_t>(p.cu_seqlens[b + 1]) - p.cu_seqlens[b];
  } else if (p.kv_len) {
    L = p.kv_len[b];
    if (L > p.kv_cap) L = p.kv_cap;
  } else {
    L = p.kv_cap;  // key-mask form without lengths: every key up to the capacity, the mask decides
  }
  if (p.kv_mask && L > p.kv_cap) L = p.kv_cap;  // the mask rows hold kv_cap keys
  return L < 0 ? 0 : static_cast<int>(L);
}

// Direct path (bf16 K and V^T, full blocks): buffer_load_dwordx4 ... lds moves a block straight into LDS without
// registers. Wave instruction j of a tile fills its rows 8 j .. 8 j + 7 (1024 consecutive bytes, lane l at
// 16 l): row R = 8 j + l / 8, physical chunk l % 8, so the logical chunk c with swz(R, c) = l % 8. The 8
// instructions of a tile go to the 4 waves two each. A lane's byte offsets from the (window, head) base depend only on the window, so
// they are computed once; a block adds kv0 rows of K / columns of V^T through the scalar offset. The buffer
// descriptors bound the reads to the window's full blocks (an out-of-range read returns zeros).
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Instruction j of a K sub-tile or of V^T fills rows 8 j .. 8 j + 7; the 8 instructions of a K sub-tile go to the
// 4 waves two each (w and w + 4), the 4 DT of V^T DT each (w + 4 t). Sub-tile 1 of K reads 64 elements further
// along every key (added to the scalar offset: the immediate offset would move the LDS destination too).
template <int DT>
struct DirectLanes {
  __amdgpu_buffer_rsrc_t k_rsrc, v_rsrc;
  uint32_t k[2];   // byte offsets of K instructions w and w + 4 for the block at key 0
  uint32_t v[DT];  // byte offsets of V^T instructions w + 4 t
  bool k_ok[Width<DT>::kSubTiles][2];  // the lane's K chunk lies inside head_dim
  bool v_ok[DT];                       // the lane's V^T row lies inside head_dim
};

// Raw buffer descriptor word 3 for 32-bit-element untyped access.
constexpr int kRsrcFlags = 0x00020000;

template <int DT>
__device__ __forceinline__ DirectLanes<DT> direct_lanes(const XattnParams& p, const uint16_t* K, const uint16_t* V,
                                                        int dchunks, int nfull, int w) {
  DirectLanes<DT> dl;
  const int lane = threadIdx.x & 63;
  const uint32_t k_bytes = static_cast<uint32_t>(((static_cast<int64_t>(nfull) * kKB - 1) * p.sk_k + p.D) * 2);
  const uint32_t v_bytes = static_cast<uint32_t>(((p.D - 1) * p.sv_d + static_cast<int64_t>(nfull) * kKB) * 2);
  dl.k_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(K), 0, k_bytes, kRsrcFlags);
  dl.v_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(V), 0, v_bytes, kRsrcFlags);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int R = 8 * (w + 4 * t) + (lane >> 3);
    const int c = swz(R, lane & 7);  // swz is an involution in c
    dl.k[t] = static_cast<uint32_t>((sigma_row(R) * p.sk_k + 8 * c) * 2);
#pragma unroll
    for (int u = 0; u < Width<DT>::kSubTiles; ++u) dl.k_ok[u][t] = 8 * u + c < dchunks;
  }
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int R = 8 * (w + 4 * t) + (lane >> 3);
    const int c = swz(R, lane & 7);
    dl.v[t] = static_cast<uint32_t>((R * p.sv_d + 8 * c) * 2);
    dl.v_ok[t] = R < 8 * dchunks;
  }
  return dl;
}

// FULL_D: head_dim = 32 DT, every lane of V^T and of K sub-tile 0 loads (no exec masking); sub-tile 1 at DT = 3
// still masks head_dim 96..127. w: the wave index (uniform).
template <int DT, bool FULL_D, bool VT_TOO = true>
__device__ __forceinline__ void stage_direct(const DirectLanes<DT>& dl, uint32_t k_soff, uint32_t v_soff, int w,
                                             uint16_t* sK, uint16_t* sV) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = w + 4 * t;
#pragma unroll
    for (int u = 0; u < Width<DT>::kSubTiles; ++u) {
      if ((FULL_D && 64 * (u + 1) <= 32 * DT) || dl.k_ok[u][t]) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(dl.k_rsrc, (lds_ptr_t)(sK + u * kKTile + 512 * j), 16, dl.k[t],
                                                 k_soff + 2 * kSub * u, 0, 0);
      }
    }
  }
  if constexpr (VT_TOO) {
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int j = w + 4 * t;
      if (FULL_D || dl.v_ok[t]) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(dl.v_rsrc, (lds_ptr_t)(sV + 512 * j), 16, dl.v[t], v_soff, 0, 0);
      }
    }
  }
}

// Row-major bf16 V of the padded layout (VROWS, direct): the instruction layout of a K sub-tile (instruction j
// fills rows 8 j .. 8 j + 7, two a wave), keys in natural order under swzv; the descriptor bounds the reads to the
// window's full blocks.
template <int DT>
struct DirectRows {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[2];                       // byte offsets of instructions w and w + 4 for the block at key 0
  bool ok[Width<DT>::kSubTiles][2];      // the lane's chunk lies inside head_dim
};

template <int DT>
__device__ __forceinline__ DirectRows<DT> direct_rows(const XattnParams& p, const uint16_t* V, int dchunks, int nfull,
                                                      int w) {
  DirectRows<DT> dr;
  const int lane = threadIdx.x & 63;
  const uint32_t bytes = static_cast<uint32_t>(((static_cast<int64_t>(nfull) * kKB - 1) * p.sv_k + p.D) * 2);
  dr.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(V), 0, bytes, kRsrcFlags);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int R = 8 * (w + 4 * t) + (lane >> 3);
    const int c = swzv(R, lane & 7);  // swzv is an involution in c
    dr.off[t] = static_cast<uint32_t>((R * p.sv_k + 8 * c) * 2);
#pragma unroll
    for (int u = 0; u < Width<DT>::kSubTiles; ++u) dr.ok[u][t] = 8 * u + c < dchunks;
  }
  return dr;
}

template <int DT, bool FULL_D>
__device__ __forceinline__ void stage_rows(const DirectRows<DT>& dr, uint32_t soff, int w, uint16_t* sV) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = w + 4 * t;
#pragma unroll
    for (int u = 0; u < Width<DT>::kSubTiles; ++u) {
      if ((FULL_D && 64 * (u + 1) <= 32 * DT) || dr.ok[u][t]) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(dr.rsrc, (lds_ptr_t)(sV + u * kKTile + 512 * j), 16, dr.off[t],
                                                 soff + 2 * kSub * u, 0, 0);
      }
    }
  }
}

// PV8 with e4m3 V^T rows whose 16-byte runs start aligned: full blocks of V^T go straight to LDS too. One
// 1024-byte buffer_load_dwordx4 ... lds fills 16 rows of 64 bytes (lane l: row 16 j + l / 4 at physical chunk
// l % 4, so logical chunk (l % 4) ^ the row's swizzle); instruction j of the 2 DT goes to wave j % 4. Rows >= D are
// never loaded (they hold zeros, or the ones row, written once).
template <int DT>
struct DirectV8 {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[(2 * DT + 3) / 4];  // per instruction of the wave (some waves one fewer)
  bool ok[(2 * DT + 3) / 4];
};

template <int DT>
__device__ __forceinline__ DirectV8<DT> direct_v8(const XattnParams& p, const uint8_t* V, int nfull, int w) {
  DirectV8<DT> dv;
  const int lane = threadIdx.x & 63;
  const uint32_t bytes = static_cast<uint32_t>((p.D - 1) * p.sv_d + static_cast<int64_t>(nfull) * kKB);
  dv.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(V), 0, bytes, kRsrcFlags);
#pragma unroll
  for (int t = 0; t < (2 * DT + 3) / 4; ++t) {
    const int R = 16 * (w + 4 * t) + (lane >> 2);
    const int c = swz8(R, lane & 3);  // swz8 is an involution in c
    dv.off[t] = static_cast<uint32_t>(R * p.sv_d + 16 * c);
    dv.ok[t] = R < p.D;
  }
  return dv;
}

// Instruction j of the direct e4m3 V^T loads (see DirectV8): 1024 bytes into rows 16 j .. 16 j + 15 of the tile.
__device__ __forceinline__ void direct_v8_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint32_t soff, uint16_t* sV,
                                               int j) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(reinterpret_cast<uint8_t*>(sV) + 1024 * j), 16, off, soff,
                                           0, 0);
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The highest index j < n with row[j] != 0 among the ones this thread reads (thread t of kThreads: 16-byte chunks
// t, t + kThreads, ... of a 16-byte aligned row, four loads in flight; the rest, or an unaligned row, byte by byte
// with eight loads in flight), or -1. The caller takes the maximum over the workgroup.
__device__ __forceinline__ int last_attended(const uint8_t* row, int n) {
  int last = -1;
  const int nvec = (reinterpret_cast<uintptr_t>(row) & 15) == 0 ? n / 16 : 0;
  for (int c0 = threadIdx.x; c0 < nvec; c0 += 4 * kThreads) {
    uint4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + u * kThreads;
      x[u] = c < nvec ? reinterpret_cast<const uint4*>(row)[c] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // the highest nonzero byte of word q: byte 4 q + (31 - clz) / 8
        if (w[q] != 0u) last = max(last, 16 * (c0 + u * kThreads) + 4 * q + ((31 - __clz(w[q])) >> 3));
      }
    }
  }
  for (int j0 = 16 * nvec + threadIdx.x; j0 < n; j0 += 8 * kThreads) {
    uint8_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = row[min(j0 + u * kThreads, n - 1)];  // no branch around the loads
#pragma unroll
    for (int u = 0; u < 8; ++u) last = (v[u] && j0 + u * kThreads < n) ? max(last, j0 + u * kThreads) : last;
  }
  return last;
}

// STAGING: kRegister (registers for every block), kDirect (direct loads for full blocks, any head_dim),
// kDirectFull (the same at head_dim 32 DT), kRegisterFull (registers at head_dim 32 DT). The last, partial block
// of a window always goes through registers. At head_dim 32 DT the score product's k-steps are all known at
// compile time, so its operand reads are issued together instead of one wait per step.
enum Staging { kRegister = 0, kDirect = 1, kDirectFull = 2, kRegisterFull = 3 };

// ONES: head_dim below 32 DT, the row sum comes from the matrix cores (V^T row D of ones). The e4m3 V^T kernel up
// to head_dim 64 is held to 168 VGPRs (three waves per SIMD; it needs 170 unbounded, without spilling at 168); the
// bf16 direct-staged ones fit by themselves.
// KMASK: a key mask (p.kv_mask) on top of the window length: the window ends at its last attended key, a block
// whose keys it all masks is skipped, one whose keys it all attends is computed as without a mask, any other masks
// its scores (the register-staged V^T form masks every block).
// PV8: e4m3 K/V take the second product on the fp8 matrix cores (see the comment at the top).
// VD8: with PV8, V^T takes direct loads for full blocks (e4m3 rows of 16-byte aligned runs).
template <bool FP8, bool VT, int STAGING, int DT, bool ONES, bool KMASK = false, bool PV8 = false, bool VD8 = false>
__global__ __launch_bounds__(kThreads, (DT == 2 && (VT || !PV8)) ? 3 : 2) void xattn_fwd_kernel(XattnParams p) {
  // The body is compiled in the device pass only: the host pass, which needs just the launch stub, otherwise
  // instantiates the staging lambdas of the key-mask kernels with direct loads and rejects their calls of the
  // device-only staging functions.
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr bool DIRECT = STAGING == kDirect || STAGING == kDirectFull;
  constexpr bool FULLK = STAGING == kDirectFull || STAGING == kRegisterFull;  // head_dim 32 DT
  static_assert(!ONES || !FULLK, "a full-width head has no padding row");
  static_assert(!PV8 || (FP8 && !DIRECT && !KMASK), "the e4m3 second product stages e4m3 K/V through registers");
  static_assert(!VD8 || (PV8 && VT), "direct e4m3 V^T loads serve the e4m3 second product");
  // bf16 P with no padding row for the row sum: the matrix cores form it from the packed P (see onesb).
  constexpr bool MSUM = !ONES && !PV8;
  // MSUM over a bf16 cache at head_dim 64: a half's second product is issued before its row sum is read back (see
  // compute). Every staging and masking takes the same form, so the layouts give the same bits. (Over an e4m3
  // cache, staged through registers, the form measured no faster.)
  constexpr bool SPEC = MSUM && !FP8 && DT == 2;
  constexpr int kSubTiles = Width<DT>::kSubTiles;
  // Row-major V with a bf16 second product: V rows in LDS, read transposed (see swzv).
  constexpr bool VROWS = !VT && !PV8;
  // V tile: V^T, 32 DT rows of 64 keys, bf16 (kRow elements a row) or e4m3 (kRow8 bytes a row); V rows in K's
  // sub-tiles.
  constexpr int kVTile = PV8 ? 32 * DT * kRow8 / 2 : (VROWS ? kSubTiles * kKTile : 32 * DT * kRow);
  // Four distinct LDS objects (not one indexed array): the compiler can then tell the direct loads into one
  // buffer from the operand reads of the other and does not wait for the loads in flight before those reads.
  __shared__ __attribute__((aligned(16))) uint16_t sK0[kSubTiles * kKTile], sK1[kSubTiles * kKTile];
  __shared__ __attribute__((aligned(16))) uint16_t sV0[kVTile], sV1[kVTile];
  __shared__ int s_window;

  // Workgroup -> (rank, head, query tile): XCD x (= id % 8) takes the (rank, head) units x, x + 8, ... with all
  // query tiles of a unit back to back. rank 0 is the window with the most keys. An XCD hands its k-th workgroup
  // to its CU k % 32, so every CU holds one unit's tile from each round of 32 and the rounds go from the longest
  // units to the shortest; odd rounds take their units in reverse, pairing a CU's long tile of one round with a
  // short one of the next (a permutation: any placement stays correct, this one only balances the CUs).
  const int64_t wg = blockIdx.x;
  int qt;
  int64_t unit;
  if ((p.B * p.H) % 8 == 0) {
    const int64_t seq = wg >> 3;
    qt = static_cast<int>(seq % p.q_tiles);
    int64_t k = seq / p.q_tiles;  // the XCD's unit index
    const int64_t per_round = kCusPerXcd / p.q_tiles;
    if (kCusPerXcd % p.q_tiles == 0 && per_round > 1) {
      const int64_t round = k / per_round;
      const int64_t full_rounds = (p.B * p.H / 8) / per_round;
      if ((round & 1) && round < full_rounds) k = round * per_round + (per_round - 1 - (k - round * per_round));
    }
    unit = (wg & 7) + 8 * k;
  } else {
    qt = static_cast<int>(wg % p.q_tiles);
    unit = wg / p.q_tiles;
  }
  const int64_t h = unit % p.H;
  const int64_t rank = unit / p.H;
  int64_t b = rank;
  if (p.B > 1 && p.B <= kMaxRankWindows) {
    // The window whose (length desc, index asc) rank is `rank`: every thread ranks its candidate windows.
    for (int64_t c = threadIdx.x; c < p.B; c += kThreads) {
      const int Lc = window_length(p, c);
      int64_t r = 0;
      for (int64_t o = 0; o < p.B; ++o) {
        const int Lo = window_length(p, o);
        r += (Lo > Lc || (Lo == Lc && o < c)) ? 1 : 0;
      }
      if (r == rank) s_window = static_cast<int>(c);
    }
    __syncthreads();
    b = s_window;
  }

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31;  // query column within the wave
  const int hh = lane >> 5;   // lane half
  const int64_t q = static_cast<int64_t>(qt) * kQTile + w * 32 + col;
  const bool q_ok = q < p.Q;

  const int64_t off = p.cu_seqlens ? p.cu_seqlens[b] : 0;
  const int L = [&]() __attribute__((always_inline)) {
    const int n = window_length(p, b);
    if constexpr (!KMASK) {
      return n;
    } else {
      // With a key mask the window ends at its last attended key: the blocks after it add nothing to O, l or m.
      // One scan of the window's mask row (a wave-uniform result; no attended key gives L = 0 and zeros).
      __shared__ int s_last;
      if (threadIdx.x == 0) s_last = -1;
      __syncthreads();
      const int last = last_attended(p.kv_mask + b * p.sm_b, n);
      if (last >= 0) atomicMax(&s_last, last);
      __syncthreads();
      return s_last + 1;
    }
  }();

  const uint16_t* Qp = static_cast<const uint16_t*>(p.q) + b * p.sq_b + h * p.sq_h;
  uint16_t* Op = static_cast<uint16_t*>(p.o) + b * p.so_b + h * p.so_h;

  float kscale = 1.f, vscale = 1.f;
  if (FP8) {
    kscale = p.k_scale[b * p.H + h];
    vscale = p.v_scale[b * p.H + h];
  }
  const float sl2 = p.scale_log2 * kscale;   // scores -> log2 units

  if (L == 0) {
    if (q_ok) {
      for (int d = hh; d < p.D; d += 2) Op[q * p.so_q + d] = 0;
    }
    return;
  }

  // The wave's Q as B operands: k-step s covers d = 16 s + 8 hh + 0..7.
  bf16x8_t qf[2 * DT];
#pragma unroll
  for (int s = 0; s < 2 * DT; ++s) {
    const int d0 = 16 * s + 8 * hh;
    uint4 raw = make_uint4(0u, 0u, 0u, 0u);
    if (q_ok && d0 < p.D) raw = *reinterpret_cast<const uint4*>(Qp + q * p.sq_q + d0);
    qf[s] = __builtin_bit_cast(bf16x8_t, raw);
  }

  using T = typename Elem<FP8>::T;
  const T* K = static_cast<const T*>(p.k) + (p.cu_seqlens ? 0 : b * p.sk_b) + h * p.sk_h + off * p.sk_k;
  const T* V = static_cast<const T*>(p.v) + (p.cu_seqlens ? 0 : b * p.sv_b) + h * p.sv_h + off * p.sv_k;
  const int dchunks = static_cast<int>(p.D / 8);
  const int Dv = static_cast<int>(p.D);
  // V^T rows allow vector loads when every 8-key run starts aligned (the base, the row stride and the offset).
  const bool vt_vec = VT && ((reinterpret_cast<uintptr_t>(V) & (FP8 ? 7 : 15)) == 0) && (p.sv_d % 8 == 0);
  const int nfull = L / kKB;           // full key blocks
  const bool tail = nfull * kKB < L;   // plus one partial block

  DirectLanes<DT> dl;
  if constexpr (DIRECT) {
    dl = direct_lanes<DT>(p, reinterpret_cast<const uint16_t*>(K), reinterpret_cast<const uint16_t*>(V), dchunks, nfull,
                      w);
    if (STAGING == kDirect && dchunks < 4 * DT) {
      // Chunks past head_dim of the K tiles that the score product reads are never loaded by direct loads; they
      // must hold zeros.
      for (int i = threadIdx.x; i < kSubTiles * kKB * 8; i += kThreads) {
        const int u = i / (kKB * 8), R = (i >> 3) % kKB, c = i & 7;
        if (8 * u + c >= dchunks) {
          const int e = u * kKTile + R * kRow + swz(R, c) * 8;
          *reinterpret_cast<uint4*>(sK0 + e) = make_uint4(0u, 0u, 0u, 0u);
          *reinterpret_cast<uint4*>(sK1 + e) = make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
    if constexpr (VROWS) {
      // Direct loads never write the chunks of V rows past head_dim: zeros, and with ONES the ones column D.
      if (dchunks < 8 * kSubTiles) {
        for (int i = threadIdx.x; i < kSubTiles * kKB * 8; i += kThreads) {
          const int u = i / (kKB * 8), R = (i >> 3) % kKB, c = i & 7;
          if (8 * u + c >= dchunks) {
            const int e = u * kKTile + R * kRow + swzv(R, c) * 8;
            const uint4 x = (ONES && 8 * u + c == dchunks) ? raw_one_first<false>() : make_uint4(0u, 0u, 0u, 0u);
            *reinterpret_cast<uint4*>(sV0 + e) = x;
            *reinterpret_cast<uint4*>(sV1 + e) = x;
          }
        }
      }
    } else if (ONES && threadIdx.x < 16) {
      // Direct loads never write V^T rows >= D: row D of both buffers holds ones for the whole kernel.
      const int R = static_cast<int>(p.D), c = threadIdx.x & 7;
      uint16_t* buf = threadIdx.x < 8 ? sV0 : sV1;
      *reinterpret_cast<uint4*>(buf + R * kRow + swz(R, c) * 8) = raw_one<false>();
    }
  }
  [[maybe_unused]] DirectRows<DT> dr;
  if constexpr (DIRECT && VROWS) {
    dr = direct_rows<DT>(p, reinterpret_cast<const uint16_t*>(V), dchunks, nfull, w);
  }

  [[maybe_unused]] DirectV8<DT> dv;
  if constexpr (VD8) {
    dv = direct_v8<DT>(p, reinterpret_cast<const uint8_t*>(V), nfull, w);
    // V^T rows D .. 32 DT - 1 of both tiles, which direct loads never write: zeros (row D ones with ONES).
    for (int i = threadIdx.x; i < (32 * DT - Dv) * 4; i += kThreads) {
      const int R = Dv + (i >> 2), c = i & 3;
      const uint32_t x = (ONES && R == Dv) ? 0x38383838u : 0u;  // e4m3 1.0
      *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(sV0) + R * kRow8 + c * 16) = make_uint4(x, x, x, x);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(sV1) + R * kRow8 + c * 16) = make_uint4(x, x, x, x);
    }
  }

  // Operand reads: lane (col, hh) takes logical chunk 2 s + hh of rows col and 32 + col of a tile; the two rows
  // share the swizzle, so four byte offsets serve K and V^T of both buffers.
  uint32_t rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) rd[s] = static_cast<uint32_t>(col * kRow * 2 + swz(col, 2 * s + hh) * 16);
  // PV8: lane (col, hh) reads keys 32 hh .. 32 hh + 31 of e4m3 V^T row 32 j + col, logical chunks 2 hh and
  // 2 hh + 1 (the swizzle depends on col only).
  [[maybe_unused]] uint32_t rdv[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) rdv[s] = static_cast<uint32_t>(col * kRow8 + swz8(col, 2 * hh + s) * 16);
  // VROWS: byte offsets of the transposed reads of output tile j (head_dim 32 j .. 32 j + 31). Within each 16-lane
  // group a ds_read_b64_tr_b16 gives lane i element i % 4 of the 8-byte reads of lanes 4 n + i / 4 (n = 0..3), so
  // lane L reads key 8 (L / 32) + (L % 16) / 4 of the k-step, head_dim 16 ((L / 16) % 2) + 4 (L % 4) .. + 3: lane
  // l then holds keys 8 (l / 32) + 0..3 of column l % 32 (and + 4..7 from the read 4 rows further), the A operand
  // of the second product. The swizzle of those rows depends on the lane only.
  [[maybe_unused]] uint32_t rvt[DT];
  if constexpr (VROWS) {
    const int row_lane = 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int flip = (row_lane >> 1) & 1;
    const int c_lane = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
#pragma unroll
    for (int j = 0; j < DT; ++j) {
      rvt[j] = static_cast<uint32_t>(((j >> 1) * kKTile + row_lane * kRow) * 2 + 16 * (4 * ((j & 1) ^ flip) + c_lane) +
                                     8 * (lane & 1));
    }
  }
  // 16-wide k-steps of the score product that head_dim reaches (2 DT at head_dim 32 DT).
  const int ksteps = FULLK ? 2 * DT : __builtin_amdgcn_readfirstlane(static_cast<int>((p.D + 15) / 16));

  // PV8 at head_dim 32 DT: the row sums of the packed P (rowsum) from v_mfma_f32_16x16x128_f8f6f4 with a ones
  // pattern as A (ones16). Read as a 16x16x128 B operand, lane l of the packed P is column l % 16, k group l / 16:
  // groups 0 and 2 hold query l % 16's 64 keys, groups 1 and 3 query 16 + l % 16's. A row 0 of ones over groups 0
  // and 2 (lanes 0 and 32) and row 4 over groups 1 and 3 (lanes 20 and 52) put query c's sum in entry 0 of lane c
  // (the C rows of lane l are 4 (l / 16) + i): lane-local, so a raise rescales it like O.
  [[maybe_unused]] f32x4_t rowsum = {0.f, 0.f, 0.f, 0.f};
  // PV8: the E8M0 scale 127 (1.0) of the A operands, in a register (a constant scale operand would be encoded as a
  // float inline constant).
  [[maybe_unused]] int unit_scale = 0;
  if constexpr (PV8) asm volatile("v_mov_b32 %0, 0x7f" : "=v"(unit_scale));
  [[maybe_unused]] i32x8_t ones16;
  if constexpr (PV8 && !ONES) {
    const int x = (lane == 0 || lane == 32 || lane == 20 || lane == 52) ? 0x38383838 : 0;  // e4m3 1.0
    ones16 = i32x8_t{x, x, x, x, x, x, x, x};
  }
  // bf16 P at head_dim 32 DT (MSUM): the half's row sums from two v_mfma_f32_16x16x32_bf16 over the packed P with
  // the same ones pattern in bf16 (a 16x16x32 B operand reads lane l of P as column l % 16, k group l / 16, as
  // above), so query c's sum is entry 0 of lane c and the VALU adds no P.
  [[maybe_unused]] bf16x8_t onesb;
  if constexpr (MSUM) {
    const bool one = lane == 0 || lane == 32 || lane == 20 || lane == 52;
#pragma unroll
    for (int i = 0; i < 8; ++i) onesb[i] = one ? static_cast<__bf16>(1.0f) : static_cast<__bf16>(0.0f);
  }
  f32x16_t o[DT];  // O^T tiles: d in [32 j, 32 j + 32)
#pragma unroll
  for (int j = 0; j < DT; ++j) o[j] = f32x16_t{0};
  float m = -INFINITY;          // stored running max (log2 units), shared by O and l
  float l = 0.f;                // MSUM: query c's row sum in lane c (lanes 32-63 hold 0)
  bool first = true;            // uniform: the window's first half always takes the max
  // KMASK: the lane's query has seen no attended key yet (m is then a placeholder 0, O and l are 0); every half
  // takes the max while any lane of the wave is in that state, so the first half with an attended key sets m to
  // that key's score however far below 0 it lies.
  [[maybe_unused]] bool placeholder = false;

  // Full block `blk` into (sK, sV): issued now, complete at the next vmem wait (direct) or at `stage_commit`
  // (registers, prefetched into `st`).
  Stage<FP8, VT, DT> st;
  auto stage_issue = [&](int blk, uint16_t* sK, uint16_t* sV) __attribute__((always_inline)) {
    if constexpr (DIRECT) {
      const int kv0 = blk * kKB;
      stage_direct<DT, STAGING == kDirectFull, VT>(dl, static_cast<uint32_t>(kv0 * p.sk_k * 2),
                                                   static_cast<uint32_t>(kv0 * 2), w, sK, sV);
      if constexpr (VROWS) stage_rows<DT, STAGING == kDirectFull>(dr, static_cast<uint32_t>(kv0 * p.sv_k * 2), w, sV);
    } else {
      stage_load<FP8, VT, DT, false, ONES, !VD8>(st, p, K, V, L, blk * kKB, dchunks, vt_vec);
      if constexpr (VD8) {
#pragma unroll
        for (int t = 0; t < (2 * DT + 3) / 4; ++t) {
          const int j = w + 4 * t;
          if (j < 2 * DT && dv.ok[t]) direct_v8_load(dv.rsrc, dv.off[t], static_cast<uint32_t>(blk * kKB), sV, j);
        }
      }
    }
  };
  auto stage_commit = [&](uint16_t* sK, uint16_t* sV) __attribute__((always_inline)) {
    if constexpr (!DIRECT) stage_store<FP8, VT, DT, ONES, PV8, !VD8>(st, sK, sV, dchunks, Dv);
  };
  // The partial block, synchronously through registers.
  auto stage_tail = [&](uint16_t* sK, uint16_t* sV) __attribute__((always_inline)) {
    Stage<FP8, VT, DT> tmp;
    stage_load<FP8, VT, DT, true, ONES>(tmp, p, K, V, L, nfull * kKB, dchunks, vt_vec);
    stage_store<FP8, VT, DT, ONES, PV8>(tmp, sK, sV, dchunks, Dv);
  };


  // The key mask of the block starting at kv0 as 64 bits (bit i: key kv0 + i is attended), wave-uniform. The
  // blocks are computed in order, so each call takes the byte the previous one fetched (lane l: key kv0 + l) and
  // fetches the next block's: its load completes under the block's compute instead of stalling the next block.
  const uint8_t* mrow = KMASK ? p.kv_mask + b * p.sm_b : nullptr;
  [[maybe_unused]] int mask_on = 0;
  auto mask_fetch = [&](int kv0) __attribute__((always_inline)) {
    if constexpr (KMASK) {
      const int j = kv0 + lane;
      mask_on = (j < L && mrow[j] != 0) ? 1 : 0;
    }
  };
  mask_fetch(0);
  auto block_bits = [&](int kv0) __attribute__((always_inline)) -> uint64_t {
    if constexpr (KMASK) {
      const uint64_t bits = __builtin_amdgcn_ballot_w64(mask_on != 0);
      mask_fetch(kv0 + kKB);
      return bits;
    } else {
      return ~0ull;
    }
  };

  // One key block from (Ks, Vt), as two 32-key halves that each run the whole online-softmax step (scores,
  // running max, exponentials, second product): a half's scores take 16 registers, which keeps four waves per
  // SIMD resident. MASKED: the partial block (keys >= L masked out).
  // PV8: the fp8 products write O^T over 16 passes, the final rows last, and this toolchain (ROCm 7.2 hipcc)
  // places too few wait states between them and the first VALU reads of O (the rows written last were read stale
  // on the GPU, in windows whose last block is the partial one). Every VALU read of O waits here explicitly first:
  // after the window's last block, and before the rescale of a raise (between blocks the next block's score
  // products and exponentials usually come first, but that distance is the compiler's choice). 64 wait states; the
  // asm takes O as an operand so that no read of it moves above the wait.
  auto settle = [&]() __attribute__((always_inline)) {
#define SVHIP_WAIT64 "s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
    if constexpr (PV8 && DT == 2) {
      asm volatile(SVHIP_WAIT64 : "+v"(o[0]), "+v"(o[1]), "+v"(rowsum));
    } else if constexpr (PV8 && DT == 3) {
      asm volatile(SVHIP_WAIT64 : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(rowsum));
    } else if constexpr (PV8) {
      static_assert(DT == 4, "head widths are 2, 3 or 4 tiles");
      asm volatile(SVHIP_WAIT64 : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]), "+v"(rowsum));
    }
#undef SVHIP_WAIT64
  };

  // PV8, the softmax of half t of a block, packed as it is formed: P = exp2(fma(S, sl2, 4 - m)), the running max
  // lifted by 2^4 so that P of scores from 2^-10 of the max upwards keeps a normal e4m3 value, straight into the
  // e4m3 B operand (v_cvt_pk_fp8_f32, round to nearest even). The lazy max with an e4m3 bound: a half whose largest
  // score passes m by more than 4.8 (P above 2^8.8 < 448) takes the slow path first, so every packed P is in range.
  // The row sum never comes from the VALU: the ones row D of V^T, or (head_dim 32 DT) a 16x16x128 product of the
  // packed P with a ones pattern (rowsum). The running max is kept an integer, so that a raise in half 1 takes
  // half 0, already packed, down by an exact power of two through the second product's E8M0 scales: `drop` counts
  // the halvings (see the second product); the row sum takes the same difference in fp32.
  auto half_pv8 = [&](int t, f32x16_t& s, uint32_t(&pf)[8], int& drop) __attribute__((always_inline)) {
    auto exps8 = [&]() __attribute__((always_inline)) {
      const float nm = kPv8Lift - m;
#pragma unroll
      for (int j = 0; j < 16; j += 4) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], sl2, nm));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j + 1], sl2, nm));
        const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j + 2], sl2, nm));
        const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j + 3], sl2, nm));
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(p0, p1, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(p2, p3, w, true);
        pf[4 * t + j / 4] = static_cast<uint32_t>(w);
      }
    };
    auto raise8 = [&](float mx) __attribute__((always_inline)) {
      settle();
      first = false;
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(mx), __float_as_int(mx), false, false);
      const float mr = __builtin_amdgcn_fmed3f(__int_as_float(sw[0]), __int_as_float(sw[1]), kFltMax);
      const float cand = __builtin_ceilf(mr * sl2);
      const float mn = cand > m ? cand : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first half, else an exact power of two
      if (t == 1) {
        const float rise = mn - m;  // m is finite after the window's first half
        drop += rise < 256.f ? static_cast<int>(rise) : 256;
      }
      m = mn;
      rowsum[0] *= alpha;
      if constexpr (!ONES) {
        if (t == 1) {
          // The row-sum product takes half 0 unscaled (its E8M0 scale blocks mix queries c and c + 16): take the
          // difference off here, the pair's half-0 sum decoded from the packed bytes.
          float h0 = 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(pf[q]), false);
            const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(pf[q]), true);
            h0 += (lo[0] + lo[1]) + (hi[0] + hi[1]);
          }
          const auto hs = __builtin_amdgcn_permlane32_swap(__float_as_int(h0), __float_as_int(h0), false, false);
          rowsum[0] -= (__int_as_float(hs[0]) + __int_as_float(hs[1])) * (1.f - alpha);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
#pragma unroll
        for (int j = 0; j < DT; ++j) o[j][i] *= alpha;
      }
      exps8();
    };
    float mx = __builtin_amdgcn_fmed3f(s[0], s[1], kFltMax);
#pragma unroll
    for (int i = 2; i < 16; i += 2) mx = max3(mx, s[i], s[i + 1]);
    exps8();
    if (first || __builtin_amdgcn_ballot_w64(__builtin_fmaf(mx, sl2, -m) > kPv8MaxHigh) != 0ull) raise8(mx);
  };

  SVHIP_TRACE(WaveTrace trace;)
  SVHIP_TRACE(trace.begin(!FP8 && !KMASK && STAGING == kDirectFull, w, lane, b, h, qt, nfull);)
  // bits: the block's key mask (block_bits, all ones without one), taken by the caller before it issues the next
  // block's loads.
  auto compute = [&](auto masked, const uint16_t* Ks, const uint16_t* Vt, int kv0, uint64_t bits)
      __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked)::value;
    SVHIP_TRACE(trace.block(MASKED ? -1 : kv0 / kKB);)
    const char* kp = reinterpret_cast<const char*>(Ks);
    const char* vp = reinterpret_cast<const char*>(Vt);
    // A key mask that masks every key of the block: the block adds nothing to O, l or m (its P are all 0), so it
    // is skipped (wave-uniform; the block's barrier is outside). Not in the register-staged V^T form, which has no
    // registers to spare for it.
    if (KMASK && (DIRECT || VROWS) && bits == 0ull) return;
    [[maybe_unused]] uint32_t pf[8];  // PV8: e4m3 P, bytes 16 t + i
    [[maybe_unused]] int drop = 0;    // PV8: halvings of half 0 since it was packed
    // S^T of keys 32 t .. 32 t + 31 of the block (LDS rows 32 t + col), keys past L (and, with a key mask, keys
    // not attended) at -inf; k-steps past head_dim (zero in Q) are skipped.
    // LEAN: one K operand in registers at a time (the rare path, where registers are short).
    auto score = [&](int t, auto lean) __attribute__((always_inline)) -> f32x16_t {
      constexpr bool LEAN = decltype(lean)::value;
      f32x16_t s;
      if constexpr (FULLK && !LEAN) {
        bf16x8_t a[2 * DT];
#pragma unroll
        for (int k = 0; k < 2 * DT; ++k) {
          a[k] = *reinterpret_cast<const bf16x8_t*>(kp + (k >> 2) * (kKTile * 2) + rd[k & 3] + t * (32 * kRow * 2));
        }
#pragma unroll
        for (int k = 0; k < 2 * DT; ++k) {
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k], qf[k], k == 0 ? f32x16_t{0} : s, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 2 * DT; ++k) {
          if (k == 0 || k < ksteps) {
            const bf16x8_t a =
                *reinterpret_cast<const bf16x8_t*>(kp + (k >> 2) * (kKTile * 2) + rd[k & 3] + t * (32 * kRow * 2));
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[k], k == 0 ? f32x16_t{0} : s, 0, 0, 0);
          }
        }
      }
      // A key mask that attends every key of a full block changes none of its scores: no masking then (except in
      // the register-staged V^T form, short of registers, which always masks).
      if (MASKED || (KMASK && (!(DIRECT || VROWS) || bits != ~0ull))) {
        // Entry i is key 32 t + (i < 8 ? 8 hh + i : 16 + 8 hh + i - 8) (PV8: 32 hh + 16 t + i); with a key mask,
        // bit i of `mine`.
        const uint32_t hb = static_cast<uint32_t>(bits >> (32 * t));
        const uint32_t mine = ((hb >> (8 * hh)) & 0xffu) | (((hb >> (16 + 8 * hh)) & 0xffu) << 8);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kin = PV8 ? 32 * hh + 16 * t + i : 32 * t + ((i < 8) ? (8 * hh + i) : (16 + 8 * hh + (i - 8)));
          if (MASKED && kv0 + kin >= L) s[i] = -INFINITY;
          if (KMASK && !((mine >> i) & 1u)) s[i] = -INFINITY;
        }
      }
      return s;
    };
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      SVHIP_TRACE(trace.mark(5 * t);)
      f32x16_t s = score(t, std::false_type{});
      if constexpr (PV8) {
        half_pv8(t, s, pf, drop);
        continue;
      }
      // P^T = exp2(sl2 S^T - m) against the running max m as it stands, as B operands: k-step ks (keys
      // 32 t + 16 ks + 8 hh + 0..7) = entries 8 ks + 0..7. On the window's first half m is -inf and the fast pass
      // gives inf or NaN, which the slow path always taken there replaces.
      // The row sum is taken over the packed (bf16-rounded) P that the second product reads, so a dominant key's
      // rounding cancels in O / l.
      bf16x8_t pb[2];
      [[maybe_unused]] float late;  // SPEC: the half's row sum, read after the second product is issued
      auto exps = [&]() __attribute__((always_inline)) {
        const float nm = -m;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            f32x2_t two = {__builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * ks + j], sl2, nm)),
                           __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * ks + j + 1], sl2, nm))};
            if constexpr (SPEC) {  // folded into the exponentials as their clamp modifier
              two[0] = __builtin_amdgcn_fmed3f(two[0], 0.f, 1.f);
              two[1] = __builtin_amdgcn_fmed3f(two[1], 0.f, 1.f);
            }
            const bf16x2_t c = __builtin_convertvector(two, bf16x2_t);
            pb[ks][j] = c[0];
            pb[ks][j + 1] = c[1];
          }
        }
      };
      // Without the ones row (MSUM): the half's row sums over the packed P from the matrix cores (query c's in
      // lane c, 0 in lanes 32-63); the VALU adds no P.
      [[maybe_unused]] auto half_sum = [&]() __attribute__((always_inline)) {
        f32x4_t h = __builtin_amdgcn_mfma_f32_16x16x32_bf16(onesb, pb[0], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        h = __builtin_amdgcn_mfma_f32_16x16x32_bf16(onesb, pb[1], h, 0, 0, 0);
        return h[0];
      };
      // The slow path: the half's max (raw scores; the chain opens with a compiler-visible v_med3_f32, med3(a, b,
      // FLT_MAX) = max(a, b) for scores below +inf, before which the compiler inserts the wait states a VALU read
      // of an MFMA result needs; the inline v_max3_f32 that follow, which the compiler does not check for that
      // hazard, read the same, by then complete, accumulator) joined with the partner lane's over
      // v_permlane32_swap, which gives (x[l % 32], x[l % 32 + 32]) in every lane, scaled to log2 units; m raised to
      // it, O and l rescaled, P redone against the new m. Every query has a key below L in the first half, so m is
      // finite after it.
      auto rebase = [&](float mx) __attribute__((always_inline)) {
        first = false;
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(mx), __float_as_int(mx), false, false);
        const float mr = __builtin_amdgcn_fmed3f(__int_as_float(sw[0]), __int_as_float(sw[1]), kFltMax);
        const float cand = SPEC ? __builtin_fmaf(mr, sl2, kSpecBias) : mr * sl2;
        float mn = (cand > m || (KMASK && placeholder)) ? cand : m;
        // Only with a key mask can a query have seen no attended key yet (every score -inf): its running max is
        // then set to 0, with O and l still 0, so that later scores are taken against a finite bias, and the lane is
        // marked so that its first attended key replaces that bias (alpha 0: O and l hold nothing to rescale).
        bool was_placeholder = false;
        if (KMASK) {
          was_placeholder = placeholder;
          placeholder = mn == -INFINITY;
          mn = placeholder ? 0.f : mn;
        }
        const float alpha = was_placeholder ? 0.f : __builtin_amdgcn_exp2f(m - mn);  // 0 on the first half
        m = mn;
        l *= alpha;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
#pragma unroll
          for (int j = 0; j < DT; ++j) o[j][i] *= alpha;
        }
      };
      auto raise = [&](float mx) __attribute__((always_inline)) {
        rebase(mx);
        exps();
      };
      auto half_max = [&](const f32x16_t& x) __attribute__((always_inline)) {
        float mx = __builtin_amdgcn_fmed3f(x[0], x[1], kFltMax);
#pragma unroll
        for (int i = 2; i < 16; i += 2) mx = max3(mx, x[i], x[i + 1]);
        return mx;
      };
      // O^T += V^T . P^T: for k-step ks, V^T columns 32 t + 16 ks + 8 hh + 0..7 are logical chunk 2 (2 t + ks) + hh
      // of rows 32 j + col.
      auto pv = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          bf16x8_t a[DT];
#pragma unroll
          for (int j = 0; j < DT; ++j) {
            if constexpr (VROWS) {
              typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
              typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;
              char* b = const_cast<char*>(vp) + rvt[j] + (32 * t + 16 * ks) * kRow * 2;
              const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(b));
              const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(b + 4 * kRow * 2));
              a[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            } else {
              a[j] = *reinterpret_cast<const bf16x8_t*>(vp + rd[2 * t + ks] + j * (32 * kRow * 2));
            }
          }
#pragma unroll
          for (int j = 0; j < DT; ++j) o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], pb[ks], o[j], 0, 0, 0);
        }
      };
      if constexpr (ONES) {
        // The half's own max decides: a score more than kMaxHigh above m raises it (P of the fast path stays
        // below 2^kMaxHigh); the row sum accumulates in O^T row D.
        const float mx = half_max(s);
        exps();
        if (first || __builtin_amdgcn_ballot_w64(__builtin_fmaf(mx, sl2, -m) > kMaxHigh || (KMASK && placeholder)) !=
                         0ull) {
          raise(mx);
        }
      } else if constexpr (SPEC) {
        // The second product does not wait for the row sum: P is formed against m as it stands (on the window's
        // first half, where m is -inf, against the half's own max), the row sum is issued, then the second
        // product, and the sum is read back after it (below), when the matrix core has long produced it.
        if (first) rebase(half_max(s));
        SVHIP_TRACE(trace.mark_after(5 * t + 1, __builtin_amdgcn_fmed3f(s[15], s[14], kFltMax));)
        exps();
        SVHIP_TRACE(trace.mark_after(5 * t + 2, __builtin_bit_cast(float, __builtin_bit_cast(uint4, pb[1]).w));)
        late = half_sum();
        __builtin_amdgcn_sched_barrier(0);  // the row sum's products go to the matrix core before the second's
      } else if constexpr (MSUM) {
        // The half's sum shows whether m still bounds its scores: above kSumHigh = 2^20 (or inf / NaN) some
        // score passed m by about 20 (log2 units). Only then (and on the window's first half, where m is -inf)
        // is the slow path taken.
        SVHIP_TRACE(trace.mark_after(5 * t + 1, __builtin_amdgcn_fmed3f(s[15], s[14], kFltMax));)
        exps();
        SVHIP_TRACE(trace.mark_after(5 * t + 2, __builtin_bit_cast(float, __builtin_bit_cast(uint4, pb[1]).w));)
        float hs = half_sum();
        SVHIP_TRACE(trace.mark_after(5 * t + 3, __builtin_amdgcn_fmed3f(hs, hs, kFltMax));)
        if (first || __builtin_amdgcn_ballot_w64(!(hs <= kSumHigh) || (KMASK && placeholder)) != 0ull) {
          raise(half_max(s));
          hs = half_sum();
        }
        l += hs;
      }
      pv();
      if constexpr (SPEC) {
        // A row sum above kSpecHigh: some score passed m by about 19 or more (log2 units), and the P of the scores
        // more than 20 above it were clamped. The half is taken back out of O (the second product again with -P;
        // l has not taken its sum), m is raised to the half's max, O and l rescaled, and the half done again; the
        // scores and P are formed again from the tile rather than held through the product. Rare: m is then within 20
        // of every score to come up to the next raise. With a key mask a query that has seen no attended key yet
        // (m a placeholder) takes this path too, as it takes the raise in the other forms.
        SVHIP_TRACE(trace.mark_after(5 * t + 3, __builtin_amdgcn_fmed3f(late, late, kFltMax));)
        if (__builtin_amdgcn_ballot_w64(!(late <= kSpecHigh) || (KMASK && placeholder)) != 0ull) {
          s = score(t, std::true_type{});
          exps();  // the same P again (the same products and m), negated
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const uint4 x = __builtin_bit_cast(uint4, pb[ks]);
            pb[ks] = __builtin_bit_cast(bf16x8_t, make_uint4(x.x ^ 0x80008000u, x.y ^ 0x80008000u, x.z ^ 0x80008000u,
                                                              x.w ^ 0x80008000u));
          }
          pv();
          rebase(half_max(s));
          exps();
          late = half_sum();
          pv();
        }
        l += late;
      }
      SVHIP_TRACE(trace.mark_after(5 * t + 4, o[DT - 1][15], l);)
    }
    if constexpr (PV8) {
      // O^T += V^T . P^T over the block's 64 keys on the fp8 matrix cores; A: V^T rows 32 j + col, keys
      // 32 hh + 0..31 (E8M0 scale 127: 1); B: the packed P, half 0 scaled by 2^-drop. The 32x32x64 form takes the
      // scale of bytes 16 b .. 16 b + 15 of column c's two lanes from lane c + 32 b (measured), so lane half 0
      // carries half 0's scale and every block belongs to one query. (The 16x16x128 row sum cannot: there block
      // (l / 32) + 2 (j / 16) of column l % 16 takes the scale of lane l % 16 + 16 block, mixing queries c and
      // c + 16; it runs unscaled, corrected in the raise.)
      const int sb = hh ? 127 : (drop < 127 ? 127 - drop : 0);
      const i32x8_t bp = {static_cast<int>(pf[0]), static_cast<int>(pf[1]), static_cast<int>(pf[2]),
                          static_cast<int>(pf[3]), static_cast<int>(pf[4]), static_cast<int>(pf[5]),
                          static_cast<int>(pf[6]), static_cast<int>(pf[7])};
#pragma unroll
      for (int j = 0; j < DT; ++j) {
        const uint4 lo = *reinterpret_cast<const uint4*>(vp + rdv[0] + j * (32 * kRow8));
        const uint4 hi = *reinterpret_cast<const uint4*>(vp + rdv[1] + j * (32 * kRow8));
        const i32x8_t a = {static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                           static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                           static_cast<int>(hi.z), static_cast<int>(hi.w)};
        o[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bp, o[j], 0, 0, 0, unit_scale, 0, sb);
      }
      if constexpr (!ONES) {
        rowsum = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones16, bp, rowsum, 0, 0, 0, 0, 0, 0);
      }
    }
  };
  using Full = std::false_type;
  using Partial = std::true_type;

  // Full block blk from (Ks, Vt) while full block blk + 1 is staged into (nK, nV). With a key mask the block's bits
  // are taken, and the next block's mask bytes fetched, before the next block's loads are issued: the wait for the
  // mask bytes (loaded during the previous block, waited for at its end) then waits for nothing in flight, where
  // after those loads it waited for them all.
  auto full_step = [&](int blk, const uint16_t* Ks, const uint16_t* Vt, uint16_t* nK, uint16_t* nV) __attribute__((always_inline)) {
    const uint64_t bits = block_bits(blk * kKB);
    stage_issue(blk + 1, nK, nV);
    compute(Full{}, Ks, Vt, blk * kKB, bits);
    stage_commit(nK, nV);
    wait_vmem();
    __syncthreads();
    SVHIP_TRACE(trace.block_end(blk, lane);)
  };

  if (nfull > 0) {
    stage_issue(0, sK0, sV0);
    stage_commit(sK0, sV0);
  } else {
    stage_tail(sK0, sV0);
  }
  wait_vmem();
  __syncthreads();
  int blk = 0;
  for (; blk + 2 < nfull; blk += 2) {
    full_step(blk, sK0, sV0, sK1, sV1);
    full_step(blk + 1, sK1, sV1, sK0, sV0);
  }
  if (blk + 1 < nfull) {
    full_step(blk, sK0, sV0, sK1, sV1);
    ++blk;
  }
  // blk is the last full block (or 0 with no full block); its tiles are the ones of its parity.
  {
    const bool odd = blk & 1;
    uint16_t* cK = odd ? sK1 : sK0;
    uint16_t* cV = odd ? sV1 : sV0;
    uint16_t* nK = odd ? sK0 : sK1;
    uint16_t* nV = odd ? sV0 : sV1;
    if (nfull > 0) {
      // The partial block's loads are in flight during the last full block (the other tiles are free since the
      // last barrier).
      const uint64_t bits = block_bits(blk * kKB);
      Stage<FP8, VT, DT> tl;
      if (tail) stage_load<FP8, VT, DT, true, ONES>(tl, p, K, V, L, nfull * kKB, dchunks, vt_vec);
      compute(Full{}, cK, cV, blk * kKB, bits);
      settle();
      if (tail) {
        stage_store<FP8, VT, DT, ONES, PV8>(tl, nK, nV, dchunks, Dv);
        wait_vmem();
        __syncthreads();
        compute(Partial{}, nK, nV, nfull * kKB, block_bits(nfull * kKB));
        settle();
      }
    } else {
      compute(Partial{}, cK, cV, 0, block_bits(0));
      settle();
    }
  }

  float lsum = l;
  if constexpr (ONES) {
    // O^T row D = the row sum, entry 4 (r / 8) of tile D / 32 in the lanes of half 0 (r = D % 32, a multiple of 8).
    const int jd = static_cast<int>(p.D) / 32, gd = (static_cast<int>(p.D) % 32) / 8;
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < DT; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (j == jd && g == gd) v = o[j][4 * g];
      }
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    lsum = __int_as_float(sw[0]);
  } else if constexpr (PV8) {
    // Query c's sum is entry 0 of lane c (lane half 0).
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(rowsum[0]), __float_as_int(rowsum[0]), false,
                                                     false);
    lsum = __int_as_float(sw[0]);
  } else {
    static_assert(MSUM, "the row sum comes from the ones row, the fp8 ones pattern or the bf16 one");
    // Query c's sum is l of lane c (lane half 0; half 1 holds 0).
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(lsum), __float_as_int(lsum), false, false);
    lsum = __int_as_float(sw[0]);
  }
  SVHIP_TRACE(trace.end(lane, lsum);)
  // A query with no attended key (only possible with a key mask) has l = 0 and O = 0: it gets zeros.
  const float inv = (KMASK && !(lsum > 0.f)) ? 0.f : vscale / lsum;
  if (q_ok) {
    // O^T entry i of tile t: d = 32 t + 8 (i / 4) + 4 hh + i % 4 ; four consecutive d per group.
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * t + 8 * g4 + 4 * hh;
        if (d0 < p.D) {
          float vals[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) vals[e] = o[t][4 * g4 + e] * inv;
          f32x2_t a = {vals[0], vals[1]}, c = {vals[2], vals[3]};
          const bf16x2_t ba = __builtin_convertvector(a, bf16x2_t);
          const bf16x2_t bc = __builtin_convertvector(c, bf16x2_t);
          uint2 packed;
          packed.x = __builtin_bit_cast(uint32_t, ba);
          packed.y = __builtin_bit_cast(uint32_t, bc);
          *reinterpret_cast<uint2*>(Op + q * p.so_q + d0) = packed;
        }
      }
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// The instantiation for DT = head_dim / 32 rounded up: bf16 K and V directly to LDS (V^T of the padded layout,
// V rows of either layout; head_dim 32 DT without exec masking), with or without a key mask; e4m3, V^T of the
// packed layout and K/V spans past 32-bit offsets through registers.
template <int DT, bool ONES>
void launch_dt(const XattnParams& p, unsigned g, hipStream_t s, bool fp8, bool pv8, bool vt, bool direct) {
  constexpr int RS = ONES ? kRegister : kRegisterFull;
  if (p.kv_mask) {  // bf16 only (checked by the entry point)
    constexpr int DS = ONES ? kDirect : kDirectFull;
    if (direct && vt) {
      xattn_fwd_kernel<false, true, DS, DT, ONES, true><<<g, kThreads, 0, s>>>(p);
    } else if (direct) {
      xattn_fwd_kernel<false, false, DS, DT, ONES, true><<<g, kThreads, 0, s>>>(p);
    } else if (vt) {
      xattn_fwd_kernel<false, true, RS, DT, ONES, true><<<g, kThreads, 0, s>>>(p);
    } else {
      xattn_fwd_kernel<false, false, RS, DT, ONES, true><<<g, kThreads, 0, s>>>(p);
    }
    return;
  }
  if (fp8 && pv8) {
    if (vt && direct) {
      xattn_fwd_kernel<true, true, RS, DT, ONES, false, true, true><<<g, kThreads, 0, s>>>(p);
    } else if (vt) {
      xattn_fwd_kernel<true, true, RS, DT, ONES, false, true><<<g, kThreads, 0, s>>>(p);
    } else {
      xattn_fwd_kernel<true, false, RS, DT, ONES, false, true><<<g, kThreads, 0, s>>>(p);
    }
  } else if (fp8) {
    if (vt) {
      xattn_fwd_kernel<true, true, RS, DT, ONES, false, false><<<g, kThreads, 0, s>>>(p);
    } else {
      xattn_fwd_kernel<true, false, RS, DT, ONES, false, false><<<g, kThreads, 0, s>>>(p);
    }
  } else if (direct && !ONES) {
    if (vt) {
      xattn_fwd_kernel<false, true, kDirectFull, DT, false><<<g, kThreads, 0, s>>>(p);
    } else {
      xattn_fwd_kernel<false, false, kDirectFull, DT, false><<<g, kThreads, 0, s>>>(p);
    }
  } else if (direct) {
    if (vt) {
      xattn_fwd_kernel<false, true, kDirect, DT, true><<<g, kThreads, 0, s>>>(p);
    } else {
      xattn_fwd_kernel<false, false, kDirect, DT, true><<<g, kThreads, 0, s>>>(p);
    }
  } else if (vt) {
    xattn_fwd_kernel<false, true, RS, DT, ONES><<<g, kThreads, 0, s>>>(p);
  } else {
    xattn_fwd_kernel<false, false, RS, DT, ONES><<<g, kThreads, 0, s>>>(p);
  }
}

// The instantiation for DT = head_dim / 32 rounded up (see launch_dt); head_dim below 32 DT takes the row sum from
// the matrix cores.
template <int DT>
void launch(const XattnParams& p, unsigned g, hipStream_t s, bool fp8, bool pv8, bool vt, bool direct) {
  if (p.D < 32 * DT) {
    launch_dt<DT, true>(p, g, s, fp8, pv8, vt, direct);
  } else {
    launch_dt<DT, false>(p, g, s, fp8, pv8, vt, direct);
  }
}

static int xattn_impl(const void* q, const void* k, const void* v, void* o, int kv_dtype, const int32_t* kv_len,
                      const int32_t* cu_seqlens, const float* k_scale, const float* v_scale, const uint8_t* kv_mask,
                      int64_t sm_b, int64_t B, int64_t H, int64_t Q, int64_t D, int64_t kv_cap, int64_t sq_b,
                      int64_t sq_h, int64_t sq_q, int64_t sk_b, int64_t sk_h, int64_t sk_k, int64_t sv_b,
                      int64_t sv_h, int64_t sv_k, int64_t sv_d, int64_t so_b, int64_t so_h, int64_t so_q,
                      float scale, void* stream, const char* name) {
  SVHIP_REQUIRE(q && k && v && o, "%s: null pointer", name);
  SVHIP_REQUIRE(B >= 0 && H >= 1 && Q >= 0, "%s: bad sizes", name);
  SVHIP_REQUIRE(D >= 8 && D <= kMaxD && D % 8 == 0, "%s: head_dim %lld unsupported (multiple of 8, <= %d)", name,
                (long long)D, kMaxD);
  SVHIP_REQUIRE(scale > 0.f && scale < 3.0e38f, "%s: softmax scale must be positive and finite", name);
  SVHIP_REQUIRE(kv_dtype == SVHIP_BF16 || kv_dtype == SVHIP_FP8_E4M3 || kv_dtype == SVHIP_FP8_E4M3_PFP8,
                "%s: kv dtype %d unsupported", name, kv_dtype);
  const bool fp8 = kv_dtype != SVHIP_BF16;
  const bool pv8 = kv_dtype == SVHIP_FP8_E4M3_PFP8;
  SVHIP_REQUIRE(!fp8 || (k_scale && v_scale), "%s: fp8 K/V need k_scale and v_scale", name);
  SVHIP_REQUIRE(!kv_mask || !fp8, "%s: the key mask takes bf16 K/V", name);
  SVHIP_REQUIRE(sv_k == 1 || sv_d == 1, "%s: V needs a unit stride along keys or head_dim", name);
  const bool vt = sv_k == 1 && sv_d != 1;
  const size_t eb = fp8 ? 1 : 2;
  // Row starts must allow 16-byte (bf16) / 8-byte (fp8) vector loads.
  const uintptr_t align = fp8 ? 8 : 16;
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && (sq_q * 2) % 16 == 0 && (sq_h * 2) % 16 == 0 &&
                    (sq_b * 2) % 16 == 0,
                "%s: Q rows must be 16-byte aligned", name);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(o) % 8 == 0 && (so_q * 2) % 8 == 0 && (so_h * 2) % 8 == 0 &&
                    (so_b * 2) % 8 == 0,
                "%s: O rows must be 8-byte aligned", name);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(k) % align == 0 && (sk_k * eb) % align == 0 &&
                    (sk_h * eb) % align == 0 && (sk_b * eb) % align == 0,
                "%s: K rows must be %d-byte aligned", name, (int)align);
  if (!vt) {
    SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(v) % align == 0 && (sv_k * eb) % align == 0 &&
                      (sv_h * eb) % align == 0 && (sv_b * eb) % align == 0,
                  "%s: V rows must be %d-byte aligned", name, (int)align);
  }
  if (B == 0 || Q == 0) return SVHIP_OK;
  SVHIP_REQUIRE(kv_cap >= 0 && kv_cap < (1ll << 31), "%s: kv_cap out of range", name);
  XattnParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.kv_len = kv_len;
  p.cu_seqlens = cu_seqlens;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.kv_mask = kv_mask;
  p.sm_b = sm_b;
  p.B = B;
  p.H = H;
  p.Q = Q;
  p.D = D;
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
  p.q_tiles = static_cast<int>(cdiv(Q, kQTile));
  const int64_t grid = static_cast<int64_t>(p.q_tiles) * H * B;
  SVHIP_REQUIRE(grid < (1ll << 31), "%s: grid too large", name);
  // Direct-to-LDS staging: bf16 K and V whose rows (and every 8-key run of V^T) start on 16-byte boundaries and
  // whose byte offsets from a (window, head) base fit 32 bits: V^T of the padded layout, row-major V of either
  // layout (a packed window starts at any key, which keeps its rows aligned but not the 8-key runs of V^T).
  // e4m3 with the fp8 second product: V^T alone takes direct loads, rows of 16-byte aligned 16-key runs.
  const bool direct =
      fp8 ? (pv8 && vt && !cu_seqlens && reinterpret_cast<uintptr_t>(v) % 16 == 0 && sv_d % 16 == 0 &&
             sv_h % 16 == 0 && sv_b % 16 == 0 && D * sv_d + kv_cap < (1ll << 32))
          : (reinterpret_cast<uintptr_t>(v) % 16 == 0 && sv_h % 8 == 0 && sv_b % 8 == 0 &&
             (kv_cap * sk_k + D) * 2 < (1ll << 32) &&
             (vt ? !cu_seqlens && sv_d % 8 == 0 && (D * sv_d + kv_cap) * 2 < (1ll << 32)
                 : sv_k % 8 == 0 && (kv_cap * sv_k + D) * 2 < (1ll << 32)));
  hipStream_t s = as_stream(stream);
  const unsigned g = static_cast<unsigned>(grid);
  if (D <= 64) {
    launch<2>(p, g, s, fp8, pv8, vt, direct);
  } else if (D <= 96) {
    launch<3>(p, g, s, fp8, pv8, vt, direct);
  } else {
    launch<4>(p, g, s, fp8, pv8, vt, direct);
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

// One workgroup per window: out[b] = 1 + the last attended key among the window's first min(kv_len[b], kv_cap)
// keys (kv_cap without kv_len), 0 when it has none.
__global__ __launch_bounds__(kThreads) void mask_lengths_kernel(const uint8_t* mask, int64_t sm_b,
                                                                const int32_t* kv_len, int64_t kv_cap, int32_t* out) {
  __shared__ int s_last;
  const int64_t b = blockIdx.x;
  int64_t n = kv_cap;
  if (kv_len) n = min(max(static_cast<int64_t>(kv_len[b]), int64_t{0}), kv_cap);
  if (threadIdx.x == 0) s_last = -1;
  __syncthreads();
  const int last = last_attended(mask + b * sm_b, static_cast<int>(n));
  if (last >= 0) atomicMax(&s_last, last);
  __syncthreads();
  if (threadIdx.x == 0) out[b] = s_last + 1;
}

}  // namespace svhip

using namespace svhip;

extern "C" int svhip_mask_lengths(const uint8_t* kv_mask, int64_t sm_b, const int32_t* kv_len, int64_t B,
                                  int64_t kv_cap, int32_t* out, void* stream) {
  const char* name = "svhip_mask_lengths";
  clear_error();
  SVHIP_REQUIRE(kv_mask && out, "%s: null pointer", name);
  SVHIP_REQUIRE(B >= 0 && B < (1ll << 31), "%s: bad window count", name);
  SVHIP_REQUIRE(kv_cap >= 0 && kv_cap < (1ll << 31), "%s: kv_cap out of range", name);
  if (B == 0) return SVHIP_OK;
  mask_lengths_kernel<<<static_cast<unsigned>(B), kThreads, 0, as_stream(stream)>>>(kv_mask, sm_b, kv_len, kv_cap,
                                                                                      out);
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}

#ifdef SVHIP_XATTN_TRACE
// Trace build only: the device buffer the instrumented kernel writes (kTraceWords words per wave), or NULL to stop.
extern "C" int svhip_xattn_trace_set(void* buffer) {
  return hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &buffer, sizeof(buffer)) == hipSuccess ? 0 : -1;
}
#endif

extern "C" int svhip_xattn_fwd(const void* q, const void* k, const void* v, void* o, int kv_dtype,
                               const int32_t* kv_len, const int32_t* cu_seqlens, const float* k_scale,
                               const float* v_scale, int64_t B, int64_t H, int64_t Q, int64_t D, int64_t kv_cap,
                               int64_t sq_b, int64_t sq_h, int64_t sq_q, int64_t sk_b, int64_t sk_h, int64_t sk_k,
                               int64_t sv_b, int64_t sv_h, int64_t sv_k, int64_t sv_d, int64_t so_b, int64_t so_h,
                               int64_t so_q, float scale, void* stream) {
  const char* name = "svhip_xattn_fwd";
  clear_error();
  SVHIP_REQUIRE(kv_len || cu_seqlens, "%s: need kv_len or cu_seqlens", name);
  return xattn_impl(q, k, v, o, kv_dtype, kv_len, cu_seqlens, k_scale, v_scale, nullptr, 0, B, H, Q, D, kv_cap, sq_b,
                    sq_h, sq_q, sk_b, sk_h, sk_k, sv_b, sv_h, sv_k, sv_d, so_b, so_h, so_q, scale, stream, name);
}

extern "C" int svhip_xattn_fwd_masked(const void* q, const void* k, const void* v, void* o, const uint8_t* kv_mask,
                                      int64_t sm_b, const int32_t* kv_len, const int32_t* cu_seqlens, int64_t B,
                                      int64_t H, int64_t Q, int64_t D, int64_t kv_cap, int64_t sq_b, int64_t sq_h,
                                      int64_t sq_q, int64_t sk_b, int64_t sk_h, int64_t sk_k, int64_t sv_b,
                                      int64_t sv_h, int64_t sv_k, int64_t sv_d, int64_t so_b, int64_t so_h,
                                      int64_t so_q, float scale, void* stream) {
  const char* name = "svhip_xattn_fwd_masked";
  clear_error();
  SVHIP_REQUIRE(kv_mask, "%s: null key mask", name);
  SVHIP_REQUIRE(!(kv_len && cu_seqlens), "%s: kv_len and cu_seqlens are exclusive", name);
  return xattn_impl(q, k, v, o, SVHIP_BF16, kv_len, cu_seqlens, nullptr, nullptr, kv_mask, sm_b, B, H, Q, D, kv_cap,
                    sq_b, sq_h, sq_q, sk_b, sk_h, sk_k, sv_b, sv_h, sv_k, sv_d, so_b, so_h, so_q, scale, stream, name);
}
