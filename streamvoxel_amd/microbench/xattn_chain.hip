// The cross-attention kernel's 32-key half (xattn_fwd_kernel at head_dim 64 over a bf16 cache) taken apart on
// gfx950: the same instructions per half with the kernel's dependencies, built up one ingredient at a time, so that
// each ingredient's cost shows at a steady number of waves per SIMD. Registers and LDS only, apart from the staged
// blocks of the last forms (read through a bounded buffer descriptor) and one store per thread.
//
//   products only        4 chained 32x32x16 score products, 2 16x16x32 row-sum products, 4 32x32x16 second products
//   softmax only         16 FMA + 16 exp2 + 8 bf16 packs on a register no product writes
//   chain                scores -> softmax -> row sums + second product, operands in registers
//   + LDS operands       the 4 score and 4 second-product A operands read from LDS every half (ds_read_b128)
//   + barrier, trigger   a workgroup barrier every second half (a 64-key block) and the row-sum ballot
//   + staging            the next block (16 KB a workgroup) loaded straight into LDS during the block, waited for
//                        before the barrier; the 8 workgroups that share a block's data sit on one XCD, as the
//                        kernel places the query tiles of a (window, head)
//   64 queries a wave    the last form with two query tiles a wave: every LDS operand read feeds two products
//   priority 1 / 2       the staged form with the wave's issue priority raised (s_setprio 1) while it issues its
//                        score products (1), or its score and second products (2), and lowered for its softmax
//   two halves at once   the staged form with a block's two halves in one stretch of code: half 1's score product
//                        issued before half 0's softmax, half 0's row sum and second product before half 1's
//                        softmax (the compiler's order), so a wave's own products run beside its own softmax;
//                        "+ rare rescales" adds the two row-sum checks as branches that rescale O (never taken)
//
// Build: python -m streamvoxel_amd.build --microbench   Run: streamvoxel_amd/microbench/xattn_chain
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);               \
      exit(1);                                                                            \
    }                                                                                     \
  } while (0)

enum Form { kProducts, kSoftmax, kChain, kLds, kBlock, kStaged };

constexpr int kTileElems = 8192;  // one block's K (8 KB) and V^T (8 KB) as bf16

__device__ __forceinline__ void softmax(const f32x16_t& s, float sl2, float nm, bf16x8_t (&pb)[2]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      f32x2_t two = {__builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * ks + j], sl2, nm)),
                     __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * ks + j + 1], sl2, nm))};
      const bf16x2_t c = __builtin_convertvector(two, bf16x2_t);
      pb[ks][j] = c[0];
      pb[ks][j + 1] = c[1];
    }
  }
}

// QT query tiles of 32 a wave (1 or 2); `kv` holds 96 units of `ublocks` 16 KB blocks (staged forms only). PRIO:
// 0 none, 1 raised around the score products, 2 around the score and the second products.
template <int FORM, int WAVES, int QT = 1, int PRIO = 0>
__global__ __launch_bounds__(256, WAVES) void half_kernel(float* out, const float* in, const uint16_t* kv,
                                                          int ublocks, int iters) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][kTileElems];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < 2 * kTileElems; i += 256) tile[i / kTileElems][i % kTileElems] = 0x3c00 + (i & 255);
  __syncthreads();
  bf16x8_t a[4], v[4], q[QT][4], ones;
  for (int k = 0; k < 4; ++k) {
    for (int i = 0; i < 8; ++i) {
      a[k][i] = (__bf16)(in[i] * (tid + k));
      v[k][i] = (__bf16)(in[16 + i] + 0.1f * tid);
      for (int u = 0; u < QT; ++u) q[u][k][i] = (__bf16)(in[8 + i] - 0.01f * k + u);
    }
  }
  for (int i = 0; i < 8; ++i) ones[i] = (__bf16)((tid & 31) == 0 ? 1.f : 0.f);
  const float sl2 = in[24] * 1e-3f, nm = -in[25];
  f32x16_t o[QT][2];
  float l[QT];
  for (int u = 0; u < QT; ++u) {
    o[u][0] = o[u][1] = f32x16_t{0};
    l[u] = 0.f;
  }
  // The staged forms: unit = the (window, head) whose blocks this workgroup reads; its 8 workgroups share
  // blockIdx % 8, hence one XCD.
  const int unit = (blockIdx.x % 8) * (gridDim.x / 64) + (blockIdx.x / 8) / 8;
  const uint32_t ubytes = static_cast<uint32_t>(ublocks) * 16384u;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(kv) + static_cast<size_t>(unit) * (ubytes / 2), 0, static_cast<int>(ubytes), 0x00020000);
  auto stage = [&](int blk, int buf) __attribute__((always_inline)) {
    const uint32_t soff = static_cast<uint32_t>(blk % ublocks) * 16384u;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = w + 4 * t;  // 16 loads of 1 KB a block, 4 a wave
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(&tile[buf][512 * j]), 16,
                                               static_cast<uint32_t>(1024 * j + 16 * lane), soff, 0, 0);
    }
  };
  if constexpr (FORM == kStaged) {
    stage(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  f32x16_t sv;  // the softmax-only form's input
  for (int i = 0; i < 16; ++i) sv[i] = in[i] * tid;
  for (int it = 0; it < iters; ++it) {
    const int t = it & 1, blk = it >> 1, buf = FORM == kStaged ? (blk & 1) : 0;
    if (FORM == kStaged && t == 0) stage(blk + 1, buf ^ 1);
    if constexpr (FORM == kSoftmax) {
      asm volatile("" : "+v"(sv));
      bf16x8_t pb[2];
      softmax(sv, sl2, nm, pb);
      asm volatile("" ::"v"(pb[0]), "v"(pb[1]));
      continue;
    }
    const char* tp = reinterpret_cast<const char*>(tile[buf]);
    bf16x8_t ak[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (FORM >= kLds) {
        ak[k] = *reinterpret_cast<const bf16x8_t*>(tp + ((lane * 16 + k * 1024 + t * 4096) & 8191));
      } else {
        asm volatile("" : "+v"(a[k]));  // an operand the compiler cannot hoist out of the loop
        ak[k] = a[k];
      }
    }
    f32x16_t s[QT];
    if constexpr (PRIO >= 1) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      s[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak[0], q[u][0], f32x16_t{0}, 0, 0, 0);
#pragma unroll
      for (int k = 1; k < 4; ++k) s[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak[k], q[u][k], s[u], 0, 0, 0);
    }
    if constexpr (PRIO >= 1) __builtin_amdgcn_s_setprio(0);
    bf16x8_t pb[QT][2];
    f32x4_t h[QT];
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      if constexpr (FORM == kProducts) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          pb[u][ks] = __builtin_bit_cast(bf16x8_t, f32x4_t{s[u][8 * ks], s[u][8 * ks + 1], s[u][8 * ks + 2],
                                                           s[u][8 * ks + 3]});
        }
      } else {
        softmax(s[u], sl2, nm, pb[u]);
      }
      h[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[u][0], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      h[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[u][1], h[u], 0, 0, 0);
    }
    if constexpr (PRIO >= 2) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8_t av[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (FORM >= kLds) {
          av[j] = *reinterpret_cast<const bf16x8_t*>(tp + 8192 + ((lane * 16 + (2 * ks + j) * 1024 + t * 4096) & 8191));
        } else {
          av[j] = v[2 * ks + j];
        }
      }
#pragma unroll
      for (int u = 0; u < QT; ++u) {
        o[u][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[0], pb[u][ks], o[u][0], 0, 0, 0);
        o[u][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[1], pb[u][ks], o[u][1], 0, 0, 0);
      }
    }
    if constexpr (PRIO >= 2) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      if constexpr (FORM >= kBlock) {
        if (__builtin_amdgcn_ballot_w64(!(h[u][0] <= 1e30f)) != 0ull) l[u] = -l[u];
      }
      l[u] += h[u][0];
    }
    if (FORM >= kBlock && t == 1) {
      if constexpr (FORM == kStaged) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  }
  float r = 0.f;
  for (int u = 0; u < QT; ++u) {
    r += l[u];
    for (int i = 0; i < 16; ++i) r += o[u][0][i] + o[u][1][i];
  }
  out[blockIdx.x * blockDim.x + tid] = r;
}

constexpr int kUnits = 128, kUnitBlocks = 128;  // 2 MB of blocks a unit, 256 MB in all (4 waves per SIMD: 1024
                                                // workgroups, units 0..127)

// Both halves of a block in one stretch (see the top). RESCALE: the row-sum checks as branches that rescale O.
template <int WAVES, bool RESCALE>
__global__ __launch_bounds__(256, WAVES) void block_kernel(float* out, const float* in, const uint16_t* kv,
                                                           int ublocks, int iters) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][kTileElems];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < 2 * kTileElems; i += 256) tile[i / kTileElems][i % kTileElems] = 0x3c00 + (i & 255);
  __syncthreads();
  bf16x8_t q[4], ones;
  for (int k = 0; k < 4; ++k) {
    for (int i = 0; i < 8; ++i) q[k][i] = (__bf16)(in[8 + i] - 0.01f * k);
  }
  for (int i = 0; i < 8; ++i) ones[i] = (__bf16)((tid & 31) == 0 ? 1.f : 0.f);
  const float sl2 = in[24] * 1e-3f, nm = -in[25];
  f32x16_t o[2];
  o[0] = o[1] = f32x16_t{0};
  float l = 0.f;
  const int unit = (blockIdx.x % 8) * (gridDim.x / 64) + (blockIdx.x / 8) / 8;
  const uint32_t ubytes = static_cast<uint32_t>(ublocks) * 16384u;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(kv) + static_cast<size_t>(unit) * (ubytes / 2), 0, static_cast<int>(ubytes), 0x00020000);
  auto stage = [&](int blk, int buf) __attribute__((always_inline)) {
    const uint32_t soff = static_cast<uint32_t>(blk % ublocks) * 16384u;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = w + 4 * t;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(&tile[buf][512 * j]), 16,
                                               static_cast<uint32_t>(1024 * j + 16 * lane), soff, 0, 0);
    }
  };
  stage(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int blk = 0; blk < iters / 2; ++blk) {
    const int buf = blk & 1;
    stage(blk + 1, buf ^ 1);
    const char* tp = reinterpret_cast<const char*>(tile[buf]);
    auto score = [&](int t) __attribute__((always_inline)) {
      bf16x8_t a[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] = *reinterpret_cast<const bf16x8_t*>(tp + ((lane * 16 + k * 1024 + t * 4096) & 8191));
      f32x16_t x = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], q[0], f32x16_t{0}, 0, 0, 0);
#pragma unroll
      for (int k = 1; k < 4; ++k) x = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k], q[k], x, 0, 0, 0);
      return x;
    };
    auto row_sum = [&](const bf16x8_t (&pb)[2]) __attribute__((always_inline)) {
      f32x4_t h = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[0], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      h = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[1], h, 0, 0, 0);
      return h[0];
    };
    auto second = [&](int t, const bf16x8_t (&pb)[2]) __attribute__((always_inline)) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const char* vp = tp + 8192;
        const bf16x8_t v0 = *reinterpret_cast<const bf16x8_t*>(vp + ((lane * 16 + (2 * ks) * 1024 + t * 4096) & 8191));
        const bf16x8_t v1 = *reinterpret_cast<const bf16x8_t*>(vp + ((lane * 16 + (2 * ks + 1) * 1024 + t * 4096) & 8191));
        o[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v0, pb[ks], o[0], 0, 0, 0);
        o[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v1, pb[ks], o[1], 0, 0, 0);
      }
    };
    const f32x16_t s0 = score(0);
    const f32x16_t s1 = score(1);
    bf16x8_t pb0[2], pb1[2];
    softmax(s0, sl2, nm, pb0);
    const float h0 = row_sum(pb0);
    __builtin_amdgcn_sched_barrier(0);
    second(0, pb0);
    softmax(s1, sl2, nm, pb1);
    const float h1 = row_sum(pb1);
    if (RESCALE && __builtin_amdgcn_ballot_w64(!(h0 <= 1e30f)) != 0ull) {
      o[0] *= 0.5f;
      o[1] *= 0.5f;
      l *= 0.5f;
    }
    l += h0;
    if (RESCALE && __builtin_amdgcn_ballot_w64(!(h1 <= 1e30f)) != 0ull) {
      o[0] *= 0.25f;
      o[1] *= 0.25f;
      l *= 0.25f;
    }
    second(1, pb1);
    l += h1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  float r = l;
  for (int i = 0; i < 16; ++i) r += o[0][i] + o[1][i];
  out[blockIdx.x * blockDim.x + tid] = r;
}

// FORM kBlockPair: block_kernel (PRIO then means RESCALE).
constexpr int kBlockPair = 100;

template <int FORM, int WAVES, int QT, int PRIO>
void launch(int grid, float* out, const float* in, const uint16_t* kv, int iters) {
  if constexpr (FORM == kBlockPair) {
    block_kernel<WAVES, PRIO != 0><<<grid, 256>>>(out, in, kv, kUnitBlocks, iters);
  } else {
    half_kernel<FORM, WAVES, QT, PRIO><<<grid, 256>>>(out, in, kv, kUnitBlocks, iters);
  }
}

template <int FORM, int WAVES, int QT = 1, int PRIO = 0>
double run(const char* name, float* out, const float* in, const uint16_t* kv, int iters, double ref_ns) {
  const int grid = 256 * WAVES;  // WAVES workgroups of 4 waves per CU: WAVES waves on every SIMD
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  launch<FORM, WAVES, QT, PRIO>(grid, out, in, kv, iters);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  const int reps = 5;
  CHECK(hipEventRecord(e0));
  for (int r = 0; r < reps; ++r) launch<FORM, WAVES, QT, PRIO>(grid, out, in, kv, iters);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  ms /= reps;
  const double ns = ms * 1e6 / (static_cast<double>(iters) * WAVES * QT);  // per 32-query half and SIMD
  if (ref_ns > 0) {
    printf("%-26s waves/SIMD %d: %7.1f ns per 32-query half per SIMD, products busy %.2f\n", name, WAVES, ns,
           ref_ns / ns);
  } else {
    printf("%-26s waves/SIMD %d: %7.1f ns per 32-query half per SIMD\n", name, WAVES, ns);
  }
  fflush(stdout);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  return ns;
}

int main() {
  float *out, *in;
  uint16_t* kv;
  const int iters = 4000;
  CHECK(hipMalloc(&out, sizeof(float) * 256 * 256 * 4));  // one float per thread at up to 4 waves per SIMD
  CHECK(hipMalloc(&in, sizeof(float) * 32));
  CHECK(hipMalloc(&kv, static_cast<size_t>(kUnits) * kUnitBlocks * 16384));
  CHECK(hipMemset(kv, 0x3c, static_cast<size_t>(kUnits) * kUnitBlocks * 16384));
  float h[32];
  for (int i = 0; i < 32; ++i) h[i] = 0.01f * (i + 1);
  CHECK(hipMemcpy(in, h, sizeof(h), hipMemcpyHostToDevice));
  const double p3 = run<kProducts, 3>("products only", out, in, kv, iters, 0);
  run<kSoftmax, 3>("softmax only", out, in, kv, iters, 0);
  run<kChain, 3>("chain", out, in, kv, iters, p3);
  run<kLds, 3>("+ LDS operands", out, in, kv, iters, p3);
  run<kBlock, 3>("+ barrier, trigger", out, in, kv, iters, p3);
  run<kStaged, 3>("+ staging", out, in, kv, iters, p3);
  run<kStaged, 2>("+ staging", out, in, kv, iters, p3);
  run<kStaged, 1>("+ staging", out, in, kv, iters, p3);
  run<kStaged, 4>("+ staging", out, in, kv, iters, p3);
  run<kChain, 4>("chain", out, in, kv, iters, p3);
  run<kStaged, 3, 2>("64 queries a wave", out, in, kv, iters, p3);
  run<kStaged, 2, 2>("64 queries a wave", out, in, kv, iters, p3);
  run<kStaged, 3, 1, 1>("+ staging, priority 1", out, in, kv, iters, p3);
  run<kStaged, 3, 1, 2>("+ staging, priority 2", out, in, kv, iters, p3);
  run<kStaged, 2, 1, 2>("+ staging, priority 2", out, in, kv, iters, p3);
  run<kStaged, 3>("+ staging", out, in, kv, iters, p3);
  run<kBlockPair, 3>("two halves at once", out, in, kv, iters, p3);
  run<kBlockPair, 3, 1, 1>("+ rare rescales", out, in, kv, iters, p3);
  run<kBlockPair, 2>("two halves at once", out, in, kv, iters, p3);
  run<kBlockPair, 1>("two halves at once", out, in, kv, iters, p3);
  CHECK(hipFree(kv));
  CHECK(hipFree(out));
  CHECK(hipFree(in));
  return 0;
}
