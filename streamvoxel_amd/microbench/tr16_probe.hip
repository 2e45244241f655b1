// The lane layout of ds_read_b64_tr_b16 (gfx950's LDS transpose load), which the cross-attention kernel uses to read
// the second product's V^T operand from row-major V in LDS. One wave, one workgroup, a 64 x 64 uint16 LDS tile
// holding each element's index; every address is 8-byte aligned and inside the tile (checked on the host first).
//   1. Five address patterns: each lane's 4 returned values are compared with the model "within each 16-lane group,
//      lane i receives element i % 4 of the 8-byte reads of lanes 4 n + i / 4, n = 0..3".
//   2. The kernel's own scheme: V rows of one 64-key block in the swizzled tile layout (chunk c of row r at physical
//      chunk c ^ 4 ((r / 2) % 2)), the per-lane offsets of output tile j, two reads per k-step (keys + 0..3, + 4..7):
//      lane l must hold keys 32 t + 16 ks + 8 (l / 32) + 0..7 of head_dim column 32 j + l % 32.
// Build: python -m streamvoxel_amd.build --microbench   Run: streamvoxel_amd/microbench/tr16_probe
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

#define CHECK(x)                                                               \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
      exit(1);                                                                 \
    }                                                                          \
  } while (0)

constexpr int kPatterns = 5;

__host__ __device__ int pattern_elem(int pattern, int l) {
  switch (pattern) {
    case 0: return l * 4;                         // contiguous 8-byte chunks of rows 0..3
    case 1: return (l % 16) * 64 + (l / 16) * 4;  // lane % 16 -> row, lane / 16 -> 4-element chunk
    case 2: return l * 64;                        // lane -> row, element 0
    case 3: return (l % 8) * 64 + (l / 8) * 4;    // lane % 8 -> row
    default: return (l % 4) * 64 + (l / 4) * 4;   // lane % 4 -> row
  }
}

__host__ __device__ int swzv(int r, int c) { return c ^ (((r >> 1) & 1) << 2); }

// Byte offset of lane l's first read for output tile j (head_dim 32 j .. 32 j + 31) of a 64 x 64 sub-tile.
__host__ __device__ int vrow_offset(int l, int j) {
  const int row_lane = 8 * (l >> 5) + ((l & 15) >> 2);
  const int flip = (row_lane >> 1) & 1;
  const int c_lane = 2 * ((l >> 4) & 1) + ((l & 3) >> 1);
  return row_lane * 128 + 16 * (4 * ((j & 1) ^ flip) + c_lane) + 8 * (l & 1);
}

// out: kPatterns x 64 lanes x 4 values, then 2 tiles x 2 t x 2 ks x 64 lanes x 8 values
__global__ void probe(uint16_t* out) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64 * 64];
  const int l = threadIdx.x;
  for (int i = l; i < 64 * 64; i += 64) tile[i] = static_cast<uint16_t>(i);
  __syncthreads();
  for (int pat = 0; pat < kPatterns; ++pat) {
    const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(tile + pattern_elem(pat, l)));
    reinterpret_cast<uint2*>(out)[pat * 64 + l] = __builtin_bit_cast(uint2, v);
  }
  __syncthreads();
  // V rows in the swizzled layout: value of (key r, head_dim d) = 64 r + d.
  for (int i = l; i < 64 * 8; i += 64) {
    const int r = i / 8, c = i % 8;
    for (int e = 0; e < 8; ++e) tile[r * 64 + swzv(r, c) * 8 + e] = static_cast<uint16_t>(64 * r + 8 * c + e);
  }
  __syncthreads();
  uint16_t* o2 = out + kPatterns * 64 * 4;
  const char* base = reinterpret_cast<const char*>(tile);
  for (int j = 0; j < 2; ++j) {
    for (int t = 0; t < 2; ++t) {
      for (int ks = 0; ks < 2; ++ks) {
        const char* b = base + vrow_offset(l, j) + (32 * t + 16 * ks) * 128;
        const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(const_cast<char*>(b)));
        const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(const_cast<char*>(b) + 512));
        uint2* dst = reinterpret_cast<uint2*>(o2 + (((j * 2 + t) * 2 + ks) * 64 + l) * 8);
        dst[0] = __builtin_bit_cast(uint2, lo);
        dst[1] = __builtin_bit_cast(uint2, hi);
      }
    }
  }
}

int main() {
  for (int pat = 0; pat < kPatterns; ++pat) {
    for (int l = 0; l < 64; ++l) {
      const int e = pattern_elem(pat, l);
      if (e < 0 || e + 4 > 64 * 64 || e % 4) {
        printf("pattern %d lane %d out of the tile\n", pat, l);
        return 1;
      }
    }
  }
  for (int l = 0; l < 64; ++l) {
    for (int j = 0; j < 2; ++j) {
      const int hi = vrow_offset(l, j) + (32 + 16) * 128 + 512;
      if (vrow_offset(l, j) % 8 || hi + 8 > 64 * 64 * 2) {
        printf("operand read of lane %d out of the tile\n", l);
        return 1;
      }
    }
  }
  const int n1 = kPatterns * 64 * 4, n2 = 2 * 2 * 2 * 64 * 8;
  uint16_t* d;
  CHECK(hipMalloc(&d, (n1 + n2) * 2));
  probe<<<1, 64>>>(d);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  uint16_t* h = static_cast<uint16_t*>(malloc((n1 + n2) * 2));
  CHECK(hipMemcpy(h, d, (n1 + n2) * 2, hipMemcpyDeviceToHost));
  int bad = 0;
  for (int pat = 0; pat < kPatterns; ++pat) {
    int pbad = 0;
    for (int l = 0; l < 64; ++l) {
      const int g = l / 16, i = l % 16;
      for (int n = 0; n < 4; ++n) {
        const int src = 16 * g + 4 * n + i / 4;  // the lane whose read supplies value n
        const int expect = pattern_elem(pat, src) + i % 4;
        if (h[(pat * 64 + l) * 4 + n] != expect) ++pbad;
      }
    }
    printf("pattern %d: %d of 256 values differ from the model\n", pat, pbad);
    bad += pbad;
  }
  int vbad = 0;
  for (int j = 0; j < 2; ++j)
    for (int t = 0; t < 2; ++t)
      for (int ks = 0; ks < 2; ++ks)
        for (int l = 0; l < 64; ++l)
          for (int e = 0; e < 8; ++e) {
            const int key = 32 * t + 16 * ks + 8 * (l / 32) + e, dcol = 32 * j + l % 32;
            if (h[n1 + (((j * 2 + t) * 2 + ks) * 64 + l) * 8 + e] != 64 * key + dcol) ++vbad;
          }
  printf("V-row operands (2 tiles x 2 halves x 2 k-steps x 64 lanes x 8 keys): %d differ from V^T\n", vbad);
  printf(bad + vbad == 0 ? "model holds\n" : "MODEL FAILS\n");
  CHECK(hipFree(d));
  free(h);
  return bad + vbad == 0 ? 0 : 1;
}
