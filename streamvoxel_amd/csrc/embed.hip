// Gather patchify: the embedding of a window's voxel tokens as patch tokens, without the one-hot tensor.
//
//   out[b, n, :] = bias + sum_{o < p^3} table[tokens[b, voxel(n, o)] * p^3 + o, :]
//
// where patch token n (row-major over the (Y/p, Z/p, X/p) patch grid) covers voxel (p*gy + dy, p*gz + dz, p*gx + dx)
// at kernel offset o = (dy*p + dz)*p + dx, and table[c * p^3 + o, :] = conv.weight[:, c, dy, dz, dx], i.e.
// Conv3d(C+1 -> W, kernel p, stride p) of the one-hot tokens (models/unconditional_md4_timefree.py:141-147) written
// as the reference's embedding bag (stream/fast_ops.py:54-75, GatherPatch). The p^3 rows are summed in fp32 in
// offset order, rounded to bf16, then the bias is added in bf16 (one more rounding), as embedding_bag(mode='sum')
// followed by `out + bias` compute it in bf16.
//
// Workgroup = 8 patch tokens of one window, 32 lanes per token, each lane 16-byte column chunks lane + 32 c; the
// table rows (reused across the batch) are gathered OB offsets at a time (8, or 4 for rows wider than 768) so that
// OB loads per chunk are in flight.
#include "common.hpp"

namespace svhip {

constexpr int kEmbedThreads = 256;
constexpr int kEmbedLanes = 32;                              // lanes per patch token
constexpr int kEmbedTokens = kEmbedThreads / kEmbedLanes;  // patch tokens per workgroup
constexpr int kEmbedMaxOffsets = 64;                        // p^3 up to 4^3
constexpr int kEmbedMaxWidth = 2048;

struct EmbedArgs {
  const int64_t* tokens;  // (b, y, z, x) at b*stb + ((y*Z) + z)*X + x
  const uint16_t* table;  // [(C+1) * p^3, W]
  const uint16_t* bias;   // [W] or null
  uint16_t* out;          // (b, n, c) at b*sob + n*son + c
  int64_t B, Y, Z, X, p, cells, W;
  int64_t stb, sob, son;
  int* bad;               // set when a token lies outside [0, cells)
};

template <int CPL>
__global__ __launch_bounds__(kEmbedThreads) void patch_embed_kernel(EmbedArgs a) {
  constexpr int OB = CPL <= 3 ? 8 : 4;
  __shared__ int s_row[kEmbedTokens][kEmbedMaxOffsets];  // table row of every (token, offset)
  const int64_t gy = a.Y / a.p, gz = a.Z / a.p, gx = a.X / a.p;
  const int64_t per_window = gy * gz * gx;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kEmbedTokens;  // flat (b, n) of slot 0
  const int p3 = static_cast<int>(a.p * a.p * a.p);
  for (int i = threadIdx.x; i < kEmbedTokens * p3; i += kEmbedThreads) {
    const int t = i / p3, o = i - t * p3;
    const int64_t flat = first + t;
    int row = 0;
    if (flat < a.B * per_window) {
      const int64_t b = flat / per_window, n = flat - b * per_window;
      const int64_t py = n / (gz * gx), pz = (n / gx) % gz, px = n % gx;
      const int dy = o / static_cast<int>(a.p * a.p), dz = (o / static_cast<int>(a.p)) % static_cast<int>(a.p);
      const int dx = o % static_cast<int>(a.p);
      const int64_t y = py * a.p + dy, z = pz * a.p + dz, x = px * a.p + dx;
      int64_t cell = a.tokens[b * a.stb + (y * a.Z + z) * a.X + x];
      if (cell < 0 || cell >= a.cells) {
        atomicOr(a.bad, 1);
        cell = 0;
      }
      row = static_cast<int>(cell) * p3 + o;
    }
    s_row[t][o] = row;
  }
  __syncthreads();
  const int t = threadIdx.x / kEmbedLanes, lane = threadIdx.x % kEmbedLanes;
  const int64_t flat = first + t;
  if (flat >= a.B * per_window) return;
  const int chunks = static_cast<int>(a.W / 8);
  float acc[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[c][j] = 0.f;
  }
  for (int o0 = 0; o0 < p3; o0 += OB) {
    uint4 w[OB][CPL];
#pragma unroll
    for (int u = 0; u < OB; ++u) {
      const int o = o0 + u;
      const uint16_t* src = a.table + static_cast<int64_t>(s_row[t][o < p3 ? o : 0]) * a.W;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = lane + kEmbedLanes * c;
        w[u][c] = (o < p3 && ch < chunks) ? *reinterpret_cast<const uint4*>(src + 8 * ch)
                                          : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    // Offsets in order: the sum of each column is taken o = 0, 1, 2, ... (zeros past p^3 leave it unchanged).
#pragma unroll
    for (int u = 0; u < OB; ++u) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t e[4] = {w[u][c].x, w[u][c].y, w[u][c].z, w[u][c].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          acc[c][j] += bf16_bits_to_float(static_cast<uint16_t>(e[j >> 1] >> (16 * (j & 1))));
        }
      }
    }
  }
  const int64_t b = flat / per_window, n = flat - b * per_window;
  uint16_t* dst = a.out + b * a.sob + n * a.son;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + kEmbedLanes * c;
    if (ch >= chunks) continue;
    uint32_t out[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float v0 = acc[c][j], v1 = acc[c][j + 1];
      bf16_round2(v0, v1);
      if (a.bias) {
        v0 += bf16_bits_to_float(a.bias[8 * ch + j]);
        v1 += bf16_bits_to_float(a.bias[8 * ch + j + 1]);
      }
      out[j / 2] = bf16_pack2(v0, v1);
    }
    *reinterpret_cast<uint4*>(dst + 8 * ch) = make_uint4(out[0], out[1], out[2], out[3]);
  }
}

}  // namespace svhip

using namespace svhip;

extern "C" int svhip_patch_embed(const int64_t* tokens, const void* table, const void* bias, void* out, int* bad,
                                 int64_t B, int64_t Y, int64_t Z, int64_t X, int64_t patch, int64_t cells, int64_t W,
                                 int64_t st_b, int64_t so_b, int64_t so_n, void* stream) {
  const char* name = "svhip_patch_embed";
  clear_error();
  SVHIP_REQUIRE(tokens && table && out && bad, "%s: null pointer", name);
  SVHIP_REQUIRE(B >= 0 && Y >= 1 && Z >= 1 && X >= 1 && cells >= 1, "%s: bad sizes", name);
  SVHIP_REQUIRE(patch >= 1 && patch * patch * patch <= kEmbedMaxOffsets && Y % patch == 0 && Z % patch == 0 &&
                    X % patch == 0,
                "%s: patch %lld must divide the window and have at most %d offsets", name, (long long)patch,
                kEmbedMaxOffsets);
  SVHIP_REQUIRE(W >= 8 && W % 8 == 0 && W <= kEmbedMaxWidth, "%s: width %lld unsupported (a multiple of 8 up to %d)",
                name, (long long)W, kEmbedMaxWidth);
  SVHIP_REQUIRE(cells * patch * patch * patch < (1ll << 31), "%s: table too large", name);
  SVHIP_REQUIRE(reinterpret_cast<uintptr_t>(table) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                    so_b % 8 == 0 && so_n % 8 == 0,
                "%s: table and output rows must start on 16-byte boundaries", name);
  const int64_t tokens_total = B * (Y / patch) * (Z / patch) * (X / patch);
  if (tokens_total == 0) return SVHIP_OK;
  EmbedArgs a{tokens, static_cast<const uint16_t*>(table), static_cast<const uint16_t*>(bias),
              static_cast<uint16_t*>(out), B, Y, Z, X, patch, cells, W, st_b, so_b, so_n, bad};
  const int64_t grid = cdiv(tokens_total, kEmbedTokens);
  SVHIP_REQUIRE(grid < (1ll << 31), "%s: grid too large", name);
  const int cpl = static_cast<int>(cdiv(W / 8, kEmbedLanes));
  hipStream_t s = as_stream(stream);
  const unsigned g = static_cast<unsigned>(grid);
  switch (cpl) {
    case 1: patch_embed_kernel<1><<<g, kEmbedThreads, 0, s>>>(a); break;
    case 2: patch_embed_kernel<2><<<g, kEmbedThreads, 0, s>>>(a); break;
    case 3: patch_embed_kernel<3><<<g, kEmbedThreads, 0, s>>>(a); break;
    case 4: patch_embed_kernel<4><<<g, kEmbedThreads, 0, s>>>(a); break;
    default: patch_embed_kernel<8><<<g, kEmbedThreads, 0, s>>>(a); break;
  }
  SVHIP_LAUNCHED(name);
  return SVHIP_OK;
}
