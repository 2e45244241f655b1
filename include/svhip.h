/*
 * libsvhip — MI355X (gfx950) kernels for StreamVoxel's per-step generation hot path, behind a plain C ABI.
 *
 * Every entry point takes caller-owned device pointers, plain sizes and strides (in elements), and a HIP stream
 * (`hipStream_t` passed as `void*`); it enqueues work on that stream and returns without synchronising, so calls
 * can be recorded into a HIP graph. No entry point allocates device memory: scratch space comes from a
 * caller-provided workspace whose size the matching `*_workspace_bytes` query returns (svhip_ease_select_noalloc
 * uses a fixed device array of the library instead).
 *
 * Return value: SVHIP_OK (0) on success, a negative status otherwise; `svhip_last_error()` then describes the
 * failure (thread-local string). No entry point aborts the process.
 *
 * Booleans are bytes holding 0 or 1 (torch.bool storage). Index order of a column window is the flat YZX order
 * `(y * Z + z) * X + x`.
 */
#ifndef SVHIP_H
#define SVHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SVHIP_FP8_E4M3_PFP8: e4m3 K/V whose attention rounds P to e4m3 for the fp8 matrix cores (see svhip_xattn_fwd). */
enum svhip_dtype { SVHIP_F32 = 0, SVHIP_BF16 = 1, SVHIP_FP8_E4M3 = 3, SVHIP_FP8_E4M3_PFP8 = 5 };

enum svhip_status { SVHIP_OK = 0, SVHIP_EINVAL = -1, SVHIP_ELAUNCH = -2, SVHIP_EWORKSPACE = -3 };

enum svhip_lel_mode { SVHIP_LEL_LAYER = 0, SVHIP_LEL_BAND = 1, SVHIP_LEL_COLUMN = 2 };

/* Library version (major * 10000 + minor * 100 + patch) and the last error of the calling thread. */
int svhip_version(void);
const char* svhip_last_error(void);

/*
 * Negative Shannon entropy per voxel, score = sum_c p_c log p_c (nats, fp32 arithmetic), for `batch` windows of
 * `n` voxels with `classes` logits each. Element (b, c, i) of `logits` is at b*stride_b + c*stride_c + i*stride_n.
 * Class-major [B,C,N] (stride_n == 1) and voxel-major [B,N,C] (stride_c == 1) layouts take vectorised paths.
 * dtype: SVHIP_F32 or SVHIP_BF16. out: fp32 [batch, n] contiguous.
 * Replaces: entropy_scores (streamvoxel/sampling/entropy.py:1-4), entropy_triton (streamvoxel/stream/fast_ops.py:420-430).
 */
int svhip_entropy(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n, int64_t stride_b,
                  int64_t stride_c, int64_t stride_n, float* out, void* stream);

/*
 * Air probability per voxel: sum over the `n_air` class ids in `air_ids` (device int32) of softmax(logits)_c.
 * Same layout rules as svhip_entropy. out: fp32 [batch, n].
 * Replaces: `logits.float().softmax(0)[air].sum(0)` (streamvoxel/stream/slot.py:126).
 */
int svhip_air_prob(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t n, int64_t stride_b,
                   int64_t stride_c, int64_t stride_n, const int32_t* air_ids, int32_t n_air, float* out,
                   void* stream);

/*
 * The same statistics over logits in the class head's patch order: patches[b, r, c] at b*stride_b + r*stride_n + c
 * (voxel-major rows of `classes` logits), where the voxel (y, z, x) of a [Y,Z,X] window sits in row
 *   r = ((y/p * (Z/p) + z/p) * (X/p) + x/p) * p^3 + ((y%p) * p + z%p) * p + x%p,   p = patch,
 * the row order of `class_head(...)` before the reshape / permute to [n, C, Y, Z, X]. patch, Y, Z, X: powers of
 * two, patch <= each; rows 16-byte aligned, classes a multiple of 16 bytes' worth of elements. out: fp32 [batch,
 * Y*Z*X] in (y, z, x) order.
 * Replaces: the permute in FastSlotForward.forward (streamvoxel/stream/fast_ops.py:305-308) and
 * UnconditionalMD4.forward (streamvoxel/models/unconditional_md4.py:126-129) followed by entropy_scores / the air
 * probability of streamvoxel/stream/slot.py:126: the permuted copy is never made.
 */
int svhip_entropy_patches(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t Y, int64_t Z,
                          int64_t X, int64_t patch, int64_t stride_b, int64_t stride_n, float* out, void* stream);
int svhip_air_prob_patches(const void* logits, int dtype, int64_t batch, int64_t classes, int64_t Y, int64_t Z,
                           int64_t X, int64_t patch, int64_t stride_b, int64_t stride_n, const int32_t* air_ids,
                           int32_t n_air, float* out, void* stream);

/*
 * Low-entropy-last update, in place on `last`:
 *   bad = (mask & air <= fp32(1 - eps)) | solid
 *   SVHIP_LEL_COLUMN: last [B,Y,Z,X] |= the top run (from y = Y-1 down) of clean voxels of every (z, x) column;
 *   SVHIP_LEL_LAYER / SVHIP_LEL_BAND: last [B,Y] |= the top run of clean layers (bands of 8 layers).
 * mask, air, solid: [B,Y,Z,X]; `mask` NULL means all true, `solid` NULL means all false.
 * Replaces: low_entropy_last_update (streamvoxel/sampling/low_entropy_last.py:8-17).
 */
int svhip_lel_update(uint8_t* last, const uint8_t* mask, const float* air, const uint8_t* solid, double eps,
                     int32_t mode, int64_t batch, int64_t Y, int64_t Z, int64_t X, void* stream);

/*
 * Global top-k mask: out[b] = the `count` largest `scores[b]` among `eligible[b]`, ties to the lower index;
 * count <= 0 selects nothing and a count above the number of eligible voxels selects all of them. The count is
 * `count_dev[b]` (device int64) when count_dev is non-NULL, else `count_host`. Scores must be finite.
 * scores fp32 [batch, n]; eligible, out: bytes [batch, n].
 * Replaces: top_mask (streamvoxel/sampling/block_quota.py:4-12), top_mask_nosync (streamvoxel/stream/fast_ops.py:433-439).
 */
int svhip_top_mask(const float* scores, const uint8_t* eligible, int64_t batch, int64_t n, const int64_t* count_dev,
                   int64_t count_host, uint8_t* out, void* stream);

/*
 * Block-quota selection of `k[b]` voxels of `mask[b]` over b^3 blocks of a [Y,Z,X] window, for `batch` windows:
 * per-block quotas apportioned from frac[b] * n_total[b, j] with the remainder handed out by ascending
 * -(fractional part) * 1e6 + pos[b, j], the quota-many highest scores taken inside each block, then a global trim
 * (more than k) or top-up (fewer) by score. bad[b] is set to 1 when the result does not hold exactly k voxels.
 *   score fp32 [B,N]; mask bytes [B,N]; k, committed int64 [B]; frac fp64 [B]; pos, n_total int64 [B, nb];
 *   chosen bytes [B,N] (written); bad bytes [B] (written), nb = N / b^3.
 * committed may be NULL: it is then derived per window on the device as sum(n_total[b]) - (non-zero mask bytes of
 * window b), the already-committed non-deferred voxels.
 * Replaces: quota_select_nosync (streamvoxel/stream/fast_ops.py:442-473) and, with committed = the number of
 * committed non-deferred voxels (or NULL), block_quota_select (streamvoxel/sampling/block_quota.py:20-38).
 */
size_t svhip_quota_select_workspace_bytes(int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block);
int svhip_quota_select(const float* score, const uint8_t* mask, int64_t batch, int64_t Y, int64_t Z, int64_t X,
                       int64_t block, const int64_t* k, const int64_t* pos, const double* frac,
                       const int64_t* n_total, const int64_t* committed, uint8_t* chosen, uint8_t* bad,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * The whole EASE selection of one solid step for `batch` windows, without host synchronisation:
 *   selectable = (tokens == mask_token) & ~last, score = entropy(logits), chosen = block-quota select
 * (as svhip_quota_select), bad = quota violation. tokens int64 [B,N]; last bytes [B,N]; logits as in
 * svhip_entropy; scores_out (optional, may be NULL) receives the fp32 scores [B,N].
 * Replaces: FastLowEntropyLastSlot.select (streamvoxel/stream/fast_ops.py:534-540) for all slots of a batch.
 */
size_t svhip_ease_select_workspace_bytes(int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block);
int svhip_ease_select(const void* logits, int dtype, int64_t classes, int64_t stride_b, int64_t stride_c,
                      int64_t stride_n, const int64_t* tokens, int64_t mask_token, const uint8_t* last,
                      int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const int64_t* k,
                      const int64_t* pos, const double* frac, const int64_t* n_total, const int64_t* committed,
                      uint8_t* chosen, uint8_t* bad, float* scores_out, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * svhip_ease_select with the scratch taken from a fixed device array of the library (48 MiB per GPU, held from
 * the library's load until the process ends) instead of a workspace argument: the call allocates nothing, for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Rejects geometries whose svhip_ease_select_workspace_bytes exceed 48 MiB (up to 92 windows of
 * 65 536 voxels at 4^3 blocks fit) with SVHIP_EINVAL, without a launch. Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, two threads) race and must be serialised by the caller. The first call on a device
 * looks up the array's address on that device (outside graph capture, so make it once before capturing).
 * No counterpart in the reference: an addition of this library for callers that cannot allocate.
 */
int svhip_ease_select_noalloc(const void* logits, int dtype, int64_t classes, int64_t stride_b, int64_t stride_c,
                              int64_t stride_n, const int64_t* tokens, int64_t mask_token, const uint8_t* last,
                              int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const int64_t* k,
                              const int64_t* pos, const double* frac, const int64_t* n_total,
                              const int64_t* committed, uint8_t* chosen, uint8_t* bad, float* scores_out,
                              void* stream);

/*
 * svhip_ease_select over logits in the class head's patch order (row map as in svhip_entropy_patches); tokens,
 * last, chosen and scores_out stay in (y, z, x) order. Workspace: svhip_ease_select_workspace_bytes.
 * Replaces: the permute of fast_ops.py:305-308 followed by FastLowEntropyLastSlot.select (fast_ops.py:534-540).
 */
int svhip_ease_select_patches(const void* logits, int dtype, int64_t classes, int64_t patch, int64_t stride_b,
                              int64_t stride_n, const int64_t* tokens, int64_t mask_token, const uint8_t* last,
                              int64_t batch, int64_t Y, int64_t Z, int64_t X, int64_t block, const int64_t* k,
                              const int64_t* pos, const double* frac, const int64_t* n_total,
                              const int64_t* committed, uint8_t* chosen, uint8_t* bad, float* scores_out,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * Cross attention over per-window, variable-length cached keys:
 *   O[b,h,q,:] = sum_{j < L_b} softmax_j(scale * Q[b,h,q,:] . K[b,h,j,:]) V[b,h,j,:]
 * with L_b = min(kv_len[b], kv_cap) (device int32 [B]) or, for the packed layout, cu_seqlens[b+1] - cu_seqlens[b] with key j of
 * window b at row cu_seqlens[b] + j. A window with L_b = 0 gets zeros. cu_seqlens stays on the device and is
 * read as given (no host check, which would need a synchronisation): it must be non-decreasing with every row
 * inside the packed K/V, as for the reference's packed attention.
 * Q, O: bf16, element (b,h,q,d) at b*s?_b + h*s?_h + q*s?_q + d. K: element (b,h,j,d) at
 * b*sk_b + h*sk_h + row*sk_k + d; V: at b*sv_b + h*sv_h + row*sv_k + d*sv_d, where either sv_d == 1 (rows of
 * head_dim, the reference layout) or sv_k == 1 (V stored transposed, keys contiguous). bf16 K and V with
 * 16-byte aligned rows take the fast staging path (V^T of the padded layout, V rows of either layout);
 * row = j, or cu_seqlens[b] + j in the packed layout (sk_b / sv_b are then ignored). kv_dtype SVHIP_BF16, or
 * e4m3 (OCP e4m3fn bytes) with per-(window, head) fp32 dequantisation scales k_scale/v_scale [B,H]:
 * SVHIP_FP8_E4M3 decodes K and V exactly to bf16 in the kernel and keeps P in bf16 (the reference's in-kernel
 * dequantisation with fp32 accumulation: within 5e-2 of fp32 attention over the unquantised K/V);
 * SVHIP_FP8_E4M3_PFP8, an opt-in outside that bar, takes P . V on the fp8 matrix cores with P rounded to e4m3 (a
 * relative rounding of 2^-4 on every softmax weight, the row sum taken over the rounded weights; up to about 8e-2
 * on rows whose logits have a standard deviation of 4). Q . K^T is a bf16 product of the exactly decoded keys in
 * both. head_dim: a multiple of 8 up to 128 (zero-padded inside the kernel to 64, 96 or 128: the 384-wide
 * model's 48, the 768-wide model's 96). fp32 accumulation.
 * scale: the softmax scale, > 0 (the reference uses 1/sqrt(head_dim)).
 * Replaces: flex_attention over PackedKeys' block mask in cross_flex (streamvoxel/stream/fast_ops.py:104-108,
 * 122-159) and the masked SDPA in SlotCrossAttention.forward / cross_sdpa (streamvoxel/stream/engine.py:28-47,
 * streamvoxel/stream/fast_ops.py:111-115).
 */
int svhip_xattn_fwd(const void* q, const void* k, const void* v, void* o, int kv_dtype, const int32_t* kv_len,
                    const int32_t* cu_seqlens, const float* k_scale, const float* v_scale, int64_t B, int64_t H,
                    int64_t Q, int64_t D, int64_t kv_cap, int64_t sq_b, int64_t sq_h, int64_t sq_q, int64_t sk_b,
                    int64_t sk_h, int64_t sk_k, int64_t sv_b, int64_t sv_h, int64_t sv_k, int64_t sv_d,
                    int64_t so_b, int64_t so_h, int64_t so_q, float scale, void* stream);

/*
 * svhip_xattn_fwd with a boolean key mask: key j of window b is attended iff kv_mask[b * sm_b + j] != 0 (bytes,
 * at least kv_cap per window; with cu_seqlens, j counts from the window's first row), within the window length
 * (kv_len[b], or the cu_seqlens length, or kv_cap when both are NULL; clamped to kv_cap, the width of the mask
 * rows). Any pattern of attended
 * keys; a query with no attended key gets zeros. bf16 K/V only.
 * Replaces: the boolean attn_mask of the masked SDPA in cross_sdpa (streamvoxel/stream/fast_ops.py:111-115) and
 * SlotCrossAttention.forward (streamvoxel/stream/engine.py:28-47), whatever the mask's shape.
 */
int svhip_xattn_fwd_masked(const void* q, const void* k, const void* v, void* o, const uint8_t* kv_mask, int64_t sm_b,
                           const int32_t* kv_len, const int32_t* cu_seqlens, int64_t B, int64_t H, int64_t Q,
                           int64_t D, int64_t kv_cap, int64_t sq_b, int64_t sq_h, int64_t sq_q, int64_t sk_b,
                           int64_t sk_h, int64_t sk_k, int64_t sv_b, int64_t sv_h, int64_t sv_k, int64_t sv_d,
                           int64_t so_b, int64_t so_h, int64_t so_q, float scale, void* stream);

/*
 * The effective window lengths of a key mask: out[b] (int32, device) = 1 + the last key j < n_b with
 * kv_mask[b * sm_b + j] != 0, or 0 when there is none, where n_b = min(kv_len[b], kv_cap) (kv_cap when kv_len is
 * NULL). Passed to svhip_xattn_fwd_masked as kv_len it gives the same output (the keys past a window's last
 * attended key add nothing) and lets the kernel rank the windows by the keys they really attend.
 * Serves: the masked SDPA of cross_sdpa (streamvoxel/stream/fast_ops.py:111-115), whose `valid` mask holds the
 * window lengths.
 */
int svhip_mask_lengths(const uint8_t* kv_mask, int64_t sm_b, const int32_t* kv_len, int64_t B, int64_t kv_cap,
                       int32_t* out, void* stream);

/*
 * Cross attention in fp32 arithmetic: fp32 q/k/v/o with the layouts and strides of svhip_xattn_fwd (elements, not
 * bytes; rows 16-byte aligned; V as rows or as V^T), padded with kv_len or packed with cu_seqlens; head_dim 16, 32,
 * 48 or 64. Every product, sum and exponential is fp32 (the VALU; no rounding of the operands), at the fp32 FMA
 * rate. A window with no key gives zeros.
 * Replaces: the SDPA of SlotCrossAttention.forward (streamvoxel/stream/engine.py:28-47) as the reference runs it on
 * fp32 tensors (its CPU path, the single-column configuration) where the window lengths hold its mask; any other
 * mask takes svhip_xattn_fwd_f32_masked.
 */
int svhip_xattn_fwd_f32(const float* q, const float* k, const float* v, float* o, const int32_t* kv_len,
                        const int32_t* cu_seqlens, int64_t B, int64_t H, int64_t Q, int64_t D, int64_t kv_cap,
                        int64_t sq_b, int64_t sq_h, int64_t sq_q, int64_t sk_b, int64_t sk_h, int64_t sk_k,
                        int64_t sv_b, int64_t sv_h, int64_t sv_k, int64_t sv_d, int64_t so_b, int64_t so_h,
                        int64_t so_q, float scale, void* stream);

/*
 * svhip_xattn_fwd_f32 with a key mask, in fp32 arithmetic: key j of window b is attended only where
 * kv_mask[b * sm_b + j] != 0 (one byte per key, any pattern; keys counted from the window's first, also in the
 * packed layout, whose windows are then cut at kv_cap keys). kv_len and cu_seqlens may both be NULL: every window
 * then spans kv_cap keys and the mask decides. A query with no attended key gets zeros (as torch's SDPA returns
 * for a fully masked row on the CPU).
 * Replaces: the masked SDPA of SlotCrossAttention.forward (streamvoxel/stream/engine.py:28-47) on fp32 tensors, its
 * mask `prefix_valid ++ local_valid` over the padded prefix and the padded local keys (engine.py:44-46).
 */
int svhip_xattn_fwd_f32_masked(const float* q, const float* k, const float* v, float* o, const uint8_t* kv_mask,
                               int64_t sm_b, const int32_t* kv_len, const int32_t* cu_seqlens, int64_t B, int64_t H,
                               int64_t Q, int64_t D, int64_t kv_cap, int64_t sq_b, int64_t sq_h, int64_t sq_q,
                               int64_t sk_b, int64_t sk_h, int64_t sk_k, int64_t sv_b, int64_t sv_h, int64_t sv_k,
                               int64_t sv_d, int64_t so_b, int64_t so_h, int64_t so_q, float scale, void* stream);

/*
 * AxialRoPE of bf16 activations: x [B,H,N,D] (element (b,h,n,d) at b*sx_b + h*sx_h + n*sx_n + d) -> out (same
 * shape, own strides; out may equal x). D, a multiple of 6, splits into three axes of D/3; in axis t the pair
 * (x[2i], x[2i+1]) (i < D/6 within the axis) turns by phase = positions[b,n,t] * freq[i] (fp32, positions element
 * (b,n,t) at b*sp_b + n*sp_n + t). sin/cos are rounded to bf16 and every product and sum to bf16, in the order of
 * the reference module. freq: fp32 [D/6], the module's `frequencies` buffer (base^(-2i/(D/3))).
 * Replaces: AxialRoPE.forward (streamvoxel/models/unconditional_md4.py:18-24) as used by cross_query and local_kv
 * (streamvoxel/stream/fast_ops.py:90-101) and RotaryCrossAttention.encode_kv
 * (streamvoxel/models/streaming_controlnet.py:31-35).
 */
int svhip_axial_rope(const void* x, void* out, const float* positions, const float* freq, int64_t B, int64_t H,
                     int64_t N, int64_t D, int64_t sx_b, int64_t sx_h, int64_t sx_n, int64_t so_b, int64_t so_h,
                     int64_t so_n, int64_t sp_b, int64_t sp_n, void* stream);

/*
 * One window of the cached cross-attention context: keys [0, P) from the prefix bank (bf16 [H,P,D], rows
 * spk_l / spv_l apart, heads spk_h / spv_h apart; already rotated), keys [P, P+L) from the local projection (bf16
 * [H,L,D]; K rotated by AxialRoPE at positions [L,3] fp32 (rows sp_l apart) when positions is not NULL, with freq
 * as for svhip_axial_rope), zeros for keys [P+L, kv_cap). Written to the window's cache: K element (h,j,d) at
 * h*sck_h + j*sck_k + d; V at h*scv_h + j*scv_k + d*scv_d with scv_d == 1 (rows) or scv_k == 1 (transposed, keys
 * contiguous). kv_dtype SVHIP_BF16, or SVHIP_FP8_E4M3: per-head scales k_scale/v_scale [H] = max(amax/448, 1e-12)
 * over the window's keys are written and the codes are round-to-nearest-even e4m3fn of x / scale; the e4m3 form
 * needs a workspace of svhip_kv_write_workspace_bytes(H, kv_cap) bytes.
 * Replaces: FastSlotForward.encode + _write (streamvoxel/stream/fast_ops.py:228-250, local_kv :90-95) and the
 * per-head amax/448 e4m3 quantisation of the cached K/V (scripts/bench_ops.py:506-522).
 */
size_t svhip_kv_write_workspace_bytes(int64_t H, int64_t kv_cap);
int svhip_kv_write(const void* prefix_k, const void* prefix_v, int64_t P, int64_t spk_h, int64_t spk_l,
                   int64_t spv_h, int64_t spv_l, const void* local_k, const void* local_v, int64_t L, int64_t slk_h,
                   int64_t slk_l, int64_t slv_h, int64_t slv_l, const float* positions, int64_t sp_l,
                   const float* freq, int64_t H, int64_t D, void* cache_k, int64_t sck_h, int64_t sck_k,
                   void* cache_v, int64_t scv_h, int64_t scv_k, int64_t scv_d, int64_t kv_cap, int kv_dtype,
                   float* k_scale, float* v_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Self-attention operands of a transformer block from its fused qkv projection: qkv bf16, element (b,n,s,h,d)
 * (s = 0 Q, 1 K, 2 V; the Linear's [3, H, D] row) at b*sx_b + n*sx_n + (s*H + h)*D + d, rows 16-byte aligned.
 * Q and K are rotated by AxialRoPE at positions [B,N,3] fp32 (element (b,n,t) at b*sp_b + n*sp_n + t) with freq
 * [D/6] exactly as svhip_axial_rope does, and written to q / k (element (b,h,n,d) at b*s?_b + h*s?_h + n*s?_n + d,
 * 16-byte aligned rows; they may be the Q / K slices of qkv itself: in place); V is written transposed to vt
 * (element (b,h,d,n) at b*svt_b + h*svt_h + d*svt_d + n, 16-byte aligned rows), the layout svhip_xattn_fwd stages
 * directly into LDS. sin / cos of a (token, pair) are evaluated once for Q and K of every head.
 * head_dim: a multiple of 24 up to 128 (48 and 96 in the shipped models).
 * Replaces: the qkv split, the two AxialRoPE calls and the layout change before F.scaled_dot_product_attention in
 * RotaryAttention.forward (streamvoxel/models/unconditional_md4_timefree.py:41-47, unconditional_md4.py:35-41).
 */
int svhip_qkv_rope(const void* qkv, const float* positions, const float* freq, int64_t B, int64_t N, int64_t H,
                   int64_t D, int64_t sx_b, int64_t sx_n, int64_t sp_b, int64_t sp_n, void* q, int64_t sq_b,
                   int64_t sq_h, int64_t sq_n, void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, void* vt,
                   int64_t svt_b, int64_t svt_h, int64_t svt_d, void* stream);

/*
 * LayerNorm over the last axis of bf16 rows, with the AdaLN modulation fused in:
 *   y = LN(x) * (1 + scale[b]) + shift[b],   LN(x) = (x - mean) / sqrt(var + eps) * weight + bias
 * x, y bf16 [B,N,W] (element (b,n,c) at b*s?_b + n*s?_n + c, 16-byte aligned rows; y may be x). weight / bias fp32
 * [W] or NULL (no affine; bias needs weight); shift / scale bf16 [B,W] (rows s_mod apart) or both NULL (no
 * modulation). Mean and biased variance in fp32; 1 + scale rounded to bf16 (as the reference's bf16 tensors
 * compute it); y rounded once. W: a multiple of 8 up to 2048.
 * Replaces: modulate(norm1(x), s1, c1) / modulate(norm2(x), s2, c2) of UnconditionalBlock.forward
 * (streamvoxel/models/unconditional_md4_timefree.py:12-13,60-63) and norm1 / norm2 of the affine block
 * (streamvoxel/models/unconditional_md4.py:44-56).
 */
int svhip_layer_norm(const void* x, void* y, const float* weight, const float* bias, const void* shift,
                     const void* scale, int64_t B, int64_t N, int64_t W, int64_t sx_b, int64_t sx_n, int64_t sy_b,
                     int64_t sy_n, int64_t s_mod, float eps, void* stream);

/*
 * The gated residual of a block, optionally followed by the next LayerNorm (+ AdaLN), in one pass:
 *   r = x + gate[b] * branch    (the product and the sum each rounded to bf16, as `x + g[:, None] * f(...)` is
 *                                in the reference's bf16 tensors; gate NULL: r = x + branch)
 *   y = LN(r) * (1 + scale[b]) + shift[b]   (as svhip_layer_norm; y NULL: only r is written)
 * x, branch, r, y bf16 [B,N,W] with 16-byte aligned rows (element (b,n,c) at b*s?_b + n*s?_n + c; r may be x);
 * gate bf16 [B,W] rows s_gate apart; weight / bias / shift / scale / s_mod / eps as for svhip_layer_norm.
 * Replaces: `x + g1[:, None] * self.attn(...)` followed by `modulate(self.norm2(x), s2, c2)`, and
 * `x + g2[:, None] * self.mlp(...)`, of UnconditionalBlock.forward
 * (streamvoxel/models/unconditional_md4_timefree.py:60-63; unconditional_md4.py:52-56 without gates).
 */
int svhip_residual_norm(const void* x, const void* branch, const void* gate, int64_t s_gate, void* r, void* y,
                        const float* weight, const float* bias, const void* shift, const void* scale, int64_t s_mod,
                        int64_t B, int64_t N, int64_t W, int64_t sx_b, int64_t sx_n, int64_t sa_b, int64_t sa_n,
                        int64_t sr_b, int64_t sr_n, int64_t sy_b, int64_t sy_n, float eps, void* stream);

/*
 * Gather patchify of voxel tokens (int64 [B,Y,Z,X], element (b,y,z,x) at b*st_b + (y*Z + z)*X + x, values in
 * [0, cells)): out[b,n,:] = bias + sum_{o < p^3} table[tokens(b, voxel(n, o)) * p^3 + o, :], patch token n row-major
 * over the (Y/p, Z/p, X/p) grid, kernel offset o = (dy*p + dz)*p + dx. table bf16 [cells * p^3, W] (16-byte aligned
 * rows) = the patch Conv3d weight permuted to [cell, dy, dz, dx, W]; bias bf16 [W] or NULL; out bf16, element
 * (b,n,c) at b*so_b + n*so_n + c. The p^3 rows are summed in fp32 in offset order and rounded to bf16, then the
 * bias is added with one more bf16 rounding. A token outside [0, cells) counts as 0 and sets *bad (device int) to
 * a non-zero value. p^3 <= 64, W a multiple of 8 up to 2048.
 * Replaces: GatherPatch.__call__ (streamvoxel/stream/fast_ops.py:54-75: patch_offsets + F.embedding_bag(mode='sum')
 * + bias), equal to the one-hot Conv3d patchify of UnconditionalMD4DiT.patchify
 * (streamvoxel/models/unconditional_md4_timefree.py:141-147).
 */
int svhip_patch_embed(const int64_t* tokens, const void* table, const void* bias, void* out, int* bad, int64_t B,
                      int64_t Y, int64_t Z, int64_t X, int64_t patch, int64_t cells, int64_t W, int64_t st_b,
                      int64_t so_b, int64_t so_n, void* stream);

/*
 * Counter-based categorical sampling of the chosen voxels of `batch` windows [Y,Z,X], at a fixed launch size.
 * Logit (b, class c, voxel v) at b*stride_b + c*stride_c + row(v)*stride_n, row(v) = v (patch == 0, YZX order) or
 * the class head's patch order (patch > 0, row map as in svhip_entropy_patches). chosen u8 [batch, N]; values
 * int16 [batch, N] gets the class of every chosen voxel and -1 elsewhere; tokens int64 [batch, N] (or NULL) gets the
 * class of every chosen voxel, other entries untouched. seed, step: device int64 [batch]. Voxel v of window b draws
 * u = (floor(w0 / 2^41) + 1/2) / 2^23 from Philox4x64-10 at counter (v, step[b], 0, 0) under key
 * (seed[b], 0x53414D504C455631) and takes the first class whose softmax CDF passes u (fp32 sums). A chosen row with
 * no finite maximum or a NaN sets *err (device int) and draws nothing: its value reads -1 and its token is left as
 * it was. classes <= 1024.
 * Replaces (as a counter-based alternative with its own random stream): the tail of
 * FastLowEntropyLastSlot.stage (streamvoxel/stream/fast_ops.py:548-553: nonzero_static -> gather -> softmax ->
 * torch.multinomial -> index_copy_), whose sizes depend on the step's k.
 */
int svhip_sample_chosen(const void* logits, int dtype, int64_t classes, int64_t patch, int64_t stride_b,
                        int64_t stride_c, int64_t stride_n, const uint8_t* chosen, int64_t* tokens, int16_t* values,
                        const int64_t* seed, const int64_t* step, int* err, int64_t batch, int64_t Y, int64_t Z,
                        int64_t X, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SVHIP_H */
