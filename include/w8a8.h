/*
 * w8a8.h -- C ABI of the MI355X (gfx950) W8A8 SmoothQuant inference path.
 *
 * Every entry point:
 *   - takes caller-allocated device pointers, plain sizes and an explicit
 *     hipStream_t (0 = the null stream the reference samples launch on);
 *   - validates every argument on the host BEFORE any HIP call and returns a
 *     status code instead of exiting (the reference calls exit(1) from its
 *     CHECK_HIP macros, rocwmma_smoothquant.cpp:35-37, common.hpp:34-46);
 *   - is asynchronous with respect to the host: work is enqueued on `stream`.
 *
 * Status codes coincide with hipError_t: 0 = success, 1 = invalid argument
 * (hipErrorInvalidValue), 801 = shape/layout not supported
 * (hipErrorNotSupported); any other value is the HIP runtime error that the
 * launch reported.  w8a8_last_error() returns a human-readable message for
 * the last failing call on the calling thread.
 *
 * fp16 tensors are passed as `const void*` / `void*` holding IEEE binary16.
 */
#ifndef W8A8_H
#define W8A8_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W8A8_SUCCESS 0
#define W8A8_ERROR_INVALID_VALUE 1
#define W8A8_ERROR_NOT_SUPPORTED 801

/* GEMM operand layouts. */
#define W8A8_LAYOUT_A_ROW_B_NK 0 /* A [M,K] row-major (lda>=K); B [N,K] K-contiguous (ldb>=K) */
#define W8A8_LAYOUT_A_COL_B_KN 1 /* A col-major (lda>=M); B [K,N] row-major (ldb>=N): the
                                    layout of rocwmma_gemm_quantized.cpp:92-95,205 */

/* GEMM output types. */
#define W8A8_OUT_I32 0 /* raw int32 accumulators (verification mode)            */
#define W8A8_OUT_F16 1 /* fp16 after the fused per-token x per-channel dequant  */

/* Version / diagnostics. */
const char* w8a8_version(void);
const char* w8a8_last_error(void);

/* ------------------------------------------------------------------------- */
/* Quantizer                                                                  */
/* ------------------------------------------------------------------------- */

/*
 * Row-wise smooth-scale + absmax int8 quantization.
 * Replaces kernel_smoothquant (rocwmma_smoothquant.cpp:58-122), launched at
 * rocwmma_smoothquant.cpp:153-155 with (dX, dS, dY, dRS, M, N, 127.f).
 *   x           fp16 [M, ldx]   (ldx = 0 means N)
 *   smooth_scale fp32 [N]
 *   y           int8 [M, ldy]   (ldy = 0 means N); row-major, i.e. the A
 *                               operand of w8a8_gemm in W8A8_LAYOUT_A_ROW_B_NK
 *   row_scale   fp32 [M]        r[m] = max_n |x*s| / quant_max
 *   quant_max   in (0, 127]
 * Any N >= 1 is accepted (the reference needs N % 8 == 0 for its vector loop).
 */
int w8a8_smoothquant(const void* x, const float* smooth_scale, int8_t* y, float* row_scale,
                     uint32_t M, uint32_t N, float quant_max, uint32_t ldx, uint32_t ldy,
                     hipStream_t stream);

/*
 * MoE smooth quantization with per-expert smooth scales.
 * Replaces kernel_moe_smoothquant (rocwmma_moe_smoothquant.cpp:69-131).
 *   x            fp16 [tokens, hidden]
 *   smooth_scale fp32 [experts, hidden]
 *   topk_ids     int32 [tokens, topk]
 *   qy           int8  [rows, hidden], row_scale fp32 [rows]
 *   dst_row      NULL  -> pair (t, slot) writes row t*topk + slot (the
 *                         reference's token-major layout, :91); rows = tokens*topk
 *                non-NULL -> int32 [tokens*topk] destination row per pair (the
 *                         expert-sorted layout produced by w8a8_moe_sort), so the
 *                         grouped GEMM reads its A operand without a gather pass;
 *                         a negative entry, or one >= rows_out, skips the pair.
 *   rows_out     rows of qy / row_scale (ignored when dst_row is NULL).
 * A pair whose expert id is outside [0, experts) writes nothing (:86-87).
 */
int w8a8_moe_smoothquant(const void* x, const float* smooth_scale, const int32_t* topk_ids,
                         int8_t* qy, float* row_scale, uint32_t tokens, uint32_t hidden,
                         uint32_t topk, uint32_t experts, float quant_max,
                         const int32_t* dst_row, uint32_t rows_out, hipStream_t stream);

/*
 * RMSNorm, optionally after a residual add, fused with the quantizer: the
 * normalised row goes to int8 + row scale without an fp16 round trip through
 * HBM.  Replaces kernel_add_rmsnorm2d_fwd (rocwmma_rmsnorm2d.cpp:127-186) or,
 * with residual = NULL, kernel_rmsnorm2d_fwd (:57-120), followed by
 * kernel_smoothquant (rocwmma_smoothquant.cpp:58-122) on their fp16 output.
 *   x, residual  fp16 [M, ldx]    (ldx = 0 means N; residual NULL = plain RMSNorm)
 *   gamma        fp32 [N]
 *   smooth_scale fp32 [N], or NULL for no quantization (q, row_scale NULL too)
 *   x_out        fp16 [M, ldx] = half(x + residual), or NULL; needs a residual;
 *                may be x or residual itself (updated in place)
 *   y            fp16 [M, ldy] normalised row (ldy = 0 means N), or NULL
 *   q, row_scale int8 [M, ldq] (ldq = 0 means N), fp32 [M]
 *   eps >= 0 (the reference uses 1e-5), quant_max in (0, 127]
 * Per row, in fp32:
 *   v = float(x) [+ float(residual)];  rstd = rsqrt(sum_n v^2 / N + eps)
 *   u = residual ? float(half(v)) : v  (the reference normalises the saved sum, :173-182)
 *   y = half((u * rstd) * gamma[n]);   q, row_scale = quantizer(y, smooth_scale)
 * At least one of x_out, y, q must be given.  The sum of squares is an fp32
 * sum in this kernel's order, so y may differ from the reference's by one
 * fp16 ulp where the two sums round differently; q and row_scale are exactly
 * w8a8_smoothquant of this call's y.
 */
int w8a8_add_rmsnorm_smoothquant(const void* x, const void* residual, const float* gamma,
                                 const float* smooth_scale, void* x_out, void* y, int8_t* q,
                                 float* row_scale, uint32_t M, uint32_t N, float eps,
                                 float quant_max, uint32_t ldx, uint32_t ldy, uint32_t ldq,
                                 hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* int8 GEMM with fused dequant                                               */
/* ------------------------------------------------------------------------- */

/*
 * Bytes of device workspace w8a8_gemm can use for this problem.  Sample
 * layout: A and B are repacked K-contiguous into it.  Primary layout: int32
 * K-split partials when the problem's tiles would fill at most half of the
 * CUs (0 otherwise); the rocWMMA split-K sample likewise takes a
 * caller-allocated workspace (rocwmma_gemm_splitk.cpp:214).
 */
size_t w8a8_gemm_workspace_size(uint32_t m, uint32_t n, uint32_t k, int layout);

/*
 * C = dequant(A . B^T).  Replaces gemm_quant_tensor_scale
 * (rocwmma_gemm_quantized.cpp:127-195) and implements its documented Mode 2
 * (:18-26), which the reference does not implement:
 *   acc[m,n] = sum_k int32(A[m,k]) * int32(B[n,k])      (exact int32)
 *   out_type W8A8_OUT_I32: C int32 [m, ldc] = acc
 *   out_type W8A8_OUT_F16: C fp16  [m, ldc] =
 *       scale_a == NULL && scale_b == NULL:
 *           half(float(acc) * (tensor_scale_a * tensor_scale_b))   (Mode 1, :189-193)
 *       otherwise:
 *           half((float(acc) * sa) * sb),  sa = scale_a ? scale_a[m] : tensor_scale_a,
 *                                          sb = scale_b ? scale_b[n] : tensor_scale_b
 * Argument order follows gemm_quant_tensor_scale (m, n, k, a, b, c, lda, ldb, ldc, scales).
 * Decode shapes (m <= 64) run a weight-streaming kernel that splits K across
 * the waves of each block and reduces the int32 partials in LDS: the role of
 * gemm_splitk_stage1/gemm_splitk_reduce (rocwmma_gemm_splitk.cpp:104-201) and
 * streamk_gemm_kernel (rocwmma_streamk_gemm.cpp:86-211), in one launch with no
 * workspace, bit-identical to the full GEMM.
 * Primary layout with a workspace (16-byte aligned, at least
 * w8a8_gemm_workspace_size bytes; NULL or smaller: not used): a problem
 * whose tiles fill at most half of the CUs runs each tile as K pieces on the
 * idle CUs, the pieces' int32 partials go to the workspace and a second
 * launch sums them, again bit-identical.  Calls sharing a workspace must be
 * ordered on one stream.
 */
int w8a8_gemm(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b, void* c,
              uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
              const float* scale_b, float tensor_scale_a, float tensor_scale_b, int out_type,
              int layout, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Stream-K GEMM: replaces streamk_gemm_kernel + streamk_reduce_kernel
 * (rocwmma_streamk_gemm.cpp:86-211, host :213-284).  Same arithmetic and
 * arguments as w8a8_gemm, primary layout only (A [m, lda] row-major, B
 * [n, ldb] K-contiguous, 16-byte aligned, lda, ldb, k multiples of 16, A and
 * B each under 2 GiB).  All tiles' k-tiles are cut into `blocks` contiguous
 * equal ranges (never more than the problem's k-tiles), one block each, as
 * the reference sample's units_per_cta (:223-226); 0: the library picks the
 * count, at most one per CU, and the tile shape from an estimate of the
 * longest block's work plus the partials it sums (any count and shape give
 * the same C); a tile
 * covered by several blocks is summed in int32 by the last of them to finish
 * (one launch, no host synchronisation), so C equals w8a8_gemm's bit for bit.
 * workspace: 16-byte aligned, w8a8_gemm_streamk_workspace_size bytes (tile
 * counters and partials; cleared by the call itself, no memset).  Calls
 * sharing a workspace must be ordered on one stream.
 */
size_t w8a8_gemm_streamk_workspace_size(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks);
int w8a8_gemm_streamk(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b,
                      void* c, uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
                      const float* scale_b, float tensor_scale_a, float tensor_scale_b,
                      int out_type, uint32_t blocks, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/*
 * The block count w8a8_gemm_streamk launches for this shape and `blocks`
 * argument (0: the count the library picks; otherwise min(blocks, the
 * problem's k-tiles)); 0 for an empty problem.  The reference sample prints
 * its num_cus (rocwmma_streamk_gemm.cpp:223-226, :268-270).
 */
uint32_t w8a8_gemm_streamk_blocks(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks);

/*
 * Sticky status of w8a8_gemm_streamk on the current device.  The last piece
 * of a split tile waits for the other pieces' partials with a bounded poll
 * (about 2^24 sleeps; never reached when every piece runs); if the bound
 * expires it still finishes the tile, so every wave exits, but that tile may
 * be wrong, and the launch sets W8A8_STREAMK_WAIT_EXPIRED in a per-device
 * word that stays set until read with clear != 0.  The query synchronizes
 * the device first (hipDeviceSynchronize), so it covers every launch already
 * enqueued on any stream; it is a diagnostic, not for hot loops.  No
 * counterpart in the reference (its reduce launch has no wait).
 */
#define W8A8_STREAMK_WAIT_EXPIRED 1u
int w8a8_gemm_streamk_status(uint32_t* flags, int clear);

/*
 * Test hook of the bounded wait above: spin_limit polls before giving up
 * (0: the default) and phantom_pieces pieces that the last piece of every
 * split tile also waits for (0: none).  With phantom_pieces > 0 every split
 * tile gives up after spin_limit polls (which must be in [1, 4096]), sums
 * the partials that are there (all of them: the real pieces have arrived)
 * and sets W8A8_STREAMK_WAIT_EXPIRED; nothing waits forever.  Process-wide;
 * call w8a8_debug_streamk_wait(0, 0) to restore the defaults.
 */
int w8a8_debug_streamk_wait(uint32_t spin_limit, uint32_t phantom_pieces);

/*
 * Bytes of the per-GPU scratch array w8a8_gemm_noalloc uses (32 MiB).
 */
#define W8A8_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * w8a8_gemm without a workspace argument and without any allocation: the
 * workspace w8a8_gemm would take (K-split partials, the sample layout's
 * repack) is a scratch array the library holds on each GPU it runs on, of
 * W8A8_NOALLOC_SCRATCH_BYTES, kept until the process ends.  Results are
 * bit-identical to w8a8_gemm given a workspace of that size.  Shapes whose
 * w8a8_gemm_workspace_size exceeds it return W8A8_ERROR_INVALID_VALUE
 * before any HIP call.  The entry point calls no allocating routine (no
 * hipMalloc / hipFree), for callers that cannot allocate: code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation.
 * Every call on one GPU shares that GPU's array, and nothing in it needs
 * clearing between calls (each call writes what it reads); calls that overlap
 * on one GPU (several streams, several host threads) race on it and must be
 * ordered.  No counterpart in the reference.
 */
int w8a8_gemm_noalloc(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b,
                      void* c, uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
                      const float* scale_b, float tensor_scale_a, float tensor_scale_b,
                      int out_type, int layout, hipStream_t stream);

/*
 * Fused SmoothQuant + W8A8 GEMM for one linear layer:
 *   (q, r) = smoothquant(x, smooth_scale)       q int8 [m, k], r fp32 [m]
 *   c      = half((float(q . w^T) * r[m]) * scale_w[n])
 *   x fp16 [m, ldx]; w int8 [n, ldw] (K-contiguous weights); c fp16 [m, ldc].
 * q and row_scale are caller-provided buffers (m*k bytes, m floats): they are
 * written, so the caller can reuse the quantized activations for several GEMMs.
 * workspace / ws_bytes: as for w8a8_gemm (primary layout; NULL, 0 allowed).
 */
int w8a8_fused_sq_gemm(const void* x, const float* smooth_scale, const int8_t* w,
                       const float* scale_w, void* c, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t ldx, uint32_t ldw, uint32_t ldc, int8_t* q, float* row_scale,
                       void* workspace, size_t ws_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* Packed ("pre-shuffled") weights                                            */
/* ------------------------------------------------------------------------- */

/*
 * Weights packed once into MFMA register order so that every wave-load of the
 * GEMM reads 1 KiB contiguous: the "pre-shuffled B" that flatmm_kernel's
 * comment describes (rocwmma_flatmm.cpp:12-16) but its code leaves row-major.
 * Layout: N padded to 64-row slabs, K to 128-deep k-tiles, 8 KiB per
 * (slab, k-tile), zero padding.
 */
size_t w8a8_pack_weights_size(uint32_t n, uint32_t k);

/* packed <- w (int8 [n, ldw], K-contiguous); packed_bytes >= w8a8_pack_weights_size. */
int w8a8_pack_weights(const int8_t* w, uint32_t n, uint32_t k, uint32_t ldw, int8_t* packed,
                      size_t packed_bytes, hipStream_t stream);

/* Smooth-scale folding modes of w8a8_quantize_weights. */
#define W8A8_FOLD_MULTIPLY 0 /* w[n,k] * smooth_scale[k]                               */
#define W8A8_FOLD_DIVIDE 1   /* w[n,k] / smooth_scale[k]: the weight side of activations
                                quantized as x * smooth_scale, so (x*s) . (w/s)^T = x . w^T */

/*
 * Offline weight preparation: SmoothQuant folding, per-output-channel absmax
 * int8 quantization and (optionally) packing, in one pass over the fp16
 * weights.  The reference has no weight-side routine (its samples take int8
 * weights as given); per row n this is the quantizer of
 * rocwmma_smoothquant.cpp:74-121 applied to the folded weights:
 *   p[k]       = float(w[n,k]) (* or /) smooth_scale[k]   (smooth_scale NULL: p = float(w))
 *   scale_w[n] = max_k |p[k]| / quant_max;  inv = scale_w[n] > 0 ? 1 / scale_w[n] : 0
 *   w_q[n,k]   = int8(clamp(rint(p[k] * inv), -quant_max, quant_max))
 * so FOLD_MULTIPLY gives exactly w8a8_smoothquant(w, smooth_scale).
 *   w          fp16 [n, ldw] (ldw = 0 means k)
 *   packed = 0 w_q int8 [n, ldq] row-major (ldq = 0 means k); out_bytes >= (n-1)*ldq + k
 *   packed = 1 w_q in the w8a8_pack_weights layout (ldq unused);
 *              out_bytes >= w8a8_pack_weights_size(n, k)
 *   scale_w    fp32 [n]: the per-channel scale the GEMMs take as scale_b
 */
int w8a8_quantize_weights(const void* w, uint32_t n, uint32_t k, uint32_t ldw,
                          const float* smooth_scale, int fold, float quant_max, int8_t* w_q,
                          uint32_t ldq, int packed, size_t out_bytes, float* scale_w,
                          hipStream_t stream);

/*
 * Bytes of device workspace w8a8_gemm_packed / w8a8_fused_sq_gemm_packed can
 * use for an m x n x k problem: the int32 split-K partials of decode shapes
 * with 32 < m <= 64 (the caller-allocated workspace of the reference's
 * split-K, rocwmma_gemm_splitk.cpp:214); 0 when the shape takes no workspace.
 */
size_t w8a8_gemm_packed_workspace_size(uint32_t m, uint32_t n, uint32_t k);

/*
 * w8a8_gemm over packed weights (layout W8A8_LAYOUT_A_ROW_B_NK, B = the packed
 * buffer of w [n, k]); same outputs bit for bit.  Requires a 16-byte aligned
 * A with lda % 16 == 0 and k % 16 == 0 (W8A8_ERROR_NOT_SUPPORTED otherwise).
 * Decode shapes (m <= 64) stream the packed weights at close to HBM rate.
 * workspace (16-byte aligned, ws_bytes >= w8a8_gemm_packed_workspace_size)
 * lets 32 < m <= 64 split K across blocks; NULL runs the unsplit kernel
 * (same results).
 */
int w8a8_gemm_packed(uint32_t m, uint32_t n, uint32_t k, const int8_t* a,
                     const int8_t* w_packed, void* c, uint32_t lda, uint32_t ldc,
                     const float* scale_a, const float* scale_b, float tensor_scale_a,
                     float tensor_scale_b, int out_type, void* workspace, size_t ws_bytes,
                     hipStream_t stream);

/*
 * w8a8_fused_sq_gemm with packed weights: the decode-time linear layer
 * (smooth-quantize the m token rows, then stream the packed weights once).
 */
int w8a8_fused_sq_gemm_packed(const void* x, const float* smooth_scale, const int8_t* w_packed,
                              const float* scale_w, void* c, uint32_t m, uint32_t n, uint32_t k,
                              uint32_t ldx, uint32_t ldc, int8_t* q, float* row_scale,
                              void* workspace, size_t ws_bytes,
                              hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* Grouped GEMM and MoE                                                       */
/* ------------------------------------------------------------------------- */

/*
 * One problem of a grouped GEMM: the fields of w8a8_gemm for the
 * W8A8_LAYOUT_A_ROW_B_NK layout.  Mirrors GroupDesc
 * (rocwmma_grouped_gemm.cpp:87-96: A, B, C, M, N, K, lda, ldb, ldc) plus the
 * dequant scales.  A group with m == 0 contributes nothing.
 */
typedef struct w8a8_group_desc {
    const int8_t* a;       /* [m, lda] */
    const int8_t* b;       /* [n, ldb] */
    void*         c;       /* [m, ldc] int32 or fp16 (per out_type) */
    const float*  scale_a; /* [m] or NULL */
    const float*  scale_b; /* [n] or NULL */
    uint32_t      m, n, k;
    uint32_t      lda, ldb, ldc;
    float         tensor_scale_a, tensor_scale_b;
} w8a8_group_desc;

/* Device workspace w8a8_grouped_gemm needs for num_groups descriptors. */
size_t w8a8_grouped_gemm_workspace_size(uint32_t num_groups);

/*
 * Runs every group's w8a8_gemm in one launch.  Replaces grouped_gemm_kernel
 * (rocwmma_grouped_gemm.cpp:104-178), whose host code uploads the descriptor
 * array with a tile_offset prefix in it (:180-226): here `groups` is a HOST array,
 * validated, then copied into `workspace` by one hipMemcpyAsync on `stream`.
 * The call returns before that copy runs: the host array must stay valid and
 * unchanged until the stream has reached it (synchronize the stream, or an
 * event recorded after the call, before reusing it).  A HIP graph that
 * captures the call records the copy, so every replay reads the host array
 * again: keep it alive and unchanged for as long as the graph may run.  Every group needs the
 * fast-path layout (16-byte aligned a/b, lda, ldb, k multiples of 16) and
 * m*lda, n*ldb < 2^31 (W8A8_ERROR_NOT_SUPPORTED otherwise).
 */
int w8a8_grouped_gemm(const w8a8_group_desc* groups, uint32_t num_groups, int out_type,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Softmax + top-k routing.  Replaces kernel_topk_softmax /
 * kernel_topk_softmax_large (rocwmma_topk_softmax.cpp:58-193).
 *   logits  [tokens, experts], fp32 (logits_f16 = 0) or fp16 (logits_f16 = 1;
 *           the reference's input type, :42)
 *   topk_weights fp32 [tokens, topk] = softmax probability of each choice
 *   topk_ids     int32 [tokens, topk], best first; ties go to the lower id.
 * experts <= 4096, topk <= experts (the reference caps at 64 experts, :172).
 */
int w8a8_topk_softmax(const void* logits, int logits_f16, float* topk_weights,
                      int32_t* topk_ids, uint32_t tokens, uint32_t experts, uint32_t topk,
                      hipStream_t stream);

/* Entries w8a8_moe_sort needs in sorted_token_ids: tokens*topk + experts*unit_size
 * (the reference's bound, rocwmma_moe_sorting.cpp:161). */
size_t w8a8_moe_sort_capacity(uint32_t tokens, uint32_t topk, uint32_t experts,
                              uint32_t unit_size);

/*
 * Sorts the (token, slot) pairs by expert.  Replaces kernel_moe_histogram,
 * kernel_prefix_sum and kernel_moe_scatter (rocwmma_moe_sorting.cpp:53-125)
 * with the same outputs, made deterministic: inside an expert, pairs keep
 * ascending order of t*topk + slot.
 *   expert_count [E], expert_start [E+1] (expert_start[E] = padded total),
 *   padded_count [E] (count rounded up to unit_size), sorted_token_ids
 *   [sorted_capacity] (token of each sorted row, -1 in padding), dst_row
 *   [tokens*topk] (sorted row of each pair, -1 for an id outside [0, E)).
 * experts <= 1024.  No memset needed before it.  Without a workspace: one
 * launch of one workgroup.  With one (4-byte aligned, at least
 * w8a8_moe_sort_workspace_size bytes: 4 * E per 1024 pairs; 0 when
 * tokens * topk <= 1024): three launches spread over 1024-pair blocks
 * (block counts, offsets, stable scatter), as the reference splits it into
 * histogram / prefix / scatter; the outputs are identical either way.
 */
size_t w8a8_moe_sort_workspace_size(uint32_t tokens, uint32_t topk, uint32_t experts);

int w8a8_moe_sort(const int32_t* topk_ids, uint32_t tokens, uint32_t topk, uint32_t experts,
                  uint32_t unit_size, int32_t* expert_count, int32_t* expert_start,
                  int32_t* padded_count, int32_t* sorted_token_ids, uint32_t sorted_capacity,
                  int32_t* dst_row, void* workspace, size_t ws_bytes, hipStream_t stream);

/*
 * Expert GEMM over expert-sorted rows (the per-expert GEMMs of
 * moe_gate_up_silu_kernel, rocwmma_fused_moe.cpp:96-158, as one grouped
 * launch).  Expert e multiplies rows [expert_start[e], expert_start[e] +
 * expert_count[e]) of a (int8 [rows, lda]) by its weights
 * w + e*w_expert_stride (int8 [n, ldw]) into the same rows of c, with
 *   c = half((float(acc) * scale_a[row]) * scale_w[e*n + col])
 * (NULL vectors fall back to the tensor scales, as in w8a8_gemm).  The
 * per-expert arrays are read on the device (the output of w8a8_moe_sort), so
 * nothing is synchronized with the host; rows outside [0, rows) are never
 * touched, whatever the arrays hold.
 * workspace (optional, 16-byte aligned, w8a8_moe_gemm_workspace_size bytes;
 * NULL or smaller: not used): when the tiles' last round would leave at
 * least half the CUs idle, its tiles are split along K over those CUs, the
 * int32 partials go to the workspace and a second launch sums them (exact:
 * results are bit-identical with and without a workspace).  The rocWMMA
 * split-K sample likewise takes a caller-allocated workspace
 * (rocwmma_gemm_splitk.cpp:214).  Calls that share a workspace must be
 * ordered on one stream.
 */
size_t w8a8_moe_gemm_workspace_size(uint32_t experts, uint32_t rows, uint32_t n, uint32_t k);

int w8a8_moe_gemm(uint32_t experts, uint32_t rows, uint32_t n, uint32_t k, const int8_t* a,
                  uint32_t lda, const int8_t* w, uint32_t ldw, uint64_t w_expert_stride, void* c,
                  uint32_t ldc, const float* scale_a, const float* scale_w,
                  float tensor_scale_a, float tensor_scale_b, const int32_t* expert_start,
                  const int32_t* expert_count, int out_type, void* workspace, size_t ws_bytes,
                  hipStream_t stream);

/*
 * SiLU(gate) * up requantization between the expert GEMMs: row r of
 * gate_up (fp16 [rows, ld_gu], gate = columns [0, inter), up = [inter, 2*inter))
 * gives a = (g / (1 + exp(-g))) * u [* smooth_scale[e*inter + j]] and the
 * SmoothQuant absmax quantization of a into q (int8 [rows, ldq]) and
 * row_scale [rows].  Only rows inside some expert's [start, start + count)
 * are written.  The reference applies SiLU to every output instead
 * (rocwmma_fused_moe.cpp:153-156); this is the gate*up form.  inter <= 32768.
 */
int w8a8_moe_silu_mul_quant(const void* gate_up, uint32_t ld_gu, const float* smooth_scale,
                            const int32_t* expert_start, const int32_t* expert_count,
                            uint32_t experts, uint32_t rows, uint32_t inter, int8_t* q,
                            uint32_t ldq, float* row_scale, float quant_max, hipStream_t stream);

/*
 * Gate_up weights in the order w8a8_moe_gate_up_silu reads: w int8
 * [experts, 2 * inter, ldw] (rows [0, inter) gate, [inter, 2 * inter) up, as
 * w8a8_moe_gemm takes them) -> w_out int8 [experts, 2 * inter, k] whose rows
 * come in blocks of 32: 16 gate rows, then the 16 up rows of the same outputs
 * (out row r = gate row (r / 32) * 16 + r % 32 for r % 32 < 16, else up row
 * (r / 32) * 16 + r % 32 - 16); scale_w [experts, 2 * inter] (optional) is
 * permuted alike into scale_w_out.  A one-time weight preparation, like
 * w8a8_pack_weights.  inter % 16 == 0; ldw = 0 means k.
 */
int w8a8_moe_interleave_gate_up(const int8_t* w, const float* scale_w, uint32_t experts,
                                uint32_t inter, uint32_t k, uint32_t ldw, int8_t* w_out,
                                float* scale_w_out, hipStream_t stream);

/* Device workspace w8a8_moe_gate_up_silu needs (the fp16 activation, per-row
 * maxima, K-split partials). */
size_t w8a8_moe_gate_up_silu_workspace_size(uint32_t rows, uint32_t inter);

/*
 * The gate_up expert GEMM with SiLU(gate) * up fused in its epilogue, then
 * the requantization for the down GEMM: the role of moe_gate_up_silu_kernel
 * (rocwmma_fused_moe.cpp:96-158, SiLU "in register, no extra global memory
 * round-trip"), computing the gated product that kernel describes (:20, :94)
 * rather than the SiLU of every output it applies (:153-156).  Per sorted row
 * r of expert e and output j < inter:
 *   g, u = fp16 dequant of the GEMM (as w8a8_moe_gemm would write them)
 *   h    = fp16(silu(g) * u)                  (fp32 product, one rounding)
 *   q[r, j], row_scale[r] = SmoothQuant of float(h) * smooth_scale[e*inter + j]
 * i.e. w8a8_moe_gemm + w8a8_moe_silu_mul_quant with the activation rounded
 * to fp16 before it is smoothed, so q may differ by one step from the
 * unfused chain.  The GEMM writes h at half the gate_up width plus, per row,
 * the maxima of |float(h) * s| over its output tiles, so the requantization
 * reads half the bytes the unfused one does and no row reduction is left.
 * a int8 [rows, lda] expert-sorted (w8a8_moe_sort order); w_interleaved from
 * w8a8_moe_interleave_gate_up ([experts, 2 * inter, k]); scale_a [rows],
 * scale_w_interleaved [experts, 2 * inter] (or tensor scales as in
 * w8a8_gemm); smooth_scale [experts, inter] or NULL; q int8 [rows, ldq]
 * (ldq = 0 means inter), row_scale [rows]: only rows inside some expert's
 * [start, start + count) are written.  workspace: 256-byte aligned,
 * w8a8_moe_gate_up_silu_workspace_size bytes.  inter % 16 == 0, inter <=
 * 32768, k % 16 == 0.
 */
int w8a8_moe_gate_up_silu(uint32_t experts, uint32_t rows, uint32_t inter, uint32_t k,
                          const int8_t* a, uint32_t lda, const int8_t* w_interleaved,
                          const float* scale_a, const float* scale_w_interleaved,
                          float tensor_scale_a, float tensor_scale_b,
                          const float* smooth_scale, const int32_t* expert_start,
                          const int32_t* expert_count, int8_t* q, uint32_t ldq, float* row_scale,
                          float quant_max, void* workspace, size_t ws_bytes, hipStream_t stream);

/*
 * Weighted combine back to token order:
 *   out[t, j] = half(sum over slots s (ascending) of
 *                    fma(topk_weights[t, s], float(y[dst_row[t*topk + s], j]), acc))
 * y fp16 [rows_y, ldy] (expert-sorted rows), out fp16 [tokens, ldo]; pairs
 * with dst_row outside [0, rows_y) are skipped.
 */
int w8a8_moe_combine(const void* y, uint32_t ldy, uint32_t rows_y, const float* topk_weights,
                     const int32_t* dst_row, uint32_t tokens, uint32_t topk, uint32_t n,
                     void* out, uint32_t ldo, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_H */
