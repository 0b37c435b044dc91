/*
 * w8a8_oracle.h -- CPU restatement of the reference's W8A8 SmoothQuant path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library (libw8a8.so) never links or calls it.
 *
 * Every function restates one reference routine operation by operation (the
 * reference file:line is given per function) so that the GPU results can be
 * compared bit-for-bit where the arithmetic is exact (int8/int32/index work),
 * and within stated tolerances where it is floating point.
 *
 * fp16 values cross this interface as raw uint16_t bit patterns.
 */
#ifndef W8A8_ORACLE_H
#define W8A8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32 conversions (exact / round-to-nearest-even). */
float    w8a8o_half_to_float(uint16_t h);
uint16_t w8a8o_float_to_half(float f);

/* Number of OpenMP threads the oracle runs with (1 when built without OpenMP). */
int w8a8o_num_threads(void);

/*
 * Row-wise SmoothQuant.  Restates kernel_smoothquant
 * (rocwmma_smoothquant.cpp:58-122):
 *   p        = float(x[m,n]) * s[n]                        (:84-85)
 *   amax     = max_n |p|                                   (:76-96)
 *   r[m]     = amax / quant_max                            (:95)
 *   inv      = r > 0 ? 1 / r : 0                           (:98)
 *   q[m,n]   = int8(min(max(rint(p * inv), -qmax), qmax))  (:110-113)
 * ldx / ldq are row strides in elements.
 */
void w8a8o_smoothquant(const uint16_t* x, const float* s, int8_t* q, float* r,
                       uint32_t M, uint32_t N, float quant_max,
                       uint32_t ldx, uint32_t ldq);

/*
 * MoE SmoothQuant.  Restates kernel_moe_smoothquant
 * (rocwmma_moe_smoothquant.cpp:69-131): flat = t*topk + slot, e = ids[flat];
 * an expert id outside [0, experts) leaves the destination row and its row
 * scale untouched (:86-87).  Destination row is `flat` (reference layout,
 * :91) or dst_row[flat] when dst_row != NULL (expert-sorted layout).
 */
void w8a8o_moe_smoothquant(const uint16_t* x, const float* s, const int32_t* topk_ids,
                           int8_t* qy, float* row_scale,
                           uint32_t tokens, uint32_t hidden, uint32_t topk,
                           uint32_t experts, float quant_max, const int32_t* dst_row);

/*
 * RMSNorm, optionally after a residual add, then the quantizer on its fp16
 * output.  Restates kernel_add_rmsnorm2d_fwd (rocwmma_rmsnorm2d.cpp:127-186)
 * or, with res == NULL, kernel_rmsnorm2d_fwd (:57-120), followed by
 * kernel_smoothquant:
 *   v[n]   = float(x[m,n]) (+ float(res[m,n]))            (:157-158 / :79-80)
 *   x_out  = half(v)                                      (:159)
 *   rstd   = rsqrt(float(sum_n v^2) / N + eps)            (:170 / :99)
 *   u[n]   = res ? float(x_out[m,n]) : v[n]               (:173-180)
 *   y[m,n] = half((u * rstd) * gamma[n])                  (:182 / :112)
 *   q, r   = w8a8o_smoothquant(y, s)                      (when q != NULL)
 * The sum of squares is taken in float64 (the reference sums in fp32 in its
 * thread and wave order, which no CPU order reproduces) and the reciprocal
 * square root is correctly rounded (the reference's rsqrtf is the GPU's).
 * Where the reference's N % 2048 != 0 tail loop counts columns twice
 * (kernel_rmsnorm2d_fwd, :83-85 after :74-82) this restates the intended sum.
 * x_out, y, q may each be NULL; x, res, x_out share ldx.
 */
void w8a8o_rmsnorm_smoothquant(const uint16_t* x, const uint16_t* res, const float* gamma,
                               const float* s, uint16_t* x_out, uint16_t* y, int8_t* q,
                               float* r, uint32_t M, uint32_t N, float eps, float quant_max,
                               uint32_t ldx, uint32_t ldy, uint32_t ldq);

/*
 * Offline weight quantization (the weight side of the path; the reference has
 * no such routine): per output channel n, the quantizer of
 * rocwmma_smoothquant.cpp:74-121 on p[k] = float(w[n,k]) * s[k] (divide = 0)
 * or float(w[n,k]) / s[k] (divide = 1), or p = float(w) when s == NULL:
 *   sb[n] = max_k |p| / quant_max;  q[n,k] = int8(clamp(rint(p * inv)))
 * Row-major output [n, ldq].
 */
void w8a8o_quantize_weights(const uint16_t* w, const float* s, int divide, float quant_max,
                            int8_t* q, float* sb, uint32_t N, uint32_t K, uint32_t ldw,
                            uint32_t ldq);

/* Operand layouts of the int8 GEMM. */
enum {
    W8A8O_LAYOUT_A_ROW_B_NK = 0, /* A [M,K] row-major (lda>=K), B [N,K] K-contiguous (ldb>=K) */
    W8A8O_LAYOUT_A_COL_B_KN = 1  /* A col-major (lda>=M), B [K,N] row-major (ldb>=N)        */
};

/*
 * int8 x int8 -> int32 GEMM.  Restates gemm_cpu_h<int8_t,int32_t,int32_t,...>
 * (common.hpp:299-345) with alpha = 1, beta = 0: d[i,j] = sum_h a(i,h)*b(h,j),
 * index lambdas per layout (common.hpp:321-327), OpenMP over rows (:329).
 * Rows [row_begin, row_end) only (row_end = M for the full product).
 */
void w8a8o_gemm_i8_i32(uint32_t M, uint32_t N, uint32_t K,
                       const int8_t* a, const int8_t* b, int32_t* c,
                       uint32_t lda, uint32_t ldb, uint32_t ldc, int layout,
                       uint32_t row_begin, uint32_t row_end);

/*
 * Dequant epilogue to fp16 (rocwmma_gemm_quantized.cpp:188-194, Mode 1, and
 * its documented Mode 2 at :18-26):
 *   both vectors NULL : out = half(float(acc) * (tsa * tsb))        (Mode 1)
 *   otherwise         : out = half((float(acc) * sa') * sb')        (Mode 2)
 *   with sa' = scale_a ? scale_a[m] : tsa, sb' = scale_b ? scale_b[n] : tsb.
 */
void w8a8o_dequant_f16(uint32_t M, uint32_t N, const int32_t* acc, uint32_t ldacc,
                       const float* scale_a, const float* scale_b,
                       float tensor_scale_a, float tensor_scale_b,
                       uint16_t* out, uint32_t ldo);

/*
 * Softmax + top-k routing (rocwmma_topk_softmax.cpp:58-131), fp32 logits.
 * Selection is made on the logits (softmax is monotonic); equal logits go to
 * the lower expert index.  (The reference's shfl_down tree, :111-119, keeps
 * the left partial on ties, which is not always the lowest index: a tie
 * between experts 2 and 4 goes to 4.  The build defines ties by index.)
 * weights = exp(l - max) * (1 / sum), the sum taken in expert order.
 */
void w8a8o_topk_softmax(const float* logits, float* topk_weights, int32_t* topk_ids,
                        uint32_t tokens, uint32_t experts, uint32_t topk);

/*
 * Counting sort of (token, slot) pairs by expert (rocwmma_moe_sorting.cpp:53-125),
 * made stable: inside an expert, pairs keep ascending flat order t*topk+slot.
 *   expert_count[e]       unpadded count
 *   expert_start[e]       padded start offset, expert_start[E] = total padded rows
 *   padded_count[e]       count rounded up to unit_size            (:96-98)
 *   sorted_token_ids[p]   token id of sorted row p, -1 in padding  (:172, :123)
 *   dst_row[flat]         sorted row of pair `flat` (-1 if its id is invalid)
 * sorted_token_ids must hold total_padded_bound = tokens*topk + experts*unit_size
 * entries (the reference's bound, :161).
 */
void w8a8o_moe_sort(const int32_t* topk_ids, uint32_t tokens, uint32_t topk,
                    uint32_t experts, uint32_t unit_size,
                    int32_t* expert_count, int32_t* expert_start, int32_t* padded_count,
                    int32_t* sorted_token_ids, int32_t* dst_row);

/*
 * MoE activation + requantization between the gate_up and down GEMMs:
 *   g = float(gu[row, j]), u = float(gu[row, inter + j])
 *   a = (g / (1 + exp(-g))) * u  [* s2[j] when s2 != NULL]
 * then the same absmax int8 quantization as w8a8o_smoothquant.
 * exp is the host libm's, so results can differ from the GPU by an ulp of `a`;
 * tests compare with +-1 LSB tolerance on q.
 */
void w8a8o_silu_mul_quant(const uint16_t* gate_up, uint32_t rows, uint32_t inter,
                          uint32_t ld_gu, const float* s2, float quant_max,
                          int8_t* q, float* row_scale, uint32_t ldq);

/*
 * Weighted top-k combine back to token order:
 *   out[t, n] = half( sum_slot fma order: acc = fma(w[t,slot], float(y[dst_row[t*topk+slot], n]), acc) )
 * slots visited in ascending order, invalid rows (dst_row < 0) skipped.
 */
void w8a8o_moe_combine(const uint16_t* y, uint32_t ldy, const float* topk_weights,
                       const int32_t* dst_row, uint32_t tokens, uint32_t topk,
                       uint32_t n, uint16_t* out, uint32_t ldo);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_ORACLE_H */
