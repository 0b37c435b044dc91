/*
 * ref_harness.h -- C entry points into the REFERENCE's own routines, compiled
 * from /root/reference by oracle/Makefile into oracle/_ref/libref.so.
 * TEST INFRASTRUCTURE ONLY: used to pin the CPU restatement in w8a8_oracle.c
 * (CPU functions) and, on the GPU box, to run the reference kernels on the
 * same seeded inputs.  All GPU pointers are device pointers; every GPU entry
 * point launches on the null stream and synchronizes, as the samples do.
 */
#pragma once
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
/* gemm_cpu_h<int8_t,int32_t,int32_t,LayoutA,LayoutB,row_major> (common.hpp:299-345),
 * alpha=1, beta=0.  layout 0: A row-major / B col-major ([N,K]); 1: A col-major / B row-major. */
void ref_gemm_cpu_i8(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b,
                     int32_t* d, uint32_t lda, uint32_t ldb, uint32_t ldd, int layout);
/* compareEqual<T> (common.hpp:347-419): returns pass flag, writes max relative error. */
int ref_compare_equal_f16(const uint16_t* a, const uint16_t* b, uint32_t size, double tol,
                          double* max_rel_err);
int ref_compare_equal_i32(const int32_t* a, const int32_t* b, uint32_t size, double tol,
                          double* max_rel_err);
/* kernel_smoothquant (rocwmma_smoothquant.cpp:58-122), grid(M) x 256 as at :153-155. */
int ref_kernel_smoothquant(const void* x, const float* s, int8_t* y, float* rs, uint32_t M,
                           uint32_t N, float quant_max);
/* kernel_moe_smoothquant (rocwmma_moe_smoothquant.cpp:69-131), grid(tokens*topk) x 256. */
int ref_kernel_moe_smoothquant(const void* x, const float* s, const int32_t* ids, int8_t* qy,
                               float* rs, uint32_t tokens, uint32_t hidden, uint32_t topk,
                               uint32_t experts, float quant_max);
/* kernel_topk_softmax (rocwmma_topk_softmax.cpp:58-131), fp16 logits, experts <= 64. */
int ref_kernel_topk_softmax(const void* logits_f16, float* w, int32_t* idx, uint32_t tokens,
                            uint32_t experts, uint32_t topk);
/* histogram + prefix + scatter (rocwmma_moe_sorting.cpp:53-125, host sequence :168-183). */
int ref_moe_sorting(const int32_t* ids, uint32_t tokens, uint32_t topk, uint32_t experts,
                    uint32_t unit_size, int32_t* count, int32_t* start, int32_t* padded,
                    int32_t* sorted, int32_t* scatter_ws);
/* kernel_rmsnorm2d_fwd (rocwmma_rmsnorm2d.cpp:57-120), grid(M) x 256 as at :215-217. */
int ref_kernel_rmsnorm2d(const void* x, const float* gamma, void* y, uint32_t M, uint32_t N,
                         uint32_t ldx, uint32_t ldy, float eps);
/* kernel_add_rmsnorm2d_fwd (rocwmma_rmsnorm2d.cpp:127-186), grid(M) x 256 as at :243-245. */
int ref_kernel_add_rmsnorm2d(const void* x, const void* residual, const float* gamma, void* y,
                             void* x_out, uint32_t M, uint32_t N, float eps);
#ifdef __cplusplus
}
#endif
