// capi.cpp -- extern "C" entry points of libw8a8.so.
//
// Each entry point validates its arguments on the host before touching HIP, so
// every error path is testable without a GPU, then enqueues the kernels on the
// caller's stream.  No entry point allocates device memory or synchronizes.
#include "../../include/w8a8.h"
#include "w8a8_internal.hpp"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char* what)
{
    if(e == hipSuccess) {
        g_err[0] = '\0';
        return W8A8_SUCCESS;
    }
    return fail((int)e, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool valid_qmax(float q) { return std::isfinite(q) && q > 0.f && q <= 127.f; }

} // namespace

extern "C" {

const char* w8a8_version(void) { return "w8a8-mi355x 0.1.0 (gfx950)"; }

const char* w8a8_last_error(void) { return g_err; }

int w8a8_smoothquant(const void* x, const float* smooth_scale, int8_t* y, float* row_scale,
                     uint32_t M, uint32_t N, float quant_max, uint32_t ldx, uint32_t ldy,
                     hipStream_t stream)
{
    if(!x || !smooth_scale || !y || !row_scale)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_smoothquant: null pointer argument");
    if(M == 0 || N == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_smoothquant: M and N must be > 0 (M=%u N=%u)",
                    M, N);
    if(!valid_qmax(quant_max))
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_smoothquant: quant_max must be in (0, 127], got %g", (double)quant_max);
    if(ldx == 0) ldx = N;
    if(ldy == 0) ldy = N;
    if(ldx < N || ldy < N)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_smoothquant: ldx=%u / ldy=%u smaller than N=%u",
                    ldx, ldy, N);
    w8a8::QuantRows p{};
    p.x    = static_cast<const uint16_t*>(x);
    p.s    = smooth_scale;
    p.q    = y;
    p.r    = row_scale;
    p.rows = M;
    p.n    = N;
    p.ldx  = ldx;
    p.ldq  = ldy;
    p.qmax = quant_max;
    return hip_status(w8a8::launch_smoothquant(p, stream), "w8a8_smoothquant");
}

int w8a8_moe_smoothquant(const void* x, const float* smooth_scale, const int32_t* topk_ids,
                         int8_t* qy, float* row_scale, uint32_t tokens, uint32_t hidden,
                         uint32_t topk, uint32_t experts, float quant_max,
                         const int32_t* dst_row, uint32_t rows_out, hipStream_t stream)
{
    if(!x || !smooth_scale || !topk_ids || !qy || !row_scale)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_moe_smoothquant: null pointer argument");
    if(tokens == 0 || hidden == 0 || topk == 0 || experts == 0)
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_moe_smoothquant: tokens, hidden, topk and experts must be > 0");
    if(topk > experts)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_moe_smoothquant: topk=%u > experts=%u", topk,
                    experts);
    if((uint64_t)tokens * topk > 0x7FFFFFFFull)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_moe_smoothquant: tokens*topk overflows int32");
    if(dst_row && rows_out == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_moe_smoothquant: rows_out must be > 0");
    if(!valid_qmax(quant_max))
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_moe_smoothquant: quant_max must be in (0, 127], got %g",
                    (double)quant_max);
    w8a8::QuantRows p{};
    p.x        = static_cast<const uint16_t*>(x);
    p.s        = smooth_scale;
    p.q        = qy;
    p.r        = row_scale;
    p.rows     = tokens * topk;
    p.n        = hidden;
    p.ldx      = hidden;
    p.ldq      = hidden;
    p.qmax     = quant_max;
    p.topk_ids = topk_ids;
    p.dst_row  = dst_row;
    p.rows_out = dst_row ? rows_out : tokens * topk;
    p.topk     = topk;
    p.experts  = experts;
    return hip_status(w8a8::launch_smoothquant(p, stream), "w8a8_moe_smoothquant");
}

static uint32_t round_up16(uint32_t v) { return (v + 15u) & ~15u; }

size_t w8a8_gemm_workspace_size(uint32_t m, uint32_t n, uint32_t k, int layout)
{
    if(layout != W8A8_LAYOUT_A_COL_B_KN) return 0;
    const size_t kp = round_up16(k);
    // repacked A [m, kp] and B [n, kp], each 256-byte aligned
    return ((size_t)m * kp + 255) / 256 * 256 + ((size_t)n * kp + 255) / 256 * 256;
}

static int validate_gemm(const char* fn, uint32_t m, uint32_t n, uint32_t k, const int8_t* a,
                         const int8_t* b, void* c, uint32_t lda, uint32_t ldb, uint32_t ldc,
                         int out_type, int layout)
{
    if(!a || !b || !c) return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(m == 0 || n == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: m, n, k must be > 0 (m=%u n=%u k=%u)", fn, m,
                    n, k);
    if(out_type != W8A8_OUT_I32 && out_type != W8A8_OUT_F16)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: unknown out_type %d", fn, out_type);
    if(layout == W8A8_LAYOUT_A_ROW_B_NK) {
        if(lda < k || ldb < k)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: lda=%u / ldb=%u smaller than k=%u", fn, lda,
                        ldb, k);
    } else if(layout == W8A8_LAYOUT_A_COL_B_KN) {
        if(lda < m || ldb < n)
            return fail(W8A8_ERROR_INVALID_VALUE,
                        "%s: sample layout needs lda >= m and ldb >= n (lda=%u m=%u ldb=%u n=%u)",
                        fn, lda, m, ldb, n);
    } else {
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: unknown layout %d", fn, layout);
    }
    if(ldc < n) return fail(W8A8_ERROR_INVALID_VALUE, "%s: ldc=%u smaller than n=%u", fn, ldc, n);
    return W8A8_SUCCESS;
}

int w8a8_gemm(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b, void* c,
              uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
              const float* scale_b, float tensor_scale_a, float tensor_scale_b, int out_type,
              int layout, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    int rc = validate_gemm("w8a8_gemm", m, n, k, a, b, c, lda, ldb, ldc, out_type, layout);
    if(rc != W8A8_SUCCESS) return rc;

    w8a8::GemmArgs g{m, n, k, a, b, c, lda, ldb, ldc, scale_a, scale_b,
                     tensor_scale_a, tensor_scale_b, out_type};

    if(layout == W8A8_LAYOUT_A_COL_B_KN) {
        const size_t need = w8a8_gemm_workspace_size(m, n, k, layout);
        if(workspace == nullptr || workspace_bytes < need) {
            // No room to repack: strided generic kernel over the sample layout.
            return hip_status(w8a8::launch_gemm_generic(g, 1, lda, 1, ldb, stream),
                              "w8a8_gemm(generic)");
        }
        if(reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
            return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_gemm: workspace must be 256-byte aligned");
        const uint32_t kp  = round_up16(k);
        int8_t*        at  = static_cast<int8_t*>(workspace);
        int8_t*        bt  = at + ((size_t)m * kp + 255) / 256 * 256;
        hipError_t     e   = w8a8::launch_transpose_i8(a, lda, at, kp, m, k, stream);
        if(e == hipSuccess) e = w8a8::launch_transpose_i8(b, ldb, bt, kp, n, k, stream);
        if(e != hipSuccess) return hip_status(e, "w8a8_gemm(repack)");
        g.a   = at;
        g.b   = bt;
        g.lda = kp;
        g.ldb = kp;
        g.k   = kp; // zero padding contributes nothing
        return hip_status(w8a8::launch_gemm_nk(g, stream), "w8a8_gemm");
    }

    if(!w8a8::gemm_fast_path_ok(g))
        return hip_status(w8a8::launch_gemm_generic(g, lda, 1, ldb, 1, stream),
                          "w8a8_gemm(generic)");
    return hip_status(w8a8::launch_gemm_nk(g, stream), "w8a8_gemm");
}

int w8a8_fused_sq_gemm(const void* x, const float* smooth_scale, const int8_t* w,
                       const float* scale_w, void* c, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t ldx, uint32_t ldw, uint32_t ldc, int8_t* q, float* row_scale,
                       hipStream_t stream)
{
    if(!x || !smooth_scale || !w || !scale_w || !c || !q || !row_scale)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_fused_sq_gemm: null pointer argument");
    if(m == 0 || n == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_fused_sq_gemm: m, n, k must be > 0");
    if(ldx == 0) ldx = k;
    if(ldw == 0) ldw = k;
    if(ldc == 0) ldc = n;
    if(ldx < k || ldw < k || ldc < n)
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_fused_sq_gemm: ldx=%u ldw=%u must be >= k=%u and ldc=%u >= n=%u", ldx,
                    ldw, k, ldc, n);
    int rc = w8a8_smoothquant(x, smooth_scale, q, row_scale, m, k, 127.f, ldx, k, stream);
    if(rc != W8A8_SUCCESS) return rc;
    return w8a8_gemm(m, n, k, q, w, c, k, ldw, ldc, row_scale, scale_w, 1.f, 1.f, W8A8_OUT_F16,
                     W8A8_LAYOUT_A_ROW_B_NK, nullptr, 0, stream);
}

size_t w8a8_pack_weights_size(uint32_t n, uint32_t k)
{
    if(n == 0 || k == 0) return 0;
    return w8a8::packed_weight_bytes(n, k);
}

int w8a8_pack_weights(const int8_t* w, uint32_t n, uint32_t k, uint32_t ldw, int8_t* packed,
                      size_t packed_bytes, hipStream_t stream)
{
    if(!w || !packed) return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_pack_weights: null pointer argument");
    if(n == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_pack_weights: n and k must be > 0");
    if(ldw == 0) ldw = k;
    if(ldw < k)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_pack_weights: ldw=%u smaller than k=%u", ldw, k);
    const size_t need = w8a8::packed_weight_bytes(n, k);
    if(packed_bytes < need)
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_pack_weights: packed buffer of %zu bytes, %zu needed", packed_bytes, need);
    if(reinterpret_cast<uintptr_t>(packed) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_pack_weights: packed must be 16-byte aligned");
    return hip_status(w8a8::launch_pack_weights(w, n, k, ldw, packed, stream), "w8a8_pack_weights");
}

int w8a8_gemm_packed(uint32_t m, uint32_t n, uint32_t k, const int8_t* a,
                     const int8_t* w_packed, void* c, uint32_t lda, uint32_t ldc,
                     const float* scale_a, const float* scale_b, float tensor_scale_a,
                     float tensor_scale_b, int out_type, hipStream_t stream)
{
    int rc = validate_gemm("w8a8_gemm_packed", m, n, k, a, w_packed, c, lda, k, ldc, out_type,
                           W8A8_LAYOUT_A_ROW_B_NK);
    if(rc != W8A8_SUCCESS) return rc;
    if(reinterpret_cast<uintptr_t>(w_packed) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_gemm_packed: w_packed must be 16-byte aligned");
    w8a8::GemmArgs g{m, n, k, a, w_packed, c, lda, k, ldc, scale_a, scale_b,
                     tensor_scale_a, tensor_scale_b, out_type};
    if(!w8a8::gemm_packed_ok(g))
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "w8a8_gemm_packed: needs 16-byte aligned A, lda %% 16 == 0, k %% 16 == 0 "
                    "and A row panels under 2 GiB (m=%u lda=%u k=%u)", m, lda, k);
    return hip_status(w8a8::launch_gemm_packed(g, stream), "w8a8_gemm_packed");
}

int w8a8_fused_sq_gemm_packed(const void* x, const float* smooth_scale, const int8_t* w_packed,
                              const float* scale_w, void* c, uint32_t m, uint32_t n, uint32_t k,
                              uint32_t ldx, uint32_t ldc, int8_t* q, float* row_scale,
                              hipStream_t stream)
{
    if(!x || !smooth_scale || !w_packed || !scale_w || !c || !q || !row_scale)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_fused_sq_gemm_packed: null pointer argument");
    if(m == 0 || n == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_fused_sq_gemm_packed: m, n, k must be > 0");
    if(ldx == 0) ldx = k;
    if(ldc == 0) ldc = n;
    if(ldx < k || ldc < n)
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_fused_sq_gemm_packed: ldx=%u must be >= k=%u and ldc=%u >= n=%u", ldx, k,
                    ldc, n);
    if(reinterpret_cast<uintptr_t>(q) % 16 != 0 || k % 16 != 0)
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "w8a8_fused_sq_gemm_packed: needs a 16-byte aligned q and k %% 16 == 0 (k=%u)", k);
    int rc = w8a8_smoothquant(x, smooth_scale, q, row_scale, m, k, 127.f, ldx, k, stream);
    if(rc != W8A8_SUCCESS) return rc;
    return w8a8_gemm_packed(m, n, k, q, w_packed, c, k, ldc, row_scale, scale_w, 1.f, 1.f,
                            W8A8_OUT_F16, stream);
}

} // extern "C"
