// capi.cpp -- extern "C" entry points of libw8a8.so.
//
// Each entry point validates its arguments on the host before touching HIP, so
// every error path is testable without a GPU, then enqueues the kernels on the
// caller's stream.  No entry point allocates device memory; only the
// diagnostic query w8a8_gemm_streamk_status synchronizes.
#include "../../include/w8a8.h"
#include "w8a8_internal.hpp"

#include <cmath>
#include <cstdarg>
#include <vector>
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

int w8a8_add_rmsnorm_smoothquant(const void* x, const void* residual, const float* gamma,
                                 const float* smooth_scale, void* x_out, void* y, int8_t* q,
                                 float* row_scale, uint32_t M, uint32_t N, float eps,
                                 float quant_max, uint32_t ldx, uint32_t ldy, uint32_t ldq,
                                 hipStream_t stream)
{
    const char* fn = "w8a8_add_rmsnorm_smoothquant";
    if(!x || !gamma) return fail(W8A8_ERROR_INVALID_VALUE, "%s: x and gamma must be given", fn);
    if(M == 0 || N == 0 || M > 0x7FFFFFFFu)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: M and N must be > 0, M < 2^31 (M=%u N=%u)", fn,
                    M, N);
    const bool quant = smooth_scale || q || row_scale;
    if(quant && !(smooth_scale && q && row_scale))
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "%s: smooth_scale, q and row_scale must be given together", fn);
    if(x_out && !residual)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: x_out needs a residual", fn);
    if(!x_out && !y && !quant)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: no output requested", fn);
    if(!(std::isfinite(eps) && eps >= 0.f))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: eps must be finite and >= 0, got %g", fn,
                    (double)eps);
    if(quant && !valid_qmax(quant_max))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: quant_max must be in (0, 127], got %g", fn,
                    (double)quant_max);
    if(ldx == 0) ldx = N;
    if(ldy == 0) ldy = N;
    if(ldq == 0) ldq = N;
    if(ldx < N || ldy < N || ldq < N)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: ldx=%u / ldy=%u / ldq=%u smaller than N=%u",
                    fn, ldx, ldy, ldq, N);
    if((uint64_t)ldx * 2 > 0x7FFFFFFFull || (uint64_t)ldy * 2 > 0x7FFFFFFFull)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: a row must stay under 2 GiB", fn);
    w8a8::NormRows p{};
    p.x     = static_cast<const uint16_t*>(x);
    p.res   = static_cast<const uint16_t*>(residual);
    p.gamma = gamma;
    p.s     = smooth_scale;
    p.x_out = static_cast<uint16_t*>(x_out);
    p.y     = static_cast<uint16_t*>(y);
    p.q     = q;
    p.r     = row_scale;
    p.rows  = M;
    p.n     = N;
    p.ldx   = ldx;
    p.ldy   = ldy;
    p.ldq   = ldq;
    p.eps   = eps;
    p.qmax  = quant ? quant_max : 127.f;
    return hip_status(w8a8::launch_rmsnorm_sq(p, stream), fn);
}

int w8a8_quantize_weights(const void* w, uint32_t n, uint32_t k, uint32_t ldw,
                          const float* smooth_scale, int fold, float quant_max, int8_t* w_q,
                          uint32_t ldq, int packed, size_t out_bytes, float* scale_w,
                          hipStream_t stream)
{
    const char* fn = "w8a8_quantize_weights";
    if(!w || !w_q || !scale_w)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(n == 0 || k == 0 || n > 0x7FFFFF00u)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: n and k must be > 0, n < 2^31 (n=%u k=%u)",
                    fn, n, k);
    if(fold != W8A8_FOLD_MULTIPLY && fold != W8A8_FOLD_DIVIDE)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: unknown fold mode %d", fn, fold);
    if(packed != 0 && packed != 1)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: packed must be 0 or 1", fn);
    if(!valid_qmax(quant_max))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: quant_max must be in (0, 127], got %g", fn,
                    (double)quant_max);
    if(ldw == 0) ldw = k;
    if(ldq == 0) ldq = k;
    if(ldw < k) return fail(W8A8_ERROR_INVALID_VALUE, "%s: ldw=%u smaller than k=%u", fn, ldw, k);
    if(packed) {
        const size_t need = w8a8::packed_weight_bytes(n, k);
        if(out_bytes < need)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: packed output needs %zu bytes, got %zu", fn,
                        need, out_bytes);
        if(reinterpret_cast<uintptr_t>(w_q) % 16)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: packed output must be 16-byte aligned", fn);
    } else {
        if(ldq < k)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: ldq=%u smaller than k=%u", fn, ldq, k);
        const size_t need = (size_t)(n - 1) * ldq + k;
        if(out_bytes < need)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: output needs %zu bytes, got %zu", fn, need,
                        out_bytes);
    }
    w8a8::WeightQuant p{};
    p.w    = static_cast<const uint16_t*>(w);
    p.s    = smooth_scale;
    p.q    = w_q;
    p.sb   = scale_w;
    p.n    = n;
    p.k    = k;
    p.ldw  = ldw;
    p.ldq  = ldq;
    p.qmax = quant_max;
    return hip_status(
        w8a8::launch_quantize_weights(p, fold == W8A8_FOLD_DIVIDE, packed == 1, stream), fn);
}

static uint32_t round_up16(uint32_t v) { return (v + 15u) & ~15u; }

size_t w8a8_gemm_workspace_size(uint32_t m, uint32_t n, uint32_t k, int layout)
{
    if(layout == W8A8_LAYOUT_A_ROW_B_NK) {
        // K-split partials for launches that fill at most half the CUs
        w8a8::GemmArgs g{m, n, k, nullptr, nullptr, nullptr, k, k, n, nullptr, nullptr, 1.f, 1.f,
                         W8A8_OUT_F16};
        return w8a8::gemm_nk_workspace_bytes(g);
    }
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

// w8a8_gemm and w8a8_gemm_noalloc (arguments validated by the caller; `fn`
// names the entry point in error messages).
static int gemm_entry(const char* fn, uint32_t m, uint32_t n, uint32_t k, const int8_t* a,
                      const int8_t* b, void* c, uint32_t lda, uint32_t ldb, uint32_t ldc,
                      const float* scale_a, const float* scale_b, float tensor_scale_a,
                      float tensor_scale_b, int out_type, int layout, void* workspace,
                      size_t workspace_bytes, hipStream_t stream)
{

    w8a8::GemmArgs g{m, n, k, a, b, c, lda, ldb, ldc, scale_a, scale_b,
                     tensor_scale_a, tensor_scale_b, out_type};

    if(layout == W8A8_LAYOUT_A_COL_B_KN) {
        const size_t need = w8a8_gemm_workspace_size(m, n, k, layout);
        if(workspace == nullptr || workspace_bytes < need) {
            // No room to repack: strided generic kernel over the sample layout.
            return hip_status(w8a8::launch_gemm_generic(g, 1, lda, 1, ldb, stream), fn);
        }
        if(reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 256-byte aligned", fn);
        const uint32_t kp  = round_up16(k);
        int8_t*        at  = static_cast<int8_t*>(workspace);
        int8_t*        bt  = at + ((size_t)m * kp + 255) / 256 * 256;
        hipError_t     e   = w8a8::launch_transpose_i8(a, lda, at, kp, m, k, stream);
        if(e == hipSuccess) e = w8a8::launch_transpose_i8(b, ldb, bt, kp, n, k, stream);
        if(e != hipSuccess) return hip_status(e, fn);
        g.a   = at;
        g.b   = bt;
        g.lda = kp;
        g.ldb = kp;
        g.k   = kp; // zero padding contributes nothing
        return hip_status(w8a8::launch_gemm_nk(g, nullptr, 0, stream), fn);
    }

    if(workspace && reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 16-byte aligned", fn);
    if(!w8a8::gemm_fast_path_ok(g))
        return hip_status(w8a8::launch_gemm_generic(g, lda, 1, ldb, 1, stream), fn);
    return hip_status(w8a8::launch_gemm_nk(g, workspace, workspace ? workspace_bytes : 0, stream),
                      fn);
}

int w8a8_gemm(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b, void* c,
              uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
              const float* scale_b, float tensor_scale_a, float tensor_scale_b, int out_type,
              int layout, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    const char* fn = "w8a8_gemm";
    int         rc = validate_gemm(fn, m, n, k, a, b, c, lda, ldb, ldc, out_type, layout);
    if(rc != W8A8_SUCCESS) return rc;
    return gemm_entry(fn, m, n, k, a, b, c, lda, ldb, ldc, scale_a, scale_b, tensor_scale_a,
                      tensor_scale_b, out_type, layout, workspace, workspace_bytes, stream);
}

int w8a8_gemm_noalloc(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b,
                      void* c, uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
                      const float* scale_b, float tensor_scale_a, float tensor_scale_b,
                      int out_type, int layout, hipStream_t stream)
{
    const char* fn = "w8a8_gemm_noalloc";
    int         rc = validate_gemm(fn, m, n, k, a, b, c, lda, ldb, ldc, out_type, layout);
    if(rc != W8A8_SUCCESS) return rc;
    const size_t need = w8a8_gemm_workspace_size(m, n, k, layout);
    if(need > W8A8_NOALLOC_SCRATCH_BYTES)
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "%s: m=%u n=%u k=%u needs %zu bytes of scratch, the library holds %zu per GPU "
                    "(call w8a8_gemm with a workspace instead)",
                    fn, m, n, k, need, (size_t)W8A8_NOALLOC_SCRATCH_BYTES);
    void*      scratch = nullptr;
    hipError_t e       = w8a8::noalloc_scratch(&scratch);
    if(e != hipSuccess) return hip_status(e, fn);
    return gemm_entry(fn, m, n, k, a, b, c, lda, ldb, ldc, scale_a, scale_b, tensor_scale_a,
                      tensor_scale_b, out_type, layout, scratch, W8A8_NOALLOC_SCRATCH_BYTES, stream);
}

size_t w8a8_gemm_streamk_workspace_size(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks)
{
    return w8a8::streamk_workspace_bytes(m, n, k, blocks);
}

int w8a8_gemm_streamk(uint32_t m, uint32_t n, uint32_t k, const int8_t* a, const int8_t* b,
                      void* c, uint32_t lda, uint32_t ldb, uint32_t ldc, const float* scale_a,
                      const float* scale_b, float tensor_scale_a, float tensor_scale_b,
                      int out_type, uint32_t blocks, void* workspace, size_t workspace_bytes,
                      hipStream_t stream)
{
    const char* fn = "w8a8_gemm_streamk";
    int rc = validate_gemm(fn, m, n, k, a, b, c, lda, ldb, ldc, out_type, W8A8_LAYOUT_A_ROW_B_NK);
    if(rc != W8A8_SUCCESS) return rc;
    w8a8::GemmArgs g{m, n, k, a, b, c, lda, ldb, ldc, scale_a, scale_b,
                     tensor_scale_a, tensor_scale_b, out_type};
    if(!w8a8::streamk_shape_ok(g))
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "%s: needs 16-byte aligned a/b, lda, ldb, k %% 16 == 0 and A, B under 2 GiB "
                    "(m=%u n=%u k=%u lda=%u ldb=%u)",
                    fn, m, n, k, lda, ldb);
    const size_t need = w8a8::streamk_workspace_bytes(m, n, k, blocks);
    if(workspace == nullptr || workspace_bytes < need)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace of %zu bytes, %zu needed", fn,
                    workspace ? workspace_bytes : (size_t)0, need);
    if(reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 16-byte aligned", fn);
    return hip_status(w8a8::launch_gemm_streamk(g, blocks, workspace, stream), fn);
}

uint32_t w8a8_gemm_streamk_blocks(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks)
{
    return w8a8::streamk_blocks(m, n, k, blocks);
}

int w8a8_gemm_streamk_status(uint32_t* flags, int clear)
{
    if(!flags) return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_gemm_streamk_status: null flags");
    *flags = 0;
    return hip_status(w8a8::streamk_status(flags, clear != 0), "w8a8_gemm_streamk_status");
}

int w8a8_debug_streamk_wait(uint32_t spin_limit, uint32_t phantom_pieces)
{
    if(phantom_pieces > 0 && (spin_limit == 0 || spin_limit > 4096))
        return fail(W8A8_ERROR_INVALID_VALUE,
                    "w8a8_debug_streamk_wait: phantom pieces need a spin limit in [1, 4096] "
                    "(got %u): the wait they force must end quickly",
                    spin_limit);
    w8a8::streamk_debug_wait(spin_limit, phantom_pieces);
    return W8A8_SUCCESS;
}

int w8a8_fused_sq_gemm(const void* x, const float* smooth_scale, const int8_t* w,
                       const float* scale_w, void* c, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t ldx, uint32_t ldw, uint32_t ldc, int8_t* q, float* row_scale,
                       void* workspace, size_t ws_bytes, hipStream_t stream)
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
                     W8A8_LAYOUT_A_ROW_B_NK, workspace, ws_bytes, stream);
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

size_t w8a8_gemm_packed_workspace_size(uint32_t m, uint32_t n, uint32_t k)
{
    if(m == 0 || n == 0 || k == 0) return 0;
    w8a8::GemmArgs g{m, n, k, nullptr, nullptr, nullptr, k, k, n, nullptr, nullptr, 1.f, 1.f,
                     W8A8_OUT_F16};
    return w8a8::packed_workspace_bytes(g);
}

int w8a8_gemm_packed(uint32_t m, uint32_t n, uint32_t k, const int8_t* a,
                     const int8_t* w_packed, void* c, uint32_t lda, uint32_t ldc,
                     const float* scale_a, const float* scale_b, float tensor_scale_a,
                     float tensor_scale_b, int out_type, void* workspace, size_t ws_bytes,
                     hipStream_t stream)
{
    int rc = validate_gemm("w8a8_gemm_packed", m, n, k, a, w_packed, c, lda, k, ldc, out_type,
                           W8A8_LAYOUT_A_ROW_B_NK);
    if(rc != W8A8_SUCCESS) return rc;
    if(reinterpret_cast<uintptr_t>(w_packed) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_gemm_packed: w_packed must be 16-byte aligned");
    if(workspace && reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "w8a8_gemm_packed: workspace must be 16-byte aligned");
    w8a8::GemmArgs g{m, n, k, a, w_packed, c, lda, k, ldc, scale_a, scale_b,
                     tensor_scale_a, tensor_scale_b, out_type};
    if(!w8a8::gemm_packed_ok(g))
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "w8a8_gemm_packed: needs 16-byte aligned A, lda %% 16 == 0, k %% 16 == 0 "
                    "and A row panels under 2 GiB (m=%u lda=%u k=%u)", m, lda, k);
    return hip_status(w8a8::launch_gemm_packed(g, workspace, workspace ? ws_bytes : 0, stream),
                      "w8a8_gemm_packed");
}

int w8a8_fused_sq_gemm_packed(const void* x, const float* smooth_scale, const int8_t* w_packed,
                              const float* scale_w, void* c, uint32_t m, uint32_t n, uint32_t k,
                              uint32_t ldx, uint32_t ldc, int8_t* q, float* row_scale,
                              void* workspace, size_t ws_bytes, hipStream_t stream)
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
    // a few rows: one kernel quantizes them per block and streams the weights
    if(w8a8::decode_fuse_ok(m, k) && reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 8 == 0
       && reinterpret_cast<uintptr_t>(smooth_scale) % 16 == 0) {
        int vrc = validate_gemm("w8a8_fused_sq_gemm_packed", m, n, k, q, w_packed, c, k, k, ldc,
                                W8A8_OUT_F16, W8A8_LAYOUT_A_ROW_B_NK);
        if(vrc != W8A8_SUCCESS) return vrc;
        if(reinterpret_cast<uintptr_t>(w_packed) % 16 != 0)
            return fail(W8A8_ERROR_INVALID_VALUE,
                        "w8a8_fused_sq_gemm_packed: w_packed must be 16-byte aligned");
        const w8a8::GemmArgs g{m, n, k, q, w_packed, c, k, k, ldc, row_scale, scale_w,
                               1.f, 1.f, W8A8_OUT_F16};
        if(w8a8::gemm_packed_ok(g)) {
            const w8a8::FuseArgs f{static_cast<const uint16_t*>(x), smooth_scale, q, row_scale,
                                   ldx, 127.f};
            return hip_status(w8a8::launch_gemm_decode_fused(g, f, stream),
                              "w8a8_fused_sq_gemm_packed");
        }
    }
    int rc = w8a8_smoothquant(x, smooth_scale, q, row_scale, m, k, 127.f, ldx, k, stream);
    if(rc != W8A8_SUCCESS) return rc;
    return w8a8_gemm_packed(m, n, k, q, w_packed, c, k, ldc, row_scale, scale_w, 1.f, 1.f,
                            W8A8_OUT_F16, workspace, ws_bytes, stream);
}

// ---------------------------------------------------------------------------
// Grouped GEMM and MoE
// ---------------------------------------------------------------------------

size_t w8a8_grouped_gemm_workspace_size(uint32_t num_groups)
{
    return ((size_t)num_groups * sizeof(w8a8_group_desc) + 255) / 256 * 256;
}

int w8a8_grouped_gemm(const w8a8_group_desc* groups, uint32_t num_groups, int out_type,
                      void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    const char* fn = "w8a8_grouped_gemm";
    if(!groups || num_groups == 0) return fail(W8A8_ERROR_INVALID_VALUE, "%s: no groups", fn);
    if(out_type != W8A8_OUT_I32 && out_type != W8A8_OUT_F16)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: unknown out_type %d", fn, out_type);
    if(!workspace || workspace_bytes < w8a8_grouped_gemm_workspace_size(num_groups))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace of %zu bytes, %zu needed", fn,
                    workspace_bytes, w8a8_grouped_gemm_workspace_size(num_groups));
    if(reinterpret_cast<uintptr_t>(workspace) % 64 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 64-byte aligned", fn);
    uint64_t   tiles[3] = {0, 0, 0}; // per tile configuration
    int        vec_ok   = 1;
    const size_t esz  = out_type == W8A8_OUT_I32 ? 4 : 2;
    for(uint32_t i = 0; i < num_groups; ++i) {
        const w8a8_group_desc& d = groups[i];
        if(d.m == 0) continue;
        if(!d.a || !d.b || !d.c)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: group %u: null pointer", fn, i);
        if(d.n == 0 || d.k == 0)
            return fail(W8A8_ERROR_INVALID_VALUE, "%s: group %u: n and k must be > 0", fn, i);
        if(d.lda < d.k || d.ldb < d.k || d.ldc < d.n)
            return fail(W8A8_ERROR_INVALID_VALUE,
                        "%s: group %u: lda=%u ldb=%u must be >= k=%u and ldc=%u >= n=%u", fn, i,
                        d.lda, d.ldb, d.k, d.ldc, d.n);
        if(reinterpret_cast<uintptr_t>(d.a) % 16 || reinterpret_cast<uintptr_t>(d.b) % 16
           || d.lda % 16 || d.ldb % 16 || d.k % 16)
            return fail(W8A8_ERROR_NOT_SUPPORTED,
                        "%s: group %u: needs 16-byte aligned a/b and lda, ldb, k %% 16 == 0", fn, i);
        if((uint64_t)d.m * d.lda > 0x7FFFFFFFull || (uint64_t)d.n * d.ldb > 0x7FFFFFFFull)
            return fail(W8A8_ERROR_NOT_SUPPORTED, "%s: group %u: operand over 2 GiB", fn, i);
        vec_ok = vec_ok && reinterpret_cast<uintptr_t>(d.c) % (4 * esz) == 0 && d.ldc % 4 == 0
                 && (d.scale_b == nullptr || reinterpret_cast<uintptr_t>(d.scale_b) % 16 == 0);
        for(int c = 0; c < 3; ++c) tiles[c] += w8a8::grouped_gemm_tiles(d.m, d.n, c);
    }
    if(tiles[2] > 0x7FFFFFFFull) return fail(W8A8_ERROR_NOT_SUPPORTED, "%s: too many tiles", fn);
    if(tiles[0] == 0) return hip_status(hipSuccess, fn);
    const int cfg = w8a8::grouped_gemm_cfg(tiles);
    hipError_t e = hipMemcpyAsync(workspace, groups, (size_t)num_groups * sizeof(w8a8_group_desc),
                                  hipMemcpyHostToDevice, stream);
    if(e == hipSuccess)
        e = w8a8::launch_grouped_gemm(static_cast<const w8a8_group_desc*>(workspace), num_groups,
                                      (uint32_t)tiles[cfg], cfg, out_type, vec_ok, stream);
    return hip_status(e, fn);
}

int w8a8_topk_softmax(const void* logits, int logits_f16, float* topk_weights,
                      int32_t* topk_ids, uint32_t tokens, uint32_t experts, uint32_t topk,
                      hipStream_t stream)
{
    const char* fn = "w8a8_topk_softmax";
    if(!logits || !topk_weights || !topk_ids)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(tokens == 0 || experts == 0 || topk == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: tokens, experts and topk must be > 0", fn);
    if(experts > 4096 || topk > experts)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: need topk <= experts <= 4096 (topk=%u experts=%u)",
                    fn, topk, experts);
    if(logits_f16 != 0 && logits_f16 != 1)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: logits_f16 must be 0 or 1", fn);
    return hip_status(w8a8::launch_topk_softmax(logits, logits_f16 == 1, topk_weights, topk_ids,
                                                tokens, experts, topk, stream),
                      fn);
}

size_t w8a8_moe_sort_capacity(uint32_t tokens, uint32_t topk, uint32_t experts, uint32_t unit_size)
{
    return (size_t)tokens * topk + (size_t)experts * unit_size;
}

size_t w8a8_moe_sort_workspace_size(uint32_t tokens, uint32_t topk, uint32_t experts)
{
    if(tokens == 0 || topk == 0 || experts == 0 || experts > 1024) return 0;
    return w8a8::moe_sort_workspace_bytes(tokens, topk, experts);
}

int w8a8_moe_sort(const int32_t* topk_ids, uint32_t tokens, uint32_t topk, uint32_t experts,
                  uint32_t unit_size, int32_t* expert_count, int32_t* expert_start,
                  int32_t* padded_count, int32_t* sorted_token_ids, uint32_t sorted_capacity,
                  int32_t* dst_row, void* workspace, size_t ws_bytes, hipStream_t stream)
{
    const char* fn = "w8a8_moe_sort";
    if(!topk_ids || !expert_count || !expert_start || !padded_count || !sorted_token_ids
       || !dst_row)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(tokens == 0 || topk == 0 || experts == 0 || unit_size == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: tokens, topk, experts, unit_size must be > 0",
                    fn);
    if(experts > 1024) return fail(W8A8_ERROR_INVALID_VALUE, "%s: experts=%u > 1024", fn, experts);
    const size_t need = w8a8_moe_sort_capacity(tokens, topk, experts, unit_size);
    if(need > 0x7FFFFFFFull)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: sorted rows overflow int32", fn);
    if(sorted_capacity < need)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: sorted_capacity=%u, %zu needed", fn,
                    sorted_capacity, need);
    if(workspace && reinterpret_cast<uintptr_t>(workspace) % 4 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 4-byte aligned", fn);
    return hip_status(w8a8::launch_moe_sort(topk_ids, tokens, topk, experts, unit_size,
                                            expert_count, expert_start, padded_count,
                                            sorted_token_ids, sorted_capacity, dst_row, workspace,
                                            workspace ? ws_bytes : 0, stream),
                      fn);
}

size_t w8a8_moe_gemm_workspace_size(uint32_t experts, uint32_t rows, uint32_t n, uint32_t k)
{
    if(experts == 0 || rows == 0 || n == 0 || k == 0) return 0;
    return w8a8::moe_gemm_workspace_bytes();
}

int w8a8_moe_gemm(uint32_t experts, uint32_t rows, uint32_t n, uint32_t k, const int8_t* a,
                  uint32_t lda, const int8_t* w, uint32_t ldw, uint64_t w_expert_stride, void* c,
                  uint32_t ldc, const float* scale_a, const float* scale_w,
                  float tensor_scale_a, float tensor_scale_b, const int32_t* expert_start,
                  const int32_t* expert_count, int out_type, void* workspace, size_t ws_bytes,
                  hipStream_t stream)
{
    const char* fn = "w8a8_moe_gemm";
    if(!a || !w || !c || !expert_start || !expert_count)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(experts == 0 || n == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: experts, n, k must be > 0", fn);
    if(out_type != W8A8_OUT_I32 && out_type != W8A8_OUT_F16)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: unknown out_type %d", fn, out_type);
    if(lda < k || ldw < k || ldc < n)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: lda=%u ldw=%u must be >= k=%u, ldc=%u >= n=%u",
                    fn, lda, ldw, k, ldc, n);
    if(w_expert_stride < (uint64_t)(n - 1) * ldw + k)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: w_expert_stride smaller than one expert", fn);
    if(reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16 || lda % 16
       || ldw % 16 || k % 16 || w_expert_stride % 16)
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "%s: needs 16-byte aligned a/w, lda, ldw, k, w_expert_stride %% 16 == 0", fn);
    if((uint64_t)rows * lda > 0x7FFFFFFFull || (uint64_t)n * ldw > 0x7FFFFFFFull)
        return fail(W8A8_ERROR_NOT_SUPPORTED, "%s: a or one expert's weights over 2 GiB", fn);
    if(workspace && reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 16-byte aligned", fn);
    if(rows == 0) return hip_status(hipSuccess, fn);
    w8a8::MoeGemmArgs g{a,    w,   c,   scale_a, scale_w, expert_start, expert_count,
                        rows, experts, n, k, lda, ldw, ldc, w_expert_stride, tensor_scale_a,
                        tensor_scale_b, out_type, workspace, workspace ? ws_bytes : 0};
    return hip_status(w8a8::launch_moe_gemm(g, stream), fn);
}

int w8a8_moe_silu_mul_quant(const void* gate_up, uint32_t ld_gu, const float* smooth_scale,
                            const int32_t* expert_start, const int32_t* expert_count,
                            uint32_t experts, uint32_t rows, uint32_t inter, int8_t* q,
                            uint32_t ldq, float* row_scale, float quant_max, hipStream_t stream)
{
    const char* fn = "w8a8_moe_silu_mul_quant";
    if(!gate_up || !expert_start || !expert_count || !q || !row_scale)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(experts == 0 || inter == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: experts and inter must be > 0", fn);
    if(inter > 32768) return fail(W8A8_ERROR_NOT_SUPPORTED, "%s: inter=%u > 32768", fn, inter);
    if(ld_gu == 0) ld_gu = 2 * inter;
    if(ldq == 0) ldq = inter;
    if(ld_gu < 2 * inter || ldq < inter)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: ld_gu=%u must be >= 2*inter and ldq=%u >= inter",
                    fn, ld_gu, ldq);
    if(!valid_qmax(quant_max))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: quant_max must be in (0, 127]", fn);
    return hip_status(w8a8::launch_silu_mul_quant(static_cast<const uint16_t*>(gate_up), ld_gu,
                                                  smooth_scale, expert_start, expert_count,
                                                  experts, rows, inter, q, ldq, row_scale,
                                                  quant_max, stream),
                      fn);
}

int w8a8_moe_interleave_gate_up(const int8_t* w, const float* scale_w, uint32_t experts,
                                uint32_t inter, uint32_t k, uint32_t ldw, int8_t* w_out,
                                float* scale_w_out, hipStream_t stream)
{
    const char* fn = "w8a8_moe_interleave_gate_up";
    if(!w || !w_out || (scale_w && !scale_w_out))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(experts == 0 || inter == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: experts, inter, k must be > 0", fn);
    if(inter % 16 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: inter=%u must be a multiple of 16", fn, inter);
    if(ldw == 0) ldw = k;
    if(ldw < k) return fail(W8A8_ERROR_INVALID_VALUE, "%s: ldw=%u smaller than k=%u", fn, ldw, k);
    return hip_status(w8a8::launch_moe_interleave_gate_up(w, scale_w, experts, inter, k, ldw,
                                                          w_out, scale_w_out, stream),
                      fn);
}

size_t w8a8_moe_gate_up_silu_workspace_size(uint32_t rows, uint32_t inter)
{
    return w8a8::moe_gate_up_silu_workspace_bytes(rows, inter);
}

int w8a8_moe_gate_up_silu(uint32_t experts, uint32_t rows, uint32_t inter, uint32_t k,
                          const int8_t* a, uint32_t lda, const int8_t* w_interleaved,
                          const float* scale_a, const float* scale_w_interleaved,
                          float tensor_scale_a, float tensor_scale_b,
                          const float* smooth_scale, const int32_t* expert_start,
                          const int32_t* expert_count, int8_t* q, uint32_t ldq, float* row_scale,
                          float quant_max, void* workspace, size_t ws_bytes, hipStream_t stream)
{
    const char* fn = "w8a8_moe_gate_up_silu";
    if(!a || !w_interleaved || !expert_start || !expert_count || !q || !row_scale || !workspace)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(experts == 0 || inter == 0 || k == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: experts, inter, k must be > 0", fn);
    if(inter % 16 != 0 || inter > 32768)
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "%s: needs inter %% 16 == 0 and inter <= 32768 (inter=%u)", fn, inter);
    if(lda == 0) lda = k;
    if(ldq == 0) ldq = inter;
    if(lda < k || ldq < inter)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: lda=%u must be >= k=%u and ldq=%u >= inter=%u",
                    fn, lda, k, ldq, inter);
    if(!valid_qmax(quant_max))
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: quant_max must be in (0, 127]", fn);
    if(reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w_interleaved) % 16
       || lda % 16 || k % 16 || reinterpret_cast<uintptr_t>(q) % 8 || ldq % 8
       || (scale_w_interleaved && reinterpret_cast<uintptr_t>(scale_w_interleaved) % 16)
       || (smooth_scale && reinterpret_cast<uintptr_t>(smooth_scale) % 16))
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "%s: needs 16-byte aligned a, w, scale_w, smooth_scale, lda, k %% 16 == 0, "
                    "8-byte aligned q and ldq %% 8 == 0",
                    fn);
    constexpr uint64_t kLimit = 0x7FFFFFFFull;
    if((uint64_t)rows * lda > kLimit || 2ull * inter * k > kLimit || (uint64_t)rows * inter * 2 > kLimit
       || (uint64_t)rows * ldq > kLimit || (uint64_t)experts * inter * 4 > kLimit)
        return fail(W8A8_ERROR_NOT_SUPPORTED,
                    "%s: a, one expert's weights, the activation, q or smooth_scale over 2 GiB", fn);
    if(reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace must be 256-byte aligned", fn);
    const size_t need = w8a8::moe_gate_up_silu_workspace_bytes(rows, inter);
    if(ws_bytes < need)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes,
                    need);
    if(rows == 0) return hip_status(hipSuccess, fn);
    w8a8::MoeSiluArgs g{a,         w_interleaved, scale_a,      scale_w_interleaved, smooth_scale,
                        expert_start, expert_count, rows,       experts,             inter,
                        k,         lda,           tensor_scale_a, tensor_scale_b,     q,
                        ldq,       row_scale,     quant_max,    workspace};
    return hip_status(w8a8::launch_moe_gate_up_silu(g, stream), fn);
}

int w8a8_moe_combine(const void* y, uint32_t ldy, uint32_t rows_y, const float* topk_weights,
                     const int32_t* dst_row, uint32_t tokens, uint32_t topk, uint32_t n,
                     void* out, uint32_t ldo, hipStream_t stream)
{
    const char* fn = "w8a8_moe_combine";
    if(!y || !topk_weights || !dst_row || !out)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: null pointer argument", fn);
    if(tokens == 0 || topk == 0 || n == 0)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: tokens, topk, n must be > 0", fn);
    if(ldy == 0) ldy = n;
    if(ldo == 0) ldo = n;
    if(ldy < n || ldo < n)
        return fail(W8A8_ERROR_INVALID_VALUE, "%s: ldy=%u / ldo=%u smaller than n=%u", fn, ldy, ldo,
                    n);
    return hip_status(w8a8::launch_moe_combine(static_cast<const uint16_t*>(y), ldy, rows_y,
                                               topk_weights, dst_row, tokens, topk, n,
                                               static_cast<uint16_t*>(out), ldo, stream),
                      fn);
}

} // extern "C"
