// Driver of the C ABI's host side for the AddressSanitizer /
// UndefinedBehaviorSanitizer build of test_sanitizers_cpu.py: libw8a8.so is
// built with its host code instrumented, and this program calls every entry
// point with arguments its validation rejects (null pointers, zero or
// oversized shapes, short strides, bad scales and workspaces) and every size
// query over a range of shapes, including the stream-K planner.  Nothing here
// reaches a kernel launch: every rejected call returns before its first HIP
// call, so no device memory is touched whether or not a GPU is present (the
// pointers below are never dereferenced).  Prints "OK <calls>" on success.
#include "../include/w8a8.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>

static int g_calls = 0;

static void reject(int rc, const char* what, int line)
{
    ++g_calls;
    const char* msg = w8a8_last_error();
    if(rc == W8A8_SUCCESS || msg == nullptr || msg[0] == '\0') {
        std::printf("FAIL line %d (%s): rc=%d msg='%s'\n", line, what, rc, msg ? msg : "(null)");
        std::exit(1);
    }
}
#define REJECT(call) reject((call), #call, __LINE__)

int main()
{
    // fake, never dereferenced: validation fails before any use
    void*          P  = reinterpret_cast<void*>(0x100000);
    const int8_t*  A  = static_cast<const int8_t*>(P);
    int8_t*        Q  = static_cast<int8_t*>(P);
    float*         F  = static_cast<float*>(P);
    int32_t*       I  = static_cast<int32_t*>(P);
    hipStream_t    st = nullptr;

    // ---- version, sizes (host arithmetic only) ------------------------------
    if(std::strstr(w8a8_version(), "gfx950") == nullptr) return 1;
    size_t sink = 0;
    const uint32_t dims[] = {1, 15, 16, 64, 127, 128, 255, 256, 511, 512, 1000, 2048, 4096,
                             14336, 28672, 65535};
    for(uint32_t m : dims)
        for(uint32_t n : dims)
            for(uint32_t k : {16u, 128u, 4096u, 14336u}) {
                sink += w8a8_gemm_workspace_size(m, n, k, W8A8_LAYOUT_A_ROW_B_NK);
                sink += w8a8_gemm_workspace_size(m, n, k, W8A8_LAYOUT_A_COL_B_KN);
                sink += w8a8_gemm_packed_workspace_size(m, n, k);
                sink += w8a8_pack_weights_size(n, k);
                if(m * (uint64_t)n <= (1ull << 26)) {
                    sink += w8a8_gemm_streamk_workspace_size(m, n, k, 0);
                    sink += w8a8_gemm_streamk_blocks(m, n, k, 0);
                    sink += w8a8_gemm_streamk_workspace_size(m, n, k, 7);
                    sink += w8a8_gemm_streamk_blocks(m, n, k, 333);
                }
            }
    for(uint32_t g : {0u, 1u, 8u, 1000u}) sink += w8a8_grouped_gemm_workspace_size(g);
    for(uint32_t t : {1u, 1000u, 4096u, 70000u})
        for(uint32_t e : {1u, 8u, 64u, 1024u}) {
            sink += w8a8_moe_sort_capacity(t, 2, e, 32);
            sink += w8a8_moe_sort_workspace_size(t, 2, e);
            sink += w8a8_moe_gemm_workspace_size(e, t * 2, 4096, 4096);
            sink += w8a8_moe_gate_up_silu_workspace_size(t * 2, 14336);
        }
    sink += w8a8_gemm_streamk_workspace_size(0, 0, 0, 0) + w8a8_gemm_streamk_blocks(0, 5, 5, 0);

    // ---- quantizers ---------------------------------------------------------
    REJECT(w8a8_smoothquant(nullptr, F, Q, F, 4, 8, 127.f, 0, 0, st));
    REJECT(w8a8_smoothquant(P, F, Q, F, 0, 8, 127.f, 0, 0, st));
    REJECT(w8a8_smoothquant(P, F, Q, F, 4, 8, 0.f, 0, 0, st));
    REJECT(w8a8_smoothquant(P, F, Q, F, 4, 8, 200.f, 0, 0, st));
    REJECT(w8a8_smoothquant(P, F, Q, F, 4, 8, 127.f, 7, 0, st));
    REJECT(w8a8_moe_smoothquant(nullptr, F, I, Q, F, 4, 8, 2, 8, 127.f, nullptr, 0, st));
    REJECT(w8a8_moe_smoothquant(P, F, I, Q, F, 0, 8, 2, 8, 127.f, nullptr, 0, st));
    REJECT(w8a8_moe_smoothquant(P, F, I, Q, F, 4, 8, 0, 8, 127.f, nullptr, 0, st));
    REJECT(w8a8_moe_smoothquant(P, F, I, Q, F, 4, 8, 2, 0, 127.f, nullptr, 0, st));
    REJECT(w8a8_add_rmsnorm_smoothquant(nullptr, P, F, F, P, P, Q, F, 4, 64, 1e-5f, 127.f, 0,
                                        0, 0, st));
    REJECT(w8a8_add_rmsnorm_smoothquant(P, nullptr, F, F, P, nullptr, Q, F, 4, 64, 1e-5f, 127.f,
                                        0, 0, 0, st));
    REJECT(w8a8_add_rmsnorm_smoothquant(P, P, F, F, P, P, Q, F, 4, 64, -1.f, 127.f, 0, 0, 0, st));
    REJECT(w8a8_add_rmsnorm_smoothquant(P, P, F, F, P, P, Q, F, 4, 64, 1e-5f, 127.f, 10, 0, 0,
                                        st));
    REJECT(w8a8_quantize_weights(nullptr, 64, 64, 0, F, W8A8_FOLD_DIVIDE, 127.f, Q, 0, 0, 4096,
                                 F, st));
    REJECT(w8a8_quantize_weights(P, 64, 64, 0, F, 7, 127.f, Q, 0, 0, 4096, F, st));
    REJECT(w8a8_quantize_weights(P, 64, 64, 0, F, W8A8_FOLD_DIVIDE, 127.f, Q, 0, 0, 100, F, st));
    REJECT(w8a8_quantize_weights(P, 64, 64, 0, F, W8A8_FOLD_DIVIDE, 127.f, Q, 0, 1, 100, F, st));

    // ---- GEMMs ----------------------------------------------------------------
    REJECT(w8a8_gemm(64, 64, 64, nullptr, A, P, 64, 64, 64, F, F, 1.f, 1.f, W8A8_OUT_F16,
                     W8A8_LAYOUT_A_ROW_B_NK, nullptr, 0, st));
    REJECT(w8a8_gemm(0, 64, 64, A, A, P, 64, 64, 64, F, F, 1.f, 1.f, W8A8_OUT_F16,
                     W8A8_LAYOUT_A_ROW_B_NK, nullptr, 0, st));
    REJECT(w8a8_gemm(64, 64, 64, A, A, P, 32, 64, 64, F, F, 1.f, 1.f, W8A8_OUT_F16,
                     W8A8_LAYOUT_A_ROW_B_NK, nullptr, 0, st));
    REJECT(w8a8_gemm(64, 64, 64, A, A, P, 64, 64, 64, F, F, 1.f, 1.f, 9,
                     W8A8_LAYOUT_A_ROW_B_NK, nullptr, 0, st));
    REJECT(w8a8_gemm(64, 64, 64, A, A, P, 64, 64, 64, F, F, 1.f, 1.f, W8A8_OUT_F16, 5, nullptr,
                     0, st));
    REJECT(w8a8_gemm_noalloc(64, 64, 64, nullptr, A, P, 64, 64, 64, F, F, 1.f, 1.f,
                             W8A8_OUT_F16, W8A8_LAYOUT_A_ROW_B_NK, st));
    REJECT(w8a8_gemm_noalloc(60000, 60000, 60000, A, A, P, 60000, 60000, 60000, F, F, 1.f, 1.f,
                             W8A8_OUT_F16, W8A8_LAYOUT_A_COL_B_KN, st));
    REJECT(w8a8_gemm_streamk(256, 256, 256, A, A, P, 256, 256, 256, nullptr, nullptr, 1.f, 1.f,
                             W8A8_OUT_F16, 0, nullptr, 0, st));
    REJECT(w8a8_gemm_streamk(256, 256, 250, A, A, P, 256, 256, 256, nullptr, nullptr, 1.f, 1.f,
                             W8A8_OUT_F16, 0, P, 1 << 20, st));
    REJECT(w8a8_gemm_streamk(256, 256, 256, A, A, P, 256, 256, 256, nullptr, nullptr, 1.f, 1.f,
                             W8A8_OUT_F16, 0, static_cast<int8_t*>(P) + 4, 1 << 20, st));
    REJECT(w8a8_gemm_streamk_status(nullptr, 1));
    REJECT(w8a8_debug_streamk_wait(0, 1));
    REJECT(w8a8_debug_streamk_wait(100000, 1));
    if(w8a8_debug_streamk_wait(0, 0) != W8A8_SUCCESS) return 1;
    REJECT(w8a8_fused_sq_gemm(nullptr, F, A, F, P, 64, 64, 64, 0, 0, 0, Q, F, nullptr, 0, st));
    REJECT(w8a8_fused_sq_gemm(P, F, A, F, P, 0, 64, 64, 0, 0, 0, Q, F, nullptr, 0, st));
    REJECT(w8a8_pack_weights(nullptr, 64, 128, 128, Q, 1 << 20, st));
    REJECT(w8a8_pack_weights(A, 64, 128, 128, Q, 16, st));
    REJECT(w8a8_gemm_packed(64, 64, 128, nullptr, A, P, 128, 64, F, F, 1.f, 1.f, W8A8_OUT_F16,
                            nullptr, 0, st));
    REJECT(w8a8_gemm_packed(64, 64, 120, A, A, P, 128, 64, F, F, 1.f, 1.f, W8A8_OUT_F16,
                            nullptr, 0, st));
    REJECT(w8a8_fused_sq_gemm_packed(nullptr, F, A, F, P, 4, 64, 128, 0, 0, Q, F, nullptr, 0,
                                     st));
    w8a8_group_desc g[2];
    std::memset(g, 0, sizeof(g));
    g[0] = {A, A, P, F, F, 64, 64, 64, 64, 64, 64, 1.f, 1.f};
    g[1] = {nullptr, A, P, F, F, 64, 64, 64, 64, 64, 64, 1.f, 1.f};
    REJECT(w8a8_grouped_gemm(g, 2, W8A8_OUT_F16, P, 1 << 20, st));
    REJECT(w8a8_grouped_gemm(nullptr, 2, W8A8_OUT_F16, P, 1 << 20, st));
    REJECT(w8a8_grouped_gemm(g, 1, W8A8_OUT_F16, P, 4, st));

    // ---- MoE --------------------------------------------------------------------
    REJECT(w8a8_topk_softmax(nullptr, 0, F, I, 16, 8, 2, st));
    REJECT(w8a8_topk_softmax(P, 0, F, I, 16, 8, 9, st));
    REJECT(w8a8_topk_softmax(P, 0, F, I, 16, 5000, 2, st));
    REJECT(w8a8_moe_sort(nullptr, 16, 2, 8, 32, I, I, I, I, 4096, I, nullptr, 0, st));
    REJECT(w8a8_moe_sort(I, 16, 2, 8, 32, I, I, I, I, 8, I, nullptr, 0, st));
    REJECT(w8a8_moe_sort(I, 16, 2, 2000, 32, I, I, I, I, 1 << 20, I, nullptr, 0, st));
    REJECT(w8a8_moe_gemm(8, 256, 64, 64, nullptr, 64, A, 64, 64 * 64, P, 64, F, F, 1.f, 1.f, I,
                         I, W8A8_OUT_F16, nullptr, 0, st));
    REJECT(w8a8_moe_gemm(8, 256, 64, 60, A, 64, A, 64, 64 * 64, P, 64, F, F, 1.f, 1.f, I, I,
                         W8A8_OUT_F16, nullptr, 0, st));
    REJECT(w8a8_moe_silu_mul_quant(nullptr, 128, F, I, I, 8, 256, 64, Q, 64, F, 127.f, st));
    REJECT(w8a8_moe_silu_mul_quant(P, 100, F, I, I, 8, 256, 64, Q, 64, F, 127.f, st));
    REJECT(w8a8_moe_interleave_gate_up(nullptr, F, 8, 64, 64, 0, Q, F, st));
    REJECT(w8a8_moe_interleave_gate_up(A, F, 8, 63, 64, 0, Q, F, st));
    REJECT(w8a8_moe_gate_up_silu(8, 256, 64, 64, nullptr, 64, A, F, F, 1.f, 1.f, F, I, I, Q, 0,
                                 F, 127.f, P, 1 << 20, st));
    REJECT(w8a8_moe_gate_up_silu(8, 256, 60, 64, A, 64, A, F, F, 1.f, 1.f, F, I, I, Q, 0, F,
                                 127.f, P, 1 << 20, st));
    REJECT(w8a8_moe_gate_up_silu(8, 256, 64, 64, A, 64, A, F, F, 1.f, 1.f, F, I, I, Q, 0, F,
                                 127.f, P, 16, st));
    REJECT(w8a8_moe_combine(nullptr, 64, 32, F, I, 16, 2, 64, P, 64, st));
    REJECT(w8a8_moe_combine(P, 32, 32, F, I, 16, 2, 64, P, 64, st));
    std::printf("OK %d (%zu)\n", g_calls, sink % 7);
    return 0;
}
