/*
 * Driver of the CPU oracle (oracle/w8a8_oracle.c) for the AddressSanitizer /
 * UndefinedBehaviorSanitizer build of test_sanitizers_cpu.py.  Every oracle
 * routine runs on small inputs held in heap buffers of exactly the size its
 * header documents (row strides wider than the rows where it takes them), so
 * a read or write one element past a buffer, a signed overflow or an
 * out-of-range shift in the oracle stops the run.  Prints "OK" on success.
 */
#include "../oracle/w8a8_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t g_state = 0x5EED5A17ull;

static uint64_t next_u64(void)
{
    /* splitmix64 */
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z          = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z          = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static float uniform(float lo, float hi)
{
    return lo + (hi - lo) * (float)((next_u64() >> 40) * (1.0 / 16777216.0));
}

static void* xmalloc(size_t bytes)
{
    void* p = malloc(bytes ? bytes : 1);
    if(!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static uint16_t* halfs(size_t n, float lo, float hi)
{
    uint16_t* h = xmalloc(n * sizeof(uint16_t));
    for(size_t i = 0; i < n; ++i) h[i] = w8a8o_float_to_half(uniform(lo, hi));
    return h;
}

static float* floats(size_t n, float lo, float hi)
{
    float* f = xmalloc(n * sizeof(float));
    for(size_t i = 0; i < n; ++i) f[i] = uniform(lo, hi);
    return f;
}

static int8_t* int8s(size_t n)
{
    int8_t* v = xmalloc(n);
    for(size_t i = 0; i < n; ++i) v[i] = (int8_t)((int)(next_u64() % 255) - 127);
    return v;
}

static void check_conversions(void)
{
    /* every binary16 bit pattern through float and back (NaNs keep NaN) */
    for(uint32_t b = 0; b < 65536; ++b) {
        const float    f = w8a8o_half_to_float((uint16_t)b);
        const uint16_t r = w8a8o_float_to_half(f);
        if(!isnan(f) && r != b) {
            printf("FAIL half round trip %u -> %u\n", b, r);
            exit(1);
        }
    }
    const float edge[] = {0.f, -0.f, 65504.f, 65520.f, 1e-8f, -1e-8f, 6e-5f, 1e30f, -1e30f, NAN,
                          INFINITY, -INFINITY};
    for(size_t i = 0; i < sizeof(edge) / sizeof(edge[0]); ++i) (void)w8a8o_float_to_half(edge[i]);
}

static void check_smoothquant(uint32_t M, uint32_t N, uint32_t ldx, uint32_t ldq)
{
    uint16_t* x = halfs((size_t)(M - 1) * ldx + N, -30.f, 30.f);
    float*    s = floats(N, 0.5f, 2.f);
    int8_t*   q = xmalloc((size_t)(M - 1) * ldq + N);
    float*    r = xmalloc(M * sizeof(float));
    w8a8o_smoothquant(x, s, q, r, M, N, 127.f, ldx, ldq);
    free(x), free(s), free(q), free(r);
}

static void check_moe_smoothquant(uint32_t T, uint32_t H, uint32_t K, uint32_t E, int sorted)
{
    uint16_t* x   = halfs((size_t)T * H, -5.f, 5.f);
    float*    s   = floats((size_t)E * H, 0.5f, 2.f);
    int32_t*  ids = xmalloc((size_t)T * K * sizeof(int32_t));
    for(uint32_t i = 0; i < T * K; ++i)
        ids[i] = (int32_t)(next_u64() % (E + 2)) - 1; /* some ids invalid (-1, E) */
    const uint32_t rows = T * K;
    int32_t*       dst  = NULL;
    if(sorted) { /* a permutation of the rows */
        dst = xmalloc(rows * sizeof(int32_t));
        for(uint32_t i = 0; i < rows; ++i) dst[i] = (int32_t)i;
        for(uint32_t i = rows; i > 1; --i) {
            const uint32_t j = (uint32_t)(next_u64() % i);
            const int32_t  t = dst[i - 1];
            dst[i - 1]       = dst[j];
            dst[j]           = t;
        }
    }
    int8_t* q = xmalloc((size_t)rows * H);
    float*  r = xmalloc(rows * sizeof(float));
    w8a8o_moe_smoothquant(x, s, ids, q, r, T, H, K, E, 127.f, dst);
    free(x), free(s), free(ids), free(dst), free(q), free(r);
}

static void check_rmsnorm(uint32_t M, uint32_t N, uint32_t ldx, int with_res, int with_q)
{
    const size_t xn = (size_t)(M - 1) * ldx + N;
    uint16_t*    x  = halfs(xn, -3.f, 3.f);
    uint16_t*    rs = with_res ? halfs(xn, -3.f, 3.f) : NULL;
    uint16_t*    xo = with_res ? xmalloc(xn * sizeof(uint16_t)) : NULL;
    float*       g  = floats(N, 0.5f, 1.5f);
    float*       s  = with_q ? floats(N, 0.5f, 2.f) : NULL;
    uint16_t*    y  = xmalloc((size_t)M * N * sizeof(uint16_t));
    int8_t*      q  = with_q ? xmalloc((size_t)M * N) : NULL;
    float*       r  = with_q ? xmalloc(M * sizeof(float)) : NULL;
    w8a8o_rmsnorm_smoothquant(x, rs, g, s, xo, y, q, r, M, N, 1e-5f, 127.f, ldx, N, N);
    free(x), free(rs), free(xo), free(g), free(s), free(y), free(q), free(r);
}

static void check_quantize_weights(uint32_t N, uint32_t K, int with_s, int divide)
{
    uint16_t* w  = halfs((size_t)N * K, -1.f, 1.f);
    float*    s  = with_s ? floats(K, 0.5f, 2.f) : NULL;
    int8_t*   q  = xmalloc((size_t)N * K);
    float*    sb = xmalloc(N * sizeof(float));
    w8a8o_quantize_weights(w, s, divide, 127.f, q, sb, N, K, K, K);
    free(w), free(s), free(q), free(sb);
}

static void check_gemm(uint32_t M, uint32_t N, uint32_t K, int layout)
{
    const uint32_t lda = layout == 0 ? K + 3 : M + 5;
    const uint32_t ldb = layout == 0 ? K + 1 : N + 2;
    const size_t   an  = layout == 0 ? (size_t)(M - 1) * lda + K : (size_t)(K - 1) * lda + M;
    const size_t   bn  = layout == 0 ? (size_t)(N - 1) * ldb + K : (size_t)(K - 1) * ldb + N;
    int8_t*        a   = int8s(an);
    int8_t*        b   = int8s(bn);
    int32_t*       c   = xmalloc((size_t)M * N * sizeof(int32_t));
    w8a8o_gemm_i8_i32(M, N, K, a, b, c, lda, ldb, N, layout, 0, M);
    float*    sa = floats(M, 1e-3f, 1e-2f);
    float*    sb = floats(N, 1e-3f, 1e-2f);
    uint16_t* o  = xmalloc((size_t)M * N * sizeof(uint16_t));
    w8a8o_dequant_f16(M, N, c, N, sa, sb, 1.f, 1.f, o, N);
    w8a8o_dequant_f16(M, N, c, N, NULL, NULL, 0.02f, 0.003f, o, N);
    w8a8o_dequant_f16(M, N, c, N, sa, NULL, 1.f, 0.5f, o, N);
    free(a), free(b), free(c), free(sa), free(sb), free(o);
}

static void check_routing(uint32_t T, uint32_t E, uint32_t K, uint32_t unit)
{
    float*   logits = floats((size_t)T * E, -3.f, 3.f);
    float*   w      = xmalloc((size_t)T * K * sizeof(float));
    int32_t* ids    = xmalloc((size_t)T * K * sizeof(int32_t));
    w8a8o_topk_softmax(logits, w, ids, T, E, K);
    int32_t* count  = xmalloc(E * sizeof(int32_t));
    int32_t* start  = xmalloc((E + 1) * sizeof(int32_t));
    int32_t* padded = xmalloc(E * sizeof(int32_t));
    int32_t* sorted = xmalloc(((size_t)T * K + (size_t)E * unit) * sizeof(int32_t));
    int32_t* dst    = xmalloc((size_t)T * K * sizeof(int32_t));
    w8a8o_moe_sort(ids, T, K, E, unit, count, start, padded, sorted, dst);
    /* combine over the sorted rows with a strided y */
    const uint32_t rows = (uint32_t)start[E], n = 40, ldy = 48;
    uint16_t*      y    = halfs(rows ? (size_t)(rows - 1) * ldy + n : 1, -2.f, 2.f);
    uint16_t*      out  = xmalloc((size_t)T * n * sizeof(uint16_t));
    if(rows) w8a8o_moe_combine(y, ldy, w, dst, T, K, n, out, n);
    free(logits), free(w), free(ids), free(count), free(start), free(padded), free(sorted);
    free(dst), free(y), free(out);
}

static void check_silu(uint32_t rows, uint32_t inter, int with_s2)
{
    const uint32_t ld = 2 * inter + 8;
    uint16_t*      gu = halfs((size_t)(rows - 1) * ld + 2 * inter, -8.f, 8.f);
    float*         s2 = with_s2 ? floats(inter, 0.5f, 2.f) : NULL;
    int8_t*        q  = xmalloc((size_t)rows * inter);
    float*         r  = xmalloc(rows * sizeof(float));
    w8a8o_silu_mul_quant(gu, rows, inter, ld, s2, 127.f, q, r, inter);
    free(gu), free(s2), free(q), free(r);
}

int main(void)
{
    check_conversions();
    check_smoothquant(1, 1, 1, 1);
    check_smoothquant(7, 1000, 1000, 1000);
    check_smoothquant(5, 4104, 4200, 4110);
    check_smoothquant(3, 8192, 8192, 8192);
    check_moe_smoothquant(9, 1024, 2, 8, 0);
    check_moe_smoothquant(13, 520, 3, 5, 1);
    check_rmsnorm(4, 1024, 1024, 0, 0);
    check_rmsnorm(3, 2050, 2056, 1, 1);
    check_rmsnorm(2, 8192, 8192, 1, 0);
    check_quantize_weights(17, 300, 1, 1);
    check_quantize_weights(5, 64, 1, 0);
    check_quantize_weights(3, 48, 0, 0);
    check_gemm(9, 17, 64, 0);
    check_gemm(13, 11, 48, 1);
    check_gemm(1, 1, 1, 0);
    check_routing(37, 8, 2, 32);
    check_routing(64, 5, 1, 1);
    check_routing(20, 64, 6, 16);
    check_silu(7, 144, 1);
    check_silu(3, 40, 0);
    printf("OK\n");
    return 0;
}
