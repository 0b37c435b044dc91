/*
 * w8a8_oracle.c -- CPU restatement of the reference's W8A8 SmoothQuant path.
 *
 * TEST INFRASTRUCTURE ONLY (see w8a8_oracle.h).  Built with -O3
 * -ffp-contract=off and without -ffast-math so every float operation is the
 * single IEEE operation the reference performs.
 */
#include "w8a8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int w8a8o_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32                                                      */
/* ------------------------------------------------------------------------- */
float w8a8o_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e    = (h >> 10) & 0x1Fu;
    uint32_t m    = h & 0x3FFu;
    uint32_t bits;
    float    f;
    if(e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        f = (float)m * (1.0f / 16777216.0f);
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if(e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t w8a8o_float_to_half(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a    = x & 0x7FFFFFFFu;
    if(a > 0x7F800000u) /* NaN: quiet, keep top payload bits */
        return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if(a >= 0x477FF000u) /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7C00u);
    if(a < 0x38800000u) { /* below 2^-14: binary16 subnormal (or rounds up to min normal) */
        float v;
        memcpy(&v, &a, 4);
        uint32_t m = (uint32_t)rintf(v * 16777216.0f); /* exact scaling, RNE */
        return (uint16_t)(sign | m);
    }
    uint32_t r = a + 0xC8000000u;          /* rebias exponent 127 -> 15 */
    r += 0xFFFu + ((r >> 13) & 1u);        /* round to nearest even on the 13 dropped bits */
    return (uint16_t)(sign | (r >> 13));
}

/* ------------------------------------------------------------------------- */
/* quantization core shared by the dense and MoE restatements                 */
/* ------------------------------------------------------------------------- */
static inline int8_t quant_one(float p, float inv, float qmax)
{
    /* rocwmma_smoothquant.cpp:110-113: float s = x*smooth*inv; rint; clamp; cast */
    float v = p * inv;
    return (int8_t)fminf(fmaxf(rintf(v), -qmax), qmax);
}

static void quant_row(const uint16_t* xrow, const float* srow, uint32_t N, float qmax,
                      int8_t* qrow, float* rs_out)
{
    /* pass 1 (rocwmma_smoothquant.cpp:76-89) */
    float amax = 0.f;
    for(uint32_t n = 0; n < N; ++n)
        amax = fmaxf(amax, fabsf(w8a8o_half_to_float(xrow[n]) * srow[n]));
    /* :95 */
    float rs = amax / qmax;
    *rs_out  = rs;
    /* :98 */
    float inv = (rs > 0.f) ? (1.f / rs) : 0.f;
    /* pass 2 (:101-121): x*s is recomputed, then multiplied by inv */
    for(uint32_t n = 0; n < N; ++n)
        qrow[n] = quant_one(w8a8o_half_to_float(xrow[n]) * srow[n], inv, qmax);
}

void w8a8o_smoothquant(const uint16_t* x, const float* s, int8_t* q, float* r,
                       uint32_t M, uint32_t N, float quant_max,
                       uint32_t ldx, uint32_t ldq)
{
#pragma omp parallel for schedule(static)
    for(long m = 0; m < (long)M; ++m)
        quant_row(x + (size_t)m * ldx, s, N, quant_max, q + (size_t)m * ldq, &r[m]);
}

void w8a8o_moe_smoothquant(const uint16_t* x, const float* s, const int32_t* topk_ids,
                           int8_t* qy, float* row_scale,
                           uint32_t tokens, uint32_t hidden, uint32_t topk,
                           uint32_t experts, float quant_max, const int32_t* dst_row)
{
    long total = (long)tokens * topk;
#pragma omp parallel for schedule(static)
    for(long flat = 0; flat < total; ++flat) {
        long    tok = flat / topk;                       /* :82 */
        int32_t e   = topk_ids[flat];                    /* :86 (tok*topk+slot == flat) */
        if(e < 0 || (uint32_t)e >= experts) continue;    /* :87 */
        long dst = dst_row ? dst_row[flat] : flat;
        if(dst < 0) continue;
        quant_row(x + (size_t)tok * hidden, s + (size_t)e * hidden, hidden, quant_max,
                  qy + (size_t)dst * hidden, &row_scale[dst]);
    }
}

/* ------------------------------------------------------------------------- */
/* weight quantization (fold + per-channel absmax)                            */
/* ------------------------------------------------------------------------- */
void w8a8o_quantize_weights(const uint16_t* w, const float* s, int divide, float quant_max,
                            int8_t* q, float* sb, uint32_t N, uint32_t K, uint32_t ldw,
                            uint32_t ldq)
{
#pragma omp parallel
    {
        float* p = (float*)malloc(sizeof(float) * K);
#pragma omp for schedule(static)
        for(long n = 0; n < (long)N; ++n) {
            const uint16_t* wr   = w + (size_t)n * ldw;
            float           amax = 0.f;
            for(uint32_t k = 0; k < K; ++k) {
                p[k] = w8a8o_half_to_float(wr[k]);
                if(s) p[k] = divide ? p[k] / s[k] : p[k] * s[k];
                amax = fmaxf(amax, fabsf(p[k]));
            }
            const float rs  = amax / quant_max;
            const float inv = (rs > 0.f) ? (1.f / rs) : 0.f;
            sb[n]           = rs;
            for(uint32_t k = 0; k < K; ++k) q[(size_t)n * ldq + k] = quant_one(p[k], inv, quant_max);
        }
        free(p);
    }
}

/* ------------------------------------------------------------------------- */
/* RMSNorm (+ residual) -> quantizer                                          */
/* ------------------------------------------------------------------------- */
void w8a8o_rmsnorm_smoothquant(const uint16_t* x, const uint16_t* res, const float* gamma,
                               const float* s, uint16_t* x_out, uint16_t* y, int8_t* q,
                               float* r, uint32_t M, uint32_t N, float eps, float quant_max,
                               uint32_t ldx, uint32_t ldy, uint32_t ldq)
{
#pragma omp parallel
    {
        float*    v  = (float*)malloc(sizeof(float) * N);
        uint16_t* yh = (uint16_t*)malloc(sizeof(uint16_t) * N);
#pragma omp for schedule(static)
        for(long m = 0; m < (long)M; ++m) {
            const uint16_t* xr = x + (size_t)m * ldx;
            const uint16_t* rr = res ? res + (size_t)m * ldx : NULL;
            /* :157-160 / :79-80: v = x (+ residual) in fp32; squares summed */
            double ss = 0.0;
            for(uint32_t n = 0; n < N; ++n) {
                v[n] = w8a8o_half_to_float(xr[n]);
                if(rr) v[n] += w8a8o_half_to_float(rr[n]);
                ss += (double)v[n] * (double)v[n];
            }
            /* :170 / :99: rstd = rsqrt(sum / N + eps), each step in fp32 */
            const float mean = (float)ss / (float)N;
            const float rstd = (float)(1.0 / sqrt((double)(mean + eps)));
            for(uint32_t n = 0; n < N; ++n) {
                float u = v[n];
                if(rr) {
                    /* :159 x_out = half(v); :173-180 normalises the saved x_out */
                    const uint16_t h = w8a8o_float_to_half(v[n]);
                    if(x_out) x_out[(size_t)m * ldx + n] = h;
                    u = w8a8o_half_to_float(h);
                }
                /* :182 / :112: f * rstd * gamma, rounded to fp16 */
                yh[n] = w8a8o_float_to_half((u * rstd) * gamma[n]);
                if(y) y[(size_t)m * ldy + n] = yh[n];
            }
            if(q) quant_row(yh, s, N, quant_max, q + (size_t)m * ldq, &r[m]);
        }
        free(v);
        free(yh);
    }
}

/* ------------------------------------------------------------------------- */
/* int8 GEMM (gemm_cpu_h semantics)                                           */
/* ------------------------------------------------------------------------- */
void w8a8o_gemm_i8_i32(uint32_t M, uint32_t N, uint32_t K,
                       const int8_t* a, const int8_t* b, int32_t* c,
                       uint32_t lda, uint32_t ldb, uint32_t ldc, int layout,
                       uint32_t row_begin, uint32_t row_end)
{
    if(row_end > M) row_end = M;
    if(layout == W8A8O_LAYOUT_A_ROW_B_NK) {
        /* aIndex = row-major (i*lda + h); bIndex = col-major (j*ldb + h) */
#pragma omp parallel for schedule(dynamic, 1)
        for(long i = row_begin; i < (long)row_end; ++i) {
            const int8_t* ar = a + (size_t)i * lda;
            for(uint32_t j = 0; j < N; ++j) {
                const int8_t* br  = b + (size_t)j * ldb;
                int32_t       acc = 0;
                for(uint32_t h = 0; h < K; ++h)
                    acc += (int32_t)ar[h] * (int32_t)br[h];
                c[(size_t)i * ldc + j] = acc;
            }
        }
    } else {
        /* aIndex = col-major (h*lda + i); bIndex = row-major (h*ldb + j) */
#pragma omp parallel for schedule(dynamic, 1)
        for(long i = row_begin; i < (long)row_end; ++i) {
            int32_t* crow = c + (size_t)i * ldc;
            for(uint32_t j = 0; j < N; ++j) crow[j] = 0;
            for(uint32_t h = 0; h < K; ++h) {
                int32_t       av = a[(size_t)h * lda + i];
                const int8_t* br = b + (size_t)h * ldb;
                for(uint32_t j = 0; j < N; ++j)
                    crow[j] += av * (int32_t)br[j];
            }
        }
    }
}

void w8a8o_dequant_f16(uint32_t M, uint32_t N, const int32_t* acc, uint32_t ldacc,
                       const float* scale_a, const float* scale_b,
                       float tensor_scale_a, float tensor_scale_b,
                       uint16_t* out, uint32_t ldo)
{
    int   mode1 = (scale_a == NULL && scale_b == NULL);
    float ab    = tensor_scale_a * tensor_scale_b; /* rocwmma_gemm_quantized.cpp:189 */
#pragma omp parallel for schedule(static)
    for(long m = 0; m < (long)M; ++m) {
        float sa = scale_a ? scale_a[m] : tensor_scale_a;
        for(uint32_t n = 0; n < N; ++n) {
            float v = (float)acc[(size_t)m * ldacc + n];
            if(mode1) {
                v = v * ab;                                    /* :192 */
            } else {
                float sb = scale_b ? scale_b[n] : tensor_scale_b;
                v        = (v * sa) * sb;
            }
            out[(size_t)m * ldo + n] = w8a8o_float_to_half(v);
        }
    }
}

/* ------------------------------------------------------------------------- */
/* MoE routing                                                                */
/* ------------------------------------------------------------------------- */
void w8a8o_topk_softmax(const float* logits, float* topk_weights, int32_t* topk_ids,
                        uint32_t tokens, uint32_t experts, uint32_t topk)
{
    for(uint32_t t = 0; t < tokens; ++t) {
        const float* row  = logits + (size_t)t * experts;
        float        wmax = -INFINITY;
        for(uint32_t e = 0; e < experts; ++e) wmax = fmaxf(wmax, row[e]);
        float wsum = 0.f;
        for(uint32_t e = 0; e < experts; ++e) wsum += expf(row[e] - wmax);
        float inv = (wsum > 0.f) ? 1.f / wsum : 0.f;
        /* iterative arg-max with lower index winning ties (:108-129) */
        uint64_t used[4] = {0, 0, 0, 0}; /* experts <= 256 */
        for(uint32_t k = 0; k < topk; ++k) {
            int32_t best = -1;
            for(uint32_t e = 0; e < experts; ++e) {
                if(used[e >> 6] >> (e & 63) & 1u) continue;
                if(best < 0 || row[e] > row[best]) best = (int32_t)e;
            }
            topk_ids[(size_t)t * topk + k] = best;
            topk_weights[(size_t)t * topk + k]
                = best >= 0 ? expf(row[best] - wmax) * inv : 0.f;
            if(best >= 0) used[best >> 6] |= (uint64_t)1 << (best & 63);
        }
    }
}

void w8a8o_moe_sort(const int32_t* topk_ids, uint32_t tokens, uint32_t topk,
                    uint32_t experts, uint32_t unit_size,
                    int32_t* expert_count, int32_t* expert_start, int32_t* padded_count,
                    int32_t* sorted_token_ids, int32_t* dst_row)
{
    size_t total = (size_t)tokens * topk;
    size_t bound = total + (size_t)experts * unit_size;
    for(uint32_t e = 0; e < experts; ++e) expert_count[e] = 0;
    for(size_t p = 0; p < total; ++p) { /* histogram (:53-77) */
        int32_t e = topk_ids[p];
        if(e >= 0 && (uint32_t)e < experts) expert_count[e]++;
    }
    int32_t off = 0; /* padded prefix (:82-101) */
    for(uint32_t e = 0; e < experts; ++e) {
        expert_start[e] = off;
        int32_t pc      = (int32_t)((expert_count[e] + unit_size - 1) / unit_size * unit_size);
        padded_count[e] = pc;
        off += pc;
    }
    expert_start[experts] = off;
    for(size_t p = 0; p < bound; ++p) sorted_token_ids[p] = -1;
    int32_t* cursor = (int32_t*)calloc(experts ? experts : 1, sizeof(int32_t));
    for(size_t p = 0; p < total; ++p) { /* stable scatter (:107-125 without atomics) */
        int32_t e = topk_ids[p];
        if(e < 0 || (uint32_t)e >= experts) {
            dst_row[p] = -1;
            continue;
        }
        int32_t slot           = expert_start[e] + cursor[e]++;
        sorted_token_ids[slot] = (int32_t)(p / topk);
        dst_row[p]             = slot;
    }
    free(cursor);
}

void w8a8o_silu_mul_quant(const uint16_t* gate_up, uint32_t rows, uint32_t inter,
                          uint32_t ld_gu, const float* s2, float quant_max,
                          int8_t* q, float* row_scale, uint32_t ldq)
{
#pragma omp parallel for schedule(static)
    for(long r = 0; r < (long)rows; ++r) {
        const uint16_t* g   = gate_up + (size_t)r * ld_gu;
        float*          act = (float*)malloc(sizeof(float) * (inter ? inter : 1));
        float           amax = 0.f;
        for(uint32_t j = 0; j < inter; ++j) {
            float gv = w8a8o_half_to_float(g[j]);
            float uv = w8a8o_half_to_float(g[inter + j]);
            float a  = (gv / (1.f + expf(-gv))) * uv;
            if(s2) a = a * s2[j];
            act[j] = a;
            amax   = fmaxf(amax, fabsf(a));
        }
        float rs      = amax / quant_max;
        row_scale[r]  = rs;
        float inv     = (rs > 0.f) ? (1.f / rs) : 0.f;
        int8_t* qrow  = q + (size_t)r * ldq;
        for(uint32_t j = 0; j < inter; ++j) qrow[j] = quant_one(act[j], inv, quant_max);
        free(act);
    }
}

void w8a8o_moe_combine(const uint16_t* y, uint32_t ldy, const float* topk_weights,
                       const int32_t* dst_row, uint32_t tokens, uint32_t topk,
                       uint32_t n, uint16_t* out, uint32_t ldo)
{
#pragma omp parallel for schedule(static)
    for(long t = 0; t < (long)tokens; ++t) {
        for(uint32_t c = 0; c < n; ++c) {
            float acc = 0.f;
            for(uint32_t k = 0; k < topk; ++k) {
                int32_t d = dst_row[(size_t)t * topk + k];
                if(d < 0) continue;
                acc = fmaf(topk_weights[(size_t)t * topk + k],
                           w8a8o_half_to_float(y[(size_t)d * ldy + c]), acc);
            }
            out[(size_t)t * ldo + c] = w8a8o_float_to_half(acc);
        }
    }
}
