// moe.hip -- the MoE pieces around the W8A8 GEMM for gfx950: top-k softmax
// routing, a deterministic expert sort, the SiLU(gate)*up requantization
// between the two expert GEMMs, the weighted combine back to token order, and
// the launchers of the grouped / MoE GEMM kernels.
#include "gemm_i8_grouped_kernel.hpp"
#include "w8a8_internal.hpp"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <mutex>

namespace w8a8 {
namespace {

// ---------------------------------------------------------------------------
// Top-k softmax (kernel_topk_softmax, rocwmma_topk_softmax.cpp:58-131).
// One wave per token.  Experts are chosen on the logits (softmax is monotonic,
// so the choice is exact), highest first, the lower expert index winning ties
// (the reference's strict '>' keeps the lower lane).  weight =
// exp(l - max) * (1 / sum_e exp(l_e - max)), as the reference computes it.
// ---------------------------------------------------------------------------
constexpr int kTopkWaves = 4;

template <bool F16>
__device__ __forceinline__ float load_logit(const void* p, size_t i)
{
    if constexpr(F16)
        return half_bits_to_float(static_cast<const uint16_t*>(p)[i]);
    else
        return static_cast<const float*>(p)[i];
}

// (value, index) of the better of two candidates: larger value, then lower index.
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi)
{
    if(ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

template <bool F16>
__global__ void __launch_bounds__(kTopkWaves* kWave)
    topk_softmax_kernel(const void* logits, float* topk_w, int32_t* topk_ids, uint32_t tokens,
                        uint32_t experts, uint32_t topk)
{
    const uint32_t tok  = blockIdx.x * kTopkWaves + threadIdx.x / kWave;
    const int      lane = threadIdx.x % kWave;
    if(tok >= tokens) return; // uniform per wave
    const size_t row = (size_t)tok * experts;

    // cross-lane steps are DPP reductions (no LDS round trips)
    float wmax = -INFINITY;
    for(uint32_t e = lane; e < experts; e += kWave) wmax = fmaxf(wmax, load_logit<F16>(logits, row + e));
    wmax = wave_max(wmax);
    float wsum = 0.f;
    for(uint32_t e = lane; e < experts; e += kWave) wsum += expf(load_logit<F16>(logits, row + e) - wmax);
    wsum            = wave_sum(wsum);
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;

    // a lane owns experts lane, lane+64, ...: `used` marks the chosen ones.
    // Per pick: each lane's best unused candidate (larger logit, then lower
    // index), the wave max of those values, then the lowest index among the
    // lanes holding that max: the same winner as a pairwise reduction.
    constexpr int kNone = 0x7FFFFFFF;
    uint64_t      used  = 0;
    for(uint32_t k = 0; k < topk; ++k) {
        float bv = -INFINITY;
        int   bi = kNone;
        int   j  = 0;
        for(uint32_t e = lane; e < experts; e += kWave, ++j)
            if(!((used >> j) & 1u)) better(bv, bi, load_logit<F16>(logits, row + e), (int)e);
        const float m = wave_max(bv);
        const int   w = wave_min_i32(bv == m ? bi : kNone);
        if(w != kNone && (uint32_t)w % kWave == (uint32_t)lane) used |= 1ull << ((uint32_t)w / kWave);
        if(lane == 0) {
            const bool ok                    = w != kNone;
            topk_ids[(size_t)tok * topk + k] = ok ? w : -1;
            topk_w[(size_t)tok * topk + k]   = ok ? expf(m - wmax) * inv : 0.f;
        }
    }
}

// ---------------------------------------------------------------------------
// Expert sort (kernel_moe_histogram / kernel_prefix_sum / kernel_moe_scatter,
// rocwmma_moe_sorting.cpp:53-125), one workgroup, deterministic: inside an
// expert, pairs keep ascending flat order t*topk + slot (the reference's
// atomic scatter gives an arbitrary order, :122-124).  Outputs are the
// reference's (count, start with start[E] = total, padded count, sorted token
// ids with -1 in padding) plus dst_row[flat], the sorted row of each pair.
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 1024;
constexpr int kSortWaves   = kSortThreads / kWave;

__global__ void __launch_bounds__(kSortThreads)
    moe_sort_kernel(const int32_t* __restrict__ ids, uint32_t total, uint32_t topk,
                    uint32_t experts, uint32_t unit, int32_t* expert_count, int32_t* expert_start,
                    int32_t* padded_count, int32_t* sorted_ids, uint32_t sorted_cap,
                    int32_t* dst_row)
{
    extern __shared__ int32_t sm[];
    int32_t*  cnt    = sm;                   // [E]
    int32_t*  start  = cnt + experts;        // [E + 1]
    int32_t*  cursor = start + experts + 1;  // [E]
    int32_t*  wcnt   = cursor + experts;     // [waves][E]
    const int tid    = threadIdx.x;
    const int wave   = tid / kWave;
    const int lane   = tid % kWave;

    for(uint32_t e = tid; e < experts; e += kSortThreads) cnt[e] = cursor[e] = 0;
    for(uint32_t i = tid; i < experts * kSortWaves; i += kSortThreads) wcnt[i] = 0;
    __syncthreads();
    for(uint32_t p = tid; p < total; p += kSortThreads) {
        const int32_t e = ids[p];
        if(e >= 0 && (uint32_t)e < experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if(wave == 0) { // padded exclusive prefix, 64 experts per step
        int32_t carry = 0;
        for(uint32_t base = 0; base < experts; base += kWave) {
            const uint32_t e   = base + lane;
            const int32_t  c   = e < experts ? cnt[e] : 0;
            const int32_t  pad = (int32_t)(((uint32_t)c + unit - 1) / unit * unit);
            int32_t        s   = pad;
#pragma unroll
            for(int d = 1; d < kWave; d <<= 1) {
                const int32_t o = __shfl_up(s, d, kWave);
                if(lane >= d) s += o;
            }
            if(e < experts) {
                start[e]        = carry + s - pad;
                expert_count[e] = c;
                expert_start[e] = carry + s - pad;
                padded_count[e] = pad;
            }
            carry += __builtin_amdgcn_readlane(s, kWave - 1);
        }
        if(lane == 0) {
            start[experts]        = carry;
            expert_start[experts] = carry;
        }
    }
    for(uint32_t i = tid; i < sorted_cap; i += kSortThreads) sorted_ids[i] = -1;
    __syncthreads();

    for(uint32_t c0 = 0; c0 < total; c0 += kSortThreads) {
        const uint32_t p     = c0 + tid;
        const int32_t  e     = p < total ? ids[p] : -1;
        const bool     valid = e >= 0 && (uint32_t)e < experts;
        // rank among this wave's earlier lanes with the same expert
        int      rank    = 0;
        uint64_t pending = __ballot(valid);
        while(pending) {
            const int      leader = __ffsll((unsigned long long)pending) - 1;
            const int32_t  le     = __builtin_amdgcn_readlane(e, leader); // leader is uniform
            const uint64_t same   = __ballot(valid && e == le);
            if(valid && e == le) rank = __popcll(same & ((1ull << lane) - 1));
            if(lane == leader) wcnt[wave * experts + le] = __popcll(same);
            pending &= ~same;
        }
        __syncthreads();
        if(valid) {
            int32_t base = cursor[e];
            for(int w = 0; w < wave; ++w) base += wcnt[w * experts + e];
            const int32_t slot = start[e] + base + rank;
            sorted_ids[slot]   = (int32_t)(p / topk);
            dst_row[p]         = slot;
        } else if(p < total) {
            dst_row[p] = -1;
        }
        __syncthreads();
        for(uint32_t x = tid; x < experts; x += kSortThreads) {
            int32_t s = 0;
            for(int w = 0; w < kSortWaves; ++w) {
                s += wcnt[w * experts + x];
                wcnt[w * experts + x] = 0;
            }
            cursor[x] += s;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Multi-block expert sort (with the caller's workspace of blocks x E ints):
// the same outputs and order as moe_sort_kernel, spread over
// ceil(total / kSortChunk) blocks of one pair per thread.
//   1. moe_sort_count_kernel: block b counts the experts of its pairs into
//      ws[b*E + e], and the grid fills sorted_ids with -1.
//   2. moe_sort_offsets_kernel (one block): per expert the exclusive prefix
//      of the block counts (in place) and the total, the padded expert
//      prefix (count, start, padded), then ws[b*E + e] += start[e].
//   3. moe_sort_scatter_kernel: block b ranks its pairs stably (lanes of a
//      wave with the same expert by ballot, waves in order through LDS) and
//      writes sorted_ids[ws[b*E + e] + rank] and dst_row.
// Blocks cover consecutive pairs, so the order inside an expert is again
// ascending flat order.
// ---------------------------------------------------------------------------
constexpr uint32_t kSortChunk = kSortThreads;

__global__ void __launch_bounds__(kSortThreads)
    moe_sort_count_kernel(const int32_t* __restrict__ ids, uint32_t total, uint32_t experts,
                          int32_t* ws, int32_t* sorted_ids, uint32_t sorted_cap)
{
    extern __shared__ int32_t cnt[]; // [E]
    const uint32_t tid = threadIdx.x;
    for(uint32_t e = tid; e < experts; e += kSortThreads) cnt[e] = 0;
    __syncthreads();
    const uint32_t p = blockIdx.x * kSortChunk + tid;
    if(p < total) {
        const int32_t e = ids[p];
        if(e >= 0 && (uint32_t)e < experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    for(uint32_t e = tid; e < experts; e += kSortThreads)
        ws[(size_t)blockIdx.x * experts + e] = cnt[e];
    for(uint32_t i = blockIdx.x * kSortThreads + tid; i < sorted_cap; i += gridDim.x * kSortThreads)
        sorted_ids[i] = -1;
}

__global__ void __launch_bounds__(kSortThreads)
    moe_sort_offsets_kernel(uint32_t blocks, uint32_t experts, uint32_t unit, int32_t* ws,
                            int32_t* expert_count, int32_t* expert_start, int32_t* padded_count)
{
    extern __shared__ int32_t sm[];
    int32_t*       cnt   = sm;           // [E]
    int32_t*       start = cnt + experts; // [E]
    const uint32_t tid   = threadIdx.x;
    const int      wave  = tid / kWave;
    const int      lane  = tid % kWave;
    for(uint32_t e = tid; e < experts; e += kSortThreads) {
        int32_t run = 0;
        for(uint32_t b = 0; b < blocks; ++b) {
            const int32_t c                = ws[(size_t)b * experts + e];
            ws[(size_t)b * experts + e]    = run;
            run                           += c;
        }
        cnt[e] = run;
    }
    __syncthreads();
    if(wave == 0) { // padded exclusive prefix, 64 experts per step
        int32_t carry = 0;
        for(uint32_t base = 0; base < experts; base += kWave) {
            const uint32_t e   = base + lane;
            const int32_t  c   = e < experts ? cnt[e] : 0;
            const int32_t  pad = (int32_t)(((uint32_t)c + unit - 1) / unit * unit);
            int32_t        s   = pad;
#pragma unroll
            for(int d = 1; d < kWave; d <<= 1) {
                const int32_t o = __shfl_up(s, d, kWave);
                if(lane >= d) s += o;
            }
            if(e < experts) {
                start[e]        = carry + s - pad;
                expert_count[e] = c;
                expert_start[e] = carry + s - pad;
                padded_count[e] = pad;
            }
            carry += __builtin_amdgcn_readlane(s, kWave - 1);
        }
        if(lane == 0) expert_start[experts] = carry;
    }
    __syncthreads();
    for(uint32_t e = tid; e < experts; e += kSortThreads) {
        const int32_t s0 = start[e];
        for(uint32_t b = 0; b < blocks; ++b) ws[(size_t)b * experts + e] += s0;
    }
}

__global__ void __launch_bounds__(kSortThreads)
    moe_sort_scatter_kernel(const int32_t* __restrict__ ids, uint32_t total, uint32_t topk,
                            uint32_t experts, const int32_t* ws, int32_t* sorted_ids,
                            int32_t* dst_row)
{
    extern __shared__ int32_t wcnt[]; // [waves][E]
    const uint32_t tid  = threadIdx.x;
    const int      wave = tid / kWave;
    const int      lane = tid % kWave;
    for(uint32_t i = tid; i < experts * kSortWaves; i += kSortThreads) wcnt[i] = 0;
    const uint32_t p     = blockIdx.x * kSortChunk + tid;
    const int32_t  e     = p < total ? ids[p] : -1;
    const bool     valid = e >= 0 && (uint32_t)e < experts;
    __syncthreads();
    int      rank    = 0;
    uint64_t pending = __ballot(valid);
    while(pending) {
        const int      leader = __ffsll((unsigned long long)pending) - 1;
        const int32_t  le     = __builtin_amdgcn_readlane(e, leader); // leader is uniform
        const uint64_t same   = __ballot(valid && e == le);
        if(valid && e == le) rank = __popcll(same & ((1ull << lane) - 1));
        if(lane == leader) wcnt[wave * experts + le] = __popcll(same);
        pending &= ~same;
    }
    __syncthreads();
    if(valid) {
        int32_t base = ws[(size_t)blockIdx.x * experts + e];
        for(int w = 0; w < wave; ++w) base += wcnt[w * experts + e];
        const int32_t slot = base + rank;
        sorted_ids[slot]   = (int32_t)(p / topk);
        dst_row[p]         = slot;
    } else if(p < total) {
        dst_row[p] = -1;
    }
}

// ---------------------------------------------------------------------------
// SiLU(gate) * up -> int8 rows for the down GEMM.  Row r of gate_up (fp16,
// gate in columns [0, inter), up in [inter, 2*inter)) gives
//   a[j] = (g / (1 + exp(-g))) * u  [* s2[e, j]]
// and the same absmax quantization as the SmoothQuant kernel.  Rows outside
// every expert's [start, start + count) (the sort's padding) are skipped.
// The row stays in registers (CPL 16-byte chunks per lane, WPR waves a row).
// ---------------------------------------------------------------------------
constexpr int kSqThreads = 256;
constexpr int kSqWaves   = kSqThreads / kWave;

struct SiluRows {
    const uint16_t* gu;
    uint32_t        ld_gu;
    const float*    s2; // [experts, inter] or null
    const int32_t*  expert_start;
    const int32_t*  expert_count;
    uint32_t        experts, rows, inter;
    int8_t*         q;
    uint32_t        ldq;
    float*          r;
    float           qmax;
    uint32_t        gu_bytes, q_bytes, s2_bytes; // buffer extents of the vector kernel
};

// Expert holding sorted row `row`, or -1 for padding / out-of-range rows
// (P: any argument block with expert_start, expert_count, experts).
template <class P>
__device__ __forceinline__ int row_expert(const P& p, uint32_t row)
{
    int lo = 0, hi = (int)p.experts - 1, e = -1;
    while(lo <= hi) { // last expert with start <= row
        const int mid = (lo + hi) / 2;
        if(p.expert_start[mid] <= (int32_t)row) {
            e  = mid;
            lo = mid + 1;
        } else {
            hi = mid - 1;
        }
    }
    if(e < 0 || (int64_t)row >= (int64_t)p.expert_start[e] + p.expert_count[e]) return -1;
    return e;
}

// Generic form (any inter, alignment and size): element loads and stores.
template <int CPL, int WPR>
__global__ void __launch_bounds__(kSqThreads) silu_quant_kernel(SiluRows p)
{
    constexpr int kRowsPerBlock = kSqWaves / WPR;
    constexpr int kSpan         = CPL * 8 * kWave;
    const int      wave = threadIdx.x / kWave;
    const int      lane = threadIdx.x % kWave;
    const int      rib  = wave / WPR;
    const int      part = wave % WPR;
    const uint32_t row  = blockIdx.x * kRowsPerBlock + rib;
    const int      e    = row < p.rows ? row_expert(p, row) : -1;
    const bool     valid = e >= 0;

    const uint16_t* g  = p.gu + (size_t)row * p.ld_gu;
    const uint16_t* u  = g + p.inter;
    const float*    s2 = p.s2 ? p.s2 + (size_t)e * p.inter : nullptr;
    const uint32_t  n  = p.inter;
    const uint32_t  base = part * kSpan + lane * 8;
    float           pv[CPL * 8];
    float           amax = 0.f;
    if(valid) {
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const uint32_t c = base + j * (8 * kWave);
#pragma unroll
            for(int x = 0; x < 8; ++x) {
                float a = 0.f;
                if(c + x < n) {
                    a = silu_mul(half_bits_to_float(g[c + x]), half_bits_to_float(u[c + x]));
                    if(s2) a *= s2[c + x];
                }
                pv[j * 8 + x] = a;
                amax          = fmaxf(amax, fabsf(a));
            }
        }
    }
    amax = wave_max(amax);
    if constexpr(WPR > 1) {
        __shared__ float red[kSqWaves];
        if(lane == 0) red[wave] = amax;
        __syncthreads();
#pragma unroll
        for(int w = 0; w < WPR; ++w) amax = fmaxf(amax, red[rib * WPR + w]);
    }
    if(!valid) return;
    const float qmax = p.qmax;
    const float rs   = amax / qmax;
    if(part == 0 && lane == 0) p.r[row] = rs;
    const float inv  = rs > 0.f ? 1.f / rs : 0.f;
    int8_t*     qrow = p.q + (size_t)row * p.ldq;
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t c = base + j * (8 * kWave);
#pragma unroll
        for(int x = 0; x < 8; ++x)
            if(c + x < n) qrow[c + x] = (int8_t)quant_i8(pv[j * 8 + x], inv, qmax);
    }
}

// Vector form (inter % 8 == 0, 16-byte aligned rows, every operand under
// 2 GiB): no per-lane branch anywhere.  All of a row's gate and up chunks go
// out at once as raw buffer loads (a chunk past the row or a row past `rows`
// gets offset kOob and reads zeros, which leave the absmax alone), the
// expert lookup runs while they are in flight, and the int8 chunks go out as
// buffer stores that kOob drops (padding rows and columns past inter).
template <int CPL, int WPR, bool S2>
__global__ void __launch_bounds__(kSqThreads) silu_quant_vec_kernel(SiluRows p)
{
    constexpr int      kRowsPerBlock = kSqWaves / WPR;
    constexpr int      kSpan         = CPL * 8 * kWave;
    constexpr uint32_t kOob          = gemm::kOob;
    const int          wave = threadIdx.x / kWave;
    const int          lane = threadIdx.x % kWave;
    const int          rib  = wave / WPR;
    const int          part = wave % WPR;
    const uint32_t     row  = blockIdx.x * kRowsPerBlock + rib;
    const uint32_t     n    = p.inter;
    const bool         in_rows = row < p.rows;

    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.gu), 0, (int)p.gu_bytes, gemm::kBufferFlags);
    uint32_t col[CPL]; // column of each 8-element chunk, or kOob
    v4i      gr[CPL], ur[CPL];
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t c  = part * kSpan + j * (8 * kWave) + lane * 8;
        col[j]            = (in_rows && c < n) ? c : kOob;
        const uint32_t vo = col[j] != kOob ? (row * p.ld_gu + c) * 2 : kOob;
        gr[j]             = __builtin_amdgcn_raw_buffer_load_b128(rg, vo, 0, 0);
        ur[j]             = __builtin_amdgcn_raw_buffer_load_b128(rg, vo, n * 2, 0);
    }
    const int  e     = in_rows ? row_expert(p, row) : -1;
    const bool valid = e >= 0;

    float pv[CPL * 8];
    float amax = 0.f;
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t gw[4] = {(uint32_t)gr[j].x, (uint32_t)gr[j].y, (uint32_t)gr[j].z,
                                (uint32_t)gr[j].w};
        const uint32_t uw[4] = {(uint32_t)ur[j].x, (uint32_t)ur[j].y, (uint32_t)ur[j].z,
                                (uint32_t)ur[j].w};
#pragma unroll
        for(int h = 0; h < 4; ++h) {
            pv[j * 8 + 2 * h]     = silu_mul(half_bits_to_float(gw[h] & 0xFFFFu),
                                             half_bits_to_float(uw[h] & 0xFFFFu));
            pv[j * 8 + 2 * h + 1] = silu_mul(half_bits_to_float(gw[h] >> 16),
                                             half_bits_to_float(uw[h] >> 16));
        }
        if constexpr(S2) {
            // s2[e, col]; a padding row (no expert) reads zeros
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(p.s2), 0, (int)p.s2_bytes, gemm::kBufferFlags);
            const uint32_t so = (valid && col[j] != kOob) ? (uint32_t)e * n * 4 + col[j] * 4 : kOob;
            const v4i      s0 = __builtin_amdgcn_raw_buffer_load_b128(rs, so, 0, 0);
            const v4i      s1 = __builtin_amdgcn_raw_buffer_load_b128(rs, so, 16, 0);
            const int      sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for(int x = 0; x < 8; ++x) pv[j * 8 + x] *= __int_as_float(sv[x]);
        }
#pragma unroll
        for(int x = 0; x < 8; ++x) amax = fmaxf(amax, fabsf(pv[j * 8 + x]));
    }
    amax = wave_max(amax);
    if constexpr(WPR > 1) {
        __shared__ float red[kSqWaves];
        if(lane == 0) red[wave] = amax;
        __syncthreads();
#pragma unroll
        for(int w = 0; w < WPR; ++w) amax = fmaxf(amax, red[rib * WPR + w]);
    }
    const float qmax = p.qmax;
    const float rs   = amax / qmax;
    if(valid && part == 0 && lane == 0) p.r[row] = rs;
    const float inv = rs > 0.f ? 1.f / rs : 0.f;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(p.q, 0, (int)p.q_bytes,
                                                                        gemm::kBufferFlags);
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const float* v = pv + j * 8;
        v2i          pk;
        pk.x = (int)cvt_pack4_i8(quant_f(v[0], inv, qmax), quant_f(v[1], inv, qmax),
                                 quant_f(v[2], inv, qmax), quant_f(v[3], inv, qmax));
        pk.y = (int)cvt_pack4_i8(quant_f(v[4], inv, qmax), quant_f(v[5], inv, qmax),
                                 quant_f(v[6], inv, qmax), quant_f(v[7], inv, qmax));
        __builtin_amdgcn_raw_buffer_store_b64(
            pk, rq, (valid && col[j] != kOob) ? row * p.ldq + col[j] : kOob, 0, 0);
    }
}

// ---------------------------------------------------------------------------
// Requantization after the gate_up GEMM's SiLU epilogue (epilogue_silu,
// gemm_i8_grouped_kernel.hpp): row r of the fp16 activation h comes with the
// per-wave maxima pmax[0..groups, r] of |float(h) * s2|, so the row scale is
// known before the row is read and each lane quantizes its chunks as they
// arrive: q = quantizer(float(h) * s2) with r = max / qmax (the SmoothQuant
// order, rocwmma_smoothquant.cpp:99-113).  Rows outside every expert's
// [start, start + count) are skipped.  inter % 8 == 0, 16-byte aligned rows.
// ---------------------------------------------------------------------------
struct SiluRequant {
    const uint16_t* h;
    uint32_t        ldh;
    const float*    pmax; // [groups, ldp] group-major
    uint32_t        ldp, groups;
    const float*    s2;   // [experts, inter] or null
    const int32_t*  expert_start;
    const int32_t*  expert_count;
    uint32_t        experts, rows, inter;
    int8_t*         q;
    uint32_t        ldq;
    float*          r;
    float           qmax;
    uint32_t        h_bytes, p_bytes, q_bytes, s2_bytes; // buffer extents (< 2 GiB)
};

// A block of kSqThreads threads takes kRqRows consecutive rows.  Phase 1:
// the rows' maxima over all groups (thread t reads row t % kRqRows of groups
// t / kRqRows, + kRqSlots, ...: kRqRows consecutive floats per group, one
// segment per wave instruction), reduced through LDS, and the rows' experts.
// Phase 2: each wave quantizes kRqRows / kSqWaves rows, kRqBatch 8-column
// chunks per lane in flight (h and s2 loads issued before any store).
// 8 rows per block: cfg5's 8448 rows make 1056 blocks, 4.1 per CU; with 16
// rows (528 blocks, 2.06 per CU) the CUs holding a third block finished alone
// (cfg5 layer 1535-1547 -> 1526-1528 us, same box, alternating).
constexpr int kRqRows  = 8;
constexpr int kRqSlots = kSqThreads / kRqRows;
constexpr int kRqBatch = 7;

template <bool S2>
__global__ void __launch_bounds__(kSqThreads) silu_requant_kernel(SiluRequant p)
{
    constexpr uint32_t kOob = gemm::kOob;
    __shared__ float   red[kRqSlots][kRqRows];
    __shared__ float   rowmax[kRqRows];
    __shared__ int     rowexp[kRqRows];
    const int          t    = threadIdx.x;
    const int          wave = t / kWave;
    const int          lane = t % kWave;
    const uint32_t     r0   = blockIdx.x * kRqRows;

    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.pmax), 0, (int)p.p_bytes, gemm::kBufferFlags);
    {
        const uint32_t row = r0 + t % kRqRows;
        float          mx  = 0.f;
        for(uint32_t g = t / kRqRows; g < p.groups; g += kRqSlots) {
            const uint32_t o = row < p.rows ? (g * p.ldp + row) * 4 : kOob;
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, o, 0, 0)));
        }
        red[t / kRqRows][t % kRqRows] = mx;
        if(t < kRqRows) rowexp[t] = r0 + t < p.rows ? row_expert(p, r0 + t) : -1;
    }
    __syncthreads();
    if(t < kRqRows) {
        float mx = 0.f;
#pragma unroll
        for(int sl = 0; sl < kRqSlots; ++sl) mx = fmaxf(mx, red[sl][t]);
        rowmax[t] = mx;
    }
    __syncthreads();

    const uint32_t n = p.inter;
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.h), 0, (int)p.h_bytes, gemm::kBufferFlags);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.s2), 0, (int)p.s2_bytes, gemm::kBufferFlags);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(p.q, 0, (int)p.q_bytes,
                                                                        gemm::kBufferFlags);
    const float qmax = p.qmax;
    for(int rr = wave; rr < kRqRows; rr += kSqWaves) {
        const uint32_t row   = r0 + rr;
        const int      e     = rowexp[rr];
        if(e < 0) continue; // wave-uniform: padding rows and rows past the end
        const float    rsc   = rowmax[rr] / qmax;
        const float    inv   = rsc > 0.f ? 1.f / rsc : 0.f;
        if(lane == 0) p.r[row] = rsc;
        for(uint32_t c0 = 0; c0 < n; c0 += kRqBatch * 8 * kWave) {
            v4i      hv[kRqBatch], s0[kRqBatch], s1[kRqBatch];
            uint32_t col[kRqBatch];
#pragma unroll
            for(int j = 0; j < kRqBatch; ++j) {
                const uint32_t c = c0 + (j * kWave + lane) * 8;
                col[j]           = c < n ? c : kOob;
                hv[j] = __builtin_amdgcn_raw_buffer_load_b128(
                    rh, col[j] != kOob ? (row * p.ldh + c) * 2 : kOob, 0, 0);
                if constexpr(S2) {
                    const uint32_t so = col[j] != kOob ? ((uint32_t)e * n + c) * 4 : kOob;
                    s0[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, so, 0, 0);
                    s1[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, so, 16, 0);
                }
            }
#pragma unroll
            for(int j = 0; j < kRqBatch; ++j) {
                const uint32_t hw[4] = {(uint32_t)hv[j].x, (uint32_t)hv[j].y, (uint32_t)hv[j].z,
                                        (uint32_t)hv[j].w};
                float          sv[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
                if constexpr(S2) {
                    const int w[8] = {s0[j].x, s0[j].y, s0[j].z, s0[j].w,
                                      s1[j].x, s1[j].y, s1[j].z, s1[j].w};
#pragma unroll
                    for(int x = 0; x < 8; ++x) sv[x] = __int_as_float(w[x]);
                }
                float v[8];
#pragma unroll
                for(int x = 0; x < 4; ++x) {
                    v[2 * x]     = half_bits_to_float(hw[x] & 0xFFFFu) * sv[2 * x];
                    v[2 * x + 1] = half_bits_to_float(hw[x] >> 16) * sv[2 * x + 1];
                }
                v2i pk;
                pk.x = (int)cvt_pack4_i8(quant_f(v[0], inv, qmax), quant_f(v[1], inv, qmax),
                                         quant_f(v[2], inv, qmax), quant_f(v[3], inv, qmax));
                pk.y = (int)cvt_pack4_i8(quant_f(v[4], inv, qmax), quant_f(v[5], inv, qmax),
                                         quant_f(v[6], inv, qmax), quant_f(v[7], inv, qmax));
                __builtin_amdgcn_raw_buffer_store_b64(
                    pk, rq, col[j] != kOob ? row * p.ldq + col[j] : kOob, 0, 0);
            }
        }
    }
}

hipError_t launch_requant(const SiluRequant& p, hipStream_t stream)
{
    const dim3 grid((p.rows + kRqRows - 1) / kRqRows);
    if(p.s2 != nullptr)
        hipLaunchKernelGGL(silu_requant_kernel<true>, grid, dim3(kSqThreads), 0, stream, p);
    else
        hipLaunchKernelGGL(silu_requant_kernel<false>, grid, dim3(kSqThreads), 0, stream, p);
    return hipGetLastError();
}

// Gate_up weights interleaved for the SiLU epilogue: output row r of expert
// e is input row (r / 32) * 16 + r % 32 for r % 32 < 16 (gate) and
// inter + (r / 32) * 16 + r % 32 - 16 otherwise (up); one block per output
// row (inter % 16 == 0, host-checked).
__global__ void __launch_bounds__(256)
    interleave_gate_up_kernel(const int8_t* __restrict__ w, const float* __restrict__ sw,
                              uint32_t inter, uint32_t k, uint32_t ldw, int8_t* __restrict__ wo,
                              float* __restrict__ swo, int vec)
{
    const uint32_t rows = 2 * inter;
    const uint32_t e = blockIdx.x / rows, r = blockIdx.x % rows;
    const uint32_t b = r / 32, x = r % 32;
    const uint32_t src = x < 16 ? b * 16 + x : inter + b * 16 + (x - 16);
    const int8_t*  in  = w + ((size_t)e * rows + src) * ldw;
    int8_t*        out = wo + ((size_t)e * rows + r) * k;
    if(vec) {
        for(uint32_t c = threadIdx.x * 16; c < k; c += 256 * 16)
            *reinterpret_cast<int4*>(out + c) = *reinterpret_cast<const int4*>(in + c);
    } else {
        for(uint32_t c = threadIdx.x; c < k; c += 256) out[c] = in[c];
    }
    if(threadIdx.x == 0 && sw != nullptr) swo[(size_t)e * rows + r] = sw[(size_t)e * rows + src];
}

template <int CPL, int WPR>
hipError_t launch_silu_rows(const SiluRows& p, bool vec, hipStream_t stream)
{
    constexpr int kRowsPerBlock = kSqWaves / WPR;
    const dim3    grid((p.rows + kRowsPerBlock - 1) / kRowsPerBlock);
    if(vec && p.s2 != nullptr)
        hipLaunchKernelGGL((silu_quant_vec_kernel<CPL, WPR, true>), grid, dim3(kSqThreads), 0,
                           stream, p);
    else if(vec)
        hipLaunchKernelGGL((silu_quant_vec_kernel<CPL, WPR, false>), grid, dim3(kSqThreads), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((silu_quant_kernel<CPL, WPR>), grid, dim3(kSqThreads), 0, stream, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weighted combine: out[t, n] = half(sum over slots, ascending, of
// fma(w[t, slot], float(y[dst_row[t*topk + slot], n]), acc)); pairs with
// dst_row < 0 are skipped.  8 columns per thread.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    moe_combine_kernel(const uint16_t* __restrict__ y, uint32_t ldy, const float* __restrict__ w,
                       const int32_t* __restrict__ dst_row, uint32_t tokens, uint32_t topk,
                       uint32_t n, uint32_t rows_y, uint16_t* __restrict__ out, uint32_t ldo,
                       int vec)
{
    const uint32_t groups = (n + 7) / 8;
    const size_t   idx    = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if(idx >= (size_t)tokens * groups) return;
    const uint32_t t  = idx / groups;
    const uint32_t c0 = (idx % groups) * 8;
    float          acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for(uint32_t s = 0; s < topk; ++s) {
        const int32_t r = dst_row[(size_t)t * topk + s];
        if(r < 0 || (uint32_t)r >= rows_y) continue;
        const float     ws  = w[(size_t)t * topk + s];
        const uint16_t* src = y + (size_t)r * ldy + c0;
        if(vec && c0 + 8 <= n) {
            const uint4    v    = *reinterpret_cast<const uint4*>(src);
            const uint32_t h[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for(int x = 0; x < 4; ++x) {
                acc[2 * x]     = __builtin_fmaf(ws, half_bits_to_float(h[x] & 0xFFFFu), acc[2 * x]);
                acc[2 * x + 1] = __builtin_fmaf(ws, half_bits_to_float(h[x] >> 16), acc[2 * x + 1]);
            }
        } else {
            for(int x = 0; x < 8; ++x)
                if(c0 + x < n) acc[x] = __builtin_fmaf(ws, half_bits_to_float(src[x]), acc[x]);
        }
    }
    uint16_t* dst = out + (size_t)t * ldo + c0;
    if(vec && c0 + 8 <= n) {
        // two roundings (the fp32 sum, then fp16): the last fma must not fold
        // into a mixed-precision fma that rounds to fp16 once
        auto pk = [&](int x) { return float2_to_half2_bits_2step(acc[x], acc[x + 1]); };
        *reinterpret_cast<uint4*>(dst) = make_uint4(pk(0), pk(2), pk(4), pk(6));
    } else {
        for(int x = 0; x < 8; ++x)
            if(c0 + x < n) dst[x] = float_to_half_bits_2step(acc[x]);
    }
}

using GemmGrouped = gemm::Cfg<256, 256, 128, 2, 2, 4, 4, 16>;
// GemmGrouped's wide partner: an expert's rest of at most 128 rows runs as
// 128 x 512 tiles (8 waves of 128 x 64, as GemmGrouped; 2 stages of 80 KiB).
using GemmGroupedWide = gemm::Cfg<128, 512, 128, 2, 1, 8, 4, 16>;
// MoE GEMM over experts of a few hundred rows: 128-row tiles waste less of
// each expert's last tile row (moe_tile_rows_128).
using GemmGroupedMid = gemm::Cfg<128, 256, 128, 3, 2, 4, 4, 16>;

// 128-row tiles when the fraction of tile rows an expert of average size
// fills, times their per-op rate relative to 256-row tiles (about 0.8,
// measured on the fused-MoE CLI shapes), beats that of 256-row tiles: ~340
// rows per expert (64 experts, top-6 of 3328 tokens) 1004 -> 1057 TOPS;
// ~550 rows (32 experts, top-5) stay on 256 rows (1516 vs 1400 TOPS).
bool moe_tile_rows_128(uint32_t rows, uint32_t experts)
{
    const double avg  = (double)rows / experts;
    const double u256 = avg / (std::ceil(avg / 256.0) * 256.0);
    const double u128 = avg / (std::ceil(avg / 128.0) * 128.0);
    return u128 * 0.8 > u256;
}

} // namespace

static_assert(sizeof(gemm::KArgs) == sizeof(w8a8_group_desc)
                  && offsetof(gemm::KArgs, m) == offsetof(w8a8_group_desc, m)
                  && offsetof(gemm::KArgs, tsb) == offsetof(w8a8_group_desc, tensor_scale_b),
              "w8a8_group_desc must have the device descriptor's layout");

hipError_t launch_topk_softmax(const void* logits, bool f16, float* w, int32_t* ids,
                               uint32_t tokens, uint32_t experts, uint32_t topk,
                               hipStream_t stream)
{
    const dim3 grid((tokens + kTopkWaves - 1) / kTopkWaves);
    if(f16)
        hipLaunchKernelGGL(topk_softmax_kernel<true>, grid, dim3(kTopkWaves * kWave), 0, stream,
                           logits, w, ids, tokens, experts, topk);
    else
        hipLaunchKernelGGL(topk_softmax_kernel<false>, grid, dim3(kTopkWaves * kWave), 0, stream,
                           logits, w, ids, tokens, experts, topk);
    return hipGetLastError();
}

size_t moe_sort_lds_bytes(uint32_t experts)
{
    return sizeof(int32_t) * ((size_t)experts * (3 + kSortWaves) + 1);
}

size_t moe_sort_workspace_bytes(uint32_t tokens, uint32_t topk, uint32_t experts)
{
    const uint64_t total = (uint64_t)tokens * topk;
    if(total <= kSortChunk) return 0; // one block: the single-workgroup kernel
    return (size_t)((total + kSortChunk - 1) / kSortChunk) * experts * sizeof(int32_t);
}

hipError_t launch_moe_sort(const int32_t* ids, uint32_t tokens, uint32_t topk, uint32_t experts,
                           uint32_t unit, int32_t* count, int32_t* start, int32_t* padded,
                           int32_t* sorted_ids, uint32_t sorted_cap, int32_t* dst_row, void* ws,
                           size_t ws_bytes, hipStream_t stream)
{
    const uint32_t total = tokens * topk;
    const size_t   need  = moe_sort_workspace_bytes(tokens, topk, experts);
    if(ws != nullptr && need > 0 && ws_bytes >= need) {
        const uint32_t blocks = (total + kSortChunk - 1) / kSortChunk;
        int32_t*       w      = static_cast<int32_t*>(ws);
        hipLaunchKernelGGL(moe_sort_count_kernel, dim3(blocks), dim3(kSortThreads),
                           experts * sizeof(int32_t), stream, ids, total, experts, w, sorted_ids,
                           sorted_cap);
        hipLaunchKernelGGL(moe_sort_offsets_kernel, dim3(1), dim3(kSortThreads),
                           2 * experts * sizeof(int32_t), stream, blocks, experts, unit, w, count,
                           start, padded);
        hipLaunchKernelGGL(moe_sort_scatter_kernel, dim3(blocks), dim3(kSortThreads),
                           (size_t)experts * kSortWaves * sizeof(int32_t), stream, ids, total, topk,
                           experts, w, sorted_ids, dst_row);
        return hipGetLastError();
    }
    const size_t lds = moe_sort_lds_bytes(experts);
    if(lds > 65536) {
        static std::once_flag once;
        std::call_once(once, [] {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(moe_sort_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            (void)hipGetLastError();
        });
    }
    hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(kSortThreads), lds, stream, ids,
                       tokens * topk, topk, experts, unit, count, start, padded, sorted_ids,
                       sorted_cap, dst_row);
    return hipGetLastError();
}

hipError_t launch_silu_mul_quant(const uint16_t* gu, uint32_t ld_gu, const float* s2,
                                 const int32_t* expert_start, const int32_t* expert_count,
                                 uint32_t experts, uint32_t rows, uint32_t inter, int8_t* q,
                                 uint32_t ldq, float* r, float qmax, hipStream_t stream)
{
    if(rows == 0) return hipSuccess;
    const uint64_t gu_bytes = ((uint64_t)(rows - 1) * ld_gu + 2ull * inter) * 2;
    const uint64_t q_bytes  = (uint64_t)(rows - 1) * ldq + inter;
    const uint64_t s2_bytes = (uint64_t)experts * inter * 4;
    SiluRows p{gu, ld_gu, s2, expert_start, expert_count, experts, rows, inter, q, ldq, r, qmax,
               (uint32_t)std::min<uint64_t>(gu_bytes, 0xFFFFFFFFull),
               (uint32_t)std::min<uint64_t>(q_bytes, 0xFFFFFFFFull),
               (uint32_t)std::min<uint64_t>(s2_bytes, 0xFFFFFFFFull)};
    constexpr uint64_t kBufLimit = 0x7FFFFFFFull; // offsets stay below kOob
    const bool vec = reinterpret_cast<uintptr_t>(gu) % 16 == 0 && ld_gu % 8 == 0
                     && inter % 8 == 0 && (s2 == nullptr || reinterpret_cast<uintptr_t>(s2) % 16 == 0)
                     && reinterpret_cast<uintptr_t>(q) % 8 == 0 && ldq % 8 == 0
                     && gu_bytes <= kBufLimit && q_bytes <= kBufLimit && s2_bytes <= kBufLimit;
    const uint32_t n = inter;
    if(n <= 512) return launch_silu_rows<1, 1>(p, vec, stream);
    if(n <= 1024) return launch_silu_rows<2, 1>(p, vec, stream);
    if(n <= 2048) return launch_silu_rows<4, 1>(p, vec, stream);
    if(n <= 4096) return launch_silu_rows<8, 1>(p, vec, stream);
    if(n <= 8192) return launch_silu_rows<16, 1>(p, vec, stream);
    if(n <= 16384) return launch_silu_rows<16, 2>(p, vec, stream);
    return launch_silu_rows<16, 4>(p, vec, stream); // inter <= 32768 (host-checked)
}

hipError_t launch_moe_interleave_gate_up(const int8_t* w, const float* sw, uint32_t experts,
                                         uint32_t inter, uint32_t k, uint32_t ldw, int8_t* wo,
                                         float* swo, hipStream_t stream)
{
    const uint64_t blocks = (uint64_t)experts * 2 * inter;
    if(blocks == 0 || k == 0) return hipSuccess;
    if(blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    const int vec = reinterpret_cast<uintptr_t>(w) % 16 == 0 && ldw % 16 == 0
                    && reinterpret_cast<uintptr_t>(wo) % 16 == 0 && k % 16 == 0;
    hipLaunchKernelGGL(interleave_gate_up_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, w,
                       sw, inter, k, ldw, wo, swo, vec);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const uint16_t* y, uint32_t ldy, uint32_t rows_y, const float* w,
                              const int32_t* dst_row, uint32_t tokens, uint32_t topk, uint32_t n,
                              uint16_t* out, uint32_t ldo, hipStream_t stream)
{
    const size_t threads = (size_t)tokens * ((n + 7) / 8);
    if(threads == 0) return hipSuccess;
    const int vec = reinterpret_cast<uintptr_t>(y) % 16 == 0 && ldy % 8 == 0
                    && reinterpret_cast<uintptr_t>(out) % 16 == 0 && ldo % 8 == 0;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0,
                       stream, y, ldy, w, dst_row, tokens, topk, n, rows_y, out, ldo, vec);
    return hipGetLastError();
}

using GemmGroupedSmall = gemm::Cfg<128, 128, 128, 3, 2, 4, 4, 16>;

namespace {
uint32_t device_cus()
{
    static const uint32_t cus = [] {
        int dev = 0, c = 256;
        if(hipGetDevice(&dev) == hipSuccess)
            (void)hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
        return (uint32_t)c;
    }();
    return cus;
}
} // namespace

hipError_t launch_grouped_gemm(const w8a8_group_desc* groups_dev, uint32_t ngroups,
                               uint32_t total_tiles, int cfg, int out_type, int vec_ok,
                               hipStream_t stream)
{
    const auto* g = reinterpret_cast<const gemm::KArgs*>(groups_dev);
    if(cfg == 1)
        return gemm::launch_grouped<GemmGroupedMid>(g, ngroups, total_tiles, out_type, vec_ok,
                                                    stream);
    if(cfg == 2)
        return gemm::launch_grouped<GemmGroupedSmall>(g, ngroups, total_tiles, out_type, vec_ok,
                                                      stream);
    return gemm::launch_grouped<GemmGrouped>(g, ngroups, total_tiles, out_type, vec_ok, stream);
}

uint32_t grouped_gemm_tiles(uint32_t m, uint32_t n, int cfg)
{
    const uint32_t bm = cfg == 0 ? 256 : 128, bn = cfg == 2 ? 128 : 256;
    return ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
}

int grouped_gemm_cfg(const uint64_t tiles[3])
{
    const uint64_t enough = (uint64_t)device_cus() * 3 / 4;
    if(tiles[0] >= enough) return 0;
    if(tiles[1] >= enough) return 1;
    return 2;
}


size_t moe_gemm_workspace_bytes()
{
    return std::max(gemm::moe_workspace_bytes<GemmGrouped>(device_cus()),
                    gemm::moe_workspace_bytes<GemmGroupedMid>(device_cus()));
}

hipError_t launch_moe_gemm(const MoeGemmArgs& a, hipStream_t stream)
{
    gemm::MoeArgs q;
    q.a            = a.a;
    q.w            = a.w;
    q.c            = a.c;
    q.sa           = a.scale_a;
    q.sw           = a.scale_w;
    q.expert_start = a.expert_start;
    q.expert_count = a.expert_count;
    q.rows         = a.rows;
    q.experts      = a.experts;
    q.n            = a.n;
    q.k            = a.k;
    q.lda          = a.lda;
    q.ldw          = a.ldw;
    q.ldc          = a.ldc;
    q.w_stride     = a.w_stride;
    q.tsa          = a.tsa;
    q.tsb          = a.tsb;
    const bool split = a.ws != nullptr && a.ws_bytes >= moe_gemm_workspace_bytes();
    q.ws           = split ? static_cast<int32_t*>(a.ws) : nullptr;
    q.cus          = split ? device_cus() : 0;
    const size_t esz    = a.out_type == W8A8_OUT_I32 ? 4 : 2;
    const int    vec_ok = reinterpret_cast<uintptr_t>(a.c) % (4 * esz) == 0 && a.ldc % 4 == 0
                       && (a.scale_w == nullptr
                           || (reinterpret_cast<uintptr_t>(a.scale_w) % 16 == 0 && a.n % 4 == 0));
    // rows (the sort's padded capacity) / experts stands for the rows per expert
    if(moe_tile_rows_128(a.rows, a.experts))
        return gemm::launch_moe<GemmGroupedMid>(q, a.out_type, vec_ok, stream);
    return gemm::launch_moe<GemmGrouped, GemmGroupedWide>(q, a.out_type, vec_ok, stream);
}

// The SiLU epilogue's tiles: wave tiles 128 columns wide (64 outputs, one
// 128-byte line of h per row and wave), otherwise as GemmGrouped /
// GemmGroupedMid (16 x 16 x 64 MFMA, whose lane layout the 32-row gate/up
// interleave matches).
using GemmSilu     = gemm::Cfg<256, 256, 128, 2, 4, 2, 4, 16>;
using GemmSiluMid  = gemm::Cfg<128, 256, 128, 3, 4, 2, 4, 16>;
using GemmSiluWide = gemm::Cfg<128, 512, 128, 2, 2, 4, 4, 16>; // GemmSilu's wide partner
static_assert(GemmSilu::kWaveN == GemmSiluMid::kWaveN, "one pmax layout for both tiles");
static_assert(gemm::Partial<GemmSilu>::kBytes == gemm::Partial<GemmGrouped>::kBytes
                  && gemm::Partial<GemmSiluMid>::kBytes == gemm::Partial<GemmGroupedMid>::kBytes,
              "the SiLU tiles' partials fit moe_gemm_workspace_bytes");
constexpr uint32_t kSiluGroupCols = GemmSilu::kWaveN; // interleaved columns per pmax entry

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

size_t moe_gate_up_silu_workspace_bytes(uint32_t rows, uint32_t inter)
{
    const size_t groups = (2ull * inter + kSiluGroupCols - 1) / kSiluGroupCols;
    return align256((size_t)rows * inter * 2) + align256((size_t)rows * groups * 4)
           + moe_gemm_workspace_bytes();
}

hipError_t launch_moe_gate_up_silu(const MoeSiluArgs& a, hipStream_t stream)
{
    if(a.rows == 0) return hipSuccess;
    const uint32_t groups = (2 * a.inter + kSiluGroupCols - 1) / kSiluGroupCols;
    int8_t*        ws     = static_cast<int8_t*>(a.ws);
    uint16_t*      h      = reinterpret_cast<uint16_t*>(ws);
    float*         pmax   = reinterpret_cast<float*>(ws + align256((size_t)a.rows * a.inter * 2));
    int32_t*       part   = reinterpret_cast<int32_t*>(
        ws + align256((size_t)a.rows * a.inter * 2) + align256((size_t)a.rows * groups * 4));

    gemm::MoeArgs q;
    q.a            = a.a;
    q.w            = a.w;
    q.c            = nullptr; // the SiLU epilogue writes h and pmax instead
    q.sa           = a.scale_a;
    q.sw           = a.scale_w;
    q.expert_start = a.expert_start;
    q.expert_count = a.expert_count;
    q.rows         = a.rows;
    q.experts      = a.experts;
    q.n            = 2 * a.inter;
    q.k            = a.k;
    q.lda          = a.lda;
    q.ldw          = a.k;
    q.ldc          = 0;
    q.w_stride     = 2ull * a.inter * a.k;
    q.tsa          = a.tsa;
    q.tsb          = a.tsb;
    q.ws           = part;
    q.cus          = device_cus();
    // pmax group-major: row stride ldp = rows
    const gemm::SiluOut so{h, pmax, a.s2, a.inter, a.rows, a.inter};
    const int vec_ok = a.scale_w == nullptr || reinterpret_cast<uintptr_t>(a.scale_w) % 16 == 0;
    hipError_t e = moe_tile_rows_128(a.rows, a.experts)
                       ? gemm::launch_moe_silu<GemmSiluMid>(q, so, vec_ok, stream)
                       : gemm::launch_moe_silu<GemmSilu, GemmSiluWide>(q, so, vec_ok, stream);
    if(e != hipSuccess) return e;

    const uint64_t h_bytes  = (uint64_t)a.rows * a.inter * 2;
    const uint64_t p_bytes  = (uint64_t)a.rows * groups * 4;
    const uint64_t q_bytes  = (uint64_t)(a.rows - 1) * a.ldq + a.inter;
    const uint64_t s2_bytes = (uint64_t)a.experts * a.inter * 4;
    const SiluRequant r{h, a.inter, pmax, a.rows, groups, a.s2, a.expert_start, a.expert_count,
                        a.experts, a.rows, a.inter, a.q, a.ldq, a.r, a.qmax, (uint32_t)h_bytes,
                        (uint32_t)p_bytes, (uint32_t)q_bytes, (uint32_t)s2_bytes};
    return launch_requant(r, stream);
}

} // namespace w8a8
