// rmsnorm_sq.hip -- RMSNorm (with optional residual add) fused with the
// row-wise SmoothQuant quantizer, for gfx950.
//
// Computation per row (kernel_add_rmsnorm2d_fwd / kernel_rmsnorm2d_fwd,
// rocwmma_rmsnorm2d.cpp:57-120, 127-186, then kernel_smoothquant,
// rocwmma_smoothquant.cpp:58-122, on the fp16 result):
//   v[n]  = float(x[n]) (+ float(res[n]))          x_out[n] = half(v[n])
//   rstd  = rsqrt(sum_n v[n]^2 / N + eps)
//   u[n]  = residual ? float(x_out[n]) : v[n]
//   y[n]  = half((u[n] * rstd) * gamma[n])
//   p[n]  = float(y[n]) * s[n];  r = max|p| / qmax;  inv = r > 0 ? 1/r : 0
//   q[n]  = int8(clamp(rint(p[n] * inv), -qmax, qmax))
// y is rounded to fp16 before it is quantized, so q and r are exactly the
// quantizer's output for the y this kernel computes, as in the unfused
// two-kernel chain.  The normalised row never goes to HBM unless the caller
// asks for y.
//
// HBM traffic per row: x 2N (+ residual 2N) read, x_out 2N (if any), q N + 4
// and y 2N (if asked) written.  gamma and s are read once per block.
//
// rmsq_stream_kernel (aligned rows, N % 8 == 0, N <= 16384): the layout of
// sq_stream_kernel -- gamma and s staged once per block in LDS (permuted so a
// wave's ds_read_b128 reads 1 KiB contiguous), groups of WPR waves walk the
// rows with a grid stride and double-buffer x and residual in registers,
// every access a buffer instruction with an out-of-range offset for masked
// lanes (no branches, exact vmcnt waits).  Two reductions per row (sum of
// squares, then absmax) go through DPP within a wave and LDS across waves.
// rmsq_generic_kernel: any stride, alignment or length; one block per row.
#include "w8a8_device.hpp"
#include "w8a8_internal.hpp"

#include <algorithm>
#include <mutex>

// Every float operation below is the IEEE operation written (no multiply-add
// contraction), and every fp16 result is rounded to fp32 first
// (float_to_half_bits_2step), so all instantiations give the same bits.
#pragma clang fp contract(off)

namespace w8a8 {
namespace {

constexpr uint32_t kOob        = 0x80000000u; // past every buffer: loads 0, stores dropped
constexpr int      kBufferFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, p ? (int)bytes : 0,
                                             kBufferFlags);
}

__device__ __forceinline__ uint32_t pack_half2(float a, float b)
{
    return float2_to_half2_bits_2step(a, b);
}

template <int CPL, int WPR, int THREADS, int BPC, bool RES, bool YOUT, bool QUANT>
__global__ void __launch_bounds__(THREADS, THREADS / 256 * BPC) // waves per SIMD for BPC blocks/CU
rmsq_stream_kernel(NormRows p, uint32_t iters)
{
    constexpr int kWaves  = THREADS / kWave;
    constexpr int kGroups = kWaves / WPR;
    constexpr int kSpan   = CPL * 8 * kWave; // columns one wave covers
    constexpr int kTotal  = kSpan * WPR;     // columns one row group covers
    static_assert(kWaves % WPR == 0, "whole row groups per block");
    // gamma at [0, kTotal), s at [kTotal, 2 kTotal) (QUANT only)
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ float red[2][kWaves];

    const int      wave = threadIdx.x / kWave;
    const int      lane = threadIdx.x % kWave;
    const int      grp  = wave / WPR;
    const int      part = wave % WPR;
    const uint32_t n    = p.n;
    const uint32_t base = part * kSpan + lane * 8;

    const uint32_t xspan = (p.rows - 1) * p.ldx * 2 + n * 2;
    const __amdgpu_buffer_rsrc_t rx  = rsrc(p.x, xspan);
    const __amdgpu_buffer_rsrc_t rr  = rsrc(p.res, xspan);
    const __amdgpu_buffer_rsrc_t rxo = rsrc(p.x_out, xspan); // NULL: every store dropped
    const __amdgpu_buffer_rsrc_t ry  = rsrc(p.y, (p.rows - 1) * p.ldy * 2 + n * 2);
    const __amdgpu_buffer_rsrc_t rq  = rsrc(p.q, (p.rows - 1) * p.ldq + n);

    uint32_t coff[CPL]; // column of each 8-element chunk, or kOob past N
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t c = base + j * (8 * kWave);
        coff[j]          = c < n ? c : kOob;
    }

    using Row = v4i[CPL];
    Row  xa, xb, ra, rb;
    auto load_row = [&](Row& xd, Row& rd, uint32_t r) {
        const bool     ok   = r < p.rows;
        const uint32_t roff = r * p.ldx * 2;
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const uint32_t off = (ok && coff[j] != kOob) ? roff + coff[j] * 2 : kOob;
            xd[j]              = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
            if constexpr(RES) rd[j] = __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0);
        }
    };

    // LDS byte offset of this lane's gamma / s values (see the staging below);
    // made opaque per pass so the compiler re-reads LDS rather than pinning
    // CPL*8 registers per vector for the whole kernel
    uint32_t l_off = (part * kSpan + lane * 4) * 4;
    auto lds4 = [&](int j, int half, int which) {
        return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(lds) + l_off
                                                + which * kTotal * 4 + j * 2048 + half * 1024);
    };
    int  slot    = 0;
    auto reduce  = [&](float v, bool is_max) {
        v = is_max ? wave_max(v) : wave_sum(v);
        if constexpr(WPR > 1) {
            if(lane == 0) red[slot][wave] = v;
            __syncthreads();
            v = red[slot][grp * WPR];
#pragma unroll
            for(int w = 1; w < WPR; ++w)
                v = is_max ? fmaxf(v, red[slot][grp * WPR + w]) : v + red[slot][grp * WPR + w];
            slot ^= 1;
        }
        return v;
    };

    auto process = [&](Row& x, const Row& res, uint32_t r) {
        const bool     valid = r < p.rows;
        const uint32_t roff  = r * p.ldx * 2;
        // 1. v = x (+ res); x_out = half(v); sum of squares in fp32
        float ss = 0.f;
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const uint32_t w[4] = {(uint32_t)x[j].x, (uint32_t)x[j].y, (uint32_t)x[j].z,
                                   (uint32_t)x[j].w};
            float v[8];
#pragma unroll
            for(int e = 0; e < 8; ++e) v[e] = half_bits_to_float((w[e / 2] >> (16 * (e % 2))) & 0xFFFFu);
            if constexpr(RES) {
                const uint32_t q4[4] = {(uint32_t)res[j].x, (uint32_t)res[j].y,
                                        (uint32_t)res[j].z, (uint32_t)res[j].w};
#pragma unroll
                for(int e = 0; e < 8; ++e)
                    v[e] += half_bits_to_float((q4[e / 2] >> (16 * (e % 2))) & 0xFFFFu);
                x[j].x = (int)pack_half2(v[0], v[1]);
                x[j].y = (int)pack_half2(v[2], v[3]);
                x[j].z = (int)pack_half2(v[4], v[5]);
                x[j].w = (int)pack_half2(v[6], v[7]);
                __builtin_amdgcn_raw_buffer_store_b128(
                    x[j], rxo, (valid && coff[j] != kOob) ? roff + coff[j] * 2 : kOob, 0, 0);
            }
#pragma unroll
            for(int e = 0; e < 8; ++e) ss += v[e] * v[e];
        }
        ss                = reduce(ss, false);
        const float rstd  = rsqrtf(ss / (float)n + p.eps);

        // 2. y = half((u * rstd) * gamma) as packed fp16 pairs (u * rstd in
        //    one v_fma_mix_f32 from the packed fp16 u); optional y store;
        //    p = y * s (again one v_fma_mix_f32 from the packed y) kept in
        //    registers for the quantize pass, and its absmax
        asm volatile("" : "+v"(l_off));
        float amax = 0.f;
        float pv[QUANT ? CPL * 8 : 1];
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const float4   g0   = lds4(j, 0, 0);
            const float4   g1   = lds4(j, 1, 0);
            const float    g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            const uint32_t w[4] = {(uint32_t)x[j].x, (uint32_t)x[j].y, (uint32_t)x[j].z,
                                   (uint32_t)x[j].w};
            uint32_t       yh[4];
#pragma unroll
            for(int e = 0; e < 4; ++e)
                yh[e] = pack_half2(mul_h16_f32<false>(w[e], rstd) * g[2 * e],
                                   mul_h16_f32<true>(w[e], rstd) * g[2 * e + 1]);
            if constexpr(YOUT)
                __builtin_amdgcn_raw_buffer_store_b128(
                    v4i{(int)yh[0], (int)yh[1], (int)yh[2], (int)yh[3]}, ry,
                    (valid && coff[j] != kOob) ? r * p.ldy * 2 + coff[j] * 2 : kOob, 0, 0);
            if constexpr(QUANT) {
                const float4 s0   = lds4(j, 0, 1);
                const float4 s1   = lds4(j, 1, 1);
                const float  s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for(int e = 0; e < 8; e += 2) {
                    pv[j * 8 + e]     = mul_h16_f32<false>(yh[e / 2], s[e]);
                    pv[j * 8 + e + 1] = mul_h16_f32<true>(yh[e / 2], s[e + 1]);
                    amax = fmaxf(fmaxf(amax, fabsf(pv[j * 8 + e])), fabsf(pv[j * 8 + e + 1]));
                }
            }
        }
        if constexpr(QUANT) {
            amax              = reduce(amax, true);
            const float qmax  = p.qmax;
            const float rs    = amax / qmax;
            if(valid && part == 0 && lane == 0) p.r[r] = rs;
            const float inv   = rs > 0.f ? 1.f / rs : 0.f;
            // 3. quantize the kept products
#pragma unroll
            for(int j = 0; j < CPL; ++j) {
                const float* v = pv + j * 8;
                v2i          pk;
                pk.x = (int)cvt_pack4_i8(quant_f(v[0], inv, qmax), quant_f(v[1], inv, qmax),
                                         quant_f(v[2], inv, qmax), quant_f(v[3], inv, qmax));
                pk.y = (int)cvt_pack4_i8(quant_f(v[4], inv, qmax), quant_f(v[5], inv, qmax),
                                         quant_f(v[6], inv, qmax), quant_f(v[7], inv, qmax));
                __builtin_amdgcn_raw_buffer_store_b64(
                    pk, rq, (valid && coff[j] != kOob) ? r * p.ldq + coff[j] : kOob, 0, 0);
            }
        }
    };

    const uint32_t stride = gridDim.x * kGroups;
    uint32_t       row    = blockIdx.x * kGroups + grp;

    // First row's loads before the staging, so the two fetches overlap.
    // gamma and s land in LDS permuted: column c = part*kSpan + j*512 + l*8 + e
    // sits at part*kSpan + j*512 + (e/4)*256 + l*4 + e%4; past N they are 0.
    load_row(xa, ra, row);
    {
        constexpr int kS4 = (kTotal + THREADS * 4 - 1) / (THREADS * 4);
        const __amdgpu_buffer_rsrc_t rg = rsrc(p.gamma, n * 4);
        const __amdgpu_buffer_rsrc_t rs = rsrc(p.s, n * 4); // NULL without QUANT
        v4i gv[kS4], sv[kS4];
#pragma unroll
        for(int i = 0; i < kS4; ++i) {
            const uint32_t c4  = (i * THREADS + threadIdx.x) * 4;
            const uint32_t off = c4 < n ? c4 * 4 : kOob;
            gv[i]              = __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0);
            if constexpr(QUANT) sv[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        }
#pragma unroll
        for(int i = 0; i < kS4; ++i) {
            const uint32_t c4 = (i * THREADS + threadIdx.x) * 4;
            if(c4 < (uint32_t)kTotal) {
                const uint32_t c  = c4 & ~7u;
                const uint32_t at = (c / 512) * 512 + ((c4 & 4u) ? 256u : 0u) + ((c % 512) / 8) * 4;
                *reinterpret_cast<v4i*>(lds + at) = gv[i];
                if constexpr(QUANT) *reinterpret_cast<v4i*>(lds + kTotal + at) = sv[i];
            }
        }
    }
    __syncthreads();

    // every wave runs the same `iters` steps, so the barriers stay uniform
    for(uint32_t it = 0; it < iters; it += 2) {
        load_row(xb, rb, row + stride);
        __builtin_amdgcn_sched_barrier(0);
        process(xa, ra, row);
        row += stride;
        if(it + 1 >= iters) break;
        load_row(xa, ra, row + stride);
        __builtin_amdgcn_sched_barrier(0);
        process(xb, rb, row);
        row += stride;
    }
}

// Any stride, alignment and length: one block per row, three passes over the
// row (the later passes re-read it, mostly from L2).
constexpr int kGenThreads = 256;

template <bool RES>
__global__ void __launch_bounds__(kGenThreads) rmsq_generic_kernel(NormRows p)
{
    __shared__ float red[2][kGenThreads / kWave];
    const uint32_t   row  = blockIdx.x;
    const int        wave = threadIdx.x / kWave;
    const uint16_t*  xr   = p.x + (size_t)row * p.ldx;
    const uint16_t*  rr   = RES ? p.res + (size_t)row * p.ldx : nullptr;
    uint16_t*        xo   = p.x_out ? p.x_out + (size_t)row * p.ldx : nullptr;

    auto block_reduce = [&](float v, int slot, bool is_max) {
        v = is_max ? wave_max(v) : wave_sum(v);
        if(threadIdx.x % kWave == 0) red[slot][wave] = v;
        __syncthreads();
        float t = red[slot][0];
#pragma unroll
        for(int w = 1; w < kGenThreads / kWave; ++w)
            t = is_max ? fmaxf(t, red[slot][w]) : t + red[slot][w];
        return t;
    };
    // u as pass 2 needs it; x_out may alias x or residual, so once written it
    // is the only copy of half(v)
    auto u_at = [&](uint32_t c) -> float {
        if constexpr(RES) {
            if(xo) return half_bits_to_float(xo[c]);
            return half_bits_to_float(float_to_half_bits_2step(half_bits_to_float(xr[c])
                                                               + half_bits_to_float(rr[c])));
        }
        return half_bits_to_float(xr[c]);
    };

    float ss = 0.f;
    for(uint32_t c = threadIdx.x; c < p.n; c += kGenThreads) {
        float v = half_bits_to_float(xr[c]);
        if constexpr(RES) {
            v += half_bits_to_float(rr[c]);
            if(xo) xo[c] = float_to_half_bits_2step(v);
        }
        ss += v * v;
    }
    ss               = block_reduce(ss, 0, false);
    const float rstd = rsqrtf(ss / (float)p.n + p.eps);
    __syncthreads(); // x_out of every thread is visible to the re-reads below

    uint16_t* yr   = p.y ? p.y + (size_t)row * p.ldy : nullptr;
    float     amax = 0.f;
    for(uint32_t c = threadIdx.x; c < p.n; c += kGenThreads) {
        const uint16_t yh = float_to_half_bits_2step((u_at(c) * rstd) * p.gamma[c]);
        if(yr) yr[c] = yh;
        if(p.q) amax = fmaxf(amax, fabsf(half_bits_to_float(yh) * p.s[c]));
    }
    if(!p.q) return; // uniform over the block
    amax            = block_reduce(amax, 1, true);
    const float rs  = amax / p.qmax;
    if(threadIdx.x == 0) p.r[row] = rs;
    const float inv = rs > 0.f ? 1.f / rs : 0.f;
    int8_t*     qr  = p.q + (size_t)row * p.ldq;
    for(uint32_t c = threadIdx.x; c < p.n; c += kGenThreads) {
        const float y = half_bits_to_float(float_to_half_bits_2step((u_at(c) * rstd) * p.gamma[c]));
        qr[c]         = (int8_t)quant_i8(y * p.s[c], inv, p.qmax);
    }
}

template <int CPL, int WPR, int THREADS, int BPC, bool RES, bool YOUT, bool QUANT>
hipError_t launch_stream_norm(const NormRows& p, hipStream_t stream)
{
    constexpr int kGroups = THREADS / kWave / WPR;
    const size_t  lds     = (size_t)CPL * 512 * WPR * sizeof(float) * (QUANT ? 2 : 1);
    // one row group must span the whole row
    if((uint64_t)CPL * 512 * WPR < p.n) return hipErrorInvalidValue;
    const void*   kernel  = reinterpret_cast<const void*>(
        rmsq_stream_kernel<CPL, WPR, THREADS, BPC, RES, YOUT, QUANT>);
    static int    max_blocks = [] {
        int dev = 0, cus = 256;
        if(hipGetDevice(&dev) == hipSuccess)
            (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        return cus * BPC;
    }();
    if(lds > 65536) {
        static std::once_flag once;
        std::call_once(once, [&] {
            (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      160 * 1024);
            (void)hipGetLastError();
        });
    }
    // every operand is addressed through a 32-bit buffer offset: launch row
    // panels whose spans stay under 2 GiB
    uint64_t row_bytes = std::max<uint64_t>((uint64_t)p.ldx * 2, std::max<uint64_t>(
                                                (uint64_t)p.ldy * 2, (uint64_t)p.ldq));
    const uint32_t panel = (uint32_t)std::min<uint64_t>(p.rows, 0x7FFFFFFFull / row_bytes);
    for(uint32_t r0 = 0; r0 < p.rows; r0 += panel) {
        NormRows q = p;
        q.rows     = std::min(panel, p.rows - r0);
        q.x        = p.x + (size_t)r0 * p.ldx;
        if(p.res) q.res = p.res + (size_t)r0 * p.ldx;
        if(p.x_out) q.x_out = p.x_out + (size_t)r0 * p.ldx;
        if(p.y) q.y = p.y + (size_t)r0 * p.ldy;
        if(p.q) q.q = p.q + (size_t)r0 * p.ldq;
        if(p.r) q.r = p.r + r0;
        const uint32_t need   = (q.rows + kGroups - 1) / kGroups;
        const uint32_t blocks = std::max<uint32_t>(1, std::min<uint32_t>(need, (uint32_t)max_blocks));
        const uint32_t iters  = (q.rows + blocks * kGroups - 1) / (blocks * kGroups);
        hipLaunchKernelGGL((rmsq_stream_kernel<CPL, WPR, THREADS, BPC, RES, YOUT, QUANT>), dim3(blocks),
                           dim3(THREADS), lds, stream, q, iters);
        const hipError_t e = hipGetLastError();
        if(e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int CPL, int WPR, int THREADS, int BPC>
hipError_t launch_by_outputs(const NormRows& p, hipStream_t stream)
{
    const bool res = p.res != nullptr, yout = p.y != nullptr, quant = p.q != nullptr;
    if(res) {
        if(yout && quant) return launch_stream_norm<CPL, WPR, THREADS, BPC, true, true, true>(p, stream);
        if(quant) return launch_stream_norm<CPL, WPR, THREADS, BPC, true, false, true>(p, stream);
        return launch_stream_norm<CPL, WPR, THREADS, BPC, true, true, false>(p, stream);
    }
    if(yout && quant) return launch_stream_norm<CPL, WPR, THREADS, BPC, false, true, true>(p, stream);
    if(quant) return launch_stream_norm<CPL, WPR, THREADS, BPC, false, false, true>(p, stream);
    return launch_stream_norm<CPL, WPR, THREADS, BPC, false, true, false>(p, stream);
}

} // namespace

hipError_t launch_rmsnorm_sq(const NormRows& p, hipStream_t stream)
{
    if(p.rows == 0) return hipSuccess;
    const auto al = [](const void* v, uintptr_t a) { return reinterpret_cast<uintptr_t>(v) % a == 0; };
    const uint32_t n = p.n;
    // 16-byte x / residual / x_out / y accesses, 8-byte q stores, rows of whole chunks
    const bool vec = n % 8 == 0 && p.ldx % 8 == 0 && p.ldy % 8 == 0 && p.ldq % 8 == 0
                     && al(p.x, 16) && al(p.res, 16) && al(p.x_out, 16) && al(p.y, 16)
                     && al(p.q, 8) && al(p.gamma, 16) && al(p.s, 16);
    // x_out without a residual is a plain copy: the generic kernel does it
    if(vec && !(p.x_out && !p.res)) {
        // two 16-byte chunks per lane and tensor: x and residual double-buffered
        // fit 128 VGPRs, i.e. two 512-thread blocks per CU
        if(n <= 1024) return launch_by_outputs<2, 1, 512, 2>(p, stream);
        if(n <= 2048) return launch_by_outputs<2, 2, 512, 2>(p, stream);
        if(n <= 4096) return launch_by_outputs<2, 4, 512, 2>(p, stream);
        if(n <= 8192) return launch_by_outputs<2, 8, 512, 2>(p, stream);
        if(n <= 16384) return launch_by_outputs<2, 16, 1024, 1>(p, stream);
    }
    if(p.res)
        hipLaunchKernelGGL(rmsq_generic_kernel<true>, dim3(p.rows), dim3(kGenThreads), 0, stream, p);
    else
        hipLaunchKernelGGL(rmsq_generic_kernel<false>, dim3(p.rows), dim3(kGenThreads), 0, stream, p);
    return hipGetLastError();
}

} // namespace w8a8
