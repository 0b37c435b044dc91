// smoothquant.hip -- row-wise smooth-scale + absmax int8 quantizer for gfx950.
//
// Computation (kernel_smoothquant, rocwmma_smoothquant.cpp:58-122, and
// kernel_moe_smoothquant, rocwmma_moe_smoothquant.cpp:69-131):
//   p = float(x[row, n]) * s[n];  r = max|p| / qmax;  inv = r > 0 ? 1/r : 0
//   q[row, n] = int8(clamp(rint(p * inv), -qmax, qmax))
//
// Design (HBM-bound: 3 bytes moved per element):
//   * One wavefront owns a row segment of CPL*512 elements; WPR wavefronts
//     share a row.  Each lane issues CPL 16-byte loads (8 fp16) so a wave
//     instruction reads 1 KiB contiguous, and the whole segment is in flight
//     at once.
//   * The smoothed row stays in VGPRs: x is read from HBM exactly once
//     (the reference re-reads it in its second pass, :101-117).
//   * absmax: DPP quad/mirror steps inside each 16-lane row + 4 readlanes;
//     rows spread over several waves merge through 16 bytes of LDS.
//   * Output: each lane packs 8 int8 and stores 8 bytes (a wave writes 512
//     contiguous bytes), straight into the row-major A operand of the GEMM.
#include "w8a8_device.hpp"
#include "w8a8_internal.hpp"

namespace w8a8 {
namespace {

constexpr int kSqThreads = 256; // 4 waves
constexpr int kSqWaves   = kSqThreads / kWave;

struct RowSrc {
    const uint16_t* x;
    const float*    s;
    long            dst;
    bool            valid;
};

template <bool MOE>
__device__ __forceinline__ RowSrc resolve_row(const QuantRows& p, uint32_t row)
{
    RowSrc rs{nullptr, nullptr, -1, false};
    if(row >= p.rows) return rs;
    if constexpr(MOE) {
        uint32_t tok = row / p.topk;
        int32_t  e   = p.topk_ids[row];
        if(e < 0 || (uint32_t)e >= p.experts) return rs;
        long dst = p.dst_row ? (long)p.dst_row[row] : (long)row;
        if(dst < 0 || dst >= (long)p.rows_out) return rs;
        rs.x   = p.x + (size_t)tok * p.ldx;
        rs.s   = p.s + (size_t)e * p.n;
        rs.dst = dst;
    } else {
        rs.x   = p.x + (size_t)row * p.ldx;
        rs.s   = p.s;
        rs.dst = row;
    }
    rs.valid = true;
    return rs;
}

// CPL: 16-byte chunks per lane; WPR: waves per row; VEC: aligned vector I/O.
template <int CPL, int WPR, bool MOE, bool VEC>
__global__ void __launch_bounds__(kSqThreads) sq_rows_kernel(QuantRows p)
{
    constexpr int kRowsPerBlock = kSqWaves / WPR;
    constexpr int kSpan         = CPL * 8 * kWave;

    const int      wave = threadIdx.x / kWave;
    const int      lane = threadIdx.x % kWave;
    const int      rib  = wave / WPR; // row in block
    const int      part = wave % WPR; // segment of the row
    const uint32_t row  = blockIdx.x * kRowsPerBlock + rib;

    RowSrc src = resolve_row<MOE>(p, row);

    float    pv[CPL * 8];
    float    amax = 0.f;
    const uint32_t n    = p.n;
    const uint32_t base = part * kSpan + lane * 8;

    if(src.valid) {
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const uint32_t c = base + j * (8 * kWave);
            if(VEC && c + 8 <= n) {
                const uint4 raw = *reinterpret_cast<const uint4*>(src.x + c);
                const float4 s0 = *reinterpret_cast<const float4*>(src.s + c);
                const float4 s1 = *reinterpret_cast<const float4*>(src.s + c + 4);
                pv[j * 8 + 0] = half_bits_to_float(raw.x & 0xFFFFu) * s0.x;
                pv[j * 8 + 1] = half_bits_to_float(raw.x >> 16) * s0.y;
                pv[j * 8 + 2] = half_bits_to_float(raw.y & 0xFFFFu) * s0.z;
                pv[j * 8 + 3] = half_bits_to_float(raw.y >> 16) * s0.w;
                pv[j * 8 + 4] = half_bits_to_float(raw.z & 0xFFFFu) * s1.x;
                pv[j * 8 + 5] = half_bits_to_float(raw.z >> 16) * s1.y;
                pv[j * 8 + 6] = half_bits_to_float(raw.w & 0xFFFFu) * s1.z;
                pv[j * 8 + 7] = half_bits_to_float(raw.w >> 16) * s1.w;
            } else {
#pragma unroll
                for(int e = 0; e < 8; ++e)
                    pv[j * 8 + e] = (c + e < n) ? half_bits_to_float(src.x[c + e]) * src.s[c + e]
                                                : 0.f;
            }
#pragma unroll
            for(int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(pv[j * 8 + e]));
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
    if(!src.valid) return;

    const float qmax = p.qmax;
    const float rs   = amax / qmax; // correctly rounded fp32 division
    if(part == 0 && lane == 0) p.r[src.dst] = rs;
    const float inv = (rs > 0.f) ? (1.f / rs) : 0.f;

    int8_t* qrow = p.q + (size_t)src.dst * p.ldq;
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t c = base + j * (8 * kWave);
        int            qi[8];
#pragma unroll
        for(int e = 0; e < 8; ++e) qi[e] = quant_i8(pv[j * 8 + e], inv, qmax);
        if(VEC && c + 8 <= n) {
            uint2 packed;
            packed.x = pack4_i8(qi[0], qi[1], qi[2], qi[3]);
            packed.y = pack4_i8(qi[4], qi[5], qi[6], qi[7]);
            *reinterpret_cast<uint2*>(qrow + c) = packed;
        } else {
#pragma unroll
            for(int e = 0; e < 8; ++e)
                if(c + e < n) qrow[c + e] = (int8_t)qi[e];
        }
    }
}

// Rows longer than the register-resident path covers: one block per row,
// two passes over x (the second pass re-reads x, mostly from L2).
template <bool MOE>
__global__ void __launch_bounds__(kSqThreads) sq_twopass_kernel(QuantRows p)
{
    __shared__ float red[kSqWaves];
    RowSrc src = resolve_row<MOE>(p, blockIdx.x);
    if(!src.valid) return; // uniform over the block
    float amax = 0.f;
    for(uint32_t c = threadIdx.x; c < p.n; c += kSqThreads)
        amax = fmaxf(amax, fabsf(half_bits_to_float(src.x[c]) * src.s[c]));
    amax = wave_max(amax);
    if(threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float rs = amax / p.qmax;
    if(threadIdx.x == 0) p.r[src.dst] = rs;
    const float inv  = (rs > 0.f) ? (1.f / rs) : 0.f;
    int8_t*     qrow = p.q + (size_t)src.dst * p.ldq;
    for(uint32_t c = threadIdx.x; c < p.n; c += kSqThreads)
        qrow[c] = (int8_t)quant_i8(half_bits_to_float(src.x[c]) * src.s[c], inv, p.qmax);
}

template <int CPL, int WPR, bool MOE>
hipError_t launch_rows(const QuantRows& p, bool vec, hipStream_t stream)
{
    constexpr int kRowsPerBlock = kSqWaves / WPR;
    dim3          grid((p.rows + kRowsPerBlock - 1) / kRowsPerBlock);
    if(vec)
        hipLaunchKernelGGL((sq_rows_kernel<CPL, WPR, MOE, true>), grid, dim3(kSqThreads), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((sq_rows_kernel<CPL, WPR, MOE, false>), grid, dim3(kSqThreads), 0,
                           stream, p);
    return hipGetLastError();
}

template <bool MOE>
hipError_t dispatch(const QuantRows& p, hipStream_t stream)
{
    // 16-byte x loads, 32-byte aligned s loads, 8-byte q stores.
    const bool vec = (reinterpret_cast<uintptr_t>(p.x) % 16 == 0) && (p.ldx % 8 == 0)
                     && (reinterpret_cast<uintptr_t>(p.s) % 16 == 0) && (!MOE || p.n % 4 == 0)
                     && (reinterpret_cast<uintptr_t>(p.q) % 8 == 0) && (p.ldq % 8 == 0);
    const uint32_t n = p.n;
    if(n <= 512) return launch_rows<1, 1, MOE>(p, vec, stream);
    if(n <= 1024) return launch_rows<2, 1, MOE>(p, vec, stream);
    if(n <= 2048) return launch_rows<4, 1, MOE>(p, vec, stream);
    if(n <= 4096) return launch_rows<8, 1, MOE>(p, vec, stream);
    if(n <= 8192) return launch_rows<16, 1, MOE>(p, vec, stream);
    if(n <= 16384) return launch_rows<16, 2, MOE>(p, vec, stream);
    if(n <= 32768) return launch_rows<16, 4, MOE>(p, vec, stream);
    hipLaunchKernelGGL((sq_twopass_kernel<MOE>), dim3(p.rows), dim3(kSqThreads), 0, stream, p);
    return hipGetLastError();
}

} // namespace

hipError_t launch_smoothquant(const QuantRows& p, hipStream_t stream)
{
    if(p.rows == 0) return hipSuccess;
    return p.topk_ids ? dispatch<true>(p, stream) : dispatch<false>(p, stream);
}

} // namespace w8a8
