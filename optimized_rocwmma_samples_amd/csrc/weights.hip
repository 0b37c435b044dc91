// weights.hip -- offline weight preparation for gfx950: SmoothQuant folding,
// per-output-channel absmax int8 quantization and packing into the layout the
// packed GEMM kernels stream (N in 64-row slabs, K in 128-deep k-tiles,
// 8 KiB per (slab, k-tile): fragment f = nt*4 + g, lane l = h*32 + r holds
// w[slab*64 + nt*32 + r, kt*128 + g*32 + h*16 : +16]).
//
// Per weight row (output channel), the quantizer's operations
// (rocwmma_smoothquant.cpp:74-121) on p = float(w) (* or /) s:
//   sb = max|p| / qmax;  inv = sb > 0 ? 1/sb : 0;  q = int8(clamp(rint(p * inv)))
// One block per (padded) row: pass 1 takes the row's absmax, pass 2 re-reads
// the row (from L2), quantizes 16 consecutive k per thread and writes them as
// one 16-byte chunk -- exactly one packed lane's fragment slice -- or as a
// row-major run.  Rows and k past the weight write zeros into the packed
// padding.  This runs once per model load; it is not on the inference path.
#include "w8a8_device.hpp"
#include "w8a8_internal.hpp"

namespace w8a8 {
namespace {

constexpr int kWqThreads = 256;

__device__ __forceinline__ size_t packed_chunk_offset(uint32_t row, uint32_t k0, uint32_t nkt)
{
    const uint32_t slab = row / 64, nt = (row % 64) / 32, r = row % 32;
    const uint32_t kt = k0 / 128, g = (k0 % 128) / 32, h = (k0 % 32) / 16;
    return (((size_t)slab * nkt + kt) * 8 + (nt * 4 + g)) * 1024 + (h * 32 + r) * 16;
}

template <bool PACKED, bool DIV>
__global__ void __launch_bounds__(kWqThreads) quant_weights_kernel(WeightQuant p)
{
    __shared__ float red[kWqThreads / kWave];
    const uint32_t   row   = blockIdx.x;
    const bool       valid = row < p.n; // packed padding rows write zeros
    const uint16_t*  wr    = p.w + (size_t)(valid ? row : 0) * p.ldw;
    auto value = [&](uint32_t c) -> float {
        const float v = half_bits_to_float(wr[c]);
        if(!p.s) return v;
        return DIV ? v / p.s[c] : v * p.s[c];
    };

    float amax = 0.f;
    if(valid)
        for(uint32_t c = threadIdx.x; c < p.k; c += kWqThreads) amax = fmaxf(amax, fabsf(value(c)));
    amax = wave_max(amax);
    if(threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float rs = amax / p.qmax;
    if(valid && threadIdx.x == 0) p.sb[row] = rs;
    const float inv = rs > 0.f ? 1.f / rs : 0.f;

    const uint32_t nkt    = (p.k + 127) / 128;
    const uint32_t chunks = PACKED ? nkt * 8 : (p.k + 15) / 16; // 16 k-values each
    for(uint32_t ch = threadIdx.x; ch < chunks; ch += kWqThreads) {
        const uint32_t k0 = ch * 16;
        int            qi[16];
#pragma unroll
        for(int e = 0; e < 16; ++e)
            qi[e] = (valid && k0 + e < p.k) ? quant_i8(value(k0 + e), inv, p.qmax) : 0;
        if constexpr(PACKED) {
            int4 v;
            v.x = (int)pack4_i8(qi[0], qi[1], qi[2], qi[3]);
            v.y = (int)pack4_i8(qi[4], qi[5], qi[6], qi[7]);
            v.z = (int)pack4_i8(qi[8], qi[9], qi[10], qi[11]);
            v.w = (int)pack4_i8(qi[12], qi[13], qi[14], qi[15]);
            *reinterpret_cast<int4*>(p.q + packed_chunk_offset(row, k0, nkt)) = v;
        } else {
            int8_t* dst = p.q + (size_t)row * p.ldq + k0;
#pragma unroll
            for(int e = 0; e < 16; ++e)
                if(k0 + e < p.k) dst[e] = (int8_t)qi[e];
        }
    }
}

template <bool PACKED>
hipError_t launch(const WeightQuant& p, bool divide, hipStream_t stream)
{
    const uint32_t rows = PACKED ? (p.n + 63) / 64 * 64 : p.n;
    if(divide)
        hipLaunchKernelGGL((quant_weights_kernel<PACKED, true>), dim3(rows), dim3(kWqThreads), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((quant_weights_kernel<PACKED, false>), dim3(rows), dim3(kWqThreads), 0,
                           stream, p);
    return hipGetLastError();
}

} // namespace

hipError_t launch_quantize_weights(const WeightQuant& p, bool divide, bool packed,
                                   hipStream_t stream)
{
    return packed ? launch<true>(p, divide, stream) : launch<false>(p, divide, stream);
}

} // namespace w8a8
