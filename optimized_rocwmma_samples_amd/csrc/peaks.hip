// peaks.hip -- measured ceilings of one MI355X, built as libw8a8_peaks.so and
// timed by bench.py beside the path's kernels (not part of the W8A8 C ABI):
//   * an int8 MFMA-only loop: v_mfma_i32_32x32x32_i8 back to back on operands
//     held in registers, nothing else in the loop -- the matrix-core rate the
//     chip sustains at the clock it holds under that load;
//   * a streaming copy: 16 bytes per lane per access, several accesses in
//     flight per lane -- the HBM rate a plain read + write stream reaches;
//   * an empty kernel -- the launch floor of back-to-back launches (timed by
//     the caller in a captured graph).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kChains = 8; // independent accumulators per wave (covers the MFMA latency)

// Each wave: kChains accumulators, `iters` rounds of kChains MFMAs.  The
// operands are pseudo-random bytes (random: a hash of the lane) or zeros, and
// are perturbed every round from the accumulators' low bits so the compiler
// cannot hoist the products; the accumulators are folded into `sink` at the
// end (one int per wave) so nothing is dead.
__global__ void __launch_bounds__(256) peak_mfma_i8_kernel(int iters, int random, int* sink)
{
    const uint32_t lane = threadIdx.x % 64;
    uint32_t       h    = (blockIdx.x * 256u + threadIdx.x) * 0x9E3779B9u + 0x7F4A7C15u;
    v4i            a, b;
    for(int i = 0; i < 4; ++i) {
        h ^= h >> 15;
        h *= 0x2C1B3C6Du;
        h ^= h >> 12;
        a[i] = random ? (int)h : 0;
        h *= 0x297A2D39u;
        h ^= h >> 15;
        b[i] = random ? (int)(h ^ lane) : 0;
    }
    v16i acc[kChains];
#pragma unroll
    for(int c = 0; c < kChains; ++c) acc[c] = v16i{0};
    for(int it = 0; it < iters; ++it) {
#pragma unroll
        for(int c = 0; c < kChains; ++c)
            acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
        // a dependency the compiler cannot see through, once per round
        asm volatile("" : "+v"(a), "+v"(b));
    }
    int s = 0;
#pragma unroll
    for(int c = 0; c < kChains; ++c)
#pragma unroll
        for(int e = 0; e < 16; ++e) s += acc[c][e];
    if(lane == 0) sink[blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64] = s;
}

// Grid-stride copy of `n16` 16-byte chunks, kUnroll loads in flight per lane.
constexpr int kUnroll = 4;
__global__ void __launch_bounds__(256) peak_copy_kernel(const v4i* __restrict__ src,
                                                        v4i* __restrict__ dst, size_t n16)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t       i      = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for(; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        v4i v[kUnroll];
#pragma unroll
        for(int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for(int u = 0; u < kUnroll; ++u) __builtin_nontemporal_store(v[u], dst + i + u * stride);
    }
    for(; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ void peak_empty_kernel() {}

} // namespace

extern "C" {

// ops one peak_mfma launch performs: blocks x 4 waves x iters x kChains x
// (2 * 32 * 32 * 32)
double w8a8_peak_mfma_ops(uint32_t blocks, uint32_t iters)
{
    return (double)blocks * 4.0 * iters * kChains * 2.0 * 32 * 32 * 32;
}

// One MFMA-only launch of `blocks` blocks of 4 waves (one wave per SIMD at one
// block per CU; use a multiple of the CU count).  sink: blocks * 4 ints.
int w8a8_peak_mfma(uint32_t blocks, uint32_t iters, int random, int* sink, hipStream_t stream)
{
    if(blocks == 0 || iters == 0 || sink == nullptr) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(peak_mfma_i8_kernel, dim3(blocks), dim3(256), 0, stream, (int)iters, random,
                       sink);
    return (int)hipGetLastError();
}

// Copy `bytes` (a multiple of 16; src, dst 16-byte aligned) with `blocks`
// blocks of 256 threads.
int w8a8_peak_copy(const void* src, void* dst, size_t bytes, uint32_t blocks, hipStream_t stream)
{
    if(!src || !dst || bytes % 16 || blocks == 0 || reinterpret_cast<uintptr_t>(src) % 16
       || reinterpret_cast<uintptr_t>(dst) % 16)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(peak_copy_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const v4i*>(src), static_cast<v4i*>(dst), bytes / 16);
    return (int)hipGetLastError();
}

int w8a8_peak_empty(hipStream_t stream)
{
    hipLaunchKernelGGL(peak_empty_kernel, dim3(1), dim3(64), 0, stream);
    return (int)hipGetLastError();
}

} // extern "C"
