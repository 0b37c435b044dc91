// peaks.hip -- measured ceilings of one MI355X, built as libw8a8_peaks.so and
// timed by bench.py beside the path's kernels (not part of the W8A8 C ABI):
//   * int8 MFMA-only loops: v_mfma_i32_32x32x32_i8 or v_mfma_i32_16x16x64_i8
//     back to back on operands held in registers, nothing else in the loop --
//     the matrix-core rate the chip sustains at the clock it holds under that
//     load;
//   * streams (read only, copy, 2:1): 16 bytes per lane per access, 8 or 16
//     accesses in flight per lane, grid-stride or contiguous per block, plain
//     or non-temporal loads -- the HBM rate a plain stream reaches, as the
//     best over those forms and the launch shapes the host sweeps;
//   * an LDS read loop: ds_read_b128 only, conflict-free, per-wave shader
//     cycles from s_memtime -- the bytes per clock one CU's LDS returns;
//   * an empty kernel -- the launch floor of back-to-back launches (timed by
//     the caller in a captured graph).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kChains = 8; // independent accumulators per wave (covers the MFMA latency)

// Each wave: kChains accumulators, `iters` rounds of kChains MFMAs.  The
// operands are pseudo-random bytes (random: a hash of the lane) or zeros; an
// empty asm statement that claims to rewrite them once per round keeps the
// compiler from hoisting or folding the products, and the accumulators are
// folded into `sink` at the end (one int per wave) so nothing is dead.  The
// operands stay the same from round to round: on MI355X, four operand sets
// rotated through a GEMM-like 4 x 2 fragment order run at the same rate
// (3.43 against 3.44 POP/s), so changing operands cost nothing measurable.
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

// The same loop on v_mfma_i32_16x16x64_i8, in blocks of 8 waves (two per
// SIMD, as the GEMM runs): one wave per SIMD cannot issue this form back to
// back (about 2.9 of 4.6 POP/s on zeros, 16 or 32 accumulators alike).  Each
// wave keeps 2 kChains accumulators of 16 x 16, so a round of a block is
// twice the 32 x 32 loop's ops; the host halves the rounds.
constexpr int kThreads16 = 512;
__global__ void __launch_bounds__(kThreads16) peak_mfma16_i8_kernel(int iters, int random,
                                                                    int* sink)
{
    const uint32_t lane = threadIdx.x % 64;
    uint32_t       h    = (blockIdx.x * kThreads16 + threadIdx.x) * 0x9E3779B9u + 0x7F4A7C15u;
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
    v4i acc[2 * kChains];
#pragma unroll
    for(int c = 0; c < 2 * kChains; ++c) acc[c] = v4i{0, 0, 0, 0};
    for(int it = 0; it < iters; ++it) {
#pragma unroll
        for(int c = 0; c < 2 * kChains; ++c)
            acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
        asm volatile("" : "+v"(a), "+v"(b));
    }
    int s = 0;
#pragma unroll
    for(int c = 0; c < 2 * kChains; ++c) s += acc[c].x + acc[c].y + acc[c].z + acc[c].w;
    if(lane == 0) sink[blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64] = s;
}

// Stream over `n16` 16-byte source chunks with kUnroll (U) loads in flight
// per lane.  MODE 0 reads only; MODE 1 copies each chunk; MODE 2 writes 8
// bytes per 16 read (the quantizer's fp16 -> int8 ratio).  Stores are
// non-temporal.  Two partitions of the chunks over the grid:
//   CONTIG = false: grid stride (lane i of the grid takes chunks i, i + G, ...);
//   CONTIG = true : block b takes the contiguous range [b n16 / B, (b+1) n16 / B)
//                   and walks it a wave instruction (1 KiB) at a time, the
//                   way the quantizer walks its rows;
// NT: loads with the non-temporal hint as well.  The host takes the best of
// these forms over several block counts and block sizes, so a kernel of the
// path that streams faster than every one of them means the ceiling is
// still low, not that the path beats the memory system.
typedef int v2i __attribute__((ext_vector_type(2)));
constexpr int kStreamThreadsMax = 1024;

template <int MODE, bool NT>
__device__ __forceinline__ v4i stream_load(const v4i* p)
{
    if constexpr(NT)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

template <int MODE, bool CONTIG, int U, bool NT>
__global__ void __launch_bounds__(kStreamThreadsMax) peak_stream_kernel(
    const v4i* __restrict__ src, void* __restrict__ dst, size_t n16, int* sink)
{
    const size_t threads = blockDim.x;
    size_t       i, end, stride;
    if constexpr(CONTIG) {
        i      = (size_t)blockIdx.x * n16 / gridDim.x + threadIdx.x;
        end    = (size_t)(blockIdx.x + 1) * n16 / gridDim.x;
        stride = threads;
    } else {
        i      = (size_t)blockIdx.x * threads + threadIdx.x;
        end    = n16;
        stride = (size_t)gridDim.x * threads;
    }
    v4i  acc = {0, 0, 0, 0};
    auto put = [&](size_t j, const v4i& v) {
        if constexpr(MODE == 1) __builtin_nontemporal_store(v, static_cast<v4i*>(dst) + j);
        if constexpr(MODE == 2)
            __builtin_nontemporal_store(v2i{v.x ^ v.y, v.z ^ v.w}, static_cast<v2i*>(dst) + j);
        if constexpr(MODE == 0) acc ^= v;
    };
    for(; i + (U - 1) * stride < end; i += U * stride) {
        v4i v[U];
#pragma unroll
        for(int u = 0; u < U; ++u) v[u] = stream_load<MODE, NT>(src + i + u * stride);
#pragma unroll
        for(int u = 0; u < U; ++u) put(i + u * stride, v[u]);
    }
    for(; i < end; i += stride) put(i, stream_load<MODE, NT>(src + i));
    if(MODE == 0 && acc.x == 0x13579BDF && acc.y == acc.z) sink[0] = acc.w; // keeps the loads live
}

// variant bits: 0 CONTIG, 1 U = 16 (else 8), 2 NT loads
template <int MODE>
hipError_t launch_stream(const v4i* s, void* d, size_t n16, uint32_t blocks, uint32_t threads,
                         int variant, int* sink, hipStream_t st)
{
#define W8A8_PEAK_STREAM(C, U, N)                                                                 \
    hipLaunchKernelGGL((peak_stream_kernel<MODE, C, U, N>), dim3(blocks), dim3(threads), 0, st, s, \
                       d, n16, sink)
    switch(variant) {
    case 0: W8A8_PEAK_STREAM(false, 8, false); break;
    case 1: W8A8_PEAK_STREAM(true, 8, false); break;
    case 2: W8A8_PEAK_STREAM(false, 16, false); break;
    case 3: W8A8_PEAK_STREAM(true, 16, false); break;
    case 4: W8A8_PEAK_STREAM(false, 8, true); break;
    case 5: W8A8_PEAK_STREAM(true, 8, true); break;
    case 6: W8A8_PEAK_STREAM(false, 16, true); break;
    default: W8A8_PEAK_STREAM(true, 16, true); break;
    }
#undef W8A8_PEAK_STREAM
    return hipGetLastError();
}

// LDS read loop.  Every lane of the block's waves reads 16 bytes per
// access (ds_read_b128; the 64 lanes of a wave on 64 consecutive chunks, so
// no bank conflicts) from a kLdsPeakBytes region `iters` times, the wave
// instructions of a block walking the region in turn, kLdsPeakBatch reads in
// flight per wave.  The empty asm after each batch keeps the compiler from
// merging or hoisting reads of one address across batches; the sums go to
// `sink`.  Shader-clock cycles of each wave's
// loop (s_memtime) go to cyc[block * 16 + wave], so bytes per clock come
// out whatever clock the chip holds.  The host launches one block per CU
// (kLdsPeakLaunch bytes of dynamic LDS each).
constexpr int kLdsPeakBytes  = 64 * 1024;
constexpr int kLdsPeakLaunch = 96 * 1024;
constexpr int kLdsPeakBatch  = 8;

__global__ void __launch_bounds__(1024) peak_lds_kernel(int iters, unsigned long long* cyc,
                                                        int* sink)
{
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, waves = blockDim.x >> 6;
    for(int i = tid; i < kLdsPeakBytes / 16; i += blockDim.x)
        reinterpret_cast<v4i*>(lds)[i] = v4i{i, i ^ 1, i ^ 2, i ^ 3};
    __syncthreads();
    v4i                      acc{0, 0, 0, 0};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for(int i = 0; i < iters; i += kLdsPeakBatch) {
        v4i v[kLdsPeakBatch];
#pragma unroll
        for(int u = 0; u < kLdsPeakBatch; ++u) {
            const int off = ((((i + u) * waves + wave) * 64 + lane) * 16) & (kLdsPeakBytes - 1);
            v[u]          = *reinterpret_cast<const v4i*>(lds + off);
        }
#pragma unroll
        for(int u = 0; u < kLdsPeakBatch; ++u) acc += v[u];
        asm volatile("" ::: "memory");
    }
    __builtin_amdgcn_s_waitcnt(0); // every read has returned
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    const int                s  = acc.x + acc.y + acc.z + acc.w;
    if(lane == 0) cyc[blockIdx.x * 16 + wave] = t1 - t0;
    sink[blockIdx.x * blockDim.x + tid] = s;
}

__global__ void peak_empty_kernel() {}

} // namespace

extern "C" {

// ops one peak_mfma launch performs (either form): blocks x 4 waves x iters
// x kChains x (2 * 32 * 32 * 32)
double w8a8_peak_mfma_ops(uint32_t blocks, uint32_t iters)
{
    return (double)blocks * 4.0 * iters * kChains * 2.0 * 32 * 32 * 32;
}

// One MFMA-only launch of `blocks` blocks (use a multiple of the CU count):
// 4 waves of the 32 x 32 x 32 form or 8 waves of the 16 x 16 x 64 form, the
// same w8a8_peak_mfma_ops either way (iters even).  mode bit 0: random (1) or
// zero (0) operands; bit 1: the 16 x 16 x 64 form.  sink: blocks * 8 ints.
int w8a8_peak_mfma(uint32_t blocks, uint32_t iters, int mode, int* sink, hipStream_t stream)
{
    if(blocks == 0 || iters == 0 || iters % 2 || sink == nullptr || mode < 0 || mode > 3)
        return (int)hipErrorInvalidValue;
    if(mode & 2)
        hipLaunchKernelGGL(peak_mfma16_i8_kernel, dim3(blocks), dim3(kThreads16), 0, stream,
                           (int)(iters / 2), mode & 1, sink);
    else
        hipLaunchKernelGGL(peak_mfma_i8_kernel, dim3(blocks), dim3(256), 0, stream, (int)iters,
                           mode & 1, sink);
    return (int)hipGetLastError();
}

// Stream `bytes` of src (a multiple of 16; src, dst 16-byte aligned) with
// `blocks` blocks of `threads` threads (64-1024, a multiple of 64) in the
// form `variant` (0-7: bit 0 contiguous ranges per block, bit 1 16 loads in
// flight per lane instead of 8, bit 2 non-temporal loads): mode 0 read only
// (dst unused, sink: one int), 1 copy to dst (`bytes` written), 2 write
// bytes / 2 to dst.
int w8a8_peak_stream(const void* src, void* dst, size_t bytes, uint32_t blocks, uint32_t threads,
                     int variant, int mode, int* sink, hipStream_t stream)
{
    if(!src || bytes % 16 || blocks == 0 || reinterpret_cast<uintptr_t>(src) % 16
       || (mode != 0 && (!dst || reinterpret_cast<uintptr_t>(dst) % 16)) || (mode == 0 && !sink)
       || mode < 0 || mode > 2 || threads < 64 || threads > kStreamThreadsMax || threads % 64
       || variant < 0 || variant > 7)
        return (int)hipErrorInvalidValue;
    const v4i* s = static_cast<const v4i*>(src);
    if(mode == 0) return (int)launch_stream<0>(s, dst, bytes / 16, blocks, threads, variant, sink, stream);
    if(mode == 1) return (int)launch_stream<1>(s, dst, bytes / 16, blocks, threads, variant, sink, stream);
    return (int)launch_stream<2>(s, dst, bytes / 16, blocks, threads, variant, sink, stream);
}

// One LDS read launch: `blocks` blocks (one per CU: use the CU count) of
// `threads` threads (64-1024, a multiple of 64), `iters` reads of 16 bytes
// per lane (a multiple of 8).  cyc: blocks * 16 entries (per-wave shader cycles), sink:
// blocks * threads ints.  Bytes read per wave: iters * 1024.
int w8a8_peak_lds(uint32_t blocks, uint32_t threads, uint32_t iters, unsigned long long* cyc,
                  int* sink, hipStream_t stream)
{
    if(blocks == 0 || iters == 0 || iters % kLdsPeakBatch || iters > (1u << 30) || threads < 64
       || threads > 1024 || threads % 64 || cyc == nullptr || sink == nullptr)
        return (int)hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(peak_lds_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
        kLdsPeakLaunch);
    if(attr != hipSuccess) return (int)attr;
    hipLaunchKernelGGL(peak_lds_kernel, dim3(blocks), dim3(threads), kLdsPeakLaunch, stream,
                       (int)iters, cyc, sink);
    return (int)hipGetLastError();
}

int w8a8_peak_empty(hipStream_t stream)
{
    hipLaunchKernelGGL(peak_empty_kernel, dim3(1), dim3(64), 0, stream);
    return (int)hipGetLastError();
}

} // extern "C"
