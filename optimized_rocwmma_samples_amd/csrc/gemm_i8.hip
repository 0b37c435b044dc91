// gemm_i8.hip -- int8 x int8 -> int32 GEMM with fused per-token x per-channel
// dequant epilogue, hand-written for gfx950 (CDNA4) on raw MFMA intrinsics.
//
// Computation (gemm_quant_tensor_scale, rocwmma_gemm_quantized.cpp:127-195,
// in its documented Mode 2, :18-26):
//   acc[m,n] = sum_k A[m,k] * B[n,k]  (int32, exact)
//   C[m,n]   = half((float(acc) * sa[m]) * sb[n])   or int32 acc
//
// Tile hierarchy
//   block : 256 (m) x 256 (n) x 64 (k), 256 threads = 4 waves in a 2x2 grid
//   wave  : 128 x 128, i.e. 4 x 4 tiles of v_mfma_i32_32x32x32_i8
//   mfma  : 32 x 32 x 32; srcA = B fragment (rows n), srcB = A fragment (rows m),
//           so D[i=n][j=m] and each lane owns one m and runs of 4 consecutive n:
//           the epilogue writes 4 fp16 (8 B) or 4 int32 (16 B) per store.
//
// Data movement
//   * global -> LDS with global_load_lds_dwordx4 (no VGPR staging): one wave
//     instruction fills 1 KiB of LDS, lane i writing bytes [16i, 16i+16).  The
//     LDS tile layout is chosen by which global 16-byte chunk each lane fetches.
//   * LDS rows are 64 B (4 chunks); chunk c of row r sits at physical chunk
//     c ^ ((r >> 2) & 3), so the 16 lanes of a ds_read_b128 quarter-wave touch
//     16 distinct 16-byte bank groups (conflict-free for A and B alike).
//   * 4-stage ring (4 x 32 KiB): tiles t+1..t+3 are in flight while tile t
//     computes.  One barrier per 64-deep k step, placed between the two
//     32-deep MFMA halves so LDS fragment reads always overlap MFMA work.
//   * Out-of-range rows / k-chunks read a 16-byte zero chunk, so edges need no
//     masking in the main loop (k must be a multiple of 16).
//   * Block order: consecutive hardware block ids are spread over the 8 XCDs;
//     they are remapped so each XCD works on a compact group of tiles (shared
//     A/B panels stay in that XCD's L2), then grouped GROUP_M rows at a time.
#include "w8a8_device.hpp"
#include "w8a8_internal.hpp"
#include "../../include/w8a8.h"

#include <mutex>

namespace w8a8 {

__device__ __attribute__((aligned(64))) int4 g_zero_chunk[4];

namespace {

constexpr int kBM       = 256;
constexpr int kBN       = 256;
constexpr int kBK       = 64;
constexpr int kStages   = 4;
constexpr int kThreads  = 256;
constexpr int kWaveM    = 128;
constexpr int kWaveN    = 128;
constexpr int kTilesM   = kWaveM / 32;
constexpr int kTilesN   = kWaveN / 32;
constexpr int kRowBytes = kBK;
constexpr int kABytes   = kBM * kRowBytes;
constexpr int kBBytes   = kBN * kRowBytes;
constexpr int kStageBytes = kABytes + kBBytes;
constexpr int kLdsBytes   = kStages * kStageBytes;
constexpr int kLoadsA     = kABytes / 1024 / (kThreads / kWave); // per wave per stage
constexpr int kLoadsB     = kBBytes / 1024 / (kThreads / kWave);
constexpr int kLoadsPerStage = kLoadsA + kLoadsB;
constexpr int kGroupM     = 8;
// sched_group_barrier instruction classes
constexpr int kSchedMfma   = 0x008;
constexpr int kSchedDsRead = 0x100;

static_assert(kLoadsA * (kThreads / kWave) * 1024 == kABytes, "A tile / wave loads");
static_assert(kLoadsB * (kThreads / kWave) * 1024 == kBBytes, "B tile / wave loads");

typedef __attribute__((address_space(3))) void lds_void_t;

struct KArgs {
    const int8_t* a;
    const int8_t* b;
    void*         c;
    const float*  sa;
    const float*  sb;
    uint32_t      m, n, k;
    uint32_t      lda, ldb, ldc;
    float         tsa, tsb;
};

// Hardware dispatches block ids round-robin over the 8 XCDs.  Return the
// logical tile id such that each XCD owns a contiguous range of logical ids.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t total)
{
    constexpr uint32_t kXcd = 8;
    const uint32_t     q    = total / kXcd;
    const uint32_t     r    = total % kXcd;
    const uint32_t     x    = bid % kXcd;
    const uint32_t     i    = bid / kXcd;
    return x * q + min(x, r) + i;
}

__device__ __forceinline__ void tile_coords(uint32_t lid, uint32_t tiles_m, uint32_t tiles_n,
                                            uint32_t& tm, uint32_t& tn)
{
    const uint32_t per_group = kGroupM * tiles_n;
    const uint32_t group     = lid / per_group;
    const uint32_t first_m   = group * kGroupM;
    const uint32_t gsize     = min(tiles_m - first_m, (uint32_t)kGroupM);
    const uint32_t in_group  = lid % per_group;
    tm                       = first_m + in_group % gsize;
    tn                       = in_group / gsize;
}

// Store 4 consecutive-n outputs of one lane.
template <int OUT>
__device__ __forceinline__ void store4(const KArgs& p, uint32_t m, uint32_t n, const int* v,
                                       float sa, const float4& sb, float ab, bool mode1,
                                       bool vec_ok)
{
    if(m >= p.m) return;
    if constexpr(OUT == W8A8_OUT_I32) {
        int32_t* dst = reinterpret_cast<int32_t*>(p.c) + (size_t)m * p.ldc + n;
        if(vec_ok && n + 4 <= p.n) {
            *reinterpret_cast<int4*>(dst) = make_int4(v[0], v[1], v[2], v[3]);
        } else {
            for(int e = 0; e < 4; ++e)
                if(n + e < p.n) dst[e] = v[e];
        }
    } else {
        const float sbv[4] = {sb.x, sb.y, sb.z, sb.w};
        uint16_t    h[4];
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            float f = (float)v[e];
            f       = mode1 ? f * ab : (f * sa) * sbv[e];
            h[e]    = float_to_half_bits(f);
        }
        uint16_t* dst = reinterpret_cast<uint16_t*>(p.c) + (size_t)m * p.ldc + n;
        if(vec_ok && n + 4 <= p.n) {
            uint2 pk;
            pk.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
            pk.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            *reinterpret_cast<uint2*>(dst) = pk;
        } else {
            for(int e = 0; e < 4; ++e)
                if(n + e < p.n) dst[e] = h[e];
        }
    }
}

// Barrier between the waves of a block without the release/acquire fences of
// __syncthreads() (those would wait for every outstanding global->LDS load,
// vmcnt(0), and serialize the prefetch ring).  LDS hazards are covered by the
// explicit s_waitcnt calls placed before each barrier.
__device__ __forceinline__ void block_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Scheduling recipe for one 32-deep MFMA half: MFMA and DS reads of the next
// fragments alternate, then the remaining MFMAs follow.  Keeping the first
// MFMA ahead of the reads means it waits only on fragments read one half earlier.
template <int ID>
__device__ __forceinline__ void interleave_mfma_ds()
{
#pragma unroll
    for(int i = 0; i < kTilesM + kTilesN; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, ID);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, ID);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kTilesM * kTilesN - (kTilesM + kTilesN), ID);
}

// Wait until at most `tiles` stages of global->LDS loads issued by this wave
// are still in flight (loads complete in order).
__device__ __forceinline__ void wait_tiles_outstanding(uint32_t tiles)
{
    static_assert(kStages <= 4, "extend the switch for deeper rings");
    switch(tiles) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<kLoadsPerStage>(); break;
    case 2: wait_vmcnt<kLoadsPerStage * 2>(); break;
    default: wait_vmcnt<kLoadsPerStage * 3>(); break;
    }
}

template <int OUT>
__global__ void __launch_bounds__(kThreads, 1) gemm_i8_nk_kernel(KArgs p, int vec_ok)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    const uint32_t tiles_m = (p.m + kBM - 1) / kBM;
    const uint32_t tiles_n = (p.n + kBN - 1) / kBN;
    uint32_t       tm, tn;
    tile_coords(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * kBM;
    const uint32_t n0 = tn * kBN;

    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int wm   = wave >> 1; // wave row in the 2x2 grid
    const int wn   = wave & 1;

    // ---- global -> LDS load descriptors (per wave, per stage) -------------
    // Wave-load j (0..15 over the block) of the A tile fills rows 16j..16j+15.
    // Lane l: row 16j + l/4, physical chunk l%4, logical chunk (l%4)^((row>>2)&3).
    const int      lrow   = lane >> 2;
    const int      lchunk = (lane & 3) ^ ((lane >> 4) & 3);
    const int8_t*  ga[kLoadsA];
    const int8_t*  gb[kLoadsB];
    bool           rowa_ok[kLoadsA], rowb_ok[kLoadsB];
#pragma unroll
    for(int i = 0; i < kLoadsA; ++i) {
        const uint32_t r = (wave * kLoadsA + i) * 16 + lrow;
        rowa_ok[i]       = (m0 + r) < p.m;
        ga[i]            = p.a + (size_t)(rowa_ok[i] ? m0 + r : 0) * p.lda + lchunk * 16;
    }
#pragma unroll
    for(int i = 0; i < kLoadsB; ++i) {
        const uint32_t r = (wave * kLoadsB + i) * 16 + lrow;
        rowb_ok[i]       = (n0 + r) < p.n;
        gb[i]            = p.b + (size_t)(rowb_ok[i] ? n0 + r : 0) * p.ldb + lchunk * 16;
    }
    const int8_t* zero = reinterpret_cast<const int8_t*>(g_zero_chunk);

    auto issue_stage = [&](int stage, uint32_t kt) {
        const uint32_t k0     = kt * kBK;
        const bool     kok    = (k0 + lchunk * 16) < p.k;
        int8_t*        sbase  = lds + stage * kStageBytes;
#pragma unroll
        for(int i = 0; i < kLoadsA; ++i) {
            const int8_t* src = (kok && rowa_ok[i]) ? ga[i] + k0 : zero;
            __builtin_amdgcn_global_load_lds(
                src, (lds_void_t*)(sbase + (wave * kLoadsA + i) * 1024), 16, 0, 0);
        }
#pragma unroll
        for(int i = 0; i < kLoadsB; ++i) {
            const int8_t* src = (kok && rowb_ok[i]) ? gb[i] + k0 : zero;
            __builtin_amdgcn_global_load_lds(
                src, (lds_void_t*)(sbase + kABytes + (wave * kLoadsB + i) * 1024), 16, 0, 0);
        }
    };

    // ---- LDS -> register fragment offsets ----------------------------------
    // Fragment row = lane%32 inside a 32-row tile, k-chunk = 2*ks + lane/32.
    const int frow = lane & 31;
    const int fswz = (frow >> 2) & 3;
    int       offa[kTilesM], offb[kTilesN];
#pragma unroll
    for(int t = 0; t < kTilesM; ++t) offa[t] = (wm * kWaveM + t * 32 + frow) * kRowBytes;
#pragma unroll
    for(int t = 0; t < kTilesN; ++t)
        offb[t] = kABytes + (wn * kWaveN + t * 32 + frow) * kRowBytes;
    int cofs[kBK / 32];
#pragma unroll
    for(int ks = 0; ks < kBK / 32; ++ks) cofs[ks] = ((2 * ks + (lane >> 5)) ^ fswz) * 16;

    v16i acc[kTilesM][kTilesN];
#pragma unroll
    for(int i = 0; i < kTilesM; ++i)
#pragma unroll
        for(int j = 0; j < kTilesN; ++j) acc[i][j] = v16i{0};

    const uint32_t nk = (p.k + kBK - 1) / kBK;

    auto load_frags = [&](const int8_t* sbase, int ks, v4i (&af)[kTilesM], v4i (&bf)[kTilesN]) {
#pragma unroll
        for(int t = 0; t < kTilesM; ++t)
            af[t] = *reinterpret_cast<const v4i*>(sbase + offa[t] + cofs[ks]);
#pragma unroll
        for(int t = 0; t < kTilesN; ++t)
            bf[t] = *reinterpret_cast<const v4i*>(sbase + offb[t] + cofs[ks]);
    };
    auto mfma_tile = [&](const v4i (&af)[kTilesM], const v4i (&bf)[kTilesN]) {
#pragma unroll
        for(int i = 0; i < kTilesM; ++i)
#pragma unroll
            for(int j = 0; j < kTilesN; ++j)
                acc[i][j]
                    = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
    };

    // ---- prologue: fill every stage of the ring ----------------------------
    uint32_t last_issued = 0; // highest tile index issued so far
#pragma unroll
    for(int s = 0; s < kStages; ++s)
        if((uint32_t)s < nk) {
            issue_stage(s, s);
            last_issued = s;
        }
    wait_tiles_outstanding(last_issued); // tile 0 landed
    block_barrier();

    v4i f0a[kTilesM], f0b[kTilesN], f1a[kTilesM], f1b[kTilesN];
    load_frags(lds, 0, f0a, f0b);

    // ---- main loop ---------------------------------------------------------
    // Per 64-deep tile kt (stage kt % S):
    //   read k-half 1 fragments; MFMA k-half 0;
    //   [all waves done reading stage kt, tile kt+1 landed] barrier;
    //   refill stage kt % S with tile kt+S; read tile kt+1 k-half 0; MFMA k-half 1.
    for(uint32_t kt = 0; kt + 1 < nk; ++kt) {
        load_frags(lds + (kt % kStages) * kStageBytes, 1, f1a, f1b);
        mfma_tile(f0a, f0b);
        interleave_mfma_ds<0>();
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0(); // this wave's reads of stage kt are done before it is refilled
        wait_tiles_outstanding(last_issued - (kt + 1));
        block_barrier();
        if(kt + kStages < nk) {
            issue_stage(kt % kStages, kt + kStages);
            last_issued = kt + kStages;
        }
        load_frags(lds + ((kt + 1) % kStages) * kStageBytes, 0, f0a, f0b);
        mfma_tile(f1a, f1b);
        interleave_mfma_ds<1>();
    }
    // last tile (peeled so the loop body has a single path for the waitcnt pass)
    load_frags(lds + ((nk - 1) % kStages) * kStageBytes, 1, f1a, f1b);
    mfma_tile(f0a, f0b);
    mfma_tile(f1a, f1b);

    // ---- epilogue ----------------------------------------------------------
    // acc[i][j][r]: m = m0 + wm*128 + i*32 + lane%32,
    //               n = n0 + wn*128 + j*32 + (r/4)*8 + (lane/32)*4 + r%4.
    const bool  mode1 = (p.sa == nullptr && p.sb == nullptr);
    const float ab    = p.tsa * p.tsb;
#pragma unroll
    for(int i = 0; i < kTilesM; ++i) {
        const uint32_t m  = m0 + wm * kWaveM + i * 32 + (lane & 31);
        float          sa = p.tsa;
        if(OUT == W8A8_OUT_F16 && p.sa != nullptr && m < p.m) sa = p.sa[m];
#pragma unroll
        for(int j = 0; j < kTilesN; ++j) {
#pragma unroll
            for(int g = 0; g < 4; ++g) {
                const uint32_t n = n0 + wn * kWaveN + j * 32 + g * 8 + (lane >> 5) * 4;
                float4         sb = make_float4(p.tsb, p.tsb, p.tsb, p.tsb);
                if(OUT == W8A8_OUT_F16 && p.sb != nullptr) {
                    if(vec_ok && n + 4 <= p.n)
                        sb = *reinterpret_cast<const float4*>(p.sb + n);
                    else {
                        if(n + 0 < p.n) sb.x = p.sb[n + 0];
                        if(n + 1 < p.n) sb.y = p.sb[n + 1];
                        if(n + 2 < p.n) sb.z = p.sb[n + 2];
                        if(n + 3 < p.n) sb.w = p.sb[n + 3];
                    }
                }
                const int v[4] = {acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1],
                                  acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]};
                store4<OUT>(p, m, n, v, sa, sb, ab, mode1, vec_ok != 0);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Generic strided kernel: one thread per output, any layout / alignment.
// ---------------------------------------------------------------------------
template <int OUT>
__global__ void __launch_bounds__(256) gemm_i8_generic_kernel(KArgs p, size_t sam, size_t sak,
                                                              size_t sbn, size_t sbk)
{
    const uint32_t n = blockIdx.x * 16 + (threadIdx.x & 15);
    const uint32_t m = blockIdx.y * 16 + (threadIdx.x >> 4);
    if(m >= p.m || n >= p.n) return;
    int32_t acc = 0;
    for(uint32_t k = 0; k < p.k; ++k)
        acc += (int32_t)p.a[m * sam + k * sak] * (int32_t)p.b[n * sbn + k * sbk];
    if constexpr(OUT == W8A8_OUT_I32) {
        reinterpret_cast<int32_t*>(p.c)[(size_t)m * p.ldc + n] = acc;
    } else {
        float f = (float)acc;
        if(p.sa == nullptr && p.sb == nullptr)
            f = f * (p.tsa * p.tsb);
        else
            f = (f * (p.sa ? p.sa[m] : p.tsa)) * (p.sb ? p.sb[n] : p.tsb);
        reinterpret_cast<uint16_t*>(p.c)[(size_t)m * p.ldc + n] = float_to_half_bits(f);
    }
}

__global__ void __launch_bounds__(256) transpose_i8_kernel(const int8_t* src, uint32_t lds_src,
                                                           int8_t* dst, uint32_t ldd,
                                                           uint32_t rows, uint32_t cols)
{
    // dst[r, c] = src[c * lds_src + r]; tile 64x64 through LDS
    __shared__ int8_t tile[64][65];
    const uint32_t r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    for(int i = threadIdx.x; i < 64 * 64; i += 256) {
        const uint32_t cc = c0 + i / 64, rr = r0 + i % 64;
        tile[i / 64][i % 64] = (cc < cols && rr < rows) ? src[(size_t)cc * lds_src + rr] : 0;
    }
    __syncthreads();
    for(int i = threadIdx.x; i < 64 * 64; i += 256) {
        const uint32_t rr = r0 + i / 64, cc = c0 + i % 64;
        if(rr < rows && cc < ldd) dst[(size_t)rr * ldd + cc] = tile[i % 64][i / 64];
    }
}

KArgs make_kargs(const GemmArgs& g)
{
    return KArgs{g.a,   g.b,   g.c,   g.scale_a, g.scale_b, g.m,   g.n,
                 g.k,   g.lda, g.ldb, g.ldc,     g.tsa,     g.tsb};
}

} // namespace

bool gemm_fast_path_ok(const GemmArgs& g)
{
    return (reinterpret_cast<uintptr_t>(g.a) % 16 == 0)
           && (reinterpret_cast<uintptr_t>(g.b) % 16 == 0) && (g.lda % 16 == 0)
           && (g.ldb % 16 == 0) && (g.k % 16 == 0);
}

hipError_t launch_gemm_nk(const GemmArgs& g, hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    const KArgs    p       = make_kargs(g);
    const uint32_t tiles   = ((g.m + kBM - 1) / kBM) * ((g.n + kBN - 1) / kBN);
    const size_t   esz     = g.out_type == W8A8_OUT_I32 ? 4 : 2;
    const int      vec_ok  = (reinterpret_cast<uintptr_t>(g.c) % (4 * esz) == 0)
                       && (g.ldc % 4 == 0)
                       && (g.scale_b == nullptr || reinterpret_cast<uintptr_t>(g.scale_b) % 16 == 0);
    // Dynamic LDS above 64 KiB: raise the per-kernel limit once (best effort;
    // the launch reports an error if the device cannot provide it).
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_nk_kernel<W8A8_OUT_I32>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_nk_kernel<W8A8_OUT_F16>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    });
    if(g.out_type == W8A8_OUT_I32)
        hipLaunchKernelGGL(gemm_i8_nk_kernel<W8A8_OUT_I32>, dim3(tiles), dim3(kThreads),
                           kLdsBytes, stream, p, vec_ok);
    else
        hipLaunchKernelGGL(gemm_i8_nk_kernel<W8A8_OUT_F16>, dim3(tiles), dim3(kThreads),
                           kLdsBytes, stream, p, vec_ok);
    return hipGetLastError();
}

hipError_t launch_gemm_generic(const GemmArgs& g, size_t sam, size_t sak, size_t sbn, size_t sbk,
                               hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    const KArgs p = make_kargs(g);
    dim3        grid((g.n + 15) / 16, (g.m + 15) / 16);
    if(g.out_type == W8A8_OUT_I32)
        hipLaunchKernelGGL(gemm_i8_generic_kernel<W8A8_OUT_I32>, grid, dim3(256), 0, stream, p,
                           sam, sak, sbn, sbk);
    else
        hipLaunchKernelGGL(gemm_i8_generic_kernel<W8A8_OUT_F16>, grid, dim3(256), 0, stream, p,
                           sam, sak, sbn, sbk);
    return hipGetLastError();
}

hipError_t launch_transpose_i8(const int8_t* src, uint32_t lds_src, int8_t* dst, uint32_t ldd,
                               uint32_t rows, uint32_t cols, hipStream_t stream)
{
    dim3 grid((rows + 63) / 64, (ldd + 63) / 64);
    hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, stream, src, lds_src, dst, ldd,
                       rows, cols);
    return hipGetLastError();
}

} // namespace w8a8
