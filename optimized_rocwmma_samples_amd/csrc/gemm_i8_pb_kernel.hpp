// gemm_i8_pb_kernel.hpp -- int8 GEMM for gfx950 with weights pre-shuffled into
// MFMA register order ("packed B"): A streams through LDS, B streams from HBM
// straight into VGPRs.
//
// Computation: acc[m,n] = sum_k A[m,k] * W[n,k];  C = half((acc * sa[m]) * sb[n])
// (gemm_quant_tensor_scale, rocwmma_gemm_quantized.cpp:127-195, Mode 2), with
// W given in the packed layout below.  This realizes the "B bypasses LDS,
// pre-shuffled weights" design the reference describes for FlatMM
// (rocwmma_flatmm.cpp:12-16) but leaves unimplemented.
//
// Packed weight layout (produced by pack_weights_kernel, w8a8_pack_weights):
//   N is padded to a multiple of 64 (a "slab"), K to a multiple of 128 (a
//   "k-tile"), pad bytes are zero.  For slab s, k-tile t, the 8 KiB block
//   ((s * nKT + t) * 8) KiB holds 8 fragments of 1 KiB, fragment f = nt*4 + g
//   (nt = 32-row half of the slab, g = 32-deep k group).  Inside a fragment,
//   lane l = h*32 + r owns 16 bytes: row s*64 + nt*32 + r, k = t*128 + g*32 +
//   h*16 + [0, 16).  That is exactly the v_mfma_i32_32x32x32_i8 operand a wave
//   holds, so one buffer_load_dwordx4 per fragment reads 1 KiB contiguous.
//
// Tile hierarchy: block BM x 256 x 128, 4 waves side by side in N; each wave
// owns BM x 64 (BM/32 x 2 MFMA tiles).  A (BM x 128 per k-tile) goes
// global -> LDS by buffer_load ... lds into a STAGES-deep ring (swizzled as in
// gemm_i8_kernel.hpp); each wave reads all A fragments from LDS and its own B
// fragments from its private register ring, DIST k-tiles ahead.  Per CU this
// keeps (STAGES-1) A tiles + DIST B tiles in flight without spending LDS on B.
#pragma once

#include "gemm_i8_kernel.hpp"

namespace w8a8 {
namespace gemm {

constexpr int kSlab      = 64;   // packed-weight rows per slab (one wave's N extent)
constexpr int kPackK     = 128;  // packed-weight k-tile
constexpr int kPackFrags = 8;    // 1 KiB fragments per (slab, k-tile)

__host__ __device__ inline uint32_t packed_ktiles(uint32_t k) { return (k + kPackK - 1) / kPackK; }
__host__ __device__ inline uint32_t packed_slabs(uint32_t n) { return (n + kSlab - 1) / kSlab; }
__host__ __device__ inline size_t   packed_bytes(uint32_t n, uint32_t k)
{
    return (size_t)packed_slabs(n) * packed_ktiles(k) * kPackFrags * 1024;
}

// One thread per 16-byte packed chunk.
__global__ void __launch_bounds__(256) pack_weights_kernel(const int8_t* __restrict__ w,
                                                           uint32_t n, uint32_t k, uint32_t ldw,
                                                           int8_t* __restrict__ out,
                                                           size_t nchunks)
{
    const size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if(idx >= nchunks) return;
    const uint32_t nkt   = packed_ktiles(k);
    const uint32_t lane  = idx % 64;
    const uint32_t frag  = (idx / 64) % kPackFrags;
    const size_t   blk   = idx / (64 * kPackFrags); // slab * nkt + ktile
    const uint32_t kt    = blk % nkt;
    const uint32_t slab  = blk / nkt;
    const uint32_t row   = slab * kSlab + (frag / 4) * 32 + lane % 32;
    const uint32_t k0    = kt * kPackK + (frag % 4) * 32 + (lane / 32) * 16;
    int4           v     = make_int4(0, 0, 0, 0);
    if(row < n) {
        const int8_t* src = w + (size_t)row * ldw + k0;
        if(k0 + 16 <= k && (reinterpret_cast<uintptr_t>(src) % 16) == 0) {
            v = *reinterpret_cast<const int4*>(src);
        } else {
            int8_t tmp[16];
            for(int e = 0; e < 16; ++e) tmp[e] = (k0 + e < k) ? src[e] : 0;
            v = *reinterpret_cast<const int4*>(tmp);
        }
    }
    reinterpret_cast<int4*>(out)[idx] = v;
}

template <int BM_, int STAGES_, int DIST_, int GROUP_M_ = 8, int WAVES_M_ = 1>
struct PbCfg {
    static constexpr int kBM      = BM_;
    static constexpr int kBN      = 4 * kSlab; // 4 waves along N x one slab each
    static constexpr int kBK      = kPackK;
    static constexpr int kStages  = STAGES_;
    static constexpr int kDist    = DIST_;    // B prefetch distance in k-tiles
    static constexpr int kGroupM  = GROUP_M_;
    static constexpr int kWavesM  = WAVES_M_; // waves along M, BM / WAVES_M rows each
    static constexpr int kWaves   = 4 * kWavesM;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kWaveM   = kBM / kWavesM;
    static constexpr int kTilesM  = kWaveM / 32;
    static constexpr int kTilesN  = kSlab / 32; // 2
    static constexpr int kChunks  = kBK / 16;   // 8 chunks per LDS row
    static constexpr int kSwzShift = 1;         // swizzle = (row >> 1) & 7
    static constexpr int kRowsPerLoad = kWave / kChunks; // 8
    static constexpr int kStageBytes  = kBM * kBK;
    static constexpr int kLdsBytes    = kStages * kStageBytes;
    static constexpr int kLoadsA  = kStageBytes / 1024 / kWaves; // A wave-loads per stage
    static constexpr int kLoadsB  = kPackFrags;                  // B fragments per k-tile
    static constexpr int kSubK    = kBK / 32;                    // 4 MFMA groups per k-tile
    static constexpr int kRing    = kDist + 1;                   // B register buffers

    static_assert(kLoadsA * kWaves * 1024 == kStageBytes, "A tile splits into wave-loads");
    static_assert(kWaveM % 32 == 0, "wave rows made of 32-row MFMA tiles");
    static_assert(kRing == 2 || kRing == 3, "B ring depth");
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 LDS per workgroup");
    static_assert(kLoadsA * (kStages - 1) + kLoadsB * (kDist + 1) < 64, "vmcnt range");
};

template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads, 1) gemm_i8_pb_kernel(KArgs p, int vec_ok)
{
    // p.b is the packed weight buffer; p.ldb is unused (the layout is fixed).
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    const uint32_t tiles_m = (p.m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n = (p.n + C::kBN - 1) / C::kBN;
    uint32_t       tm, tn;
    tile_coords<C::kGroupM>(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * C::kBM;
    const uint32_t n0 = tn * C::kBN;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int wm   = wave / 4; // rows wm*kWaveM ...
    const int wn   = wave % 4; // slab n0/64 + wn
    const uint32_t nkt = packed_ktiles(p.k);

    // ---- A: global -> LDS (swizzled rows of 128 bytes) --------------------
    const int lrow = lane / C::kChunks;
    uint32_t  va[C::kLoadsA];
    int       cha[C::kLoadsA];
#pragma unroll
    for(int i = 0; i < C::kLoadsA; ++i) {
        const uint32_t r = (wave * C::kLoadsA + i) * C::kRowsPerLoad + lrow;
        cha[i]           = (lane % C::kChunks) ^ ((r >> C::kSwzShift) & (C::kChunks - 1));
        va[i]            = (m0 + r) < p.m ? (m0 + r) * p.lda + cha[i] * 16 : kOob;
    }
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.a), 0, (int)(p.m * p.lda), kBufferFlags);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

    auto issue_a = [&](int stage, uint32_t kt) {
        const uint32_t k0     = kt * C::kBK;
        const bool     full_k = k0 + C::kBK <= p.k;
        const uint32_t sbase  = lds0 + stage * C::kStageBytes + wave * (C::kLoadsA * 1024);
#pragma unroll
        for(int i = 0; i < C::kLoadsA; ++i) {
            const uint32_t v = (full_k || k0 + cha[i] * 16 < p.k) ? va[i] : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_void_t*)(uintptr_t)(sbase + i * 1024), 16, v, k0, 0, 0);
        }
    };

    // ---- B: packed weights -> VGPR ring ------------------------------------
    const uint32_t slab = n0 / kSlab + wn;
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.b), 0, (int)packed_bytes(p.n, p.k), kBufferFlags);
    const uint32_t vbl = slab * nkt * (kPackFrags * 1024) + lane * 16; // per-lane offset
    using BTile = v4i[C::kLoadsB];
    BTile bq[C::kRing];
    auto issue_b = [&](BTile& dst, uint32_t kt) {
        // A tile past K reads at voffset kOob: past the buffer whether or not
        // the range check includes soffset, so zeros and no memory traffic.
        const bool     live = kt < nkt;
        const uint32_t v    = live ? vbl : kOob;
        const uint32_t kofs = live ? kt * (kPackFrags * 1024) : 0u;
#pragma unroll
        for(int f = 0; f < C::kLoadsB; ++f)
            dst[f] = __builtin_amdgcn_raw_buffer_load_b128(rb, v, kofs + f * 1024, 0);
    };

    // ---- A fragments from LDS ----------------------------------------------
    const int frow = lane & 31;
    const int fswz = (frow >> C::kSwzShift) & (C::kChunks - 1);
    int       offa[C::kTilesM];
#pragma unroll
    for(int t = 0; t < C::kTilesM; ++t) offa[t] = (wm * C::kWaveM + t * 32 + frow) * C::kBK;
    int cofs[C::kSubK];
#pragma unroll
    for(int g = 0; g < C::kSubK; ++g) cofs[g] = ((2 * g + (lane >> 5)) ^ fswz) * 16;

    using FragA = v4i[C::kTilesM];
    auto load_a = [&](const int8_t* sbase, int g, FragA& af) {
#pragma unroll
        for(int t = 0; t < C::kTilesM; ++t)
            af[t] = *reinterpret_cast<const v4i*>(sbase + offa[t] + cofs[g]);
    };

    v16i acc[C::kTilesM][C::kTilesN];
#pragma unroll
    for(int i = 0; i < C::kTilesM; ++i)
#pragma unroll
        for(int j = 0; j < C::kTilesN; ++j) acc[i][j] = v16i{0};

    auto mfma_group = [&](const FragA& af, const BTile& bt, int g) {
#pragma unroll
        for(int i = 0; i < C::kTilesM; ++i)
#pragma unroll
            for(int j = 0; j < C::kTilesN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bt[j * 4 + g], af[i], acc[i][j],
                                                                  0, 0, 0);
    };
    constexpr int kMfma = C::kTilesM * C::kTilesN;

    // ---- prologue -----------------------------------------------------------
#pragma unroll
    for(int s = 0; s < C::kStages; ++s) issue_a(s, s);
#pragma unroll
    for(int d = 0; d < C::kDist; ++d) issue_b(bq[d], d);
    // A tile 0 landed: everything issued after it may stay in flight
    wait_vmcnt<C::kLoadsA * (C::kStages - 1) + C::kLoadsB * C::kDist>();
    block_barrier();

    FragA fa[2];
    load_a(lds, 0, fa[0]);

    // One k-tile: groups 0..2 read the next group's A fragments as they go;
    // then [reads of this stage done, next A tile landed] barrier; refill the
    // stage with tile kt+STAGES, prefetch B tile kt+DIST, read the next tile's
    // group-0 fragments and run the last group.  Tiles past K are issued as
    // zero loads so every count below is a constant.
    auto step = [&](uint32_t kt, BTile& bcur, BTile& bnext_slot) {
        const int8_t* sbase = lds + (kt % C::kStages) * C::kStageBytes;
#pragma unroll
        for(int g = 0; g + 1 < C::kSubK; ++g) {
            load_a(sbase, g + 1, fa[(g + 1) & 1]);
            mfma_group(fa[g & 1], bcur, g);
            interleave_mfma_ds<kMfma, C::kTilesM, 0>();
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        // A tile kt+1 landed: keep in flight at most the loads of the last
        // STAGES-2 A refills and DIST B prefetches (all issued after it).
        wait_vmcnt<C::kLoadsA * (C::kStages - 2) + C::kLoadsB * C::kDist>();
        block_barrier();
        issue_a(kt % C::kStages, kt + C::kStages);
        issue_b(bnext_slot, kt + C::kDist);
        load_a(lds + ((kt + 1) % C::kStages) * C::kStageBytes, 0, fa[0]);
        mfma_group(fa[1], bcur, C::kSubK - 1);
        interleave_mfma_vmem_ds<kMfma, C::kLoadsA + C::kLoadsB, C::kTilesM, 1>();
    };

    uint32_t kt = 0;
    if constexpr(C::kRing == 3) {
        for(; kt + 3 <= nkt; kt += 3) {
            step(kt + 0, bq[0], bq[2]);
            step(kt + 1, bq[1], bq[0]);
            step(kt + 2, bq[2], bq[1]);
        }
        if(kt < nkt) step(kt, bq[0], bq[2]);
        if(kt + 1 < nkt) step(kt + 1, bq[1], bq[0]);
    } else {
        for(; kt + 2 <= nkt; kt += 2) {
            step(kt + 0, bq[0], bq[1]);
            step(kt + 1, bq[1], bq[0]);
        }
        if(kt < nkt) step(kt, bq[0], bq[1]);
    }
    wait_vmcnt<0>(); // no global->LDS write may outlive the workgroup's LDS

    // ---- epilogue ----------------------------------------------------------
    // acc[i][j][r]: m = m0 + wm*kWaveM + i*32 + lane%32,
    //               n = n0 + wn*64 + j*32 + (r/4)*8 + (lane/32)*4 + r%4.
    const bool  mode1 = (p.sa == nullptr && p.sb == nullptr);
    const float ab    = p.tsa * p.tsb;
#pragma unroll
    for(int i = 0; i < C::kTilesM; ++i) {
        const uint32_t m  = m0 + wm * C::kWaveM + i * 32 + (lane & 31);
        float          sa = p.tsa;
        if(OUT == W8A8_OUT_F16 && p.sa != nullptr && m < p.m) sa = p.sa[m];
#pragma unroll
        for(int j = 0; j < C::kTilesN; ++j) {
#pragma unroll
            for(int g = 0; g < 4; ++g) {
                const uint32_t n  = n0 + wn * kSlab + j * 32 + g * 8 + (lane >> 5) * 4;
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

template <class C, int OUT>
void raise_lds_limit_pb_once()
{
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_pb_kernel<C, OUT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
        (void)hipGetLastError();
    });
}

// Launch one packed-weight configuration.  Preconditions (host-checked): a is
// 16-byte aligned with lda % 16 == 0, M*lda < 2^31, packed_bytes(n, k) < 2^31.
template <class C>
hipError_t launch_pb(const KArgs& p, int out_type, int vec_ok, hipStream_t stream)
{
    const uint32_t tiles = ((p.m + C::kBM - 1) / C::kBM) * ((p.n + C::kBN - 1) / C::kBN);
    if(out_type == W8A8_OUT_I32) {
        raise_lds_limit_pb_once<C, W8A8_OUT_I32>();
        hipLaunchKernelGGL((gemm_i8_pb_kernel<C, W8A8_OUT_I32>), dim3(tiles), dim3(C::kThreads),
                           C::kLdsBytes, stream, p, vec_ok);
    } else {
        raise_lds_limit_pb_once<C, W8A8_OUT_F16>();
        hipLaunchKernelGGL((gemm_i8_pb_kernel<C, W8A8_OUT_F16>), dim3(tiles), dim3(C::kThreads),
                           C::kLdsBytes, stream, p, vec_ok);
    }
    return hipGetLastError();
}

inline hipError_t launch_pack_weights(const int8_t* w, uint32_t n, uint32_t k, uint32_t ldw,
                                      int8_t* out, hipStream_t stream)
{
    const size_t chunks = packed_bytes(n, k) / 16;
    hipLaunchKernelGGL(pack_weights_kernel, dim3((chunks + 255) / 256), dim3(256), 0, stream, w,
                       n, k, ldw, out, chunks);
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
