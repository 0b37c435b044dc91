// gemm_i8_decode_wide_kernel.hpp -- decode GEMM for 32 < M <= 64 over packed
// weights, with the activation tile shared through LDS and split-K across
// blocks into a caller workspace.
//
// Why a second decode kernel: in gemm_i8_decode_kernel every block reads the
// whole A (M x its K range) for only NT*32 weight rows, so at M = 64 the A
// re-reads equal or exceed the weight bytes and the register ring for both
// operands caps the waves per CU.  Here
//   * a block covers WV*32 weight rows (each wave a 32-row half slab of the
//     packed layout, streamed into a RING-deep register ring), and its waves
//     share each 64 x 128 A k-tile, loaded once per block into an LDS ring by
//     LDS-DMA buffer loads (8 KiB per k-tile in 1 KiB wave-loads over the waves) and read back
//     as MFMA fragments (16-byte chunks XOR-swizzled by row: conflict-free);
//   * blockIdx.y splits K; each split writes its int32 partial tile to the
//     workspace [split][M][ldw] with plain stores, and decode_reduce_kernel
//     sums the splits in split order and runs the dequant epilogue (integer
//     sums: exact, so the result equals the unsplit GEMM bit for bit).  With
//     one split the kernel runs the epilogue itself.
// One barrier per k-tile keeps the A ring consistent: at iteration t every
// wave has finished reading stage t-1, which the refill then overwrites.
#pragma once

#include "gemm_i8_pb_kernel.hpp"

namespace w8a8 {
namespace gemm {

template <int WV_, int RING_>
struct DecWideCfg {
    static constexpr int kMT         = 2;                // 64 A rows
    static constexpr int kWaves      = WV_;              // weight half-slabs per block
    static constexpr int kRing       = RING_;            // W ring = A stages (prefetch RING-1)
    static constexpr int kThreads    = kWaves * kWave;
    static constexpr int kRows       = kWaves * 32;      // weight rows per block
    static constexpr int kAStage     = kMT * 32 * kPackK; // 8 KiB
    static constexpr int kLdsBytes   = kRing * kAStage;
    static constexpr int kALoads     = kAStage / 1024 / kWaves; // A wave-loads per wave
    static constexpr int kOpsPerTile = 4 + kALoads;              // W frags + A wave-loads
    static_assert(kWaves % 2 == 0, "whole 64-row slabs per block");
    static_assert(kALoads >= 1 && kAStage / 1024 % kWaves == 0,
                  "A k-tile splits into whole wave-loads per wave");
    static_assert(kRing >= 2 && kRing <= 4, "ring depth");
    static_assert(kOpsPerTile * (kRing - 1) < 64, "vmcnt range");
};

// OUT = W8A8_OUT_I32 / W8A8_OUT_F16: the final output (one split).  PARTIAL:
// int32 partials to ws + split * m * ldw.
constexpr int kOutPartial = 2;

template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads) gemm_i8_decode_wide_kernel(KArgs p, int vec_ok,
                                                                          int32_t* ws,
                                                                          uint32_t ldw,
                                                                          uint32_t per)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    const int      wave  = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int      lane  = threadIdx.x % kWave;
    const uint32_t nbase = blockIdx.x * C::kRows + wave * 32; // this wave's first weight row
    const uint32_t nkt   = packed_ktiles(p.k);
    const uint32_t kt0   = min(nkt, blockIdx.y * per);
    const uint32_t kt1   = min(nkt, kt0 + per);

    // packed weights: half slab (nbase/64, (nbase%64)/32), fragment g of k-tile
    // kt at slab*nkt*8 KiB + kt*8 KiB + nt*4 KiB + g*1 KiB + lane*16
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.b), 0, (int)packed_bytes(p.n, p.k), kBufferFlags);
    const uint32_t vb = nbase < p.n ? (nbase / kSlab) * nkt * (kPackFrags * 1024)
                                          + ((nbase % kSlab) / 32) * 4096 + lane * 16
                                    : kOob;
    // A k-tile -> LDS: wave-load j (= wave * kALoads + i) fills rows 8j ..
    // 8j+7, lane l writes physical chunk l%8 of row 8j + l/8, i.e. fetches
    // logical chunk (l%8) ^ swz(row)
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.a), 0, (int)((p.m - 1) * p.lda + p.k), kBufferFlags);
    uint32_t achunk[C::kALoads], va[C::kALoads];
#pragma unroll
    for(int i = 0; i < C::kALoads; ++i) {
        const uint32_t arow = (wave * C::kALoads + i) * 8 + lane / 8;
        achunk[i]           = (lane % 8) ^ ((arow >> 1) & 7);
        va[i]               = arow < p.m ? arow * p.lda + achunk[i] * 16 : kOob;
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

    using WTile = v4i[4];
    WTile bq[C::kRing];
    // k-tiles outside [kt0, kt1) read at kOob: zeros, no memory traffic, and
    // every wave keeps the same count of loads in flight
    auto issue = [&](int slot, uint32_t kt) {
        const bool     live = kt < kt1;
        const uint32_t vbb  = live ? vb : kOob;
        const uint32_t kofs = live ? kt * (kPackFrags * 1024) : 0u;
#pragma unroll
        for(int g = 0; g < 4; ++g)
            bq[slot][g] = __builtin_amdgcn_raw_buffer_load_b128(rb, vbb, kofs + g * 1024,
                                                                kDecodeWeightPolicy);
#pragma unroll
        for(int i = 0; i < C::kALoads; ++i) {
            const uint32_t kk = kt * kPackK + achunk[i] * 16;
            const uint32_t v  = (live && va[i] != kOob && kk < p.k) ? va[i] + kt * kPackK : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_void_t*)(uintptr_t)(lds0 + slot * C::kAStage + (wave * C::kALoads + i) * 1024),
                16, v, 0, 0, 0);
        }
    };

    v16i acc[C::kMT];
#pragma unroll
    for(int i = 0; i < C::kMT; ++i) acc[i] = v16i{0};

    // A fragment (i, g) for lane l: row i*32 + l%32, logical chunk 2g + l/32
    const int frow = lane & 31;
    const int fswz = (frow >> 1) & 7;
    auto compute = [&](int slot) {
        const int8_t* st = lds + slot * C::kAStage;
#pragma unroll
        for(int g = 0; g < 4; ++g)
#pragma unroll
            for(int i = 0; i < C::kMT; ++i) {
                const int chunk = (2 * g + (lane >> 5)) ^ fswz;
                const v4i af = *reinterpret_cast<const v4i*>(st + (i * 32 + frow) * kPackK + chunk * 16);
                acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bq[slot][g], af, acc[i], 0, 0, 0);
            }
    };

    // ---- stream [kt0, kt1) ----------------------------------------------------
#pragma unroll
    for(int d = 0; d + 1 < C::kRing; ++d) issue(d, kt0 + d);
    auto step = [&](int slot, uint32_t kt) {
        wait_vmcnt<C::kOpsPerTile * (C::kRing - 2)>(); // k-tile kt landed (this wave)
        block_barrier(); // ... and every wave's A part; stage slot-1 is read by all
        issue((slot + C::kRing - 1) % C::kRing, kt + C::kRing - 1);
        compute(slot);
    };
    for(uint32_t kt = kt0; kt < kt1; kt += C::kRing) {
#pragma unroll
        for(int d = 0; d < C::kRing; ++d)
            if(kt + d < kt1) step(d, kt + d); // uniform
    }
    wait_vmcnt<0>(); // no global->LDS write may outlive the workgroup's LDS

    // ---- output ------------------------------------------------------------------
    // acc[i][r]: m = i*32 + lane%32, n = nbase + (r/4)*8 + (lane/32)*4 + r%4
    const bool  mode1 = (p.sa == nullptr && p.sb == nullptr);
    const float ab    = p.tsa * p.tsb;
#pragma unroll
    for(int i = 0; i < C::kMT; ++i) {
        const uint32_t m = i * 32 + (lane & 31);
        if(m >= p.m) continue;
        float sa = p.tsa;
        if(OUT == W8A8_OUT_F16 && p.sa != nullptr) sa = p.sa[m];
#pragma unroll
        for(int q = 0; q < 4; ++q) {
            const uint32_t n = nbase + q * 8 + (lane >> 5) * 4;
            if(n >= p.n) continue;
            const int v[4] = {acc[i][q * 4 + 0], acc[i][q * 4 + 1], acc[i][q * 4 + 2],
                              acc[i][q * 4 + 3]};
            if constexpr(OUT == kOutPartial) {
                // ldw % 4 == 0 and n % 4 == 0: one 16-byte store, in bounds
                int32_t* dst = ws + ((size_t)blockIdx.y * p.m + m) * ldw + n;
                *reinterpret_cast<int4*>(dst) = make_int4(v[0], v[1], v[2], v[3]);
            } else {
                float4 sb = make_float4(p.tsb, p.tsb, p.tsb, p.tsb);
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
                store4<OUT>(p, m, n, v, sa, sb, ab, mode1, vec_ok != 0);
            }
        }
    }
}

// Sum the splits of each 4-wide run of n (in split order) and run the epilogue.
template <int OUT>
__global__ void __launch_bounds__(256) decode_reduce_kernel(KArgs p, int vec_ok,
                                                            const int32_t* __restrict__ ws,
                                                            uint32_t ldw, uint32_t splits)
{
    const uint32_t runs = ldw / 4;
    const size_t   idx  = blockIdx.x * (size_t)256 + threadIdx.x;
    if(idx >= (size_t)p.m * runs) return;
    const uint32_t m = idx / runs;
    const uint32_t n = (idx % runs) * 4;
    if(n >= p.n) return;
    int4 s = make_int4(0, 0, 0, 0);
    for(uint32_t z = 0; z < splits; ++z) {
        const int4 v = *reinterpret_cast<const int4*>(ws + ((size_t)z * p.m + m) * ldw + n);
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
    }
    const bool  mode1 = (p.sa == nullptr && p.sb == nullptr);
    const float ab    = p.tsa * p.tsb;
    float       sa    = p.tsa;
    if(OUT == W8A8_OUT_F16 && p.sa != nullptr) sa = p.sa[m];
    float4 sb = make_float4(p.tsb, p.tsb, p.tsb, p.tsb);
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
    const int v[4] = {s.x, s.y, s.z, s.w};
    store4<OUT>(p, m, n, v, sa, sb, ab, mode1, vec_ok != 0);
}

// Workspace row stride (int32) and bytes for `splits` K splits of an m x n GEMM.
inline uint32_t decode_ws_ld(uint32_t n) { return (n + 3) / 4 * 4; }
inline size_t   decode_ws_bytes(uint32_t m, uint32_t n, uint32_t splits)
{
    return splits > 1 ? (size_t)splits * m * decode_ws_ld(n) * sizeof(int32_t) : 0;
}

// Preconditions (checked by the caller): packed weights, 32 < m <= 64,
// 16-byte aligned A with lda % 16 == 0, k % 16 == 0, (m-1)*lda + k < 2^31,
// packed_bytes(n, k) < 2^31; ws holds decode_ws_bytes(m, n, splits).
template <class C>
hipError_t launch_decode_wide(const KArgs& p, int out_type, int vec_ok, int32_t* ws,
                              uint32_t splits, hipStream_t stream)
{
    const uint32_t nkt  = packed_ktiles(p.k);
    const uint32_t per  = (nkt + splits - 1) / splits;
    splits              = (nkt + per - 1) / per; // no empty split
    const dim3     grid((p.n + C::kRows - 1) / C::kRows, splits);
    const uint32_t ldw  = decode_ws_ld(p.n);
    if(splits == 1) {
        if(out_type == W8A8_OUT_I32)
            hipLaunchKernelGGL((gemm_i8_decode_wide_kernel<C, W8A8_OUT_I32>), grid,
                               dim3(C::kThreads), C::kLdsBytes, stream, p, vec_ok, ws, ldw, per);
        else
            hipLaunchKernelGGL((gemm_i8_decode_wide_kernel<C, W8A8_OUT_F16>), grid,
                               dim3(C::kThreads), C::kLdsBytes, stream, p, vec_ok, ws, ldw, per);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((gemm_i8_decode_wide_kernel<C, kOutPartial>), grid, dim3(C::kThreads),
                       C::kLdsBytes, stream, p, vec_ok, ws, ldw, per);
    hipError_t e = hipGetLastError();
    if(e != hipSuccess) return e;
    const size_t items  = (size_t)p.m * (ldw / 4);
    const dim3   rgrid((uint32_t)((items + 255) / 256));
    if(out_type == W8A8_OUT_I32)
        hipLaunchKernelGGL((decode_reduce_kernel<W8A8_OUT_I32>), rgrid, dim3(256), 0, stream, p,
                           vec_ok, ws, ldw, splits);
    else
        hipLaunchKernelGGL((decode_reduce_kernel<W8A8_OUT_F16>), rgrid, dim3(256), 0, stream, p,
                           vec_ok, ws, ldw, splits);
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
