// gemm_i8_decode_kernel.hpp -- skinny (decode) int8 GEMM for gfx950:
// M <= 64 tokens, HBM-bound weight streaming, over plain [N, K] weights or
// weights packed in MFMA register order (gemm_i8_pb_kernel.hpp).
//
// Computation: acc[m,n] = sum_k A[m,k] * W[n,k]; C = half((acc * sa[m]) * sb[n])
// (the split-K decode role of gemm_splitk_stage1 + gemm_splitk_reduce,
// rocwmma_gemm_splitk.cpp:104-201, and of streamk_gemm_kernel,
// rocwmma_streamk_gemm.cpp:86-211), with int32 partials instead of fp32 so
// the reduction is exact and order-free.
//
// Design: the weight bytes are read exactly once, so the kernel is a stream.
//   * One block per NT*32 weight rows (half or all of a 64-row packed slab);
//     its KW waves split the K range in contiguous chunks (split-K inside the
//     block: no workspace, no global atomics, no cross-XCD fences).
//   * Each wave streams its weight fragments (packed: 1 KiB contiguous per
//     buffer_load_dwordx4; plain: 32 rows x 32 bytes) into a register ring
//     RING-1 k-tiles ahead, and reads
//     the matching A fragments (M <= 64 rows, L2-resident) directly into
//     registers; rows >= M read zeros through the buffer range check.
//   * v_mfma_i32_32x32x32_i8 with A padded to 32 (MT=1) or 64 (MT=2) rows:
//     the MFMA work is far below the weight-stream time, so padding is free.
//   * The KW partial tiles meet in LDS (register order, 1 KiB per fragment);
//     wave w then sums fragments w, w+KW, ... and runs the dequant epilogue.
#pragma once

#include "gemm_i8_pb_kernel.hpp"

namespace w8a8 {
namespace gemm {

// Cache policy of the weight stream: non-temporal.  Every weight byte is read
// once per call and a layer's weights do not fit the MALL beside the rest of
// a model, so nothing is lost by not keeping them.
constexpr int kDecodeWeightPolicy = 2;

template <int MT_, int NT_, int KW_, int RING_>
struct DecCfg {
    static constexpr int kMT      = MT_;            // 32-row m tiles (1 or 2)
    static constexpr int kNT      = NT_;            // 32-row weight tiles per block (1 or 2)
    static constexpr int kKW      = KW_;            // waves per block (k split)
    static constexpr int kRing    = RING_;          // register ring depth (prefetch RING-1)
    static constexpr int kThreads = kKW * kWave;
    static constexpr int kFrags   = kMT * kNT * 4;  // v4i accumulator fragments per lane
    static constexpr int kWaveLds = kFrags * 1024;  // one wave's partial tile in LDS
    static constexpr int kLdsBytes = kKW * kWaveLds;
    static_assert(kMT == 1 || kMT == 2, "decode handles up to 64 rows per block");
    static_assert(kNT == 1 || kNT == 2, "a block covers half a slab or a whole one");
    static_assert(kRing >= 2 && kRing <= 6, "ring depth");
    static_assert(kLdsBytes <= 128 * 1024, "partials must fit in LDS");
};

// SmoothQuant of the activation rows folded into the decode kernel (m <=
// kFuseRows, packed weights): every block quantizes the rows itself into LDS
// (a few KiB, read from L2 while the block's first weight fragments are in
// flight) and block (0, 0) also writes q and the row scales.  Same
// per-element operations as the quantizer kernels (rocwmma_smoothquant.cpp:
// 58-122): p = float(x) * s; r = max|p| / qmax; inv = r > 0 ? 1 / r : 0;
// q = int8(clamp(rint(p * inv), -qmax, qmax)); the maximum does not depend
// on the order of the reduction, so q and r are bit-identical.  One row: the
// prologue grows with the rows every block quantizes, and from two rows on
// the separate quantizer launch is as fast or faster (M = 4, N = 28672,
// K = 8192: 55.0 fused against 41.9 us; with the kernel built for up to 4
// rows, M = 1 ran 8.1 / 5.0 us at 4096^2 / 1024^2 against 7.2 / 4.1 us
// built for one).
constexpr uint32_t kFuseRows = 1;
// LDS row pitch = ka + kFusePad: the fused rows' 16-byte fragment reads at one
// k offset (up to kFuseRows rows x 2 lane halves) then fall on distinct bank groups.
constexpr uint32_t kFusePad = 32;
struct FuseQ {
    const uint16_t* x;    // [m, ldx] fp16 activations (16-byte aligned rows)
    const float*    s;    // [k] smoothing scale (16-byte aligned)
    int8_t*         q;    // [m, k] quantized rows out
    float*          r;    // [m] row scales out
    uint32_t        ldx;  // ldx % 8 == 0
    uint32_t        ka;   // LDS row length: k rounded up to kPackK (zero padded)
    uint32_t        pitch; // LDS row pitch: ka + kFusePad
    float           qmax;
};

// Block-wide: quantize the m (<= kFuseRows) rows into qa (pitch fq.pitch) and
// return their row scales in rs.  red: LDS scratch of KW * kFuseRows floats.
template <class C>
__device__ __forceinline__ void fuse_quantize(const FuseQ& fq, uint32_t m, uint32_t k, int8_t* qa,
                                              float* red, float (&rs)[kFuseRows])
{
    const uint32_t tid    = threadIdx.x;
    const int      lane   = tid % kWave;
    const int      wave   = tid / kWave;
    const uint32_t chunks = k / 8;
    auto smoothed = [&](uint32_t r, uint32_t c, float (&v)[8]) {
        const v4i    raw = *reinterpret_cast<const v4i*>(fq.x + (size_t)r * fq.ldx + c * 8);
        const float4 s0  = *reinterpret_cast<const float4*>(fq.s + c * 8);
        const float4 s1  = *reinterpret_cast<const float4*>(fq.s + c * 8 + 4);
        v[0] = half_bits_to_float((uint32_t)raw.x & 0xFFFFu) * s0.x;
        v[1] = half_bits_to_float((uint32_t)raw.x >> 16) * s0.y;
        v[2] = half_bits_to_float((uint32_t)raw.y & 0xFFFFu) * s0.z;
        v[3] = half_bits_to_float((uint32_t)raw.y >> 16) * s0.w;
        v[4] = half_bits_to_float((uint32_t)raw.z & 0xFFFFu) * s1.x;
        v[5] = half_bits_to_float((uint32_t)raw.z >> 16) * s1.y;
        v[6] = half_bits_to_float((uint32_t)raw.w & 0xFFFFu) * s1.z;
        v[7] = half_bits_to_float((uint32_t)raw.w >> 16) * s1.w;
    };
    float amax[kFuseRows];
#pragma unroll
    for(uint32_t r = 0; r < kFuseRows; ++r) amax[r] = 0.f;
    for(uint32_t c = tid; c < chunks; c += C::kThreads) {
#pragma unroll
        for(uint32_t r = 0; r < kFuseRows; ++r) {
            if(r < m) {
                float v[8];
                smoothed(r, c, v);
#pragma unroll
                for(int e = 0; e < 8; ++e) amax[r] = fmaxf(amax[r], fabsf(v[e]));
            }
        }
    }
#pragma unroll
    for(uint32_t r = 0; r < kFuseRows; ++r) {
        amax[r] = wave_max(amax[r]);
        if(lane == 0) red[wave * kFuseRows + r] = amax[r];
    }
    __syncthreads();
    float inv[kFuseRows];
    const bool first_block = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
    for(uint32_t r = 0; r < kFuseRows; ++r) {
        float a = 0.f;
#pragma unroll
        for(int w = 0; w < C::kKW; ++w) a = fmaxf(a, red[w * kFuseRows + r]);
        rs[r]  = a / fq.qmax;
        inv[r] = rs[r] > 0.f ? 1.f / rs[r] : 0.f;
        if(first_block && tid == r && r < m) fq.r[r] = rs[r];
    }
    // rows of kPackK-padded chunks; the padding is zero
    for(uint32_t c = tid; c < fq.ka / 8; c += C::kThreads) {
#pragma unroll
        for(uint32_t r = 0; r < kFuseRows; ++r) {
            if(r < m) {
                v2i pk = {0, 0};
                if(c < chunks) {
                    float v[8];
                    smoothed(r, c, v);
                    pk.x = (int)cvt_pack4_i8(quant_f(v[0], inv[r], fq.qmax), quant_f(v[1], inv[r], fq.qmax),
                                             quant_f(v[2], inv[r], fq.qmax), quant_f(v[3], inv[r], fq.qmax));
                    pk.y = (int)cvt_pack4_i8(quant_f(v[4], inv[r], fq.qmax), quant_f(v[5], inv[r], fq.qmax),
                                             quant_f(v[6], inv[r], fq.qmax), quant_f(v[7], inv[r], fq.qmax));
                    if(first_block) *reinterpret_cast<v2i*>(fq.q + (size_t)r * k + c * 8) = pk;
                }
                *reinterpret_cast<v2i*>(qa + r * fq.pitch + c * 8) = pk;
            }
        }
    }
    __syncthreads();
}

// PACKED: p.b is the packed weight buffer (p.ldb unused).  Otherwise p.b is
// W [n, ldb] with K contiguous.
template <class C, int OUT, bool PACKED, bool FUSE = false>
__global__ void __launch_bounds__(C::kThreads) gemm_i8_decode_kernel(KArgs p, int vec_ok, FuseQ fq)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    const uint32_t nbase = blockIdx.x * (C::kNT * 32); // first weight row of the block
    const uint32_t mbase = blockIdx.y * (C::kMT * 32);
    const int      wave  = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int      lane  = threadIdx.x % kWave;
    const uint32_t nkt   = packed_ktiles(p.k);
    const uint32_t per   = (nkt + C::kKW - 1) / C::kKW;
    const uint32_t kt0   = min(nkt, wave * per);
    const uint32_t kt1   = min(nkt, kt0 + per);

    // ---- operands -----------------------------------------------------------
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.b), 0,
        PACKED ? (int)packed_bytes(p.n, p.k) : (int)((p.n - 1) * p.ldb + p.k), kBufferFlags);
    // packed: fragment f of k-tile kt of this block at
    //   slab*nkt*8 KiB + kt*8 KiB + ((nbase%64)/32)*4 KiB + f*1 KiB + lane*16
    // plain: fragment (j, g) for lane l: row nbase + j*32 + l%32,
    //   k = kt*128 + g*32 + (l/32)*16
    const uint32_t vb = PACKED ? (nbase / kSlab) * nkt * (kPackFrags * 1024)
                                     + ((nbase % kSlab) / 32) * 4096 + lane * 16
                               : 0u;
    uint32_t vbr[C::kNT];
#pragma unroll
    for(int j = 0; j < C::kNT; ++j) {
        const uint32_t row = nbase + j * 32 + (lane & 31);
        vbr[j]             = row < p.n ? row * p.ldb + (lane >> 5) * 16 : kOob;
    }
    // A's range ends at the last row's K-th byte (not m*lda: the caller's
    // buffer need not hold the last row's padding)
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.a), 0, (int)((p.m - 1) * p.lda + p.k), kBufferFlags);
    // A fragment (i, g) for lane l: row mbase + i*32 + l%32, k = k0 + g*32 + (l/32)*16.
    uint32_t va[C::kMT];
#pragma unroll
    for(int i = 0; i < C::kMT; ++i) {
        const uint32_t row = mbase + i * 32 + (lane & 31);
        va[i]              = row < p.m ? row * p.lda + (lane >> 5) * 16 : kOob;
    }

    using BTile = v4i[C::kNT * 4];
    using ATile = v4i[C::kMT * 4];
    BTile bq[C::kRing];
    ATile aq[C::kRing];
    // FUSE: the quantized rows in LDS after the partials area, pitch fq.pitch
    int8_t* qa = lds + C::kLdsBytes;
    auto issue_b = [&](int slot, uint32_t kt) {
        // k-tiles outside [kt0, kt1) read at kOob: zeros, no memory traffic
        const bool live = kt < kt1;
        if constexpr(PACKED) {
            const uint32_t vbb  = live ? vb : kOob;
            const uint32_t kofs = live ? kt * (kPackFrags * 1024) : 0u;
#pragma unroll
            for(int f = 0; f < C::kNT * 4; ++f)
                bq[slot][f] = __builtin_amdgcn_raw_buffer_load_b128(rb, vbb, kofs + f * 1024,
                                                                   kDecodeWeightPolicy);
        } else {
            // chunks at k >= K read zeros (k % 16 == 0, so a chunk is all in or out)
#pragma unroll
            for(int g = 0; g < 4; ++g) {
                const uint32_t kk = kt * kPackK + g * 32 + (lane >> 5) * 16;
#pragma unroll
                for(int j = 0; j < C::kNT; ++j) {
                    const uint32_t v
                        = (live && kk < p.k && vbr[j] != kOob) ? vbr[j] + kt * kPackK + g * 32 : kOob;
                    bq[slot][j * 4 + g] = __builtin_amdgcn_raw_buffer_load_b128(rb, v, 0, kDecodeWeightPolicy);
                }
            }
        }
    };
    auto issue_a = [&](int slot, uint32_t kt) {
        const bool live = kt < kt1;
        if constexpr(FUSE) {
#pragma unroll
            for(int i = 0; i < C::kMT; ++i) {
                const uint32_t row = mbase + i * 32 + (lane & 31);
                const bool     use = live && row < p.m;
                // Lanes past the last row read that row's bytes (one address,
                // a broadcast, not a bank conflict) and drop them; past kt1
                // every lane reads row 0's first bytes.  The address stays
                // inside the quantized rows whatever the lane.
                const uint32_t rowc = row < p.m ? row : p.m - 1;
                const int8_t*  src  = qa + (live ? rowc * fq.pitch + kt * kPackK : 0u) + (lane >> 5) * 16;
#pragma unroll
                for(int g = 0; g < 4; ++g) {
                    const v4i v         = *reinterpret_cast<const v4i*>(src + g * 32);
                    aq[slot][i * 4 + g] = use ? v : v4i{0};
                }
            }
            return;
        }
#pragma unroll
        for(int i = 0; i < C::kMT; ++i) {
            // The k offset goes into voffset so the range check sees it: the
            // last row's k >= K reads past the buffer and returns zeros.  For
            // other rows k >= K reads the next row's bytes, which meet zero
            // weights (packed padding or masked chunks) and add nothing.
            const uint32_t v = (live && va[i] != kOob) ? va[i] + kt * kPackK : kOob;
#pragma unroll
            for(int g = 0; g < 4; ++g)
                aq[slot][i * 4 + g] = __builtin_amdgcn_raw_buffer_load_b128(ra, v + g * 32, 0, 0);
        }
    };
    auto issue = [&](int slot, uint32_t kt) {
        issue_b(slot, kt);
        issue_a(slot, kt);
    };

    v16i acc[C::kMT][C::kNT];
#pragma unroll
    for(int i = 0; i < C::kMT; ++i)
#pragma unroll
        for(int j = 0; j < C::kNT; ++j) acc[i][j] = v16i{0};

    auto compute = [&](int slot) {
#pragma unroll
        for(int g = 0; g < 4; ++g)
#pragma unroll
            for(int i = 0; i < C::kMT; ++i)
#pragma unroll
                for(int j = 0; j < C::kNT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                        bq[slot][j * 4 + g], aq[slot][i * 4 + g], acc[i][j], 0, 0, 0);
    };

    // ---- stream the wave's k range with a RING-deep register ring ----------
    float rs[kFuseRows];
    if constexpr(FUSE) {
        // the first weight fragments load while the block quantizes A
#pragma unroll
        for(int d = 0; d + 1 < C::kRing; ++d) issue_b(d, kt0 + d);
        fuse_quantize<C>(fq, p.m, p.k, qa, reinterpret_cast<float*>(lds), rs);
#pragma unroll
        for(int d = 0; d + 1 < C::kRing; ++d) issue_a(d, kt0 + d);
    } else {
#pragma unroll
        for(int d = 0; d + 1 < C::kRing; ++d) issue(d, kt0 + d);
    }
    // slot d of a round holds k-tile kt + d; before computing it, the slot
    // freed one step earlier is refilled RING - 1 k-tiles ahead (tiles past
    // kt1 read nothing)
    uint32_t kt = kt0;
    for(; kt + C::kRing <= kt1; kt += C::kRing) {
#pragma unroll
        for(int d = 0; d < C::kRing; ++d) {
            issue((d + C::kRing - 1) % C::kRing, kt + d + C::kRing - 1);
            compute(d);
        }
    }
#pragma unroll
    for(int d = 0; d + 1 < C::kRing; ++d) {
        if(kt + d < kt1) {
            if(kt + d + C::kRing - 1 < kt1) issue((d + C::kRing - 1) % C::kRing, kt + d + C::kRing - 1);
            compute(d);
        }
    }

    // ---- reduce the KW partials through LDS --------------------------------
    int8_t* mine = lds + wave * C::kWaveLds + lane * 16;
#pragma unroll
    for(int i = 0; i < C::kMT; ++i)
#pragma unroll
        for(int j = 0; j < C::kNT; ++j)
#pragma unroll
            for(int q = 0; q < 4; ++q)
                *reinterpret_cast<v4i*>(mine + ((i * C::kNT + j) * 4 + q) * 1024)
                    = v4i{acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2],
                          acc[i][j][q * 4 + 3]};
    __syncthreads();

    const bool  mode1 = (p.sa == nullptr && p.sb == nullptr);
    const float ab    = p.tsa * p.tsb;
    for(int f = wave; f < C::kFrags; f += C::kKW) {
        v4i s = v4i{0};
        for(int w = 0; w < C::kKW; ++w)
            s += *reinterpret_cast<const v4i*>(lds + w * C::kWaveLds + f * 1024 + lane * 16);
        // fragment f = (i*NT + j)*4 + q: m = mbase + i*32 + lane%32,
        // n = nbase + j*32 + q*8 + (lane/32)*4 + [0, 4)
        const int      i  = f / (4 * C::kNT);
        const int      j  = (f / 4) % C::kNT;
        const int      q  = f % 4;
        const uint32_t m  = mbase + i * 32 + (lane & 31);
        const uint32_t n  = nbase + j * 32 + q * 8 + (lane >> 5) * 4;
        float          sa = p.tsa;
        if constexpr(FUSE) {
            // this block's own row scales (block (0, 0) may still be writing p.sa)
#pragma unroll
            for(uint32_t r = 0; r < kFuseRows; ++r)
                if(m == r) sa = rs[r];
        } else if(OUT == W8A8_OUT_F16 && p.sa != nullptr && m < p.m) {
            sa = p.sa[m];
        }
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
        const int v[4] = {s[0], s[1], s[2], s[3]};
        store4<OUT>(p, m, n, v, sa, sb, ab, mode1, vec_ok != 0);
    }
}

// Preconditions (checked by the caller): 16-byte aligned A and B with
// lda % 16 == 0, ldb % 16 == 0, k % 16 == 0; (m-1)*lda + k < 2^31; the
// weights under 2^31 bytes (packed_bytes(n, k), or (n-1)*ldb + k).
template <class C, bool PACKED>
hipError_t launch_decode(const KArgs& p, int out_type, int vec_ok, hipStream_t stream)
{
    using K32 = decltype(&gemm_i8_decode_kernel<C, W8A8_OUT_I32, PACKED>);
    const K32 kern[2] = {&gemm_i8_decode_kernel<C, W8A8_OUT_I32, PACKED>,
                         &gemm_i8_decode_kernel<C, W8A8_OUT_F16, PACKED>};
    if constexpr(C::kLdsBytes > 65536) {
        static std::once_flag once;
        std::call_once(once, [&] {
            for(auto k : kern)
                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          C::kLdsBytes);
            (void)hipGetLastError();
        });
    }
    const dim3 grid((p.n + C::kNT * 32 - 1) / (C::kNT * 32), (p.m + C::kMT * 32 - 1) / (C::kMT * 32));
    hipLaunchKernelGGL(kern[out_type == W8A8_OUT_I32 ? 0 : 1], grid, dim3(C::kThreads),
                       C::kLdsBytes, stream, p, vec_ok, FuseQ{});
    return hipGetLastError();
}

// The decode kernel with the activation quantization folded in (packed
// weights, fp16 output, p.m <= kFuseRows, C::kMT == 1).  p.sa must be fq.r.
// The host checks C::kLdsBytes + p.m * fq.pitch <= 160 KiB.
template <class C>
hipError_t launch_decode_fused(const KArgs& p, const FuseQ& fq, int vec_ok, hipStream_t stream)
{
    static_assert(C::kMT == 1, "one 32-row m tile holds the fused rows");
    const void* kern = reinterpret_cast<const void*>(
        &gemm_i8_decode_kernel<C, W8A8_OUT_F16, true, true>);
    static std::once_flag once;
    std::call_once(once, [&] {
        (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipGetLastError();
    });
    const dim3 grid((p.n + C::kNT * 32 - 1) / (C::kNT * 32), 1);
    hipLaunchKernelGGL((gemm_i8_decode_kernel<C, W8A8_OUT_F16, true, true>), grid,
                       dim3(C::kThreads), C::kLdsBytes + p.m * fq.pitch, stream, p, vec_ok, fq);
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
