// gemm_i8_kernel.hpp -- int8 x int8 -> int32 GEMM tile kernel for gfx950 with a
// fused per-token x per-channel dequant epilogue, templated on the tile shape.
//
// Computation (gemm_quant_tensor_scale, rocwmma_gemm_quantized.cpp:127-195, in
// its documented Mode 2, :18-26):
//   acc[m,n] = sum_k A[m,k] * B[n,k]                 (int32, exact)
//   C[m,n]   = half((float(acc) * sa[m]) * sb[n])    or the int32 acc itself
// A is [M,K] row-major, B is [N,K] K-contiguous (both operands K-major).
//
// Tile hierarchy (Cfg): block BM x BN x BK, WAVES_M x WAVES_N waves, each wave
// owning a (BM/WAVES_M) x (BN/WAVES_N) tile of 16 x 16 v_mfma_i32_16x16x64_i8
// blocks (or 32 x 32 v_mfma_i32_32x32x32_i8 ones, Cfg's MFMA_ parameter).
// The MFMA is issued with srcA = B fragment (rows n) and srcB = A fragment
// (rows m): D[i=n][j=m], so each lane owns one m and runs of 4 consecutive n
// (Acc<C>'s quads) and the epilogue writes 4 fp16 (8 B) or 4 int32 (16 B)
// per store.
//
// Data movement
//   * global -> LDS with global_load_lds_dwordx4 (no VGPR staging): one wave
//     instruction fills 1 KiB of LDS, lane i writing bytes [16i, 16i+16); the
//     LDS layout is chosen by which global 16-byte chunk each lane fetches.
//   * An LDS row holds the BK bytes of one m (or n); with C = BK/16 chunks per
//     row, chunk c of row r is stored at chunk c ^ ((r >> log2(16/C)) & (C-1)).
//     The 16 lanes of each ds_read_b128 quarter-wave (16 consecutive rows, same
//     logical chunk) then hit 16 distinct 16-byte bank groups: conflict-free.
//   * STAGES-deep ring: tiles t+1..t+STAGES-1 are in flight while t computes.
//     One barrier per BK-deep tile, placed before the last MFMA k-group so
//     LDS fragment reads always overlap MFMA work (FragPipe).
//   * Loads are raw buffer loads into LDS: per-lane offsets are fixed, the
//     tile's k offset is the uniform soffset, and out-of-range rows / k-chunks
//     use an offset past the buffer, which reads as zeros; edges need no
//     masking in the main loop (K must be a multiple of 16).
//   * Block order: hardware block ids go round-robin over the 8 XCDs; they are
//     remapped so each XCD owns a contiguous run of tiles (shared A/B panels
//     stay in one L2), grouped GROUP_M tile-rows at a time.
//   * fp16 epilogue: the dequantized tile goes through the idle LDS ring so
//     that every lane stores 16 contiguous bytes and a wave store fills whole
//     128-byte lines (epilogue_f16_lds); storing straight from the MFMA
//     layout spreads each wave store over 32 lines and cost 6-13% of the
//     GEMM time at the Llama projection shapes.
#pragma once

#include "../../include/w8a8.h"
#include "w8a8_device.hpp"

#include <mutex>
#include <type_traits>

namespace w8a8 {

namespace gemm {

// MFMA_: the matrix instruction of the tile body, 32 for v_mfma_i32_32x32x32_i8
// or 16 for v_mfma_i32_16x16x64_i8.  Both retire the same int8 ops per cycle
// and read the same LDS bytes per op for a given wave tile; on MI355X under
// the power limit the 16 x 16 x 64 form sustains ~14% more ops on random
// operands (3.60 against 3.16 POP/s in a loop fed from LDS like the tile
// body; plausibly because it reads and writes half the accumulator bytes per
// op).
template <int BM_, int BN_, int BK_, int STAGES_, int WAVES_M_, int WAVES_N_, int GROUP_M_ = 8,
          int MFMA_ = 32>
struct Cfg {
    static constexpr int kBM      = BM_;
    static constexpr int kBN      = BN_;
    static constexpr int kBK      = BK_;
    static constexpr int kStages  = STAGES_;
    static constexpr int kWavesM  = WAVES_M_;
    static constexpr int kWavesN  = WAVES_N_;
    static constexpr int kGroupM  = GROUP_M_;
    static constexpr int kWaves   = kWavesM * kWavesN;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kWaveM   = kBM / kWavesM;
    static constexpr int kWaveN   = kBN / kWavesN;
    static constexpr int kMfma    = MFMA_;
    static constexpr int kTilesM  = kWaveM / kMfma;      // MFMA blocks per wave tile
    static constexpr int kTilesN  = kWaveN / kMfma;
    static constexpr int kChunks  = kBK / 16;           // 16-byte chunks per LDS row
    static constexpr int kSwzShift = kChunks == 8 ? 1 : (kChunks == 4 ? 2 : 3);
    static constexpr int kRowsPerLoad = kWave / kChunks; // rows one wave-load fills
    static constexpr int kABytes  = kBM * kBK;
    static constexpr int kBBytes  = kBN * kBK;
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int kLdsBytes   = kStages * kStageBytes;
    static constexpr int kLoadsA  = kABytes / 1024 / kWaves; // wave-loads per wave per stage
    static constexpr int kLoadsB  = kBBytes / 1024 / kWaves;
    static constexpr int kLoads   = kLoadsA + kLoadsB;
    static constexpr int kMfmaK   = kMfma == 32 ? 32 : 64; // depth of one MFMA
    static constexpr int kSubK    = kBK / kMfmaK;        // MFMA k-groups per tile

    static_assert(kChunks == 2 || kChunks == 4 || kChunks == 8, "BK in {32, 64, 128}");
    // the fragment slots alternate by k-group parity within a k-tile, and the
    // first group of every k-tile uses slot 0
    static_assert(kSubK % 2 == 0, "fragment ping-pong needs an even k-group count per k-tile");
    static_assert(kLoadsA * kWaves * 1024 == kABytes && kLoadsB * kWaves * 1024 == kBBytes,
                  "tile bytes must split evenly into 1 KiB wave-loads");
    static_assert(kMfma == 32 || kMfma == 16, "32x32x32 or 16x16x64 MFMA");
    static_assert(kBK % kMfmaK == 0, "whole MFMA k-groups per tile");
    static_assert(kWaveM % 32 == 0 && kWaveN % 32 == 0, "wave tile of whole 32-row passes");
    static_assert(kStages >= 2, "at least double buffering");
    static_assert(kLoads * (kStages - 1) < 64, "vmcnt counter range");
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 LDS per workgroup");
};

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

typedef __attribute__((address_space(3))) void lds_void_t;

// sched_group_barrier instruction classes
constexpr int kSchedMfma   = 0x008;
constexpr int kSchedVmemRd = 0x020;
constexpr int kSchedDsRead = 0x100;

// Buffer resource word 3 for gfx9 raw buffers (32-bit data format, no swizzle)
// and the byte offset that lies past every operand (operands stay < 2 GiB).
constexpr int      kBufferFlags = 0x00020000;
constexpr uint32_t kOob         = 0x80000000u;

// Hardware dispatches block ids round-robin over the 8 XCDs.  Return the
// logical tile id such that each XCD owns a contiguous range of logical ids.
__host__ __device__ inline uint32_t xcd_remap(uint32_t bid, uint32_t total)
{
    constexpr uint32_t kXcd = 8;
    const uint32_t     q    = total / kXcd;
    const uint32_t     r    = total % kXcd;
    const uint32_t     x    = bid % kXcd;
    const uint32_t     i    = bid / kXcd;
    return x * q + (x < r ? x : r) + i;
}

template <int GROUP_M>
__host__ __device__ inline void tile_coords(uint32_t lid, uint32_t tiles_m, uint32_t tiles_n,
                                            uint32_t& tm, uint32_t& tn)
{
    const uint32_t per_group = GROUP_M * tiles_n;
    const uint32_t group     = lid / per_group;
    const uint32_t first_m   = group * GROUP_M;
    const uint32_t gsize     = tiles_m - first_m < (uint32_t)GROUP_M ? tiles_m - first_m : GROUP_M;
    const uint32_t in_group  = lid % per_group;
    tm                       = first_m + in_group % gsize;
    tn                       = in_group / gsize;
}

// Barrier between the waves of a block without the release/acquire fences of
// __syncthreads() (those wait for every outstanding global->LDS load, vmcnt(0),
// and would serialize the prefetch ring).  LDS hazards are covered by the
// explicit s_waitcnt calls placed before each barrier.
__device__ __forceinline__ void block_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One MFMA k-group (32 x 32 x 32 form): MFMAs and the DS reads of the next
// fragments alternate, then the remaining MFMAs follow.  The first MFMA stays
// ahead of the reads so it waits only on fragments read one group earlier.
template <int NMFMA, int NDS, int ID>
__device__ __forceinline__ void interleave_mfma_ds()
{
    constexpr int kPairs = NDS < NMFMA ? NDS : NMFMA;
#pragma unroll
    for(int i = 0; i < kPairs; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, ID);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, ID);
    }
    if constexpr(NMFMA > kPairs)
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, NMFMA - kPairs, ID);
    if constexpr(NDS > kPairs)
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, NDS - kPairs, ID);
}

// The group after the barrier also issues the refill of the freed stage:
// steps of (one MFMA, its share of global->LDS loads, its share of DS reads),
// then the remaining MFMAs.
template <int I, int STEPS, int NVMEM, int NDS, int ID>
__device__ __forceinline__ void interleave_step()
{
    if constexpr(I < STEPS) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, ID);
        constexpr int nv = (I + 1) * NVMEM / STEPS - I * NVMEM / STEPS;
        constexpr int nd = (I + 1) * NDS / STEPS - I * NDS / STEPS;
        if constexpr(nv > 0) __builtin_amdgcn_sched_group_barrier(kSchedVmemRd, nv, ID);
        if constexpr(nd > 0) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, nd, ID);
        interleave_step<I + 1, STEPS, NVMEM, NDS, ID>();
    }
}

template <int NMFMA, int NVMEM, int NDS, int ID>
__device__ __forceinline__ void interleave_mfma_vmem_ds()
{
    constexpr int kSteps = NMFMA;
    interleave_step<0, kSteps, NVMEM, NDS, ID>();
}

// One 16 x 16 x 64 k-group (FragPipe): per outer fragment, its INNER MFMAs,
// then the read of its next fragment (and of one next inner fragment in the
// first INNER of them) and its share of NVMEM global -> LDS loads.
template <int I, int OUTER, int INNER, int NVMEM, int ID>
__device__ __forceinline__ void interleave_rows16()
{
    if constexpr(I < OUTER) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, INNER, ID);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, I < INNER ? 2 : 1, ID);
        constexpr int nv = (I + 1) * NVMEM / OUTER - I * NVMEM / OUTER;
        if constexpr(nv > 0) __builtin_amdgcn_sched_group_barrier(kSchedVmemRd, nv, ID);
        interleave_rows16<I + 1, OUTER, INNER, NVMEM, ID>();
    }
}

// The int32 accumulators of one wave tile, in the lane layout of the tile's
// MFMA (srcA = B fragment, srcB = A fragment, so D[n][m]).  Epilogues see
// them as quads: 4 outputs of one row m at 4 consecutive columns n, quad
// (qm, qn) at wave-tile row row(qm) and first column col(qn):
//   MFMA 32: r[i][j] is the 32 x 32 block (i, j); quad (qm, qn) is
//     r[qm][qn / 4][4 (qn % 4) ...], m = 32 qm + lane % 32,
//     n = 32 (qn / 4) + 8 (qn % 4) + 4 (lane / 32);
//   MFMA 16: r[i][j] is the 16 x 16 block (i, j) and quad (i, j) itself,
//     m = 16 qm + lane % 16, n = 16 qn + 4 (lane / 16).
// Quads are numbered q = qm * kQuadsN + qn (the K-split partial layout).
template <class C>
struct Acc {
    static constexpr bool kBig    = C::kMfma == 32;
    static constexpr int  kQuadsM = C::kTilesM;
    static constexpr int  kQuadsN = kBig ? C::kTilesN * 4 : C::kTilesN;
    static constexpr int  kQuads  = kQuadsM * kQuadsN;
    using Block                   = std::conditional_t<kBig, v16i, v4i>;
    Block r[C::kTilesM][C::kTilesN];

    __device__ static __forceinline__ int row(int qm, int lane)
    {
        return kBig ? qm * 32 + (lane & 31) : qm * 16 + (lane & 15);
    }
    __device__ static __forceinline__ int col(int qn, int lane)
    {
        return kBig ? (qn >> 2) * 32 + (qn & 3) * 8 + (lane >> 5) * 4 : qn * 16 + (lane >> 4) * 4;
    }
    __device__ __forceinline__ void zero()
    {
#pragma unroll
        for(int i = 0; i < C::kTilesM; ++i)
#pragma unroll
            for(int j = 0; j < C::kTilesN; ++j) r[i][j] = Block{0};
    }
    __device__ __forceinline__ v4i quad(int qm, int qn) const
    {
        if constexpr(kBig) {
            const v16i& b = r[qm][qn >> 2];
            const int   o = (qn & 3) * 4;
            return v4i{b[o], b[o + 1], b[o + 2], b[o + 3]};
        } else {
            return r[qm][qn];
        }
    }
    __device__ __forceinline__ void add(int qm, int qn, const v4i& v)
    {
        if constexpr(kBig) {
            v16i&     b = r[qm][qn >> 2];
            const int o = (qn & 3) * 4;
            b[o] += v.x, b[o + 1] += v.y, b[o + 2] += v.z, b[o + 3] += v.w;
        } else {
            r[qm][qn] += v;
        }
    }
    // r += the products of one k-group's fragments
    __device__ __forceinline__ void mfma(const v4i (&af)[C::kTilesM], const v4i (&bf)[C::kTilesN])
    {
#pragma unroll
        for(int i = 0; i < C::kTilesM; ++i)
#pragma unroll
            for(int j = 0; j < C::kTilesN; ++j) {
                if constexpr(kBig)
                    r[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], r[i][j], 0, 0, 0);
                else
                    r[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], r[i][j], 0, 0, 0);
            }
    }
};

// LDS -> register fragments of one k-group.  Fragment t of A covers wave-tile
// rows [t kMfma, (t + 1) kMfma): lane l reads row t kMfma + l % kMfma, 16
// bytes at k-chunk (kMfmaK / 16) g + l / kMfma of the k-tile, i.e. the
// chunk it was swizzled to (same rule as the loads).  B alike.  Both
// operands use the same lane -> k mapping, so the sum over k is the full dot
// product whatever order the MFMA reduces it in.  The row's swizzle bits lie
// below bit 4, so they come from the lane alone.
template <class C>
struct FragReader {
    using FragA = v4i[C::kTilesM];
    using FragB = v4i[C::kTilesN];
    int offa, offb;       // byte offsets of fragment 0 within a stage
    int cofs[C::kSubK];   // byte offset of each k-group's chunk

    __device__ __forceinline__ FragReader(int wm, int wn, int lane)
    {
        const int frow = lane % C::kMfma;
        const int fswz = (frow >> C::kSwzShift) & (C::kChunks - 1);
        offa           = (wm * C::kWaveM + frow) * C::kBK;
        offb           = C::kABytes + (wn * C::kWaveN + frow) * C::kBK;
        constexpr int kPerG = C::kMfmaK / 16; // 16-byte k-chunks per lane group and k-group
#pragma unroll
        for(int g = 0; g < C::kSubK; ++g)
            cofs[g] = ((kPerG * g + lane / C::kMfma) ^ fswz) * 16;
    }
    __device__ __forceinline__ v4i a(const int8_t* sbase, int g, int t) const
    {
        return *reinterpret_cast<const v4i*>(sbase + offa + t * C::kMfma * C::kBK + cofs[g]);
    }
    __device__ __forceinline__ v4i b(const int8_t* sbase, int g, int t) const
    {
        return *reinterpret_cast<const v4i*>(sbase + offb + t * C::kMfma * C::kBK + cofs[g]);
    }
    __device__ __forceinline__ void load(const int8_t* sbase, int g, FragA& af, FragB& bf) const
    {
#pragma unroll
        for(int t = 0; t < C::kTilesM; ++t) af[t] = a(sbase, g, t);
#pragma unroll
        for(int t = 0; t < C::kTilesN; ++t) bf[t] = b(sbase, g, t);
    }
};

// The k-loop's fragment registers, and one k-group of MFMAs with the reads of
// the next k-group's fragments interleaved.  Slot s = k-group parity (even
// kSubK, so k-group g of every k-tile uses slot g & 1).
//   MFMA 32: two full fragment sets; a group reads the next into the other.
//   MFMA 16: the operand with more fragments per wave tile is the outer one
//     (A unless the wave tile is wider than tall): one register set, the next
//     group's outer fragment t read into fragment t's registers right after
//     its MFMAs have issued, (outer - 1) x inner MFMAs before its first use;
//     the inner fragments ping-pong, next inner fragment t read after outer
//     fragment t (the earliest slots, so they have the most time to land
//     before the next group starts).  A 128 x 64 wave tile holds 64 fragment
//     VGPRs instead of 96, which keeps its loop within 256 VGPRs.
// NVMEM: global -> LDS loads issued just before, spread over the group.
template <class C>
struct FragPipe {
    static constexpr bool kBig       = C::kMfma == 32;
    static constexpr bool kRowsOuter = C::kTilesM >= C::kTilesN;
    static constexpr int  kOuter     = kRowsOuter ? C::kTilesM : C::kTilesN;
    static constexpr int  kInner     = kRowsOuter ? C::kTilesN : C::kTilesM;
    static constexpr int  kMfmaN     = C::kTilesM * C::kTilesN;
    static constexpr int  kDs        = C::kTilesM + C::kTilesN;
    FragReader<C> fr;
    // MFMA 32 registers
    v4i fa[kBig ? 2 : 1][kBig ? C::kTilesM : 1];
    v4i fb[kBig ? 2 : 1][kBig ? C::kTilesN : 1];
    // MFMA 16 registers
    v4i fo[kBig ? 1 : kOuter];
    v4i fi[kBig ? 1 : 2][kBig ? 1 : kInner];

    __device__ __forceinline__ FragPipe(int wm, int wn, int lane) : fr(wm, wn, lane) {}

    __device__ __forceinline__ v4i outer(const int8_t* sbase, int g, int t) const
    {
        return kRowsOuter ? fr.a(sbase, g, t) : fr.b(sbase, g, t);
    }
    __device__ __forceinline__ v4i inner(const int8_t* sbase, int g, int t) const
    {
        return kRowsOuter ? fr.b(sbase, g, t) : fr.a(sbase, g, t);
    }
    // the 16 x 16 x 64 MFMAs of outer fragment o with inner set s
    __device__ __forceinline__ void mfma_outer(Acc<C>& acc, int s, int o)
    {
#pragma unroll
        for(int x = 0; x < kInner; ++x) {
            const int i = kRowsOuter ? o : x, j = kRowsOuter ? x : o;
            const v4i& a = kRowsOuter ? fo[o] : fi[s][x];
            const v4i& b = kRowsOuter ? fi[s][x] : fo[o];
            acc.r[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, a, acc.r[i][j], 0, 0, 0);
        }
    }

    __device__ __forceinline__ void first(const int8_t* sbase)
    {
        if constexpr(kBig) {
            fr.load(sbase, 0, fa[0], fb[0]);
        } else {
#pragma unroll
            for(int t = 0; t < kOuter; ++t) fo[t] = outer(sbase, 0, t);
#pragma unroll
            for(int t = 0; t < kInner; ++t) fi[0][t] = inner(sbase, 0, t);
        }
    }

    template <int NVMEM>
    __device__ __forceinline__ void step(Acc<C>& acc, int s, const int8_t* sbase_n, int g_n)
    {
        if constexpr(kBig) {
            fr.load(sbase_n, g_n, fa[s ^ 1], fb[s ^ 1]);
            acc.mfma(fa[s], fb[s]);
            if constexpr(NVMEM > 0)
                interleave_mfma_vmem_ds<kMfmaN, NVMEM, kDs, 1>();
            else
                interleave_mfma_ds<kMfmaN, kDs, 0>();
        } else {
#pragma unroll
            for(int o = 0; o < kOuter; ++o) {
                mfma_outer(acc, s, o);
                fo[o] = outer(sbase_n, g_n, o);
                if(o < kInner) fi[s ^ 1][o] = inner(sbase_n, g_n, o);
            }
            interleave_rows16<0, kOuter, kInner, NVMEM, (NVMEM > 0 ? 1 : 0)>();
        }
    }
    // a k-group with no fragments to read next: MFMAs only, with the NVMEM
    // global -> LDS loads issued just before spread over them
    template <int NVMEM = 0>
    __device__ __forceinline__ void last(Acc<C>& acc, int s)
    {
        if constexpr(kBig) {
            acc.mfma(fa[s], fb[s]);
        } else {
#pragma unroll
            for(int o = 0; o < kOuter; ++o) mfma_outer(acc, s, o);
        }
        if constexpr(NVMEM > 0) interleave_mfma_vmem_ds<kMfmaN, NVMEM, 0, 1>();
    }
};

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
            h[e]    = float_to_half_bits_2step(f);
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

// Dequant scales of one lane's outputs in a wave tile (quad layout of
// Acc<C>): sa[qm] for the lane's row in each quad row, sb[qn] for each run
// of 4 columns.  Tensor-scale mode (no scale vectors) folds tsa * tsb into sa
// and sets sb to 1, which is exact, so every output is (acc * sa) * sb.  On
// tiles that lie inside the matrix the loads are unconditional: they all go
// out back to back and the epilogue waits for them once (per-group guarded
// loads each waited for their own result and serialized eight memory
// latencies).
template <class C>
struct EpiScales {
    using A = Acc<C>;
    float  sa[A::kQuadsM];
    float4 sb[A::kQuadsN];

    __device__ __forceinline__ void load(const KArgs& p, uint32_t m0, uint32_t n0, int wm, int wn,
                                         int lane, int vec_ok)
    {
        const uint32_t mb = m0 + wm * C::kWaveM;
        const uint32_t nb = n0 + wn * C::kWaveN;
        if(p.sa == nullptr && p.sb == nullptr) {
            const float ab = p.tsa * p.tsb;
#pragma unroll
            for(int i = 0; i < A::kQuadsM; ++i) sa[i] = ab;
#pragma unroll
            for(int j = 0; j < A::kQuadsN; ++j) sb[j] = make_float4(1.f, 1.f, 1.f, 1.f);
            return;
        }
        if(p.sa == nullptr) {
#pragma unroll
            for(int i = 0; i < A::kQuadsM; ++i) sa[i] = p.tsa;
        } else if(m0 + C::kBM <= p.m) {
#pragma unroll
            for(int i = 0; i < A::kQuadsM; ++i) sa[i] = p.sa[mb + A::row(i, lane)];
        } else {
#pragma unroll
            for(int i = 0; i < A::kQuadsM; ++i) {
                const uint32_t m = mb + A::row(i, lane);
                sa[i]            = m < p.m ? p.sa[m] : p.tsa;
            }
        }
        if(p.sb == nullptr) {
#pragma unroll
            for(int j = 0; j < A::kQuadsN; ++j) sb[j] = make_float4(p.tsb, p.tsb, p.tsb, p.tsb);
        } else if(vec_ok && n0 + C::kBN <= p.n) {
#pragma unroll
            for(int j = 0; j < A::kQuadsN; ++j)
                sb[j] = *reinterpret_cast<const float4*>(p.sb + nb + A::col(j, lane));
        } else {
#pragma unroll
            for(int j = 0; j < A::kQuadsN; ++j) {
                const uint32_t n = nb + A::col(j, lane);
                float4         v = make_float4(p.tsb, p.tsb, p.tsb, p.tsb);
                if(n + 0 < p.n) v.x = p.sb[n + 0];
                if(n + 1 < p.n) v.y = p.sb[n + 1];
                if(n + 2 < p.n) v.z = p.sb[n + 2];
                if(n + 3 < p.n) v.w = p.sb[n + 3];
                sb[j] = v;
            }
        }
    }
};

// fp16 epilogue through LDS.  The MFMA result layout gives each lane runs of 4
// consecutive n in 32 different rows, so storing straight from registers
// scatters every wave store over 32 cache lines in 16-byte pieces.  Instead
// each wave dequantizes its kWaveM x kWaveN tile into its own slice of the
// (now idle) LDS ring, rows of kWaveN fp16 with 16-byte chunks XOR-swizzled
// by row, then reads it back row-contiguous: every lane stores 16 bytes and
// a wave store covers whole 128-byte lines of 64 // (kWaveN / 8) rows.
// fp16 output rows staged in LDS as rows of kRowChunks 16-byte chunks (8
// columns each).  In the MFMA layout lane (row, half = lane >> 5) holds
// columns [4 * half, 4 * half + 4) of a chunk and writes them as 8 bytes; the
// read-back takes whole chunks.  An 8-byte write is served per half-wave (32
// rows, one half) over 32 banks = 128 bytes, so the chunk is XOR-swizzled with
// the row bits above the rows that share a 128-byte window and the half flips
// with row bit 3: the 32 writes then fill each of the window's 16 8-byte slots
// twice, with no conflict cycles.  The read-back reads each chunk as its two
// halves, each from where it was put.
template <int kRowChunks>
struct StageSwz {
    static_assert(kRowChunks == 4 || kRowChunks == 8 || kRowChunks == 16, "row of 4-16 chunks");
    static constexpr int kSwz   = kRowChunks < 8 ? kRowChunks : 8;
    static constexpr int kShift = kRowChunks == 4 ? 1 : 0; // 64-byte rows: two per window
    __device__ static __forceinline__ int  chunk(int ch, int row) { return ch ^ ((row >> kShift) & (kSwz - 1)); }
    __device__ static __forceinline__ int  half(int h, int row) { return h ^ ((row >> 3) & 1); }
};

template <class C>
__device__ __forceinline__ void epilogue_f16_lds(const KArgs& p, uint32_t m0, uint32_t n0,
                                                 int vec_ok, int8_t* lds, int slot, int lane,
                                                 int wm, int wn, const Acc<C>& acc,
                                                 const EpiScales<C>& sc)
{
    constexpr int kRowBytes  = C::kWaveN * 2;
    constexpr int kRowChunks = kRowBytes / 16;
    constexpr int kRowsPerSt = kWave / kRowChunks; // rows one wave store covers
    static_assert(kRowChunks == 4 || kRowChunks == 8 || kRowChunks == 16, "row of 4-16 chunks");
    static_assert(C::kWaves * C::kWaveM * kRowBytes <= C::kLdsBytes, "staging fits the ring");
    using S = StageSwz<kRowChunks>;

    // every wave's fragment reads and LDS loads are done: the ring is free
    block_barrier();
    int8_t* stage = lds + slot * (C::kWaveM * kRowBytes);
    using A       = Acc<C>;
#pragma unroll
    for(int i = 0; i < A::kQuadsM; ++i) {
        const int row = A::row(i, lane);
#pragma unroll
        for(int j = 0; j < A::kQuadsN; ++j) {
            const int    col    = A::col(j, lane);
            const v4i    v      = acc.quad(i, j);
            const float4 sb     = sc.sb[j];
            const int    vv[4]  = {v.x, v.y, v.z, v.w};
            const float  sbv[4] = {sb.x, sb.y, sb.z, sb.w};
            float        f[4];
#pragma unroll
            for(int e = 0; e < 4; ++e) f[e] = ((float)vv[e] * sc.sa[i]) * sbv[e];
            // two roundings (fp32 product, then fp16), as the reference's
            // float epilogue does: never one fused mixed-precision multiply
            const int phys = S::chunk(col >> 3, row);
            v2i       pk;
            pk.x = (int)float2_to_half2_bits_2step(f[0], f[1]);
            pk.y = (int)float2_to_half2_bits_2step(f[2], f[3]);
            *reinterpret_cast<v2i*>(stage + row * kRowBytes + phys * 16
                                    + S::half((col >> 2) & 1, row) * 8) = pk;
        }
    }
    // a wave reads back only what it wrote itself: LDS returns each wave's
    // accesses in order, so no barrier is needed between the two phases
    const bool     st16  = vec_ok && (reinterpret_cast<uintptr_t>(p.c) % 16 == 0) && (p.ldc % 8 == 0);
    const int      chunk = lane % kRowChunks;
    const uint32_t n     = n0 + wn * C::kWaveN + chunk * 8;
    // a tile wholly inside C with 16-byte rows: every store is a whole chunk
    const bool     inner = st16 && m0 + C::kBM <= p.m && n0 + C::kBN <= p.n;
    constexpr int  kSt   = C::kWaveM / kRowsPerSt; // stores per lane
    constexpr int  kBat  = kSt < 4 ? kSt : 4;
    static_assert(kSt % kBat == 0, "whole batches");
#pragma unroll
    for(int q0 = 0; q0 < kSt; q0 += kBat) {
        // a batch of reads before its stores; each 16-byte chunk in one
        // ds_read_b128, its halves swapped back where the writes swapped them
        // (free when row bit 3 is fixed per read, as with 8-chunk rows; a
        // select per dword otherwise).  Two 8-byte reads per chunk instead
        // hit the same half of each chunk from four rows of a half-wave: 256
        // LDS bank-conflict cycles per 128 x 128 tile.
        v4i out[kBat];
#pragma unroll
        for(int b = 0; b < kBat; ++b) {
            const int     row = (q0 + b) * kRowsPerSt + lane / kRowChunks;
            const int8_t* src = stage + row * kRowBytes + S::chunk(chunk, row) * 16;
            const v4i     v   = *reinterpret_cast<const v4i*>(src);
            out[b]            = S::half(0, row) ? v4i{v.z, v.w, v.x, v.y} : v;
        }
#pragma unroll
        for(int b = 0; b < kBat; ++b) {
            const uint32_t m   = m0 + wm * C::kWaveM + (q0 + b) * kRowsPerSt + lane / kRowChunks;
            const v4i      v   = out[b];
            uint16_t*      dst = reinterpret_cast<uint16_t*>(p.c) + (size_t)m * p.ldc + n;
            if(inner) {
                *reinterpret_cast<v4i*>(dst) = v;
                continue;
            }
            if(m >= p.m || n >= p.n) continue;
            if(st16 && n + 8 <= p.n) {
                *reinterpret_cast<v4i*>(dst) = v;
            } else {
                const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
                for(int e = 0; e < 8; ++e)
                    if(n + e < p.n) dst[e] = (uint16_t)(w[e / 2] >> (16 * (e % 2)));
            }
        }
    }
}

// int32 accumulators of one tile as a K-split partial: quad q of thread t
// (Acc<C> numbering, 4 ints) at ints (q * kThreads + t) * 4, so every store
// and load of a quad is contiguous.
template <class C>
struct Partial {
    static constexpr int    kBlocks = Acc<C>::kQuads;
    static constexpr size_t kInts   = (size_t)kBlocks * C::kThreads * 4;
    static constexpr size_t kBytes  = kInts * 4;
    // fixup blocks of kFixupWaves waves: the tile's epilogue in kPieces blocks
    static constexpr int    kFixupWaves = 2;
    static constexpr int    kPieces     = C::kWaves / kFixupWaves;
    static constexpr int    kFixupLds   = kFixupWaves * C::kWaveM * C::kWaveN * 2;
    static_assert(C::kWaves % kFixupWaves == 0, "whole fixup blocks");
};

// K pieces of a split tile: at most kMaxParts, each at least kMinKtPerPart
// k-tiles (shorter pieces do not repay the partial traffic).
constexpr uint32_t kMaxParts     = 8;
constexpr uint32_t kMinKtPerPart = 16;

template <class C>
__device__ __forceinline__ void store_partial(int32_t* part, const Acc<C>& acc)
{
    using A = Acc<C>;
#pragma unroll
    for(int i = 0; i < A::kQuadsM; ++i)
#pragma unroll
        for(int j = 0; j < A::kQuadsN; ++j) {
            const int q = i * A::kQuadsN + j;
            *reinterpret_cast<v4i*>(part + ((size_t)q * C::kThreads + threadIdx.x) * 4)
                = acc.quad(i, j);
        }
}

// acc += one partial, for thread `tid` of the tile's layout.  The loads go out
// in batches of kBatch into a register array before any add, so a thread
// keeps kBatch loads in flight.
template <class C>
__device__ __forceinline__ void add_partial(const int32_t* part, uint32_t tid, Acc<C>& acc)
{
    using A              = Acc<C>;
    constexpr int kBatch = A::kQuads < 16 ? A::kQuads : 16;
    static_assert(A::kQuads % kBatch == 0, "whole batches");
#pragma unroll
    for(int b = 0; b < A::kQuads; b += kBatch) {
        v4i v[kBatch];
#pragma unroll
        for(int x = 0; x < kBatch; ++x)
            v[x] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(
                part + ((size_t)(b + x) * C::kThreads + tid) * 4));
        __builtin_amdgcn_sched_barrier(0); // every load of the batch issued before the adds
#pragma unroll
        for(int x = 0; x < kBatch; ++x)
            acc.add((b + x) / A::kQuadsN, (b + x) % A::kQuadsN, v[x]);
    }
}

template <class C, int OUT>
__device__ __forceinline__ void tile_epilogue_sc(const KArgs& p, uint32_t m0, uint32_t n0,
                                                 int vec_ok, int8_t* lds,
                                                 const Acc<C>& acc, int wave_base,
                                                 const EpiScales<C>& sc);

// The int32 accumulators of one BM x BN output tile at (m0, n0) of problem
// p over k-tiles [kt0, kt0 + nk) (nk >= 1), computed by the whole block;
// `lds` is the block's kLdsBytes ring, free again when this returns.
// SCALES: the fp16 epilogue's scales go into `sc` while the last k-tile's
// MFMAs run.
template <class C, bool SCALES>
__device__ __forceinline__ void gemm_tile_acc(const KArgs& p, uint32_t m0, uint32_t n0,
                                              int vec_ok, int8_t* lds, uint32_t kt0,
                                              uint32_t nk, Acc<C>& acc, EpiScales<C>& sc)
{
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform
    const int lane = threadIdx.x % kWave;
    const int wm   = wave / C::kWavesN;
    const int wn   = wave % C::kWavesN;

    // ---- global -> LDS load descriptors -----------------------------------
    // Wave-load j of the A (or B) tile fills rows kRowsPerLoad*j ... ; lane l
    // covers row kRowsPerLoad*j + l / kChunks at physical chunk l % kChunks and
    // therefore fetches logical chunk (l % kChunks) ^ swizzle(row).
    // Loads are raw buffer loads: the per-lane byte offset is fixed for the
    // whole K loop, the tile's k offset travels in the uniform soffset, and a
    // row past the matrix gets offset kOob, which the buffer range check turns
    // into zeros (the host keeps each operand under 2 GiB).
    const int lrow = lane / C::kChunks;
    uint32_t  va[C::kLoadsA], vb[C::kLoadsB]; // per-lane byte offsets (k0 excluded)
    int       cha[C::kLoadsA], chb[C::kLoadsB];
#pragma unroll
    for(int i = 0; i < C::kLoadsA; ++i) {
        const uint32_t r = (wave * C::kLoadsA + i) * C::kRowsPerLoad + lrow;
        cha[i]           = (lane % C::kChunks) ^ ((r >> C::kSwzShift) & (C::kChunks - 1));
        va[i]            = (m0 + r) < p.m ? (m0 + r) * p.lda + cha[i] * 16 : kOob;
    }
#pragma unroll
    for(int i = 0; i < C::kLoadsB; ++i) {
        const uint32_t r = (wave * C::kLoadsB + i) * C::kRowsPerLoad + lrow;
        chb[i]           = (lane % C::kChunks) ^ ((r >> C::kSwzShift) & (C::kChunks - 1));
        vb[i]            = (n0 + r) < p.n ? (n0 + r) * p.ldb + chb[i] * 16 : kOob;
    }
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.a), 0, (int)(p.m * p.lda), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.b), 0, (int)(p.n * p.ldb), kBufferFlags);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds; // LDS byte address of the ring

    auto issue_stage = [&](int stage, uint32_t kt) {
        const uint32_t k0     = (kt0 + kt) * C::kBK;
        const bool     full_k = k0 + C::kBK <= p.k; // uniform: only a K tail is partial
        const uint32_t sbase  = lds0 + stage * C::kStageBytes + wave * (C::kLoadsA * 1024);
        const uint32_t sbaseb = lds0 + stage * C::kStageBytes + C::kABytes
                                + wave * (C::kLoadsB * 1024);
#pragma unroll
        for(int i = 0; i < C::kLoadsA; ++i) {
            const uint32_t v = (full_k || k0 + cha[i] * 16 < p.k) ? va[i] : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_void_t*)(uintptr_t)(sbase + i * 1024), 16, v, k0, 0, 0);
        }
#pragma unroll
        for(int i = 0; i < C::kLoadsB; ++i) {
            const uint32_t v = (full_k || k0 + chb[i] * 16 < p.k) ? vb[i] : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (lds_void_t*)(uintptr_t)(sbaseb + i * 1024), 16, v, k0, 0, 0);
        }
    };

    // ---- LDS -> register fragments (FragPipe) --------------------------------
    FragPipe<C> fp(wm, wn, lane);
    acc.zero();

    // ---- prologue: fill every stage of the ring ----------------------------
    // Tiles past K are still issued (every lane then reads kOob: zeros, no
    // memory traffic), so each wave always has the same loads in flight and
    // every wait below is a compile-time count.
#pragma unroll
    for(int s = 0; s < C::kStages; ++s) issue_stage(s, s);
    wait_vmcnt<C::kLoads * (C::kStages - 1)>(); // tile 0 landed
    block_barrier();
    fp.first(lds);

    // ---- main loop (the last tile is peeled: one path for the waitcnt pass) -
    // Per tile kt: k-groups 0..S-2 read the next group's fragments as they
    // go; then [all reads of stage kt done, tile kt+1 landed] barrier; the
    // last group refills stage kt with tile kt+S and reads tile kt+1 group 0.
    for(uint32_t kt = 0; kt + 1 < nk; ++kt) {
        const int8_t* sbase = lds + (kt % C::kStages) * C::kStageBytes;
#pragma unroll
        for(int g = 0; g + 1 < C::kSubK; ++g) fp.template step<0>(acc, g & 1, sbase, g + 1);
        constexpr int gl = C::kSubK - 1;
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0(); // this wave's reads of stage kt are done before it is refilled
        wait_vmcnt<C::kLoads * (C::kStages - 2)>(); // tile kt+1 landed
        block_barrier();
        issue_stage(kt % C::kStages, kt + C::kStages);
        fp.template step<C::kLoads>(acc, gl & 1, lds + ((kt + 1) % C::kStages) * C::kStageBytes,
                                    0);
    }
    // the fp16 epilogue's scales load while the last tile's MFMAs run
    if constexpr(SCALES) sc.load(p, m0, n0, wm, wn, lane, vec_ok);
    {
        const int8_t* sbase = lds + ((nk - 1) % C::kStages) * C::kStageBytes;
#pragma unroll
        for(int g = 0; g + 1 < C::kSubK; ++g) fp.template step<0>(acc, g & 1, sbase, g + 1);
        fp.last(acc, (C::kSubK - 1) & 1);
    }
    wait_vmcnt<0>(); // no global->LDS write may outlive the workgroup's LDS
}

// One BM x BN output tile at (m0, n0) of problem p, computed by the whole
// block; `lds` is the block's kLdsBytes ring.  Shared by the plain, grouped
// and MoE kernels, which differ only in how a block finds its tile.
// PART: only k-tiles [kt0, kt0 + nkt) are summed and the int32 accumulators
// go to `part` (store_partial layout) instead of through the epilogue.
template <class C, int OUT, bool PART = false>
__device__ __forceinline__ void gemm_tile(const KArgs& p, uint32_t m0, uint32_t n0, int vec_ok,
                                          int8_t* lds, uint32_t kt0 = 0, uint32_t nkt = 0,
                                          int32_t* part = nullptr)
{
    Acc<C>       acc;
    EpiScales<C> sc;
    if constexpr(PART) {
        gemm_tile_acc<C, false>(p, m0, n0, vec_ok, lds, kt0, nkt, acc, sc);
        store_partial<C>(part, acc);
    } else {
        gemm_tile_acc<C, OUT == W8A8_OUT_F16>(p, m0, n0, vec_ok, lds, 0,
                                              (p.k + C::kBK - 1) / C::kBK, acc, sc);
        tile_epilogue_sc<C, OUT>(p, m0, n0, vec_ok, lds, acc, 0, sc);
    }
}

// Quad (qm, qn) of a wave's Acc<C> holds outputs m = m0 + wm*kWaveM +
// row(qm), n = n0 + wn*kWaveN + col(qn) + 0..3.
// A block may hold only waves wave_base, wave_base + 1, ... of the tile (the
// split-tile fixup); each wave stages through LDS slice threadIdx.x / 64.
// sc: the fp16 path's scales, loaded by the caller (unused for int32 output).
template <class C, int OUT>
__device__ __forceinline__ void tile_epilogue_sc(const KArgs& p, uint32_t m0, uint32_t n0,
                                                 int vec_ok, int8_t* lds, const Acc<C>& acc,
                                                 int wave_base, const EpiScales<C>& sc)
{
    const int   slot  = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int   wave  = wave_base + slot;
    const int   lane  = threadIdx.x % kWave;
    const int   wm    = wave / C::kWavesN;
    const int   wn    = wave % C::kWavesN;
    const bool  mode1 = (p.sa == nullptr && p.sb == nullptr);
    const float ab    = p.tsa * p.tsb;
    if constexpr(OUT == W8A8_OUT_F16) {
        epilogue_f16_lds<C>(p, m0, n0, vec_ok, lds, slot, lane, wm, wn, acc, sc);
        return;
    }
    // int32 output: straight from the registers
    using A = Acc<C>;
#pragma unroll
    for(int i = 0; i < A::kQuadsM; ++i) {
        const uint32_t m = m0 + wm * C::kWaveM + A::row(i, lane);
#pragma unroll
        for(int j = 0; j < A::kQuadsN; ++j) {
            const uint32_t n    = n0 + wn * C::kWaveN + A::col(j, lane);
            const v4i      q    = acc.quad(i, j);
            const int      v[4] = {q.x, q.y, q.z, q.w};
            store4<OUT>(p, m, n, v, p.tsa, make_float4(p.tsb, p.tsb, p.tsb, p.tsb), ab, mode1,
                        vec_ok != 0);
        }
    }
}

// Epilogue of a tile whose scales are not loaded yet (K-split fixups,
// grouped and MoE fixups): one batch of scale loads, then the epilogue.
template <class C, int OUT>
__device__ __forceinline__ void tile_epilogue(const KArgs& p, uint32_t m0, uint32_t n0,
                                              int vec_ok, int8_t* lds, const Acc<C>& acc,
                                              int wave_base = 0)
{
    EpiScales<C> sc;
    if constexpr(OUT == W8A8_OUT_F16) {
        const int wave = wave_base + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
        sc.load(p, m0, n0, wave / C::kWavesN, wave % C::kWavesN, threadIdx.x % kWave, vec_ok);
    }
    tile_epilogue_sc<C, OUT>(p, m0, n0, vec_ok, lds, acc, wave_base, sc);
}

template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads, 1) gemm_i8_tile_kernel(KArgs p, int vec_ok)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const uint32_t tiles_m = (p.m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n = (p.n + C::kBN - 1) / C::kBN;
    uint32_t       tm, tn;
    tile_coords<C::kGroupM>(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
    gemm_tile<C, OUT>(p, tm * C::kBM, tn * C::kBN, vec_ok, lds);
}

// K split of a launch whose tiles fill at most half of the CUs: logical
// block b runs piece b % parts of tile b / parts (k-tiles [part * nk / parts,
// (part + 1) * nk / parts)) and stores its int32 accumulators to
// ws + b * Partial<C>::kInts; gemm_i8_split_fixup_kernel then sums each
// tile's pieces in order (exact) and runs the tile epilogue, in kPieces
// blocks of kFixupWaves waves per tile.  Logical ids are contiguous per XCD
// (xcd_remap): the tiles of one XCD share their B panels in its L2, so each
// weight panel comes from HBM once (with hardware ids the GROUP_M tiles of a
// panel sat on different XCDs and each fetched it: M=512 K=14336 N=4096 read
// the weights four times).
template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads, 1)
    gemm_i8_split_kernel(KArgs p, int vec_ok, int32_t* ws, uint32_t parts)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const uint32_t tiles_m = (p.m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n = (p.n + C::kBN - 1) / C::kBN;
    const uint32_t lid  = xcd_remap(blockIdx.x, gridDim.x);
    const uint32_t slot = lid / parts, part = lid % parts;
    uint32_t       tm, tn;
    tile_coords<C::kGroupM>(slot, tiles_m, tiles_n, tm, tn);
    const uint32_t nk  = (p.k + C::kBK - 1) / C::kBK;
    const uint32_t kt0 = part * nk / parts, kt1 = (part + 1) * nk / parts;
    gemm_tile<C, OUT, true>(p, tm * C::kBM, tn * C::kBN, vec_ok, lds, kt0, kt1 - kt0,
                            ws + (size_t)lid * Partial<C>::kInts);
}

template <class C, int OUT>
__global__ void __launch_bounds__(Partial<C>::kFixupWaves * kWave, 1)
    gemm_i8_split_fixup_kernel(KArgs p, int vec_ok, const int32_t* ws, uint32_t parts)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const uint32_t tiles_m   = (p.m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n   = (p.n + C::kBN - 1) / C::kBN;
    const uint32_t slot      = blockIdx.x / Partial<C>::kPieces;
    const int      wave_base = (int)(blockIdx.x % Partial<C>::kPieces) * Partial<C>::kFixupWaves;
    uint32_t       tm, tn;
    tile_coords<C::kGroupM>(slot, tiles_m, tiles_n, tm, tn);
    Acc<C> acc;
    acc.zero();
    const uint32_t tid = wave_base * kWave + threadIdx.x;
    for(uint32_t part = 0; part < parts; ++part)
        add_partial<C>(ws + (size_t)(slot * parts + part) * Partial<C>::kInts, tid, acc);
    tile_epilogue<C, OUT>(p, tm * C::kBM, tn * C::kBN, vec_ok, lds, acc, wave_base);
}

template <class C, int OUT>
void raise_lds_limit_once()
{
    // Dynamic LDS above 64 KiB: raise the per-kernel limit once per kernel
    // (best effort; the launch itself reports an error if it cannot be met).
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_tile_kernel<C, OUT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
        (void)hipGetLastError();
    });
}

template <class C, int OUT>
void raise_split_lds_once()
{
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_split_kernel<C, OUT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
        (void)hipGetLastError();
    });
}

// Launch one configuration; the caller has validated the fast-path
// preconditions (16-byte aligned a/b, lda/ldb/k multiples of 16).
template <class C>
hipError_t launch_cfg(const KArgs& p, int out_type, int vec_ok, hipStream_t stream)
{
    const uint32_t tiles = ((p.m + C::kBM - 1) / C::kBM) * ((p.n + C::kBN - 1) / C::kBN);
    if(out_type == W8A8_OUT_I32) {
        raise_lds_limit_once<C, W8A8_OUT_I32>();
        hipLaunchKernelGGL((gemm_i8_tile_kernel<C, W8A8_OUT_I32>), dim3(tiles), dim3(C::kThreads),
                           C::kLdsBytes, stream, p, vec_ok);
    } else {
        raise_lds_limit_once<C, W8A8_OUT_F16>();
        hipLaunchKernelGGL((gemm_i8_tile_kernel<C, W8A8_OUT_F16>), dim3(tiles), dim3(C::kThreads),
                           C::kLdsBytes, stream, p, vec_ok);
    }
    return hipGetLastError();
}

// Split launch (see gemm_i8_split_kernel): ws holds tiles * parts partials.
template <class C>
hipError_t launch_cfg_split(const KArgs& p, int out_type, int vec_ok, int32_t* ws,
                            uint32_t parts, hipStream_t stream)
{
    const uint32_t tiles  = ((p.m + C::kBM - 1) / C::kBM) * ((p.n + C::kBN - 1) / C::kBN);
    const dim3     grid(tiles * parts), fgrid(tiles * Partial<C>::kPieces);
    const dim3     fblock(Partial<C>::kFixupWaves * kWave);
    if(out_type == W8A8_OUT_I32) {
        raise_split_lds_once<C, W8A8_OUT_I32>();
        hipLaunchKernelGGL((gemm_i8_split_kernel<C, W8A8_OUT_I32>), grid, dim3(C::kThreads),
                           C::kLdsBytes, stream, p, vec_ok, ws, parts);
        hipLaunchKernelGGL((gemm_i8_split_fixup_kernel<C, W8A8_OUT_I32>), fgrid, fblock,
                           Partial<C>::kFixupLds, stream, p, vec_ok, ws, parts);
    } else {
        raise_split_lds_once<C, W8A8_OUT_F16>();
        hipLaunchKernelGGL((gemm_i8_split_kernel<C, W8A8_OUT_F16>), grid, dim3(C::kThreads),
                           C::kLdsBytes, stream, p, vec_ok, ws, parts);
        hipLaunchKernelGGL((gemm_i8_split_fixup_kernel<C, W8A8_OUT_F16>), fgrid, fblock,
                           Partial<C>::kFixupLds, stream, p, vec_ok, ws, parts);
    }
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
