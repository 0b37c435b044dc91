// gemm_i8_persist_kernel.hpp -- persistent variant of the int8 tile GEMM for
// launches of several tiles per CU with an fp16 output.
//
// Same arithmetic, operand layout, LDS ring and MFMA schedule as
// gemm_i8_tile_kernel (gemm_i8_kernel.hpp); what differs is how a CU moves
// from one tile to the next.  A one-tile-per-block launch pays, per tile, a
// workgroup launch, a cold prologue (two k-tiles fetched before any MFMA) and
// an epilogue whose stores every CU issues at the same moment.  Here:
//   * one block per CU walks a fixed list of tiles: the tiles of its XCD's
//     contiguous range, round-robin over the XCD's blocks (the same L2
//     locality as the remapped one-tile launch);
//   * the stage ring runs across tile boundaries: the last k-steps of tile j
//     already fetch tile j+1's first k-tiles, so the next tile starts with its
//     operands in LDS;
//   * the epilogue stages through its own LDS slice (32 rows per pass), not
//     the ring, which holds the next tile's operands;
//   * every wave issues exactly kStores buffer stores per tile (rows or
//     columns past the matrix use an offset past the buffer, which drops the
//     store), so the first wait of the next tile can leave those stores in
//     flight with an exact vmcnt and they drain behind its MFMAs.
// Results are bit-identical to gemm_i8_tile_kernel: the same k-order per tile
// and the same epilogue arithmetic.
#pragma once

#include "gemm_i8_kernel.hpp"

namespace w8a8 {
namespace gemm {

// Cache-policy operand of the buffer builtins: the NT (non-temporal) bit.
constexpr int kCpolNonTemporal = 2;
// MI355X's last-level cache (MALL, AMD Infinity Cache): 256 MB.
constexpr uint64_t kMallBytes = 256ull << 20;

template <class C>
struct Persist {
    static constexpr int kRowBytes    = C::kWaveN * 2;           // one staged fp16 row
    static constexpr int kRowChunks   = kRowBytes / 16;
    static constexpr int kRowsPerSt   = kWave / kRowChunks;       // rows per wave store
    static constexpr int kPassRows    = 32;                       // rows staged per pass
    static constexpr int kPasses      = C::kWaveM / kPassRows;
    static constexpr int kQmPerPass   = kPassRows / C::kMfma;     // quad rows per pass
    static constexpr int kStPerPass   = kPassRows / kRowsPerSt;
    static constexpr int kStores      = kPasses * kStPerPass;     // per wave per tile
    static constexpr int kSliceBytes  = kPassRows * kRowBytes;    // per wave
    static constexpr int kLdsBytes    = C::kLdsBytes + C::kWaves * kSliceBytes;
    static_assert(kRowChunks == 4 || kRowChunks == 8 || kRowChunks == 16, "row of 4-16 chunks");
    static_assert(kPassRows % kRowsPerSt == 0, "whole stores per pass");
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 LDS per workgroup");
    static_assert(C::kLoads * (C::kStages - 2) + kStores < 64, "vmcnt counter range");
};

// fp16 epilogue of one wave tile through the wave's LDS slice, 32 rows per
// pass; every lane issues exactly Persist<C>::kStores 16-byte stores.  The
// host guarantees N % 8 == 0, ldc % 8 == 0 and a 16-byte aligned C, so an
// 8-column chunk is either inside the matrix or entirely past it.
// NT: non-temporal stores, for outputs of at least a quarter of the MALL.
// Larger than the MALL they cannot stay resident, and
// write-allocating them leaves it full of dirty lines that the next kernel
// pays to write back (the quantizer that follows the 470 MB gate_up output of
// cfg3 runs 62 instead of 89 us).  From a quarter of it they still crowd out
// the next kernels' operands: cfg3's qkv and o_proj outputs (100 / 67 MB)
// stored this way take the step from 1.493 to 1.463-1.476 ms (same box,
// alternating).
template <class C, bool NT>
__device__ __forceinline__ void epilogue_f16_persist(const KArgs& p, __amdgpu_buffer_rsrc_t rc,
                                                     uint32_t m0, uint32_t n0, int8_t* slice,
                                                     int lane, int wm, int wn, const Acc<C>& acc,
                                                     const EpiScales<C>& sc)
{
    using P               = Persist<C>;
    using S               = StageSwz<P::kRowChunks>;
    using A               = Acc<C>;
    const int      chunk  = lane % P::kRowChunks;
    const uint32_t n      = n0 + wn * C::kWaveN + chunk * 8;
    const bool     n_in   = n < p.n;
#pragma unroll
    for(int pass = 0; pass < P::kPasses; ++pass) {
#pragma unroll
        for(int i = pass * P::kQmPerPass; i < (pass + 1) * P::kQmPerPass; ++i) {
            const int row = A::row(i, lane) - pass * P::kPassRows; // row within the slice
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
                const int phys = S::chunk(col >> 3, row);
                v2i       pk;
                pk.x = (int)float2_to_half2_bits_2step(f[0], f[1]);
                pk.y = (int)float2_to_half2_bits_2step(f[2], f[3]);
                *reinterpret_cast<v2i*>(slice + row * P::kRowBytes + phys * 16
                                        + S::half((col >> 2) & 1, row) * 8) = pk;
            }
        }
        // read the pass back row-contiguous, all its reads before its stores;
        // each 16-byte chunk in one ds_read_b128, its halves swapped back in
        // registers where the writes swapped them (S::half: row bit 3).  With
        // 8 rows per store, row bit 3 of read q is q's own low bit, a
        // compile-time fact (the lane itself is opaque here), so the swap is
        // a register renaming.  Two 8-byte reads per chunk instead (the lane
        // offset unknown to the compiler) cost 512 LDS bank-conflict cycles
        // per tile: four rows of a half-wave then hit the same half of every
        // chunk.  A wave's LDS accesses complete in order, so the next pass's
        // writes cannot overtake these reads.
        static_assert(P::kRowsPerSt == 8, "row bit 3 of a read-back row is q's low bit");
        v4i out[P::kStPerPass];
#pragma unroll
        for(int q = 0; q < P::kStPerPass; ++q) {
            const int     r   = q * P::kRowsPerSt + lane / P::kRowChunks;
            const int8_t* src = slice + r * P::kRowBytes + S::chunk(chunk, r) * 16;
            const v4i     v   = *reinterpret_cast<const v4i*>(src);
            out[q]            = (q & 1) ? v4i{v.z, v.w, v.x, v.y} : v;
        }
        // row mr + q * kRowsPerSt at byte offset off0 + q * step (in range rows
        // only: the host keeps every element offset of C below 2^31)
        const uint32_t mr   = m0 + wm * C::kWaveM + pass * P::kPassRows + lane / P::kRowChunks;
        const uint32_t off0 = (mr * p.ldc + n) * 2;
        const uint32_t step = P::kRowsPerSt * p.ldc * 2;
#pragma unroll
        for(int q = 0; q < P::kStPerPass; ++q) {
            const uint32_t off = (mr + q * P::kRowsPerSt < p.m && n_in) ? off0 + q * step : kOob;
            __builtin_amdgcn_raw_buffer_store_b128(out[q], rc, off, 0, NT ? kCpolNonTemporal : 0);
        }
    }
}

template <class C>
__global__ void __launch_bounds__(C::kThreads, 1) gemm_i8_persist_kernel(KArgs p, int vec_ok, int nt)
{
    using P = Persist<C>;
    static_assert(C::kStages >= 2, "ring");
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    // ---- this block's tiles -------------------------------------------------
    // XCD x (block ids x, x + 8, ...) owns logical tiles [start_x, end_x); its
    // per = gridDim.x / 8 blocks take them round-robin.  The host launches a
    // multiple of 8 blocks.
    const uint32_t tiles_m = (p.m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n = (p.n + C::kBN - 1) / C::kBN;
    const uint32_t total   = tiles_m * tiles_n;
    const uint32_t per     = gridDim.x / 8;
    const uint32_t x = blockIdx.x % 8, bi = blockIdx.x / 8;
    const uint32_t q = total / 8, rr = total % 8;
    const uint32_t first = x * q + min(x, rr) + bi;
    const uint32_t end   = (x + 1) * q + min(x + 1, rr);
    const uint32_t count = first < end ? (end - first + per - 1) / per : 0;
    if(count == 0) return; // whole block: no barrier is left waiting
    auto tile_of = [&](uint32_t j, uint32_t& m0, uint32_t& n0) {
        uint32_t tm, tn;
        tile_coords<C::kGroupM>(first + j * per, tiles_m, tiles_n, tm, tn);
        m0 = tm * C::kBM;
        n0 = tn * C::kBN;
    };

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int wm   = wave / C::kWavesN;
    const int wn   = wave % C::kWavesN;

    // ---- global -> LDS loads (layout as in gemm_tile) -----------------------
    // Wave-load i of the A (B) tile fills tile rows rowA(i) (rowB(i)); the
    // lane fetches logical chunk chunk_of(row) of its row.  Rows and chunks are
    // recomputed from the lane where needed (a tile change, a K tail) rather
    // than held in registers across the loop.
    const int lrow = lane / C::kChunks;
    auto rowA = [&](int i) { return (uint32_t)((wave * C::kLoadsA + i) * C::kRowsPerLoad + lrow); };
    auto rowB = [&](int i) { return (uint32_t)((wave * C::kLoadsB + i) * C::kRowsPerLoad + lrow); };
    auto chunk_of = [&](uint32_t r) {
        return (uint32_t)((lane % C::kChunks) ^ ((r >> C::kSwzShift) & (C::kChunks - 1)));
    };
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.a), 0, (int)(p.m * p.lda), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.b), 0, (int)(p.n * p.ldb), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        p.c, 0, (int)(((p.m - 1) * p.ldc + p.n) * 2), kBufferFlags);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

    // load cursor: the next k-step to fetch is k-tile lkt of tile lj; va / vb
    // hold that tile's per-lane offsets (all kOob once the list is exhausted,
    // so the ring keeps a fixed number of loads in flight to the end)
    const uint32_t nk = (p.k + C::kBK - 1) / C::kBK;
    uint32_t       lj = 0, lkt = 0;
    uint32_t       va[C::kLoadsA], vb[C::kLoadsB];
    auto set_load_tile = [&](uint32_t j) {
        uint32_t m0 = 0, n0 = 0;
        const bool live = j < count;
        if(live) tile_of(j, m0, n0);
#pragma unroll
        for(int i = 0; i < C::kLoadsA; ++i) {
            const uint32_t r = rowA(i);
            va[i] = (live && m0 + r < p.m) ? (m0 + r) * p.lda + chunk_of(r) * 16 : kOob;
        }
#pragma unroll
        for(int i = 0; i < C::kLoadsB; ++i) {
            const uint32_t r = rowB(i);
            vb[i] = (live && n0 + r < p.n) ? (n0 + r) * p.ldb + chunk_of(r) * 16 : kOob;
        }
    };
    set_load_tile(0);
    auto issue_next = [&](int stage) {
        const uint32_t k0     = lkt * C::kBK;
        const bool     full_k = k0 + C::kBK <= p.k; // uniform: only a K tail is partial
        const uint32_t sbase  = lds0 + stage * C::kStageBytes + wave * (C::kLoadsA * 1024);
        const uint32_t sbaseb = lds0 + stage * C::kStageBytes + C::kABytes
                                + wave * (C::kLoadsB * 1024);
#pragma unroll
        for(int i = 0; i < C::kLoadsA; ++i) {
            const uint32_t v = (full_k || k0 + chunk_of(rowA(i)) * 16 < p.k) ? va[i] : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_void_t*)(uintptr_t)(sbase + i * 1024), 16, v, k0, 0, 0);
        }
#pragma unroll
        for(int i = 0; i < C::kLoadsB; ++i) {
            const uint32_t v = (full_k || k0 + chunk_of(rowB(i)) * 16 < p.k) ? vb[i] : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (lds_void_t*)(uintptr_t)(sbaseb + i * 1024), 16, v, k0, 0, 0);
        }
        if(++lkt == nk) {
            lkt = 0;
            set_load_tile(++lj);
        }
    };

    // ---- LDS -> register fragments (as in gemm_tile) -------------------------
    FragPipe<C> fp(wm, wn, lane);
    Acc<C>      acc;

    int8_t* slice = lds + C::kLdsBytes + wave * P::kSliceBytes;

    // ---- prologue: the first S k-steps --------------------------------------
#pragma unroll
    for(int s = 0; s < C::kStages; ++s) issue_next(s);
    wait_vmcnt<C::kLoads * (C::kStages - 1)>();
    block_barrier();

    fp.first(lds);

    // ---- tiles ----------------------------------------------------------------
    // Every k-step: MFMA groups 0..S-2 read the next group's fragments; then
    // [this wave's reads of the stage done, the next k-step landed] barrier;
    // the freed stage is refilled with the k-step S ahead (possibly the next
    // tile's), and the last group reads the next k-step's group 0.
    uint32_t step = 0;
    // one k-step; after_epi: the previous tile's epilogue stores are the
    // youngest memory operations and may stay in flight at the wait.
    // last: the tile's last k-step, whose final k-group reads no fragments;
    // the next k-step's first ones are read after the epilogue, so they do
    // not occupy registers through it.
    auto kstep = [&](bool after_epi, auto last) {
        const int8_t* sbase = lds + (step % C::kStages) * C::kStageBytes;
#pragma unroll
        for(int g = 0; g + 1 < C::kSubK; ++g) fp.template step<0>(acc, g & 1, sbase, g + 1);
        constexpr int gl = C::kSubK - 1;
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        if(after_epi)
            wait_vmcnt<C::kLoads * (C::kStages - 2) + P::kStores>();
        else
            wait_vmcnt<C::kLoads * (C::kStages - 2)>();
        block_barrier();
        issue_next(step % C::kStages);
        if constexpr(decltype(last)::value)
            fp.template last<C::kLoads>(acc, gl & 1);
        else
            fp.template step<C::kLoads>(acc, gl & 1,
                                        lds + ((step + 1) % C::kStages) * C::kStageBytes, 0);
        ++step;
    };
    for(uint32_t j = 0; j < count; ++j) {
        uint32_t m0, n0;
        tile_of(j, m0, n0);
        acc.zero();
        for(uint32_t kt = 0; kt + 1 < nk; ++kt) kstep(kt == 0 && j > 0, std::false_type{});
        // last k-step peeled: the epilogue's scales load while it runs.  The
        // lane id is made opaque per tile so that the epilogue's per-lane
        // addresses are computed here, not hoisted out of the tile loop and
        // held in registers across the k-loop
        int elane = lane;
        asm volatile("" : "+v"(elane));
        EpiScales<C> sc;
        sc.load(p, m0, n0, wm, wn, elane, vec_ok);
        kstep(nk == 1 && j > 0, std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
        if(nt)
            epilogue_f16_persist<C, true>(p, rc, m0, n0, slice, elane, wm, wn, acc, sc);
        else
            epilogue_f16_persist<C, false>(p, rc, m0, n0, slice, elane, wm, wn, acc, sc);
        __builtin_amdgcn_sched_barrier(0);
        // the next k-step (landed at the last barrier, not refilled since)
        fp.first(lds + (step % C::kStages) * C::kStageBytes);
    }
    wait_vmcnt<0>(); // no global->LDS write may outlive the workgroup's LDS
}

template <class C>
void raise_persist_lds_once()
{
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_persist_kernel<C>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  Persist<C>::kLdsBytes);
        (void)hipGetLastError();
    });
}

// Whether the persistent kernel applies: fp16 output, several tiles per CU
// (blocks = CUs, a multiple of 8), 8-column chunks that never straddle N,
// 16-byte aligned rows of C, and C within the 32-bit buffer range.
template <class C>
bool persist_ok(const KArgs& p, int vec_ok, uint32_t cus)
{
    const uint64_t tiles = (uint64_t)((p.m + C::kBM - 1) / C::kBM) * ((p.n + C::kBN - 1) / C::kBN);
    return vec_ok && cus >= 8 && cus % 8 == 0 && tiles >= 2ull * cus && p.n % 8 == 0
           && p.ldc % 8 == 0 && reinterpret_cast<uintptr_t>(p.c) % 16 == 0
           && ((uint64_t)(p.m - 1) * p.ldc + p.n) * 2 < 0x80000000ull;
}

template <class C>
hipError_t launch_cfg_persist(const KArgs& p, int vec_ok, uint32_t cus, hipStream_t stream)
{
    raise_persist_lds_once<C>();
    const int nt = (uint64_t)p.m * p.ldc * 2 >= kMallBytes / 4;
    hipLaunchKernelGGL((gemm_i8_persist_kernel<C>), dim3(cus), dim3(C::kThreads),
                       Persist<C>::kLdsBytes, stream, p, vec_ok, nt);
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
