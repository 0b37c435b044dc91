// gemm_i8_grouped_kernel.hpp -- grouped int8 GEMMs for gfx950 built on the
// tile body of gemm_i8_kernel.hpp.
//
//   * gemm_i8_grouped_kernel: G independent problems given as an array of
//     descriptors in device memory (the role of grouped_gemm_kernel and its
//     GroupDesc array, rocwmma_grouped_gemm.cpp:87-178).  The reference looks
//     up a block's group by binary search over a host-computed tile_offset
//     array (:112-122); here every wave scans the descriptors' tile counts
//     with a wave prefix sum, so no second array has to be kept in sync.
//   * gemm_i8_moe_kernel: the MoE form.  A holds the expert-sorted token rows
//     (w8a8_moe_sort order), weights are [E, N, K], and the per-expert row
//     counts and first rows live in device memory (written by the sort
//     kernel), so nothing returns to the host between routing and the GEMM.
//     The grid is sized for the worst case and surplus blocks exit at once.
// In both, a block's linear tile id goes through the XCD remap over the real
// tile count and then GROUP_M grouping inside its group.
#pragma once

#include "gemm_i8_kernel.hpp"

namespace w8a8 {
namespace gemm {

// Wave-uniform search over `count` slots with tiles(i) tiles each (0 for
// i >= count): total tile count and, for tile index `target`, the slot that
// holds it and the index of that slot's first tile.  Returns false when
// target >= total.
template <class F>
__device__ __forceinline__ bool find_slot(uint32_t count, uint32_t target, F tiles,
                                          uint32_t& slot, uint32_t& first, uint32_t& total)
{
    const int lane  = threadIdx.x % kWave;
    uint32_t  carry = 0;
    bool      found = false;
    slot = first = 0;
    for(uint32_t base = 0; base < count; base += kWave) {
        const uint32_t i = base + lane;
        const uint32_t t = i < count ? tiles(i) : 0u;
        uint32_t       s = t;
#pragma unroll
        for(int d = 1; d < kWave; d <<= 1) {
            const uint32_t o = __shfl_up(s, d, kWave);
            if(lane >= d) s += o;
        }
        const uint32_t incl = s + carry;
        if(!found) {
            const uint64_t hit = __ballot(incl > target);
            if(hit) {
                const int l = __ffsll((unsigned long long)hit) - 1;
                slot        = base + l;
                // one lane's value read by every lane: uniform, and said so
                // (a shuffle result is otherwise taken as divergent, and so is
                // everything derived from it: the tile's loads would then run
                // in readfirstlane loops)
                first       = __builtin_amdgcn_readfirstlane(__shfl(incl - t, l, kWave));
                found       = true;
            }
        }
        carry = __builtin_amdgcn_readfirstlane(__shfl(incl, kWave - 1, kWave));
    }
    total = carry;
    return found;
}

// Local tile id -> (tm, tn) with GROUP_M grouping inside one problem.
template <class C>
__host__ __device__ inline void local_tile(uint32_t id, uint32_t m, uint32_t n, uint32_t& m0,
                                           uint32_t& n0)
{
    const uint32_t tiles_m = (m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n = (n + C::kBN - 1) / C::kBN;
    uint32_t       tm, tn;
    tile_coords<C::kGroupM>(id, tiles_m, tiles_n, tm, tn);
    m0 = tm * C::kBM;
    n0 = tn * C::kBN;
}

template <class C>
__device__ __forceinline__ uint32_t problem_tiles(uint32_t m, uint32_t n)
{
    return ((m + C::kBM - 1) / C::kBM) * ((n + C::kBN - 1) / C::kBN);
}

// Descriptors: KArgs per group (field order of w8a8_group_desc).
template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads, 1)
    gemm_i8_grouped_kernel(const KArgs* __restrict__ groups, uint32_t ngroups, int vec_ok)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    auto tiles = [&](uint32_t i) { return problem_tiles<C>(groups[i].m, groups[i].n); };
    uint32_t g, first, total;
    find_slot(ngroups, 0xFFFFFFFFu, tiles, g, first, total); // total only
    if(blockIdx.x >= total) return;
    const uint32_t lid = xcd_remap(blockIdx.x, total);
    find_slot(ngroups, lid, tiles, g, first, total);
    const KArgs p = groups[g];
    uint32_t    m0, n0;
    local_tile<C>(lid - first, p.m, p.n, m0, n0);
    gemm_tile<C, OUT>(p, m0, n0, vec_ok, lds);
}

struct MoeArgs {
    const int8_t*  a;            // [rows, lda] expert-sorted activations
    const int8_t*  w;            // expert e at w + e * w_stride: [n, ldw]
    void*          c;            // [rows, ldc]
    const float*   sa;           // [rows] or null
    const float*   sw;           // [experts, n] or null
    const int32_t* expert_start; // [experts] first row of each expert
    const int32_t* expert_count; // [experts] rows of each expert
    uint32_t       rows;         // rows of a / c / sa: an expert's rows are clamped to it
    uint32_t       experts, n, k, lda, ldw, ldc;
    uint64_t       w_stride;     // elements between consecutive experts' weights
    float          tsa, tsb;
    int32_t*       ws;           // tail-split partials (cus slots of Partial<C>) or null
    uint32_t       cus;          // compute units the split fills (0: no split)
};

// Tail split.  With T equal tiles on `cus` CUs the last round holds
// L = T % cus tiles and leaves the other CUs idle for a whole tile time.
// When L <= cus / 2 each of those L tiles is cut along K into `parts` pieces
// (L * parts <= cus) whose int32 partials go to the workspace; the fixup
// kernel sums them (exact) and runs the usual epilogue.  Tiles [0, base) run
// whole, as without a split.
struct TailSplit {
    uint32_t base, left, parts;
};

__host__ __device__ inline TailSplit tail_split(uint32_t total, uint32_t cus, uint32_t nk,
                                                bool enabled)
{
    TailSplit s{total, 0u, 1u};
    if(!enabled || cus < 2) return s;
    const uint32_t left = total % cus;
    if(left == 0 || left > cus / 2) return s;
    uint32_t parts = cus / left;
    parts          = parts < nk / kMinKtPerPart ? parts : nk / kMinKtPerPart;
    parts          = parts < kMaxParts ? parts : kMaxParts;
    if(parts < 2) return s;
    return TailSplit{total - left, left, parts};
}

// Rows of expert e, clamped to the buffers: a corrupt count can never make a
// block read or write outside a, c or sa.
__device__ __forceinline__ uint32_t moe_rows_of(const MoeArgs& q, uint32_t e)
{
    const int32_t st = q.expert_start[e], cnt = q.expert_count[e];
    if(st < 0 || cnt <= 0 || (uint32_t)st >= q.rows) return 0u;
    return min((uint32_t)cnt, q.rows - (uint32_t)st);
}

// MoE tile shapes.  C is the block tile; W, its wide partner, has half the
// rows and twice the columns in the same block of waves (W = C: no wide
// tiles).  An expert's rows split into whole C tile rows and a rest; a rest
// of at most W::kBM rows runs as one row of W tiles, which covers its
// outputs with half the MFMA work of a C tile row, a larger rest as one more
// C row.  (A top-k routing leaves many experts a rest of a few dozen rows:
// an expert of 1050 rows takes 4 C rows + 1 W row instead of 5 C rows.)
// Logical tile order: expert by expert, its C tiles (GROUP_M order) and then
// its W tiles, so a W tile reads its weight rows soon after the expert's C
// tiles did.
template <class C, class W>
struct MoeShape {
    static constexpr bool kWide = !std::is_same<C, W>::value;
    static_assert(!kWide || (2 * W::kBM == C::kBM && W::kBN == 2 * C::kBN
                             && W::kThreads == C::kThreads && W::kBK == C::kBK),
                  "W: half the rows and twice the columns of C, the same block and BK");

    // rows of an expert that C tiles cover (the rest, if any, is W's)
    __host__ __device__ static uint32_t c_rows(uint32_t rows)
    {
        const uint32_t rest = rows % C::kBM;
        return kWide && rest != 0 && rest <= (uint32_t)W::kBM ? rows - rest : rows;
    }
    __host__ __device__ static uint32_t c_tiles(uint32_t rows, uint32_t n)
    {
        return (c_rows(rows) + C::kBM - 1) / C::kBM * ((n + C::kBN - 1) / C::kBN);
    }
    __host__ __device__ static uint32_t w_tiles(uint32_t rows, uint32_t n)
    {
        return c_rows(rows) != rows ? (n + W::kBN - 1) / W::kBN : 0u;
    }
    __host__ __device__ static uint32_t tiles(uint32_t rows, uint32_t n)
    {
        return c_tiles(rows, n) + w_tiles(rows, n);
    }
    // origin of the expert's tile `local` (< tiles(rows, n)); wide: a W tile
    __host__ __device__ static void origin(uint32_t local, uint32_t rows, uint32_t n,
                                           uint32_t& m0, uint32_t& n0, bool& wide)
    {
        const uint32_t nc = c_tiles(rows, n);
        wide              = local >= nc;
        if(wide) {
            m0 = c_rows(rows);
            n0 = (local - nc) * W::kBN;
        } else {
            local_tile<C>(local, c_rows(rows), n, m0, n0);
        }
    }
};

template <class C, class W>
__device__ __forceinline__ uint32_t moe_total_tiles(const MoeArgs& q)
{
    uint32_t e, first, total;
    find_slot(q.experts, 0xFFFFFFFFu,
              [&](uint32_t i) { return MoeShape<C, W>::tiles(moe_rows_of(q, i), q.n); }, e, first,
              total);
    return total;
}

// Problem, expert, first row, tile origin and shape (wide: W) of logical
// MoE tile `lid` (< total).
template <class C, class W, int OUT>
__device__ __forceinline__ void moe_tile(const MoeArgs& q, uint32_t lid, KArgs& p, uint32_t& m0,
                                         uint32_t& n0, uint32_t& e, uint32_t& row0, bool& wide)
{
    using S = MoeShape<C, W>;
    uint32_t first, total;
    find_slot(q.experts, lid, [&](uint32_t i) { return S::tiles(moe_rows_of(q, i), q.n); }, e,
              first, total);
    // wave-uniform values, said so: the operand buffer resources built from
    // them must be scalar, or every load of the tile runs in a readfirstlane
    // loop
    e     = __builtin_amdgcn_readfirstlane(e);
    row0  = __builtin_amdgcn_readfirstlane((uint32_t)q.expert_start[e]);
    p.a   = q.a + (size_t)row0 * q.lda;
    p.b   = q.w + (size_t)e * q.w_stride;
    p.c   = static_cast<int8_t*>(q.c) + (size_t)row0 * q.ldc * (OUT == W8A8_OUT_I32 ? 4 : 2);
    p.sa  = q.sa ? q.sa + row0 : nullptr;
    p.sb  = q.sw ? q.sw + (size_t)e * q.n : nullptr;
    p.m   = moe_rows_of(q, e);
    p.n   = q.n;
    p.k   = q.k;
    p.lda = q.lda;
    p.ldb = q.ldw;
    p.ldc = q.ldc;
    p.tsa = q.tsa;
    p.tsb = q.tsb;
    S::origin(lid - first, p.m, p.n, m0, n0, wide);
}

// ---------------------------------------------------------------------------
// SiLU(gate) * up epilogue of the MoE gate_up GEMM (w8a8_moe_gate_up_silu).
// The weights' rows come interleaved in blocks of 32: 16 gate rows, then the
// 16 up rows of the same outputs (w8a8_moe_interleave_gate_up).  In the
// 16 x 16 MFMA layout a lane holds, for each 16-column MFMA tile, a run of
// 4 columns 4 (lane / 16) + e; with that interleave tile 2 p is gate and
// tile 2 p + 1 is up of the same 4 outputs
//   o = n0 / 2 + wn * kWaveN / 2 + 16 p + 4 (lane / 16) + e,
// so silu(g) * u is formed in registers: g and u rounded to fp16 (the values
// the unfused gate_up GEMM would write), a = silu_mul_epi(g, u) in fp32, h =
// fp16(a).  h is written at half the gate_up width, and each wave writes,
// per row, the max over its kWaveN / 2 outputs of |float(h) * s2[e, o]| to
// pmax[n0 / kWaveN + wn][row] (group-major, so a wave's rows are contiguous
// floats): the requantization then knows every row's scale
// before it reads the row.  The SiLU kernels use wave tiles kWaveN = 128
// wide, so each wave's h rows are 128-byte lines.
// ---------------------------------------------------------------------------
struct SiluOut {
    uint16_t*    h;    // [rows, ldh] fp16 activation (columns [0, inter))
    float*       pmax; // [groups, ldp] group-major, groups = ceil(2 * inter / kWaveN), ldp >= rows
    const float* s2;   // [experts, inter] smooth scale of the down GEMM's input, or null
    uint32_t     ldh, ldp, inter;
};

// One tile's epilogue for waves wave_base, wave_base + 1, ... of the tile;
// h and pmax point at the expert's first row, s2 at its vector (or null).
// The weights come interleaved in blocks of 32 rows, 16 gate rows then the
// 16 up rows of the same outputs, so in the 16 x 16 MFMA layout (Acc<C>)
// quad 2 p of a lane holds the gates and quad 2 p + 1 the ups of its outputs
// 16 p + 4 (lane / 16) + 0..3 of the wave's kWaveN / 2.
template <class C>
__device__ __forceinline__ void epilogue_silu(const KArgs& p, uint32_t m0, uint32_t n0,
                                              int8_t* lds, int wave_base, const Acc<C>& acc,
                                              const EpiScales<C>& sc, uint16_t* h, float* pmax,
                                              const float* s2, uint32_t ldh, uint32_t ldp,
                                              uint32_t inter)
{
    static_assert(C::kMfma == 16, "SiLU epilogue: 16 x 16 MFMA layout");
    using A                  = Acc<C>;
    constexpr int kPairs     = A::kQuadsN / 2;
    constexpr int kOutCols   = C::kWaveN / 2;
    constexpr int kRowBytes  = kOutCols * 2;
    constexpr int kRowChunks = kRowBytes / 16;
    constexpr int kRowsPerSt = kWave / kRowChunks;
    static_assert(kRowChunks == 4 || kRowChunks == 8 || kRowChunks == 16, "row of 4-16 chunks");
    static_assert(C::kWaveN % 32 == 0, "whole 32-row interleave blocks per wave");
    using S = StageSwz<kRowChunks>;
    const int      slot = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int      wave = wave_base + slot;
    const int      lane = threadIdx.x % kWave;
    const int      wm   = wave / C::kWavesN;
    const int      wn   = wave % C::kWavesN;
    const int      lgrp = lane >> 4; // 4-column group of the lane's quads
    const uint32_t oc0  = n0 / 2 + wn * kOutCols;
    // waves wholly past the last interleaved column (a partial last N tile)
    // have no pmax entry and store nothing
    const bool     live = n0 + wn * C::kWaveN < p.n;
    float* const   pcol = pmax + (size_t)(n0 / C::kWaveN + wn) * ldp;

    // s2 of this lane's outputs (1 without s2; 0 past inter, where g = u = 0)
    float s2v[kPairs][4];
#pragma unroll
    for(int q = 0; q < kPairs; ++q) {
        const uint32_t o = oc0 + q * 16 + lgrp * 4;
        if(s2 != nullptr && o + 4 <= inter) {
            const float4 v = *reinterpret_cast<const float4*>(s2 + o);
            s2v[q][0] = v.x, s2v[q][1] = v.y, s2v[q][2] = v.z, s2v[q][3] = v.w;
        } else {
#pragma unroll
            for(int e = 0; e < 4; ++e)
                s2v[q][e] = o + e < inter ? (s2 != nullptr ? s2[o + e] : 1.f) : 0.f;
        }
    }

    block_barrier(); // every wave's fragment reads and LDS loads are done: the ring is free
    int8_t* stage = lds + slot * (C::kWaveM * kRowBytes);
#pragma unroll
    for(int i = 0; i < A::kQuadsM; ++i) {
        const int row = A::row(i, lane);
        float     mx  = 0.f;
#pragma unroll
        for(int q = 0; q < kPairs; ++q) {
            const v4i    gq     = acc.quad(i, 2 * q);
            const v4i    uq     = acc.quad(i, 2 * q + 1);
            const float4 sg     = sc.sb[2 * q];
            const float4 su     = sc.sb[2 * q + 1];
            const int    gv[4]  = {gq.x, gq.y, gq.z, gq.w};
            const int    uv[4]  = {uq.x, uq.y, uq.z, uq.w};
            const float  sgv[4] = {sg.x, sg.y, sg.z, sg.w};
            const float  suv[4] = {su.x, su.y, su.z, su.w};
            float        act[4];
#pragma unroll
            for(int e = 0; e < 4; ++e) {
                // g and u rounded to fp16 together, as the unfused GEMM stores them
                const uint32_t gu = float2_to_half2_bits_2step(
                    ((float)gv[e] * sc.sa[i]) * sgv[e], ((float)uv[e] * sc.sa[i]) * suv[e]);
                act[e] = silu_mul_epi(half_bits_to_float(gu & 0xFFFFu), half_bits_to_float(gu >> 16));
            }
            const uint32_t h01 = float2_to_half2_bits_2step(act[0], act[1]);
            const uint32_t h23 = float2_to_half2_bits_2step(act[2], act[3]);
            const uint32_t hb[4] = {h01 & 0xFFFFu, h01 >> 16, h23 & 0xFFFFu, h23 >> 16};
#pragma unroll
            for(int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(half_bits_to_float(hb[e]) * s2v[q][e]));
            const int oc   = q * 16 + lgrp * 4; // output column within the wave
            const int phys = S::chunk(oc >> 3, row);
            v2i       pk;
            pk.x = (int)h01;
            pk.y = (int)h23;
            *reinterpret_cast<v2i*>(stage + row * kRowBytes + phys * 16
                                    + S::half((oc >> 2) & 1, row) * 8) = pk;
        }
        // the row's other three column groups
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const uint32_t m = m0 + wm * C::kWaveM + row;
        if(lgrp == 0 && live && m < p.m) pcol[m] = mx;
    }
    // a wave reads back only what it wrote itself (LDS returns a wave's
    // accesses in order)
    const int      chunk = lane % kRowChunks;
    const uint32_t o     = oc0 + chunk * 8;
    constexpr int  kSt   = C::kWaveM / kRowsPerSt; // stores per lane
    constexpr int  kBat  = kSt < 4 ? kSt : 4;
    static_assert(kSt % kBat == 0, "whole batches");
#pragma unroll
    for(int q0 = 0; q0 < kSt; q0 += kBat) {
        // a batch of reads before its stores: each chunk in one
        // ds_read_b128, its halves swapped back where the writes swapped them
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
            const uint32_t m = m0 + wm * C::kWaveM + (q0 + b) * kRowsPerSt + lane / kRowChunks;
            if(m < p.m && o < inter) *reinterpret_cast<v4i*>(h + (size_t)m * ldh + o) = out[b];
        }
    }
}

// One whole MoE tile of shape X (C or W) with its epilogue.
template <class X, int OUT, bool SILU>
__device__ __forceinline__ void moe_whole(const KArgs& p, uint32_t m0, uint32_t n0, uint32_t e,
                                          uint32_t row0, const SiluOut& so, uint32_t nk,
                                          int vec_ok, int8_t* lds)
{
    if constexpr(SILU) {
        Acc<X>       acc;
        EpiScales<X> sc;
        gemm_tile_acc<X, true>(p, m0, n0, vec_ok, lds, 0, nk, acc, sc);
        epilogue_silu<X>(p, m0, n0, lds, 0, acc, sc, so.h + (size_t)row0 * so.ldh, so.pmax + row0,
                         so.s2 ? so.s2 + (size_t)e * so.inter : nullptr, so.ldh, so.ldp,
                         so.inter);
    } else {
        gemm_tile<X, OUT>(p, m0, n0, vec_ok, lds);
    }
}

// The fixup of a split MoE tile of shape X for this block's waves: sum the
// parts' partials (slots slot * parts ...) and run the epilogue.
template <class X, int OUT, bool SILU>
__device__ __forceinline__ void moe_fix(const MoeArgs& q, const KArgs& p, uint32_t m0,
                                        uint32_t n0, uint32_t e, uint32_t row0, const SiluOut& so,
                                        uint32_t slot, uint32_t parts, int wave_base, int vec_ok,
                                        int8_t* lds)
{
    Acc<X> acc;
    acc.zero();
    const uint32_t tid = wave_base * kWave + threadIdx.x;
    for(uint32_t part = 0; part < parts; ++part)
        add_partial<X>(q.ws + (size_t)(slot * parts + part) * Partial<X>::kInts, tid, acc);
    if constexpr(SILU) {
        const int    wave = wave_base + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
        EpiScales<X> sc;
        sc.load(p, m0, n0, wave / X::kWavesN, wave % X::kWavesN, threadIdx.x % kWave, vec_ok);
        epilogue_silu<X>(p, m0, n0, lds, wave_base, acc, sc, so.h + (size_t)row0 * so.ldh,
                         so.pmax + row0,
                         so.s2 ? so.s2 + (size_t)e * so.inter : nullptr, so.ldh, so.ldp,
                         so.inter);
    } else {
        tile_epilogue<X, OUT>(p, m0, n0, vec_ok, lds, acc, wave_base);
    }
}

// MoE GEMM over C tiles and, for the experts' short rests, W tiles
// (MoeShape); W = C: C tiles only.  The two shapes have the same wave tile,
// so they share the partial slot layout and the fixup blocks.
template <class C, class W, int OUT, bool SILU = false>
__global__ void __launch_bounds__(C::kThreads, 1) gemm_i8_moe_kernel(MoeArgs q, int vec_ok,
                                                                      SiluOut so)
{
    static_assert(Partial<W>::kInts == Partial<C>::kInts
                      && Partial<W>::kPieces == Partial<C>::kPieces
                      && Partial<W>::kFixupLds == Partial<C>::kFixupLds,
                  "W and C share the partial slots and the fixup blocks");
    constexpr bool kWide = MoeShape<C, W>::kWide;
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const uint32_t  total = moe_total_tiles<C, W>(q);
    const uint32_t  nk    = (q.k + C::kBK - 1) / C::kBK;
    const TailSplit sp    = tail_split(total, q.cus, nk, q.ws != nullptr);
    KArgs           p;
    uint32_t        m0, n0, e, row0;
    bool            wide;
    if(blockIdx.x < sp.base) {
        moe_tile<C, W, OUT>(q, xcd_remap(blockIdx.x, sp.base), p, m0, n0, e, row0, wide);
        if(kWide && wide)
            moe_whole<W, OUT, SILU>(p, m0, n0, e, row0, so, nk, vec_ok, lds);
        else
            moe_whole<C, OUT, SILU>(p, m0, n0, e, row0, so, nk, vec_ok, lds);
        return;
    }
    const uint32_t x = blockIdx.x - sp.base;
    if(x >= sp.left * sp.parts) return;
    const uint32_t slot = x / sp.parts, part = x % sp.parts;
    const uint32_t kt0 = part * nk / sp.parts, kt1 = (part + 1) * nk / sp.parts;
    moe_tile<C, W, OUT>(q, sp.base + slot, p, m0, n0, e, row0, wide);
    int32_t* const ws = q.ws + (size_t)x * Partial<C>::kInts;
    if(kWide && wide)
        gemm_tile<W, OUT, true>(p, m0, n0, vec_ok, lds, kt0, kt1 - kt0, ws);
    else
        gemm_tile<C, OUT, true>(p, m0, n0, vec_ok, lds, kt0, kt1 - kt0, ws);
}

// Split tiles, kPieces blocks each: a block holds kFixupWaves of the tile's
// waves, sums their accumulators over the parts in order and runs their part
// of the tile epilogue.
template <class C, class W, int OUT, bool SILU = false>
__global__ void __launch_bounds__(Partial<C>::kFixupWaves * kWave, 1)
    gemm_i8_moe_fixup_kernel(MoeArgs q, int vec_ok, SiluOut so)
{
    constexpr bool kWide = MoeShape<C, W>::kWide;
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const uint32_t  total     = moe_total_tiles<C, W>(q);
    const uint32_t  nk        = (q.k + C::kBK - 1) / C::kBK;
    const TailSplit sp        = tail_split(total, q.cus, nk, q.ws != nullptr);
    const uint32_t  slot      = blockIdx.x / Partial<C>::kPieces;
    const int       wave_base = (int)(blockIdx.x % Partial<C>::kPieces) * Partial<C>::kFixupWaves;
    if(slot >= sp.left) return;
    KArgs    p;
    uint32_t m0, n0, e, row0;
    bool     wide;
    moe_tile<C, W, OUT>(q, sp.base + slot, p, m0, n0, e, row0, wide);
    if(kWide && wide)
        moe_fix<W, OUT, SILU>(q, p, m0, n0, e, row0, so, slot, sp.parts, wave_base, vec_ok, lds);
    else
        moe_fix<C, OUT, SILU>(q, p, m0, n0, e, row0, so, slot, sp.parts, wave_base, vec_ok, lds);
}

// One flag per (configs, output type, kernel kind): the two output types of a
// kernel share a function-pointer type, so the kernel itself cannot key it.
// The dynamic LDS is the larger of the two tiles' rings.
template <class C, class W>
constexpr int moe_lds_bytes()
{
    return C::kLdsBytes > W::kLdsBytes ? C::kLdsBytes : W::kLdsBytes;
}

template <class C, int OUT, int KIND, class W = C>
void raise_lds_once(const void* kern)
{
    static std::once_flag once;
    std::call_once(once, [&] {
        (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  moe_lds_bytes<C, W>());
        (void)hipGetLastError();
    });
}

template <class C>
hipError_t launch_grouped(const KArgs* groups_dev, uint32_t ngroups, uint32_t total_tiles,
                          int out_type, int vec_ok, hipStream_t stream)
{
    if(total_tiles == 0) return hipSuccess;
    if(out_type == W8A8_OUT_I32) {
        raise_lds_once<C, W8A8_OUT_I32, 0>(reinterpret_cast<const void*>(gemm_i8_grouped_kernel<C, W8A8_OUT_I32>));
        hipLaunchKernelGGL((gemm_i8_grouped_kernel<C, W8A8_OUT_I32>), dim3(total_tiles),
                           dim3(C::kThreads), C::kLdsBytes, stream, groups_dev, ngroups, vec_ok);
    } else {
        raise_lds_once<C, W8A8_OUT_F16, 0>(reinterpret_cast<const void*>(gemm_i8_grouped_kernel<C, W8A8_OUT_F16>));
        hipLaunchKernelGGL((gemm_i8_grouped_kernel<C, W8A8_OUT_F16>), dim3(total_tiles),
                           dim3(C::kThreads), C::kLdsBytes, stream, groups_dev, ngroups, vec_ok);
    }
    return hipGetLastError();
}

// Grid bound: every expert's last m tile may be partial, so at most
// ceil(rows / BM) + experts C tile rows in total (a row of W tiles replaces
// one C row and has at most as many tiles); a tail split adds at most
// cus - 1 blocks.  The fixup launch has kPieces blocks per split tile (at
// most cus / 2 split tiles).
template <class C>
size_t moe_workspace_bytes(uint32_t cus)
{
    return (size_t)cus * Partial<C>::kBytes;
}

template <class C>
uint64_t moe_grid_bound(const MoeArgs& q)
{
    const uint32_t tiles_n = (q.n + C::kBN - 1) / C::kBN;
    return ((uint64_t)(q.rows + C::kBM - 1) / C::kBM + q.experts) * tiles_n;
}

template <class C, class W, int OUT, bool SILU>
hipError_t launch_moe_kernels(const MoeArgs& q, const SiluOut& so, int vec_ok, hipStream_t stream)
{
    const uint64_t bound = moe_grid_bound<C>(q);
    if(bound == 0) return hipSuccess;
    const bool     split = q.ws != nullptr && q.cus >= 2;
    const uint64_t grid  = bound + (split ? q.cus : 0);
    const uint32_t fixup_blocks = q.cus / 2 * Partial<C>::kPieces;
    if(grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    constexpr int kLds = moe_lds_bytes<C, W>();
    raise_lds_once<C, OUT, (SILU ? 2 : 1), W>(
        reinterpret_cast<const void*>(gemm_i8_moe_kernel<C, W, OUT, SILU>));
    hipLaunchKernelGGL((gemm_i8_moe_kernel<C, W, OUT, SILU>), dim3((uint32_t)grid),
                       dim3(C::kThreads), kLds, stream, q, vec_ok, so);
    if(split)
        hipLaunchKernelGGL((gemm_i8_moe_fixup_kernel<C, W, OUT, SILU>), dim3(fixup_blocks),
                           dim3(Partial<C>::kFixupWaves * kWave), Partial<C>::kFixupLds, stream,
                           q, vec_ok, so);
    return hipGetLastError();
}

// C tiles and, for the experts' rests of at most W::kBM rows, W tiles (W = C:
// C tiles only).
template <class C, class W = C>
hipError_t launch_moe(const MoeArgs& q, int out_type, int vec_ok, hipStream_t stream)
{
    return out_type == W8A8_OUT_I32
               ? launch_moe_kernels<C, W, W8A8_OUT_I32, false>(q, SiluOut{}, vec_ok, stream)
               : launch_moe_kernels<C, W, W8A8_OUT_F16, false>(q, SiluOut{}, vec_ok, stream);
}

// The gate_up GEMM with the SiLU epilogue (q.n = 2 * inter interleaved
// columns, fp16 scales path; the caller checked vec_ok and the alignment of
// h, ldh and s2).  Both tiles' waves are kWaveN wide, the width of one pmax
// group.
template <class C, class W = C>
hipError_t launch_moe_silu(const MoeArgs& q, const SiluOut& so, int vec_ok, hipStream_t stream)
{
    static_assert(C::kWaveN == W::kWaveN, "one pmax group per wave column in both tiles");
    return launch_moe_kernels<C, W, W8A8_OUT_F16, true>(q, so, vec_ok, stream);
}

} // namespace gemm
} // namespace w8a8
