// gemm_i8_streamk_kernel.hpp -- stream-K schedule of the int8 tile GEMM.
//
// The reference's stream-K sample (rocwmma_streamk_gemm.cpp:86-211) gives each
// of #CU blocks a contiguous range of "SK units" (tile, 16-deep k slice),
// flushes fp32 partials into a workspace with atomics and sums them in a
// second launch.  Here the unit is one BK-deep k-tile of a BM x BN tile and
// the sum is exact and happens in the same launch:
//   * tiles [t0, t0 + ntiles) (logical ids in tile_coords order) hold
//     T = ntiles * nk k-tiles; block lb of G takes [lb*T/G, (lb+1)*T/G), so
//     ranges differ by at most one k-tile.  Logical block ids are contiguous
//     per XCD (xcd_remap), so neighbouring ranges share one L2.
//   * A range covers whole tiles (the plain epilogue) and pieces of at most
//     two partly covered tiles.  Each piece runs the same k-loop as the tile
//     kernel over its k-tiles, then announces itself on the tile's arrival
//     counter.  Every piece but the last to arrive stores its int32
//     accumulators to a workspace slot and bumps the tile's done counter;
//     the last one waits for that counter (only on pieces that have already
//     arrived, so are running and need nothing further to finish), adds the
//     other pieces' partials to its own and runs the tile's epilogue.
//     Partials and counters move with device-scope accesses (kCpolDevice,
//     relaxed agent-scope atomics) and explicit waits, not fences.
//     Integer addition is exact, so every tile equals the unsplit kernel's
//     bit for bit, whatever the arrival order.
//   * Slots: a tile with P pieces uses P - 1 consecutive slots, after those of
//     the tiles before it; the slot count of tile t is the number of block
//     ranges that start strictly inside it (SkPlan::cut).
//   * The two counters per tile are cleared by streamk_clear_kernel, launched
//     just before on the stream (a kernel, not a memset: the pair may be
//     captured into a HIP graph).
#pragma once

#include "gemm_i8_kernel.hpp"

namespace w8a8 {
namespace gemm {

struct SkPlan {
    uint32_t nk;     // k-tiles per tile
    uint32_t ntiles; // tiles of the stream-K part
    uint32_t blocks; // G; the host keeps G <= ntiles * nk

    __host__ __device__ uint64_t total() const { return (uint64_t)ntiles * nk; }
    __host__ __device__ uint64_t start(uint32_t b) const { return (uint64_t)b * total() / blocks; }
    // the block whose range holds k-tile i: the largest b with start(b) <= i
    __host__ __device__ uint32_t block_of(uint64_t i) const
    {
        return (uint32_t)(((i + 1) * blocks - 1) / total());
    }
    // blocks that contribute to tile t
    __host__ __device__ uint32_t pieces(uint32_t t) const
    {
        return block_of((uint64_t)(t + 1) * nk - 1) - block_of((uint64_t)t * nk) + 1;
    }
    // block b's range starts strictly inside a tile: one more piece there
    __host__ __device__ bool cut(uint32_t b) const
    {
        return b >= 1 && b < blocks && start(b) % nk != 0;
    }
    // the most pieces any tile has: 1 + the most cuts (block ranges starting
    // strictly inside a tile) that fall in one tile.  Block starts increase,
    // so the cuts of one tile are consecutive blocks: O(blocks), not O(tiles)
    __host__ __device__ uint32_t max_pieces() const
    {
        uint32_t best = 1, run = 1;
        uint64_t cur = ~0ull;
        for(uint32_t b = 1; b < blocks; ++b) {
            if(!cut(b)) continue;
            const uint64_t t = start(b) / nk;
            run              = t == cur ? run + 1 : 2;
            cur              = t;
            best             = run > best ? run : best;
        }
        return best;
    }
    // workspace: 2 counters per tile (256-byte aligned), then the slots
    __host__ __device__ size_t sync_bytes() const { return ((size_t)ntiles * 8 + 255) / 256 * 256; }
};

// Host: partial slots of a plan (the number of interior cuts).
inline uint32_t sk_slots(const SkPlan& s)
{
    uint32_t n = 0;
    for(uint32_t b = 1; b < s.blocks; ++b) n += s.cut(b);
    return n;
}

template <class C>
size_t sk_workspace_bytes(const SkPlan& s)
{
    return s.sync_bytes() + (size_t)sk_slots(s) * Partial<C>::kBytes;
}

// Cache policy operand of the buffer builtins: SC1, device scope.  A store
// with it is acknowledged only once it is coherent device-wide, and a load
// with it is never served from another XCD's stale copy: the per-access form
// of a relaxed atomic at agent scope.  The pieces of a tile exchange their
// partials this way; an agent-scope fence would instead write back every
// dirty line of the XCD's L2 (buffer_wbl2) once per piece, which measured
// about 100 us per launch.
constexpr int kCpolDevice = 16;

template <class C>
__device__ __forceinline__ void store_partial_dev(int32_t* part, const Acc<C>& acc)
{
    using A = Acc<C>;
    const __amdgpu_buffer_rsrc_t r
        = __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)Partial<C>::kBytes, kBufferFlags);
#pragma unroll
    for(int i = 0; i < A::kQuadsM; ++i)
#pragma unroll
        for(int j = 0; j < A::kQuadsN; ++j) {
            const int q = i * A::kQuadsN + j;
            __builtin_amdgcn_raw_buffer_store_b128(acc.quad(i, j), r,
                                                   (uint32_t)(q * C::kThreads + threadIdx.x) * 16,
                                                   0, kCpolDevice);
        }
}

// acc += one partial (store_partial layout), read with device scope in
// batches that keep every load of a batch in flight before the adds.
template <class C>
__device__ __forceinline__ void add_partial_dev(const int32_t* part, Acc<C>& acc)
{
    using A              = Acc<C>;
    constexpr int kBatch = A::kQuads < 8 ? A::kQuads : 8;
    static_assert(A::kQuads % kBatch == 0, "whole batches");
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(part), 0, (int)Partial<C>::kBytes, kBufferFlags);
#pragma unroll
    for(int b = 0; b < A::kQuads; b += kBatch) {
        v4i v[kBatch];
#pragma unroll
        for(int x = 0; x < kBatch; ++x)
            v[x] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                                 r, (uint32_t)((b + x) * C::kThreads + threadIdx.x) * 16,
                                                 0, kCpolDevice));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for(int x = 0; x < kBatch; ++x) acc.add((b + x) / A::kQuadsN, (b + x) % A::kQuadsN, v[x]);
    }
}

// Polls of the done counter before a finishing block gives up.  Unreached in
// a correct launch (the pieces waited for have arrived and only store and
// count); the bound keeps every wave's exit certain.
constexpr uint32_t kSkSpinLimit = 1u << 24;

// The bounded wait's report.  A last piece whose wait expires still sums the
// slots and runs the epilogue (every wave exits), but that tile may hold
// stale partials, so it sets kSkWaitExpired in *status, a device word that
// stays set until the host reads and clears it (w8a8_gemm_streamk_status).
// spin: polls before giving up (kSkSpinLimit).  phantom: pieces the last
// piece waits for beyond the real ones, 0 except from the host's test hook,
// which forces the give-up path without a piece that never arrives.
constexpr uint32_t kSkWaitExpired = 1u;
struct SkWatch {
    uint32_t* status;
    uint32_t  spin;
    uint32_t  phantom;
};

__global__ void __launch_bounds__(256) streamk_clear_kernel(uint32_t* sync, uint32_t n)
{
    for(uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) sync[i] = 0;
}

template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads, 1)
    gemm_i8_streamk_kernel(KArgs p, int vec_ok, uint32_t t0, SkPlan sk, uint32_t* sync,
                           int32_t* part, SkWatch watch)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    __shared__ uint32_t bcast[2];
    const uint32_t tiles_m = (p.m + C::kBM - 1) / C::kBM;
    const uint32_t tiles_n = (p.n + C::kBN - 1) / C::kBN;
    const uint32_t lb      = xcd_remap(blockIdx.x, gridDim.x);
    const uint64_t end     = sk.start(lb + 1);
    uint64_t       it      = sk.start(lb);
    for(bool first = true; it < end; first = false) {
        const uint32_t t  = (uint32_t)(it / sk.nk);
        const uint32_t k0 = (uint32_t)(it - (uint64_t)t * sk.nk);
        const uint32_t k1 = (uint32_t)min<uint64_t>(sk.nk, k0 + (end - it));
        it += k1 - k0;
        if(!first) __syncthreads(); // the last piece's LDS reads are done
        uint32_t tm, tn;
        tile_coords<C::kGroupM>(t0 + t, tiles_m, tiles_n, tm, tn);
        const uint32_t m0 = tm * C::kBM, n0 = tn * C::kBN;
        Acc<C>         acc;
        EpiScales<C>   unused;
        gemm_tile_acc<C, false>(p, m0, n0, vec_ok, lds, k0, k1 - k0, acc, unused);
        if(k0 != 0 || k1 != sk.nk) {
            // ---- a piece: arrival order, and this tile's first slot -------
            uint32_t* arrive = sync + 2 * t;
            uint32_t* done   = arrive + 1;
            if(threadIdx.x == 0) {
                bcast[0] = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                bcast[1] = 0;
            }
            __syncthreads();
            uint32_t mine = 0; // cut blocks whose range starts before this tile
            for(uint32_t b = threadIdx.x + 1; b < sk.blocks; b += blockDim.x)
                mine += sk.cut(b) && sk.start(b) < (uint64_t)t * sk.nk;
            if(mine) atomicAdd(&bcast[1], mine);
            __syncthreads();
            // wave-uniform (read from LDS, so taken as divergent unless said:
            // the partial slot's buffer resource would then be rebuilt in a
            // readfirstlane loop around every store and load)
            const uint32_t order  = __builtin_amdgcn_readfirstlane(bcast[0]);
            const uint32_t base   = __builtin_amdgcn_readfirstlane(bcast[1]);
            const uint32_t pieces = sk.pieces(t);
            if(order + 1 < pieces) {
                store_partial_dev<C>(part + (size_t)(base + order) * Partial<C>::kInts, acc);
                wait_vmcnt<0>(); // this wave's partial is coherent device-wide
                __syncthreads(); // ... and every other wave's
                if(threadIdx.x == 0)
                    __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                continue;
            }
            // the last piece to arrive: wait for the others' partials, sum
            if(threadIdx.x == 0) {
                const uint32_t want  = pieces + watch.phantom;
                uint32_t       polls = 0;
                while(__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1
                          < want
                      && ++polls < watch.spin)
                    __builtin_amdgcn_s_sleep(2);
                if(__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 < want)
                    __hip_atomic_fetch_or(watch.status, kSkWaitExpired, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            for(uint32_t q = 0; q + 1 < pieces; ++q)
                add_partial_dev<C>(part + (size_t)(base + q) * Partial<C>::kInts, acc);
        }
        tile_epilogue<C, OUT>(p, m0, n0, vec_ok, lds, acc);
    }
}

template <class C, int OUT>
void raise_streamk_lds_once()
{
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_streamk_kernel<C, OUT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
        (void)hipGetLastError();
    });
}

// Stream-K launch over logical tiles [t0, t0 + s.ntiles) with s.blocks blocks;
// ws holds sk_workspace_bytes<C>(s) bytes (16-byte aligned).
template <class C>
hipError_t launch_cfg_streamk(const KArgs& p, int out_type, int vec_ok, uint32_t t0,
                              const SkPlan& s, void* ws, const SkWatch& watch, hipStream_t stream)
{
    uint32_t*      sync = static_cast<uint32_t*>(ws);
    int32_t*       part = reinterpret_cast<int32_t*>(static_cast<int8_t*>(ws) + s.sync_bytes());
    const uint32_t n    = 2 * s.ntiles;
    hipLaunchKernelGGL(streamk_clear_kernel, dim3(std::min<uint32_t>((n + 255) / 256, 64)),
                       dim3(256), 0, stream, sync, n);
    if(out_type == W8A8_OUT_I32) {
        raise_streamk_lds_once<C, W8A8_OUT_I32>();
        hipLaunchKernelGGL((gemm_i8_streamk_kernel<C, W8A8_OUT_I32>), dim3(s.blocks),
                           dim3(C::kThreads), C::kLdsBytes, stream, p, vec_ok, t0, s, sync, part,
                           watch);
    } else {
        raise_streamk_lds_once<C, W8A8_OUT_F16>();
        hipLaunchKernelGGL((gemm_i8_streamk_kernel<C, W8A8_OUT_F16>), dim3(s.blocks),
                           dim3(C::kThreads), C::kLdsBytes, stream, p, vec_ok, t0, s, sync, part,
                           watch);
    }
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
