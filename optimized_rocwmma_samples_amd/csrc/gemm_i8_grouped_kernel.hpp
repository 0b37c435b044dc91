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
                first       = __shfl(incl - t, l, kWave);
                found       = true;
            }
        }
        carry = __shfl(incl, kWave - 1, kWave);
    }
    total = carry;
    return found;
}

// Local tile id -> (tm, tn) with GROUP_M grouping inside one problem.
template <class C>
__device__ __forceinline__ void local_tile(uint32_t id, uint32_t m, uint32_t n, uint32_t& m0,
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
};

template <class C, int OUT>
__global__ void __launch_bounds__(C::kThreads, 1) gemm_i8_moe_kernel(MoeArgs q, int vec_ok)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const uint32_t tiles_n = (q.n + C::kBN - 1) / C::kBN;
    // rows of expert e, clamped to the buffers: a corrupt count can never
    // make a block read or write outside a, c or sa
    auto rows_of = [&](uint32_t e) -> uint32_t {
        const int32_t st = q.expert_start[e], cnt = q.expert_count[e];
        if(st < 0 || cnt <= 0 || (uint32_t)st >= q.rows) return 0u;
        return min((uint32_t)cnt, q.rows - (uint32_t)st);
    };
    auto tiles = [&](uint32_t e) { return (rows_of(e) + C::kBM - 1) / C::kBM * tiles_n; };
    uint32_t e, first, total;
    find_slot(q.experts, 0xFFFFFFFFu, tiles, e, first, total);
    if(blockIdx.x >= total) return;
    const uint32_t lid = xcd_remap(blockIdx.x, total);
    find_slot(q.experts, lid, tiles, e, first, total);
    const uint32_t row0 = (uint32_t)q.expert_start[e];
    KArgs          p;
    p.a   = q.a + (size_t)row0 * q.lda;
    p.b   = q.w + (size_t)e * q.w_stride;
    p.c   = static_cast<int8_t*>(q.c) + (size_t)row0 * q.ldc * (OUT == W8A8_OUT_I32 ? 4 : 2);
    p.sa  = q.sa ? q.sa + row0 : nullptr;
    p.sb  = q.sw ? q.sw + (size_t)e * q.n : nullptr;
    p.m   = rows_of(e);
    p.n   = q.n;
    p.k   = q.k;
    p.lda = q.lda;
    p.ldb = q.ldw;
    p.ldc = q.ldc;
    p.tsa = q.tsa;
    p.tsb = q.tsb;
    uint32_t m0, n0;
    local_tile<C>(lid - first, p.m, p.n, m0, n0);
    gemm_tile<C, OUT>(p, m0, n0, vec_ok, lds);
}

// One flag per (config, output type, kernel kind): the two output types of a
// kernel share a function-pointer type, so the kernel itself cannot key it.
template <class C, int OUT, int KIND>
void raise_lds_once(const void* kern)
{
    static std::once_flag once;
    std::call_once(once, [&] {
        (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  C::kLdsBytes);
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
// ceil(rows / BM) + experts m tiles in total.
template <class C>
hipError_t launch_moe(const MoeArgs& q, int out_type, int vec_ok, hipStream_t stream)
{
    const uint32_t tiles_n = (q.n + C::kBN - 1) / C::kBN;
    const uint64_t bound   = ((uint64_t)(q.rows + C::kBM - 1) / C::kBM + q.experts) * tiles_n;
    if(bound == 0) return hipSuccess;
    if(bound > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if(out_type == W8A8_OUT_I32) {
        raise_lds_once<C, W8A8_OUT_I32, 1>(reinterpret_cast<const void*>(gemm_i8_moe_kernel<C, W8A8_OUT_I32>));
        hipLaunchKernelGGL((gemm_i8_moe_kernel<C, W8A8_OUT_I32>), dim3((uint32_t)bound),
                           dim3(C::kThreads), C::kLdsBytes, stream, q, vec_ok);
    } else {
        raise_lds_once<C, W8A8_OUT_F16, 1>(reinterpret_cast<const void*>(gemm_i8_moe_kernel<C, W8A8_OUT_F16>));
        hipLaunchKernelGGL((gemm_i8_moe_kernel<C, W8A8_OUT_F16>), dim3((uint32_t)bound),
                           dim3(C::kThreads), C::kLdsBytes, stream, q, vec_ok);
    }
    return hipGetLastError();
}

} // namespace gemm
} // namespace w8a8
