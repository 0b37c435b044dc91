// Reference MoE counting sort, compiled from /root/reference/rocwmma_moe_sorting.cpp.
#include <algorithm>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <random>
#include <vector>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include "ref_harness.h"
#define main ref_moe_sorting_sample_main
namespace ref_sort {
#include "rocwmma_moe_sorting.cpp"
}
#undef main
#undef CHECK_HIP

// Same launch sequence as the sample's timed lambda (rocwmma_moe_sorting.cpp:168-183).
extern "C" int ref_moe_sorting(const int32_t* ids, uint32_t tokens, uint32_t topk,
                               uint32_t experts, uint32_t unit_size, int32_t* count,
                               int32_t* start, int32_t* padded, int32_t* sorted,
                               int32_t* scatter_ws)
{
    const uint32_t total        = tokens * topk;
    const uint32_t total_padded = total + experts * unit_size;
    hipError_t     e            = hipMemset(count, 0, experts * sizeof(int32_t));
    if(e == hipSuccess) e = hipMemset(scatter_ws, 0, experts * sizeof(int32_t));
    if(e == hipSuccess) e = hipMemset(sorted, -1, total_padded * sizeof(int32_t));
    if(e != hipSuccess) return (int)e;
    dim3 block(ref_sort::TBLOCK), grid((total + ref_sort::TBLOCK - 1) / ref_sort::TBLOCK);
    hipLaunchKernelGGL(ref_sort::kernel_moe_histogram, grid, block, experts * sizeof(int32_t), 0,
                       ids, count, total, experts);
    hipLaunchKernelGGL(ref_sort::kernel_prefix_sum, dim3(1), dim3(1), 0, 0, count, start, padded,
                       experts, unit_size);
    hipLaunchKernelGGL(ref_sort::kernel_moe_scatter, grid, block, 0, 0, ids, start, sorted,
                       scatter_ws, tokens, topk, experts);
    e = hipGetLastError();
    if(e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}
