// Reference kernel_topk_softmax, compiled from /root/reference/rocwmma_topk_softmax.cpp.
#include <algorithm>
#include <cmath>
#include <iomanip>
#include <iostream>
#include <limits>
#include <vector>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include "ref_harness.h"
#define main ref_topk_softmax_sample_main
namespace ref_topk {
#include "rocwmma_topk_softmax.cpp"
}
#undef main
#undef CHECK_HIP

extern "C" int ref_kernel_topk_softmax(const void* logits_f16, float* w, int32_t* idx,
                                       uint32_t tokens, uint32_t experts, uint32_t topk)
{
    if(experts > ref_topk::WARP_SIZE) return (int)hipErrorInvalidValue;
    dim3 grid((tokens + ref_topk::WARPS_PER_BLOCK - 1) / ref_topk::WARPS_PER_BLOCK);
    hipLaunchKernelGGL(ref_topk::kernel_topk_softmax, grid, dim3(ref_topk::TBLOCK), 0, 0,
                       static_cast<const __half*>(logits_f16), w, idx, tokens, experts, topk);
    hipError_t e = hipGetLastError();
    if(e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}
