// Reference kernel_moe_smoothquant, compiled from /root/reference/rocwmma_moe_smoothquant.cpp.
#include <algorithm>
#include <cmath>
#include <iostream>
#include <limits>
#include <random>
#include <set>
#include <vector>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include "ref_harness.h"
#define main ref_moe_smoothquant_sample_main
namespace ref_moe_sq {
#include "rocwmma_moe_smoothquant.cpp"
}
#undef main
#undef CHECK_HIP

extern "C" int ref_kernel_moe_smoothquant(const void* x, const float* s, const int32_t* ids,
                                          int8_t* qy, float* rs, uint32_t tokens, uint32_t hidden,
                                          uint32_t topk, uint32_t experts, float quant_max)
{
    hipLaunchKernelGGL(ref_moe_sq::kernel_moe_smoothquant, dim3(tokens * topk),
                       dim3(ref_moe_sq::TBLOCK), 0, 0, static_cast<const __half*>(x), s, ids, qy,
                       rs, tokens, hidden, topk, experts, quant_max);
    hipError_t e = hipGetLastError();
    if(e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}
