// Reference kernel_smoothquant, compiled from /root/reference/rocwmma_smoothquant.cpp.
#include <cmath>
#include <iostream>
#include <limits>
#include <vector>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include "ref_harness.h"
#define main ref_smoothquant_sample_main
namespace ref_sq {
#include "rocwmma_smoothquant.cpp"
}
#undef main
#undef CHECK_HIP

extern "C" int ref_kernel_smoothquant(const void* x, const float* s, int8_t* y, float* rs,
                                      uint32_t M, uint32_t N, float quant_max)
{
    hipLaunchKernelGGL(ref_sq::kernel_smoothquant, dim3(M), dim3(ref_sq::TBLOCK), 0, 0,
                       static_cast<const __half*>(x), s, y, rs, M, N, quant_max);
    hipError_t e = hipGetLastError();
    if(e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}
