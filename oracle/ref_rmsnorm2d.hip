// Reference kernel_rmsnorm2d_fwd / kernel_add_rmsnorm2d_fwd, compiled from
// /root/reference/rocwmma_rmsnorm2d.cpp (test infrastructure only).
#include <cmath>
#include <iostream>
#include <vector>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include "ref_harness.h"
#define main ref_rmsnorm2d_sample_main
namespace ref_rms {
#include "rocwmma_rmsnorm2d.cpp"
}
#undef main
#undef CHECK_HIP

extern "C" int ref_kernel_rmsnorm2d(const void* x, const float* gamma, void* y, uint32_t M,
                                    uint32_t N, uint32_t ldx, uint32_t ldy, float eps)
{
    hipLaunchKernelGGL(ref_rms::kernel_rmsnorm2d_fwd, dim3(M), dim3(ref_rms::TBLOCK), 0, 0,
                       static_cast<const __half*>(x), gamma, static_cast<__half*>(y), M, N, ldx,
                       ldy, eps);
    hipError_t e = hipGetLastError();
    if(e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}

extern "C" int ref_kernel_add_rmsnorm2d(const void* x, const void* residual, const float* gamma,
                                        void* y, void* x_out, uint32_t M, uint32_t N, float eps)
{
    hipLaunchKernelGGL(ref_rms::kernel_add_rmsnorm2d_fwd, dim3(M), dim3(ref_rms::TBLOCK), 0, 0,
                       static_cast<const __half*>(x), static_cast<const __half*>(residual), gamma,
                       static_cast<__half*>(y), static_cast<__half*>(x_out), M, N, eps);
    hipError_t e = hipGetLastError();
    if(e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}
