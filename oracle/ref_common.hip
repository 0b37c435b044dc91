// Reference CPU GEMM and comparator, compiled from /root/reference/common.hpp.
#include <hip/hip_runtime.h>
#include <rocwmma/rocwmma.hpp>
#include "common.hpp"
#include "ref_harness.h"

extern "C" void ref_gemm_cpu_i8(uint32_t m, uint32_t n, uint32_t k, const int8_t* a,
                                const int8_t* b, int32_t* d, uint32_t lda, uint32_t ldb,
                                uint32_t ldd, int layout)
{
    using rocwmma::col_major;
    using rocwmma::row_major;
    if(layout == 0)
        gemm_cpu_h<int8_t, int32_t, int32_t, row_major, col_major, row_major>(
            m, n, k, a, b, d, d, lda, ldb, ldd, ldd, 1, 0);
    else
        gemm_cpu_h<int8_t, int32_t, int32_t, col_major, row_major, row_major>(
            m, n, k, a, b, d, d, lda, ldb, ldd, ldd, 1, 0);
}

extern "C" int ref_compare_equal_f16(const uint16_t* a, const uint16_t* b, uint32_t size,
                                     double tol, double* max_rel_err)
{
    auto r = compareEqual<rocwmma::float16_t>(reinterpret_cast<const rocwmma::float16_t*>(a),
                                              reinterpret_cast<const rocwmma::float16_t*>(b),
                                              size, tol);
    *max_rel_err = r.second;
    return r.first ? 1 : 0;
}

extern "C" int ref_compare_equal_i32(const int32_t* a, const int32_t* b, uint32_t size,
                                     double tol, double* max_rel_err)
{
    auto r = compareEqual<int32_t>(a, b, size, tol);
    *max_rel_err = r.second;
    return r.first ? 1 : 0;
}
