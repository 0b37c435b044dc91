// gemm_i8.hip -- launchers of the int8 GEMM: the gfx950 MFMA tile kernel
// (gemm_i8_kernel.hpp), a generic strided kernel for shapes the tile kernel
// does not take (k % 16 != 0, unaligned operands) and the repack used for the
// reference sample's A col-major / B [K,N] layout.
#include "gemm_i8_kernel.hpp"
#include "w8a8_internal.hpp"

#include <algorithm>
#include <mutex>

namespace w8a8 {

namespace {

using gemm::KArgs;

// Production tile configuration.
using GemmMain = gemm::Cfg<256, 256, 128, 2, 2, 4>;

// ---------------------------------------------------------------------------
// Generic strided kernel: one thread per output, any layout / alignment.
// ---------------------------------------------------------------------------
template <int OUT>
__global__ void __launch_bounds__(256) gemm_i8_generic_kernel(KArgs p, size_t sam, size_t sak,
                                                              size_t sbn, size_t sbk)
{
    const uint32_t n = blockIdx.x * 16 + (threadIdx.x & 15);
    const uint32_t m = blockIdx.y * 16 + (threadIdx.x >> 4);
    if(m >= p.m || n >= p.n) return;
    int32_t acc = 0;
    for(uint32_t k = 0; k < p.k; ++k)
        acc += (int32_t)p.a[m * sam + k * sak] * (int32_t)p.b[n * sbn + k * sbk];
    if constexpr(OUT == W8A8_OUT_I32) {
        reinterpret_cast<int32_t*>(p.c)[(size_t)m * p.ldc + n] = acc;
    } else {
        float f = (float)acc;
        if(p.sa == nullptr && p.sb == nullptr)
            f = f * (p.tsa * p.tsb);
        else
            f = (f * (p.sa ? p.sa[m] : p.tsa)) * (p.sb ? p.sb[n] : p.tsb);
        reinterpret_cast<uint16_t*>(p.c)[(size_t)m * p.ldc + n] = float_to_half_bits(f);
    }
}

__global__ void __launch_bounds__(256) transpose_i8_kernel(const int8_t* src, uint32_t lds_src,
                                                           int8_t* dst, uint32_t ldd,
                                                           uint32_t rows, uint32_t cols)
{
    // dst[r, c] = src[c * lds_src + r]; tile 64x64 through LDS
    __shared__ int8_t tile[64][65];
    const uint32_t r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    for(int i = threadIdx.x; i < 64 * 64; i += 256) {
        const uint32_t cc = c0 + i / 64, rr = r0 + i % 64;
        tile[i / 64][i % 64] = (cc < cols && rr < rows) ? src[(size_t)cc * lds_src + rr] : 0;
    }
    __syncthreads();
    for(int i = threadIdx.x; i < 64 * 64; i += 256) {
        const uint32_t rr = r0 + i / 64, cc = c0 + i % 64;
        if(rr < rows && cc < ldd) dst[(size_t)rr * ldd + cc] = tile[i % 64][i / 64];
    }
}

KArgs make_kargs(const GemmArgs& g)
{
    return KArgs{g.a,   g.b,   g.c,   g.scale_a, g.scale_b, g.m,   g.n,
                 g.k,   g.lda, g.ldb, g.ldc,     g.tsa,     g.tsb};
}

} // namespace

bool gemm_fast_path_ok(const GemmArgs& g)
{
    return (reinterpret_cast<uintptr_t>(g.a) % 16 == 0)
           && (reinterpret_cast<uintptr_t>(g.b) % 16 == 0) && (g.lda % 16 == 0)
           && (g.ldb % 16 == 0) && (g.k % 16 == 0);
}

hipError_t launch_gemm_nk(const GemmArgs& g, hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    const size_t esz    = g.out_type == W8A8_OUT_I32 ? 4 : 2;
    const int    vec_ok = (reinterpret_cast<uintptr_t>(g.c) % (4 * esz) == 0) && (g.ldc % 4 == 0)
                       && (g.scale_b == nullptr
                           || reinterpret_cast<uintptr_t>(g.scale_b) % 16 == 0);
    // The tile kernel addresses each operand through a buffer resource whose
    // out-of-range offsets read as zero; keep every launch's A and B under
    // 2 GiB by splitting M and N into row panels (multiples of the tile).
    constexpr size_t kLimit = 0x7FFFFFFFull;
    const uint32_t   mstep  = (uint32_t)std::min<size_t>(
        g.m, std::max<size_t>(GemmMain::kBM, kLimit / g.lda / GemmMain::kBM * GemmMain::kBM));
    const uint32_t nstep = (uint32_t)std::min<size_t>(
        g.n, std::max<size_t>(GemmMain::kBN, kLimit / g.ldb / GemmMain::kBN * GemmMain::kBN));
    for(uint32_t m0 = 0; m0 < g.m; m0 += mstep) {
        for(uint32_t n0 = 0; n0 < g.n; n0 += nstep) {
            KArgs p = make_kargs(g);
            p.m     = std::min(mstep, g.m - m0);
            p.n     = std::min(nstep, g.n - n0);
            p.a     = g.a + (size_t)m0 * g.lda;
            p.b     = g.b + (size_t)n0 * g.ldb;
            p.c     = static_cast<int8_t*>(g.c) + ((size_t)m0 * g.ldc + n0) * esz;
            p.sa    = g.scale_a ? g.scale_a + m0 : nullptr;
            p.sb    = g.scale_b ? g.scale_b + n0 : nullptr;
            hipError_t e = gemm::launch_cfg<GemmMain>(p, g.out_type, vec_ok, stream);
            if(e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

hipError_t launch_gemm_generic(const GemmArgs& g, size_t sam, size_t sak, size_t sbn, size_t sbk,
                               hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    const KArgs p = make_kargs(g);
    dim3        grid((g.n + 15) / 16, (g.m + 15) / 16);
    if(g.out_type == W8A8_OUT_I32)
        hipLaunchKernelGGL(gemm_i8_generic_kernel<W8A8_OUT_I32>, grid, dim3(256), 0, stream, p,
                           sam, sak, sbn, sbk);
    else
        hipLaunchKernelGGL(gemm_i8_generic_kernel<W8A8_OUT_F16>, grid, dim3(256), 0, stream, p,
                           sam, sak, sbn, sbk);
    return hipGetLastError();
}

hipError_t launch_transpose_i8(const int8_t* src, uint32_t lds_src, int8_t* dst, uint32_t ldd,
                               uint32_t rows, uint32_t cols, hipStream_t stream)
{
    dim3 grid((rows + 63) / 64, (ldd + 63) / 64);
    hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, stream, src, lds_src, dst, ldd,
                       rows, cols);
    return hipGetLastError();
}

} // namespace w8a8
