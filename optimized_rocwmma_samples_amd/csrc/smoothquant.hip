// smoothquant.hip -- row-wise smooth-scale + absmax int8 quantizer for gfx950.
//
// Computation (kernel_smoothquant, rocwmma_smoothquant.cpp:58-122, and
// kernel_moe_smoothquant, rocwmma_moe_smoothquant.cpp:69-131):
//   p = float(x[row, n]) * s[n];  r = max|p| / qmax;  inv = r > 0 ? 1/r : 0
//   q[row, n] = int8(clamp(rint(p * inv), -qmax, qmax))
//
// Two kernels, the same per-element operations (bit-identical results):
//   * sq_stream_kernel (dense rows, 16-byte aligned, N % 8 == 0, N <= 32768):
//     s staged once per block in LDS, one block per CU walking the rows with
//     a grid stride and double-buffering them in registers (described at the
//     kernel);
//   * sq_rows_kernel / sq_twopass_kernel: everything else (the MoE gather,
//     unaligned or odd-length rows, very long rows).
//
// sq_rows_kernel (HBM-bound: 3 bytes moved per element):
//   * One wavefront owns a row segment of CPL*512 elements; WPR wavefronts
//     share a row.  Each lane issues CPL 16-byte loads (8 fp16) so a wave
//     instruction reads 1 KiB contiguous, and the whole segment is in flight
//     at once.
//   * The smoothed row stays in VGPRs: x is read from HBM exactly once
//     (the reference re-reads it in its second pass, :101-117).
//   * absmax: DPP quad/mirror steps inside each 16-lane row + 4 readlanes;
//     rows spread over several waves merge through 16 bytes of LDS.
//   * Output: each lane packs 8 int8 and stores 8 bytes (a wave writes 512
//     contiguous bytes), straight into the row-major A operand of the GEMM.
#include "w8a8_device.hpp"
#include "w8a8_internal.hpp"

#include <algorithm>
#include <mutex>

namespace w8a8 {
namespace {

constexpr int kSqThreads = 256; // 4 waves
// Cache-policy operand of the buffer builtins: the NT (non-temporal) bit.
constexpr int kCpolNt = 2;
constexpr int kSqWaves   = kSqThreads / kWave;

struct RowSrc {
    const uint16_t* x;
    const float*    s;
    long            dst;
    bool            valid;
};

template <bool MOE>
__device__ __forceinline__ RowSrc resolve_row(const QuantRows& p, uint32_t row)
{
    RowSrc rs{nullptr, nullptr, -1, false};
    if(row >= p.rows) return rs;
    if constexpr(MOE) {
        uint32_t tok = row / p.topk;
        int32_t  e   = p.topk_ids[row];
        if(e < 0 || (uint32_t)e >= p.experts) return rs;
        long dst = p.dst_row ? (long)p.dst_row[row] : (long)row;
        if(dst < 0 || dst >= (long)p.rows_out) return rs;
        rs.x   = p.x + (size_t)tok * p.ldx;
        rs.s   = p.s + (size_t)e * p.n;
        rs.dst = dst;
    } else {
        rs.x   = p.x + (size_t)row * p.ldx;
        rs.s   = p.s;
        rs.dst = row;
    }
    rs.valid = true;
    return rs;
}

// CPL: 16-byte chunks per lane; WPR: waves per row; VEC: aligned vector I/O.
template <int CPL, int WPR, bool MOE, bool VEC>
__global__ void __launch_bounds__(kSqThreads) sq_rows_kernel(QuantRows p)
{
    constexpr int kRowsPerBlock = kSqWaves / WPR;
    constexpr int kSpan         = CPL * 8 * kWave;

    const int      wave = threadIdx.x / kWave;
    const int      lane = threadIdx.x % kWave;
    const int      rib  = wave / WPR; // row in block
    const int      part = wave % WPR; // segment of the row
    const uint32_t row  = blockIdx.x * kRowsPerBlock + rib;

    RowSrc src = resolve_row<MOE>(p, row);

    float    pv[CPL * 8];
    float    amax = 0.f;
    const uint32_t n    = p.n;
    const uint32_t base = part * kSpan + lane * 8;

    if(src.valid) {
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const uint32_t c = base + j * (8 * kWave);
            if(VEC && c + 8 <= n) {
                const uint4 raw = *reinterpret_cast<const uint4*>(src.x + c);
                const float4 s0 = *reinterpret_cast<const float4*>(src.s + c);
                const float4 s1 = *reinterpret_cast<const float4*>(src.s + c + 4);
                pv[j * 8 + 0] = mul_h16_f32<false>(raw.x, s0.x);
                pv[j * 8 + 1] = mul_h16_f32<true>(raw.x, s0.y);
                pv[j * 8 + 2] = mul_h16_f32<false>(raw.y, s0.z);
                pv[j * 8 + 3] = mul_h16_f32<true>(raw.y, s0.w);
                pv[j * 8 + 4] = mul_h16_f32<false>(raw.z, s1.x);
                pv[j * 8 + 5] = mul_h16_f32<true>(raw.z, s1.y);
                pv[j * 8 + 6] = mul_h16_f32<false>(raw.w, s1.z);
                pv[j * 8 + 7] = mul_h16_f32<true>(raw.w, s1.w);
            } else {
#pragma unroll
                for(int e = 0; e < 8; ++e)
                    pv[j * 8 + e] = (c + e < n) ? half_bits_to_float(src.x[c + e]) * src.s[c + e]
                                                : 0.f;
            }
#pragma unroll
            for(int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(pv[j * 8 + e]));
        }
    }

    amax = wave_max(amax);
    if constexpr(WPR > 1) {
        __shared__ float red[kSqWaves];
        if(lane == 0) red[wave] = amax;
        __syncthreads();
#pragma unroll
        for(int w = 0; w < WPR; ++w) amax = fmaxf(amax, red[rib * WPR + w]);
    }
    if(!src.valid) return;

    const float qmax = p.qmax;
    const float rs   = amax / qmax; // correctly rounded fp32 division
    if(part == 0 && lane == 0) p.r[src.dst] = rs;
    const float inv = (rs > 0.f) ? (1.f / rs) : 0.f;

    int8_t* qrow = p.q + (size_t)src.dst * p.ldq;
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t c = base + j * (8 * kWave);
        const float*   v = pv + j * 8;
        if(VEC && c + 8 <= n) {
            uint2 packed;
            packed.x = cvt_pack4_i8(quant_f(v[0], inv, qmax), quant_f(v[1], inv, qmax),
                                    quant_f(v[2], inv, qmax), quant_f(v[3], inv, qmax));
            packed.y = cvt_pack4_i8(quant_f(v[4], inv, qmax), quant_f(v[5], inv, qmax),
                                    quant_f(v[6], inv, qmax), quant_f(v[7], inv, qmax));
            *reinterpret_cast<uint2*>(qrow + c) = packed;
        } else {
#pragma unroll
            for(int e = 0; e < 8; ++e)
                if(c + e < n) qrow[c + e] = (int8_t)quant_i8(v[e], inv, qmax);
        }
    }
}

// Rows longer than the register-resident path covers: one block per row,
// two passes over x (the second pass re-reads x, mostly from L2).
template <bool MOE>
__global__ void __launch_bounds__(kSqThreads) sq_twopass_kernel(QuantRows p)
{
    __shared__ float red[kSqWaves];
    RowSrc src = resolve_row<MOE>(p, blockIdx.x);
    if(!src.valid) return; // uniform over the block
    float amax = 0.f;
    for(uint32_t c = threadIdx.x; c < p.n; c += kSqThreads)
        amax = fmaxf(amax, fabsf(half_bits_to_float(src.x[c]) * src.s[c]));
    amax = wave_max(amax);
    if(threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float rs = amax / p.qmax;
    if(threadIdx.x == 0) p.r[src.dst] = rs;
    const float inv  = (rs > 0.f) ? (1.f / rs) : 0.f;
    int8_t*     qrow = p.q + (size_t)src.dst * p.ldq;
    for(uint32_t c = threadIdx.x; c < p.n; c += kSqThreads)
        qrow[c] = (int8_t)quant_i8(half_bits_to_float(src.x[c]) * src.s[c], inv, p.qmax);
}

// ---------------------------------------------------------------------------
// Streaming quantizer for the dense case (aligned rows, N % 8 == 0, N <= 32768).
//   * s is staged once per block in LDS, permuted so that each ds_read_b128 of
//     a wave reads 1 KiB contiguous (conflict-free); rows then never re-read
//     s from L2, and no register holds it.
//   * A group of WPR waves owns one row at a time (CPL 16-byte chunks per
//     lane), the block's groups walk the rows with a grid stride, and each
//     wave loads its next row into a second register buffer while it reduces
//     and quantizes the current one: HBM reads stay in flight across rows.
//   * The smoothed values are recomputed from x and the LDS copy of s in the
//     quantize pass instead of being kept in registers, so a wave holds only
//     2 x CPL x 4 VGPRs of row data.
// Results are bit-identical to sq_rows_kernel: same per-element operations.
// ---------------------------------------------------------------------------

// Bytes of x or q one streaming launch addresses at most (below the kernel's
// out-of-range row offset, 0x7FFFFFF0).
constexpr uint64_t kPanelBytes = 0x7F000000ull;

// NT: x is read with the non-temporal cache policy (it is read once); NTS:
// q is stored with it too.
template <int CPL, int WPR, int THREADS, bool NT = false, bool NTS = false>
__global__ void __launch_bounds__(THREADS) sq_stream_kernel(QuantRows p, uint32_t iters)
{
    constexpr int kStreamThreads = THREADS;
    constexpr int kStreamWaves   = THREADS / kWave;
    extern __shared__ __attribute__((aligned(16))) float s_lds[]; // kSpan * WPR floats
    __shared__ float red[2][kStreamWaves];
    constexpr int      kGroups = kStreamWaves / WPR;
    static_assert(kStreamWaves % WPR == 0, "whole row groups per block");
    constexpr int      kSpan   = CPL * 8 * kWave; // columns one wave covers
    constexpr uint32_t kOobOff = 0x80000000u;     // past every buffer: loads 0, stores dropped
    const int      wave = threadIdx.x / kWave;
    const int      lane = threadIdx.x % kWave;
    const int      grp  = wave / WPR;
    const int      part = wave % WPR;
    const uint32_t n    = p.n;
    const uint32_t base = part * kSpan + lane * 8;

    // Operands through buffer resources: rows past the end and columns past N
    // use an offset beyond the buffer (loads read 0, stores are dropped), so
    // the hot loop has no branches and every wave always has exactly CPL loads
    // per row in flight; the wait before a row is processed then leaves the
    // next row's loads outstanding.
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.x), 0, (int)((p.rows - 1) * p.ldx * 2 + n * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        p.q, 0, (int)((p.rows - 1) * p.ldq + n), 0x00020000);

    // Offsets of a chunk = the row's base + the chunk's column offset.  A
    // column past N has offset kOobOff and a row past the end the base
    // kOobRow: every sum of an in-range row and column stays below the
    // buffer's size (< 2^31), and every other sum lies in [2^31, 2^32) (no
    // wrap), past the buffer: one add per chunk, no select.
    // (The host keeps both buffers under kPanelBytes < kOobRow.)
    constexpr uint32_t kOobRow = 0x7FFFFFF0u;
    uint32_t coff[CPL]; // q byte offset of each chunk in a row (its column), or kOobOff
    uint32_t xoff[CPL]; // x byte offset of each chunk in a row, or kOobOff
#pragma unroll
    for(int j = 0; j < CPL; ++j) {
        const uint32_t c = base + j * (8 * kWave);
        coff[j]          = c < n ? c : kOobOff;
        xoff[j]          = c < n ? 2 * c : kOobOff;
    }

    using Row = v4i[CPL];
    Row  xa, xb;
    auto load_row = [&](Row& dst, uint32_t r) {
        const uint32_t roff = r < p.rows ? r * p.ldx * 2 : kOobRow;
#pragma unroll
        for(int j = 0; j < CPL; ++j)
            dst[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, roff + xoff[j], 0,
                                                           NT ? kCpolNt : 0);
    };
    // LDS offset of this lane's s values; made opaque once per row (below) so
    // the compiler re-reads s from LDS instead of pinning CPL*8 registers to it
    // for the whole kernel, which would cap the CU at one block
    uint32_t s_off = (part * kSpan + lane * 4) * 4;
    // the 8 products x*s of chunk j (mul_h16_f32: one instruction each)
    auto smoothed = [&](const v4i& raw, int j, float* v) {
        const float4 s0 = *reinterpret_cast<const float4*>(
            reinterpret_cast<const char*>(s_lds) + s_off + j * 2048);
        const float4 s1 = *reinterpret_cast<const float4*>(
            reinterpret_cast<const char*>(s_lds) + s_off + j * 2048 + 1024);
        v[0] = mul_h16_f32<false>((uint32_t)raw.x, s0.x);
        v[1] = mul_h16_f32<true>((uint32_t)raw.x, s0.y);
        v[2] = mul_h16_f32<false>((uint32_t)raw.y, s0.z);
        v[3] = mul_h16_f32<true>((uint32_t)raw.y, s0.w);
        v[4] = mul_h16_f32<false>((uint32_t)raw.z, s1.x);
        v[5] = mul_h16_f32<true>((uint32_t)raw.z, s1.y);
        v[6] = mul_h16_f32<false>((uint32_t)raw.w, s1.z);
        v[7] = mul_h16_f32<true>((uint32_t)raw.w, s1.w);
    };
    auto process = [&](const Row& x, uint32_t r, int parity) {
        asm volatile("" : "+v"(s_off));
        // columns past N hold x = 0 and s = 0: they add nothing to the max.
        // The products stay in registers for the quantize pass.
        float pv[CPL * 8];
        float amax = 0.f;
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            smoothed(x[j], j, pv + j * 8);
#pragma unroll
            for(int e = 0; e < 8; e += 2)
                amax = fmaxf(fmaxf(amax, fabsf(pv[j * 8 + e])), fabsf(pv[j * 8 + e + 1]));
        }
        amax = wave_max(amax);
        if constexpr(WPR > 1) {
            if(lane == 0) red[parity][wave] = amax;
            __syncthreads();
#pragma unroll
            for(int w = 0; w < WPR; ++w) amax = fmaxf(amax, red[parity][grp * WPR + w]);
        }
        const bool  valid = r < p.rows;
        const float qmax  = p.qmax;
        const float rs    = amax / qmax;
        if(valid && part == 0 && lane == 0) p.r[r] = rs;
        const float    inv  = rs > 0.f ? 1.f / rs : 0.f;
        const uint32_t qoff = valid ? r * p.ldq : kOobRow;
#pragma unroll
        for(int j = 0; j < CPL; ++j) {
            const float* v = pv + j * 8;
            v2i          pk;
            pk.x = (int)cvt_pack4_i8(quant_f(v[0], inv, qmax), quant_f(v[1], inv, qmax),
                                     quant_f(v[2], inv, qmax), quant_f(v[3], inv, qmax));
            pk.y = (int)cvt_pack4_i8(quant_f(v[4], inv, qmax), quant_f(v[5], inv, qmax),
                                     quant_f(v[6], inv, qmax), quant_f(v[7], inv, qmax));
            __builtin_amdgcn_raw_buffer_store_b64(pk, rq, qoff + coff[j], 0, NTS ? kCpolNt : 0);
        }
    };

    const uint32_t stride = gridDim.x * kGroups;
    uint32_t       row    = blockIdx.x * kGroups + grp;

    // The first row's loads go out before s is staged, so the two fetches
    // overlap.  s lands in LDS permuted so that each ds_read_b128 of a wave
    // reads 1 KiB contiguous (conflict-free): column c = part*kSpan + j*512 +
    // l*8 + e of a row sits at part*kSpan + j*512 + (e/4)*256 + l*4 + e%4.
    // Columns past N are stored as 0.
    load_row(xa, row);
    {
        constexpr int kTotal = kSpan * WPR;
        constexpr int kS4    = (kTotal + kStreamThreads * 4 - 1) / (kStreamThreads * 4);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(p.s), 0, (int)(n * 4), 0x00020000);
        v4i sv[kS4];
#pragma unroll
        for(int i = 0; i < kS4; ++i) {
            const uint32_t c4 = (i * kStreamThreads + threadIdx.x) * 4;
            sv[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, c4 < n ? c4 * 4 : kOobOff, 0, 0);
        }
#pragma unroll
        for(int i = 0; i < kS4; ++i) {
            const uint32_t c4 = (i * kStreamThreads + threadIdx.x) * 4;
            if(c4 < (uint32_t)kTotal) {
                const uint32_t c    = c4 & ~7u;
                const uint32_t slot = (c / 512) * 512 + ((c4 & 4u) ? 256u : 0u) + ((c % 512) / 8) * 4;
                *reinterpret_cast<v4i*>(s_lds + slot) = sv[i];
            }
        }
    }
    __syncthreads();

    // every wave runs the same `iters` steps, so the barriers stay uniform
    // (sched_barrier: the next row's loads are issued before the wait for the
    // current row, never sunk below it by the scheduler)
    for(uint32_t it = 0; it < iters; it += 2) {
        load_row(xb, row + stride);
        __builtin_amdgcn_sched_barrier(0);
        process(xa, row, 0);
        row += stride;
        if(it + 1 >= iters) break;
        load_row(xa, row + stride);
        __builtin_amdgcn_sched_barrier(0);
        process(xb, row, 1);
        row += stride;
    }
}

// THREADS per block, BPC resident blocks per CU (the grid is BPC x CUs, each
// block walking rows with a grid stride).
template <int CPL, int WPR, int THREADS, int BPC = 1, bool NT = false, bool NTS = false>
hipError_t launch_stream(const QuantRows& p, hipStream_t stream)
{
    constexpr int  kGroups = THREADS / kWave / WPR;
    const size_t   lds     = (size_t)CPL * 512 * WPR * sizeof(float);
    // one row group must span the whole row
    if((uint64_t)CPL * 512 * WPR < p.n) return hipErrorInvalidValue;
    static int     max_blocks = [] {
        int dev = 0, cus = 256;
        if(hipGetDevice(&dev) == hipSuccess)
            (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        return cus * BPC;
    }();
    if(lds > 65536) {
        static std::once_flag once;
        std::call_once(once, [] {
            (void)hipFuncSetAttribute(
                reinterpret_cast<const void*>(sq_stream_kernel<CPL, WPR, THREADS, NT, NTS>),
                hipFuncAttributeMaxDynamicSharedMemorySize, 131072);
            (void)hipGetLastError();
        });
    }
    // x and q are addressed through 32-bit buffer offsets: launch row panels
    // whose x and q spans both stay under kPanelBytes (the kernel's
    // out-of-range sentinels lie above it)
    const uint64_t rows_x = kPanelBytes / ((uint64_t)p.ldx * 2);
    const uint64_t rows_q = kPanelBytes / (uint64_t)p.ldq;
    // (a single row spans only its own n columns, whatever the strides)
    const uint32_t panel  = (uint32_t)std::max<uint64_t>(
        1, std::min<uint64_t>(p.rows, std::min(rows_x, rows_q)));
    for(uint32_t r0 = 0; r0 < p.rows; r0 += panel) {
        QuantRows q = p;
        q.rows      = std::min(panel, p.rows - r0);
        q.x         = p.x + (size_t)r0 * p.ldx;
        q.q         = p.q + (size_t)r0 * p.ldq;
        q.r         = p.r + r0;
        const uint32_t need   = (q.rows + kGroups - 1) / kGroups;
        const uint32_t blocks = std::max<uint32_t>(1, std::min<uint32_t>(need, (uint32_t)max_blocks));
        const uint32_t iters  = (q.rows + blocks * kGroups - 1) / (blocks * kGroups);
        hipLaunchKernelGGL((sq_stream_kernel<CPL, WPR, THREADS, NT, NTS>), dim3(blocks), dim3(THREADS), lds,
                           stream, q, iters);
        const hipError_t e = hipGetLastError();
        if(e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int CPL, int WPR, bool MOE>
hipError_t launch_rows(const QuantRows& p, bool vec, hipStream_t stream)
{
    constexpr int kRowsPerBlock = kSqWaves / WPR;
    dim3          grid((p.rows + kRowsPerBlock - 1) / kRowsPerBlock);
    if(vec)
        hipLaunchKernelGGL((sq_rows_kernel<CPL, WPR, MOE, true>), grid, dim3(kSqThreads), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((sq_rows_kernel<CPL, WPR, MOE, false>), grid, dim3(kSqThreads), 0,
                           stream, p);
    return hipGetLastError();
}

template <bool MOE>
hipError_t dispatch(const QuantRows& p, hipStream_t stream)
{
    // 16-byte x loads, 32-byte aligned s loads, 8-byte q stores.
    const bool vec = (reinterpret_cast<uintptr_t>(p.x) % 16 == 0) && (p.ldx % 8 == 0)
                     && (reinterpret_cast<uintptr_t>(p.s) % 16 == 0) && (!MOE || p.n % 4 == 0)
                     && (reinterpret_cast<uintptr_t>(p.q) % 8 == 0) && (p.ldq % 8 == 0);
    const uint32_t n = p.n;
    if constexpr(!MOE) {
        // aligned dense rows: the streaming kernel (s in LDS, rows double-buffered)
        if(vec && n % 8 == 0) {
            // (configurations chosen by a sweep on MI355X over CPL, WPR,
            // block size and blocks per CU, cache-warm and cache-cold)
            // A few rows (decode): the launch is latency-bound, so each row
            // is spread over all 16 waves of a 1024-thread block.
            if(p.rows <= 64 && n > 4096 && n <= 8192) return launch_stream<1, 16, 1024>(p, stream);
            if(p.rows <= 64 && n > 8192 && n <= 16384) return launch_stream<2, 16, 1024>(p, stream);
            if(n <= 512) return launch_stream<1, 1, 512>(p, stream);
            if(n <= 1024) return launch_stream<2, 1, 512>(p, stream);
            if(n <= 2048) return launch_stream<4, 1, 512>(p, stream);
            // Up to 4096 columns (cold, MALL-rotated buffers): below 1024
            // rows two blocks of 256 threads per CU with a row over two waves
            // (512 x 4096: 4.1 us); from 1024 rows x is read non-temporally
            // (it is read once) and one wave holds a whole row, so its max
            // needs no cross-wave merge: two blocks of 256 threads per CU
            // (2048 x 4096: 9.1 -> 7.3 us, 3328 rows 12.9 -> 10.2 us), except
            // 4096 to 32767 rows, where four blocks of 256 threads with a row
            // over two waves keep more rows in flight (8192 rows: 17.4 us
            // against 18.1), and from 32768 rows, where one 512-thread block
            // of rows over two waves walks them (131072 rows: 307 -> 275 us)
            if(n <= 4096 && p.rows < 1024) return launch_stream<4, 2, 256, 2>(p, stream);
            if(n <= 4096 && p.rows >= 4096 && p.rows < 32768)
                return launch_stream<4, 2, 256, 4, true>(p, stream);
            // (1024-4095 rows also store q non-temporally: 2048 x 4096 cold
            // 7.4 -> 6.5 us; from 4096 rows it no longer pays, 8192 rows 17.6
            // against 18.4 us)
            if(n <= 4096 && p.rows >= 32768) return launch_stream<4, 2, 512, 1, true>(p, stream);
            if(n <= 4096) return launch_stream<8, 1, 256, 2, true, true>(p, stream);
            if(n <= 8192) return launch_stream<4, 4, 512, 2>(p, stream);
            // two row groups of 8 waves per 1024-thread block (4 chunks per
            // lane), x read non-temporally: n = 14336 cold, 2048 / 8192 rows
            // 19.4 -> 16.7 / 64.2 -> 58.0 us
            if(n <= 16384) return launch_stream<4, 8, 1024, 1, true>(p, stream);
            if(n <= 32768) return launch_stream<4, 16, 1024>(p, stream);
        }
    }
    if(n <= 512) return launch_rows<1, 1, MOE>(p, vec, stream);
    if(n <= 1024) return launch_rows<2, 1, MOE>(p, vec, stream);
    if(n <= 2048) return launch_rows<4, 1, MOE>(p, vec, stream);
    if(n <= 4096) return launch_rows<8, 1, MOE>(p, vec, stream);
    if(n <= 8192) return launch_rows<16, 1, MOE>(p, vec, stream);
    if(n <= 16384) return launch_rows<16, 2, MOE>(p, vec, stream);
    if(n <= 32768) return launch_rows<16, 4, MOE>(p, vec, stream);
    hipLaunchKernelGGL((sq_twopass_kernel<MOE>), dim3(p.rows), dim3(kSqThreads), 0, stream, p);
    return hipGetLastError();
}

} // namespace

hipError_t launch_smoothquant(const QuantRows& p, hipStream_t stream)
{
    if(p.rows == 0) return hipSuccess;
    return p.topk_ids ? dispatch<true>(p, stream) : dispatch<false>(p, stream);
}

} // namespace w8a8
