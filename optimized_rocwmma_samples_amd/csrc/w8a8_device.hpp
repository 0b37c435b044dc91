// w8a8_device.hpp -- gfx950 device helpers shared by the W8A8 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w8a8 {

typedef int   v2i __attribute__((ext_vector_type(2)));
typedef int   v4i __attribute__((ext_vector_type(4)));
typedef int   v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1      = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2      = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowMirror     = 0x140; // lane i <- lane 15-i inside each row of 16
constexpr int kDppRowHalfMirror = 0x141; // lane i <- lane 7-i inside each half-row of 8

template <int Ctrl>
__device__ __forceinline__ float dpp_mov(float v)
{
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// Max over all 64 lanes; the result is wave-uniform.  max is exact, so the
// reduction order cannot change the value.
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_mov<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_mov<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_mov<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppRowMirror>(v));
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

template <int Ctrl>
__device__ __forceinline__ int dpp_mov_i32(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, Ctrl, 0xF, 0xF, false);
}

// Min over all 64 lanes of an int; the result is wave-uniform.
__device__ __forceinline__ int wave_min_i32(int v)
{
    v = min(v, dpp_mov_i32<kDppQuadXor1>(v));
    v = min(v, dpp_mov_i32<kDppQuadXor2>(v));
    v = min(v, dpp_mov_i32<kDppRowHalfMirror>(v));
    v = min(v, dpp_mov_i32<kDppRowMirror>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Sum over all 64 lanes in a fixed order (quad butterflies, half-row and row
// mirrors, then the four row totals left to right); the result is
// wave-uniform and the same on every call for the same inputs.
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_mov<kDppQuadXor1>(v);
    v += dpp_mov<kDppQuadXor2>(v);
    v += dpp_mov<kDppRowHalfMirror>(v);
    v += dpp_mov<kDppRowMirror>(v);
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return ((r0 + r1) + r2) + r3;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h16)
{
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)h16);
    return (float)h;
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f)
{
    _Float16 h = (_Float16)f; // v_cvt_f16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

// fp16 of an fp32 result, rounded in two IEEE steps: the producing operation
// rounds to fp32, then the conversion rounds to fp16.  The empty asm makes the
// fp32 value opaque, so the compiler cannot fold the producing multiply or add
// into a mixed-precision FMA that rounds to fp16 once (which differs where the
// fp32 result lands exactly between two fp16 values).
__device__ __forceinline__ uint16_t float_to_half_bits_2step(float f)
{
    asm("" : "+v"(f));
    return float_to_half_bits(f);
}

// Two fp32 results as packed fp16 (a in the low half), each rounded in the
// same two steps as float_to_half_bits_2step: one v_cvt_pk_f16_f32 on gfx950
// (round to nearest even, as v_cvt_f16_f32) instead of two conversions and a
// merge.
__device__ __forceinline__ uint32_t float2_to_half2_bits_2step(float a, float b)
{
    typedef float    f2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    asm("" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t{a, b}), h2_t));
}

// int8 quantization of one smoothed value (reference order: (x*s)*inv, rint,
// clamp to +-qmax, rocwmma_smoothquant.cpp:110-113).
__device__ __forceinline__ int quant_i8(float p, float inv, float qmax)
{
    float v = p * inv;
    return (int)fminf(fmaxf(__builtin_rintf(v), -qmax), qmax);
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d)
{
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16)
           | ((uint32_t)d << 24);
}

// The quantizer's arithmetic in fewer VALU instructions, same results.
//
// float(x) * s for the fp16 x in the low (HI = false) or high half of a
// packed pair, in one v_fma_mix_f32: the fp16 operand converts exactly and
// x * s + 0 is rounded once, so the value is float(x) * s except that an
// exact -0 product comes out +0, which nothing downstream tells apart (|p|
// and rint(p * inv) are the same for both).
template <bool HI>
__device__ __forceinline__ float mul_h16_f32(uint32_t h2, float s)
{
    float r;
    if constexpr(HI)
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=v"(r)
            : "v"(h2), "v"(s));
    else
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s));
    return r;
}

// rint(p * inv) clamped to [-qmax, qmax], as a float: quant_i8 before its
// conversion.  v_med3_f32 of (v, -qmax, qmax) is the clamp in one
// instruction, NaN included: with a NaN operand it returns the min3 of its
// operands, -qmax, which is what fminf(fmaxf(NaN, -qmax), qmax) gives.
__device__ __forceinline__ float quant_f(float p, float inv, float qmax)
{
    return __builtin_amdgcn_fmed3f(__builtin_rintf(p * inv), -qmax, qmax);
}

// Four quant_f results (integer-valued, within +-127) converted to int8 and
// packed (a in the low byte): each v_cvt_i32_f32 writes its low byte straight
// into its byte of the result (SDWA dst_sel, the other bytes kept), so the
// packing costs no instruction beyond the conversions.
__device__ __forceinline__ uint32_t cvt_pack4_i8(float a, float b, float c, float d)
{
    uint32_t r;
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD"
        : "=v"(r)
        : "v"(a));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
        : "+v"(r)
        : "v"(b));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
        : "+v"(r)
        : "v"(c));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
        : "+v"(r)
        : "v"(d));
    return r;
}

// (g / (1 + exp(-g))) * u in about a third of the instructions of expf and
// the IEEE division (the requantization is VALU-bound with those):
//   exp(-g) = 2^(ph + pl), ph + pl = -g * log2(e) with log2(e) in two parts
//   and the product's rounding error recovered by an fma, so v_exp_f32 of ph
//   times (1 + pl ln 2) is within about an ulp of exp(-g);
//   g / d from v_rcp_f32 and one residual correction (the quotient is then
//   the correctly rounded one except in rare near-halfway cases).
// Where exp(-g) overflows (ph >= 128) the division gives -0, for g = +inf it
// gives +inf; both are selected explicitly.
__device__ __forceinline__ float silu_mul(float g, float u)
{
    constexpr float kLog2eHi = 1.44269502162933349609375f;   // float(log2 e)
    constexpr float kLog2eLo = 1.925963033500011079e-8f;     // log2 e - kLog2eHi
    constexpr float kLn2     = 0.693147180559945309f;
    const float ph = -g * kLog2eHi;
    const float pl = __builtin_fmaf(-g, kLog2eLo, __builtin_fmaf(-g, kLog2eHi, -ph));
    float       e  = __builtin_amdgcn_exp2f(ph);
    e              = __builtin_fmaf(e, pl * kLn2, e);
    const float d  = 1.f + e;
    const float r  = __builtin_amdgcn_rcpf(d);
    const float q0 = g * r;
    float       q  = __builtin_fmaf(__builtin_fmaf(-d, q0, g), r, q0);
    q              = ph >= 128.f ? -0.f : q;
    q              = g == __builtin_inff() ? g : q;
    return q * u;
}

// silu(g) * u for the gate_up GEMM's SiLU epilogue, where it runs inside the
// compute-bound GEMM: exp(-g) as one v_exp_f32 of -g * log2(e) and the
// quotient from v_rcp_f32, with no correction steps (a few ulps of fp32,
// ahead of a rounding to fp16).  As g -> -inf exp(-g) overflows and the
// product gives -0 (g = -inf selected explicitly); g = +inf gives +inf * u.
__device__ __forceinline__ float silu_mul_epi(float g, float u)
{
    constexpr float kLog2e = 1.44269502162933349609375f;
    const float     r      = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e));
    const float     s      = g == -__builtin_inff() ? -0.f : g * r;
    return s * u;
}

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left at their maxima (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_lgkmcnt0()
{
    __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
}

} // namespace w8a8
