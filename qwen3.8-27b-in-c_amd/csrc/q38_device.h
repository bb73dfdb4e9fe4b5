/* Device helpers shared by the gfx950 kernels. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q38 {

constexpr int kQK = 256;
constexpr int kQ4K = 12;
constexpr int kQ6K = 14;
constexpr int kIQ1M = 29;

/* Q38Q8KBlock as stored in HBM: fp32 scale @0, int8 quants @4, int16 sums @260. */
constexpr int kQ8KBytes = 292;

/* Exact IEEE binary16 -> binary32 (handles subnormals, inf and NaN). */
__device__ __forceinline__ float f16_to_f32(uint32_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h & 0xffffu)));
}

/* Signed 8-bit 4-way dot product with accumulate: v_dot4_i32_i8. */
__device__ __forceinline__ int dot4(int a, int b, int c)
{
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

/* Same with a zero accumulator.  The builtin is lowered to v_dot4c plus a
 * v_mov that clears the tied accumulator; the three-operand encoding written
 * as inline assembly computed wrong sums in a kernel here (inline assembly
 * is outside the compiler's hazard handling), so it is not used. */
__device__ __forceinline__ int dot4z(int a, int b)
{
    return __builtin_amdgcn_sdot4(a, b, 0, false);
}

/* 24-bit signed multiply / multiply-add (full-rate v_mul_i32_i24 /
 * v_mad_i32_i24); operands must fit in 24 bits. */
__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

/* Lane exchanges inside a quad (DPP quad_perm); every lane of the quad is
 * active wherever these are used, so bound_ctrl never applies. */
__device__ __forceinline__ int quad_xor1(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);
}
__device__ __forceinline__ int quad_xor2(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);
}
__device__ __forceinline__ int quad_sum(int v)
{
    v += quad_xor1(v);
    return v + quad_xor2(v);
}

/* Whole-wavefront reductions with DPP row operations (no LDS traffic);
 * every lane must be active and the result is uniform.  Within each row of
 * 16 lanes: quad swaps, row_half_mirror, row_mirror; then row_bcast15 into
 * rows 1 and 3 and row_bcast31 into rows 2 and 3, so lane 63 holds the
 * total. */
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_move(int old, int v)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}

/* maximum over the wavefront of non-NaN values (fmaxf) */
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, __int_as_float(dpp_move<0xB1>(0, __float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x4E>(0, __float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x141>(0, __float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x140>(0, __float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x142, 0xA>(__float_as_int(v), __float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x143, 0xC>(__float_as_int(v), __float_as_int(v))));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_move_f64(double v)
{
    const int lo = dpp_move<CTRL, ROWS>(0, __double2loint(v)), hi = dpp_move<CTRL, ROWS>(0, __double2hiint(v));
    return __hiloint2double(hi, lo);
}

/* sum over the wavefront (rows outside a broadcast's row mask add 0.0) */
__device__ __forceinline__ double wave_sum(double v)
{
    v += dpp_move_f64<0xB1>(v);
    v += dpp_move_f64<0x4E>(v);
    v += dpp_move_f64<0x141>(v);
    v += dpp_move_f64<0x140>(v);
    v += dpp_move_f64<0x142, 0xA>(v);
    v += dpp_move_f64<0x143, 0xC>(v);
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 63),
                            __builtin_amdgcn_readlane(__double2loint(v), 63));
}

/* IEEE correctly rounded fp32 division and square root.  In this toolchain
 * __fdiv_rn is plain '/', and __fsqrt_rn is the approximate native square
 * root unless OCML_BASIC_ROUNDED_OPERATIONS is defined, so neither is used;
 * '/' and __builtin_sqrtf are correctly rounded under
 * -fhip-fp32-correctly-rounded-divide-sqrt (set in the Makefile). */
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }
__device__ __forceinline__ float sqrt_rn(float a) { return __builtin_sqrtf(a); }

__device__ __forceinline__ float fmul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fadd_rn(float a, float b) { return __fadd_rn(a, b); }

}  // namespace q38
