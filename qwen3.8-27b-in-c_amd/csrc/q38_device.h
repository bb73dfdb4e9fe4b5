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

/* Lane exchanges inside a quad (DPP quad_perm). */
__device__ __forceinline__ int quad_xor1(int v)
{
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ int quad_xor2(int v)
{
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
}
__device__ __forceinline__ int quad_sum(int v)
{
    v += quad_xor1(v);
    return v + quad_xor2(v);
}

__device__ __forceinline__ float fmul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fadd_rn(float a, float b) { return __fadd_rn(a, b); }

}  // namespace q38
