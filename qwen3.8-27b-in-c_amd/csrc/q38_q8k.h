/* Q8_K quantisation of one 256-element block by one wavefront (device side). */
#pragma once

#include "q38_device.h"

namespace q38 {

/* Lane l holds elements 4l..4l+3 of the block in v[].  Restates
 * q38_quantize_q8_k (src/qwen38/qwen38_quant.c:50-88): the block maximum is
 * the signed value of the FIRST element holding the largest |x| (NaN never
 * wins), inverse = -127/max (IEEE division), quants are round-half-even via
 * the 1.5*2^23 shift and clamped above at 127, sums are per 16 elements,
 * scale = 1/inverse.  An all-zero block stores zeros.  `blk` is the 292-byte
 * block in memory (fp32 scale @0, int8 quants @4, int16 sums @260). */
__device__ __forceinline__ void wave_quantize_q8k(const float v[4], uint8_t *__restrict__ blk, int lane)
{
    float amax = 0.0f;
    int idx = 0x7fffffff;
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        if (a > amax) { amax = a; idx = 4 * lane + i; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(amax, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (oa > amax || (oa == amax && oi < idx)) { amax = oa; idx = oi; }
    }
    if (amax == 0.0f) {
        reinterpret_cast<uint32_t *>(blk + 4)[lane] = 0u;
        if (lane < 16) reinterpret_cast<int16_t *>(blk + 260)[lane] = 0;
        if (lane == 0) *reinterpret_cast<float *>(blk) = 0.0f;
        return;
    }
    const int k = idx & 3;
    const float mine = k == 0 ? v[0] : k == 1 ? v[1] : k == 2 ? v[2] : v[3];
    const float maximum = __shfl(mine, idx >> 2, 64);
    const float inv = div_rn(-127.0f, maximum);

    uint32_t packed = 0;
    int sum = 0;
    for (int i = 0; i < 4; ++i) {
        const float shifted = __fadd_rn(__fmul_rn(inv, v[i]), 12582912.0f);
        int q = (int)(__float_as_uint(shifted) & 0x007fffffu) - 0x00400000;
        if (q > 127) q = 127;
        sum += q;
        packed |= (static_cast<uint32_t>(q) & 0xffu) << (8 * i);
    }
    reinterpret_cast<uint32_t *>(blk + 4)[lane] = packed;
    sum = quad_sum(sum);
    if ((lane & 3) == 0) reinterpret_cast<int16_t *>(blk + 260)[lane >> 2] = static_cast<int16_t>(sum);
    if (lane == 0) *reinterpret_cast<float *>(blk) = div_rn(1.0f, inv);
}

}  // namespace q38
