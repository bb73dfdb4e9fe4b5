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

/* wave_quantize_q8k for K blocks at once (block k at blk + k * stride),
 * with the K reductions interleaved so their cross-lane latencies overlap.
 * Same results as K separate calls. */
template <int K>
__device__ __forceinline__ void wave_quantize_q8k_multi(const float (&v)[K][4], uint8_t *__restrict__ blk,
                                                        size_t stride, int lane)
{
    float amax[K];
    int idx[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        amax[k] = 0.0f;
        idx[k] = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = fabsf(v[k][i]);
            if (a > amax[k]) { amax[k] = a; idx[k] = 4 * lane + i; }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float oa[K];
        int oi[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            oa[k] = __shfl_xor(amax[k], off, 64);
            oi[k] = __shfl_xor(idx[k], off, 64);
        }
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (oa[k] > amax[k] || (oa[k] == amax[k] && oi[k] < idx[k])) { amax[k] = oa[k]; idx[k] = oi[k]; }
    }
    float maximum[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int e = idx[k] & 3;
        const float mine = e == 0 ? v[k][0] : e == 1 ? v[k][1] : e == 2 ? v[k][2] : v[k][3];
        maximum[k] = __shfl(mine, (idx[k] >> 2) & 63, 64);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        uint8_t *b = blk + k * stride;
        if (amax[k] == 0.0f) {   /* uniform over the wave */
            reinterpret_cast<uint32_t *>(b + 4)[lane] = 0u;
            if (lane < 16) reinterpret_cast<int16_t *>(b + 260)[lane] = 0;
            if (lane == 0) *reinterpret_cast<float *>(b) = 0.0f;
            continue;
        }
        const float inv = div_rn(-127.0f, maximum[k]);
        uint32_t packed = 0;
        int sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float shifted = __fadd_rn(__fmul_rn(inv, v[k][i]), 12582912.0f);
            int qv = (int)(__float_as_uint(shifted) & 0x007fffffu) - 0x00400000;
            if (qv > 127) qv = 127;
            sum += qv;
            packed |= (static_cast<uint32_t>(qv) & 0xffu) << (8 * i);
        }
        reinterpret_cast<uint32_t *>(b + 4)[lane] = packed;
        sum = quad_sum(sum);
        if ((lane & 3) == 0) reinterpret_cast<int16_t *>(b + 260)[lane >> 2] = static_cast<int16_t>(sum);
        if (lane == 0) *reinterpret_cast<float *>(b) = div_rn(1.0f, inv);
    }
}

}  // namespace q38
