/* Q8_K quantisation of one 256-element block by one wavefront (device side). */
#pragma once

#include "q38_device.h"

namespace q38 {

/* Lane l holds elements 4l..4l+3 of a 256-element block in v[].  The
 * signed value of the FIRST element holding the largest |x| (NaN never
 * wins; 0 when every |x| is 0 or NaN): the wave maximum of |x| by DPP, then
 * one ballot per element slot finds the lowest element index 4l + i that
 * holds it, and its lane supplies the value. */
__device__ __forceinline__ float block_signed_max(const float (&v)[4])
{
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) a = fmaxf(a, fabsf(v[i]));
    const float amax = wave_max(a);
    int best = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned long long m = __ballot(fabsf(v[i]) == amax);
        if (m) best = min(best, 4 * (int)__builtin_ctzll(m) + i);
    }
    /* `best` is uniform: read the four candidates of its lane into scalars
     * and select among those (a select over v[] would index it) */
    const int src = (best >> 2) & 63, e = best & 3;
    const int c0 = __builtin_amdgcn_readlane(__float_as_int(v[0]), src);
    const int c1 = __builtin_amdgcn_readlane(__float_as_int(v[1]), src);
    const int c2 = __builtin_amdgcn_readlane(__float_as_int(v[2]), src);
    const int c3 = __builtin_amdgcn_readlane(__float_as_int(v[3]), src);
    const float mine = __int_as_float(e == 0 ? c0 : e == 1 ? c1 : e == 2 ? c2 : c3);
    return amax == 0.0f ? 0.0f : mine;
}

/* Restates q38_quantize_q8_k (src/qwen38/qwen38_quant.c:50-88) for one
 * block held as above: maximum as block_signed_max, inverse = -127/max (IEEE
 * division), quants round-half-even via the 1.5*2^23 shift and clamped above
 * at 127, sums per 16 elements, scale = 1/inverse; an all-zero block stores
 * zeros.  `blk` is the 292-byte block in memory (fp32 scale @0, int8 quants
 * @4, int16 sums @260). */
__device__ __forceinline__ void q8k_store(const float (&v)[4], float maximum, uint8_t *__restrict__ blk, int lane)
{
    if (maximum == 0.0f) {   /* uniform over the wave */
        reinterpret_cast<uint32_t *>(blk + 4)[lane] = 0u;
        if (lane < 16) reinterpret_cast<int16_t *>(blk + 260)[lane] = 0;
        if (lane == 0) *reinterpret_cast<float *>(blk) = 0.0f;
        return;
    }
    const float inv = div_rn(-127.0f, maximum);
    uint32_t packed = 0;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float shifted = __fadd_rn(__fmul_rn(inv, v[i]), 12582912.0f);
        const int qv = min((int)(__float_as_uint(shifted) & 0x007fffffu) - 0x00400000, 127);
        sum += qv;
        packed |= (static_cast<uint32_t>(qv) & 0xffu) << (8 * i);
    }
    reinterpret_cast<uint32_t *>(blk + 4)[lane] = packed;
    sum = quad_sum(sum);
    if ((lane & 3) == 0) reinterpret_cast<int16_t *>(blk + 260)[lane >> 2] = static_cast<int16_t>(sum);
    if (lane == 0) *reinterpret_cast<float *>(blk) = div_rn(1.0f, inv);
}

__device__ __forceinline__ void wave_quantize_q8k(const float v[4], uint8_t *__restrict__ blk, int lane)
{
    const float w[4] = {v[0], v[1], v[2], v[3]};
    q8k_store(w, block_signed_max(w), blk, lane);
}

/* wave_quantize_q8k for K blocks at once (block k at blk + k * stride);
 * the K reductions are independent, so their latencies overlap.  Same
 * results as K separate calls. */
template <int K>
__device__ __forceinline__ void wave_quantize_q8k_multi(const float (&v)[K][4], uint8_t *__restrict__ blk,
                                                        size_t stride, int lane)
{
    float maximum[K];
#pragma unroll
    for (int k = 0; k < K; ++k) maximum[k] = block_signed_max(v[k]);
#pragma unroll
    for (int k = 0; k < K; ++k) q8k_store(v[k], maximum[k], blk + k * stride, lane);
}

}  // namespace q38
