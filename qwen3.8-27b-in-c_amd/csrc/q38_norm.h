/* RMSNorm / L2-norm building blocks shared by the decode kernels: the
 * reference's double-precision squared sums and the fused residual add +
 * RMSNorm + Q8_K of one hidden row. */
#pragma once

#include "q38_device.h"
#include "q38_math.h"
#include "q38_q8k.h"

namespace q38 {

/* ---- exact sequential double sums ---------------------------------------- */

/* The reference norms compute sum += (double)(x[i]*x[i]) for i = 0..n-1 in
 * order and use only a monotone, float-rounded function of the sum:
 * (float)(sum / n) for RMSNorm (qwen38_model.c:426-435) and (float)sum for
 * the L2 norm (:608-614).  The block first sums in parallel (any order);
 * for non-negative terms both that sum and the sequential one are within
 * (n + 8) * 2^-53 relative of the exact sum, far inside the 2^-36 margin used
 * here for n <= 65536.  If the float result is the same at both ends of the
 * margin it is the reference's result; otherwise (about one call in 4000,
 * and always for NaN) one thread redoes the sequential loop.  `post` is the
 * float-rounding step. */
template <int THREADS, typename Post>
__device__ float block_sum_finish(double s, const float *x, int n, Post post)
{
    static_assert(THREADS % 64 == 0 && THREADS <= 1024, "block size");
    __shared__ double partial[THREADS / 64];
    __shared__ float result;
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double total = 0.0;
        for (int w = 0; w < THREADS / 64; ++w) total += partial[w];
        const float lo = post(total * (1.0 - 0x1p-36));
        const float hi = post(total * (1.0 + 0x1p-36));
        if (lo == hi) {
            result = lo;
        } else {
            double seq = 0.0;
            for (int i = 0; i < n; ++i) seq += (double)__fmul_rn(x[i], x[i]);
            result = post(seq);
        }
    }
    __syncthreads();
    const float r = result;
    __syncthreads();
    return r;
}

/* block_sum_finish over a vector the block reads itself */
template <int THREADS, typename Post>
__device__ float block_sum_squares(const float *x, int n, Post post)
{
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += THREADS) {
        const float v = x[i];
        s += (double)__fmul_rn(v, v);
    }
    return block_sum_finish<THREADS>(s, x, n, post);
}

struct MeanPost {
    double n;
    __device__ float operator()(double s) const { return (float)(s / n); }
};
struct FloatPost {
    __device__ float operator()(double s) const { return (float)s; }
};

/* ---- RMSNorm + Q8_K of one row ---------------------------------------------- */

/* One block of T threads over one row of N = 4*T*NV floats at h.  ADD: the
 * row first becomes h + branch (the residual add of qwen38_model.c:975/983,
 * written back to h).  Then y = (x * scale) * w with scale =
 * 1/sqrtf(mean + 1e-6) (q38_rmsnorm, :426-435), written to norm_out (when
 * not null) and quantised to Q8_K into q_out (when not null): float4
 * f = tid + T*j holds elements 4f..4f+3, i.e. lane `tid % 64` of Q8_K
 * block (T/64)*j + tid/64, so each wavefront quantises whole blocks. */
template <int T, int NV, bool ADD>
__device__ __forceinline__ void rmsnorm_quant_row(float *__restrict__ norm_out, uint8_t *__restrict__ q_out,
                                                  float *__restrict__ h, const float *__restrict__ branch,
                                                  const float *__restrict__ weight)
{
    static_assert(T % 64 == 0, "whole wavefronts");
    constexpr int N = 4 * T * NV;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    /* the weights do not depend on the row: load them with the row */
    const float4 *w4 = reinterpret_cast<const float4 *>(weight);
    float4 w[NV], x[NV];
    for (int j = 0; j < NV; ++j) w[j] = w4[tid + T * j];
    for (int j = 0; j < NV; ++j) x[j] = reinterpret_cast<const float4 *>(h)[tid + T * j];
    if (ADD) {
        const float4 *b = reinterpret_cast<const float4 *>(branch);
        for (int j = 0; j < NV; ++j) {
            const float4 bj = b[tid + T * j];
            x[j].x = __fadd_rn(x[j].x, bj.x);
            x[j].y = __fadd_rn(x[j].y, bj.y);
            x[j].z = __fadd_rn(x[j].z, bj.z);
            x[j].w = __fadd_rn(x[j].w, bj.w);
            reinterpret_cast<float4 *>(h)[tid + T * j] = x[j];
        }
    }
    double s = 0.0;
    for (int j = 0; j < NV; ++j) {
        s += (double)__fmul_rn(x[j].x, x[j].x);
        s += (double)__fmul_rn(x[j].y, x[j].y);
        s += (double)__fmul_rn(x[j].z, x[j].z);
        s += (double)__fmul_rn(x[j].w, x[j].w);
    }
    const float mean = block_sum_finish<T>(s, h, N, MeanPost{(double)N});
    const float scale = rms_scale(mean);
    float v[NV][4];
    for (int j = 0; j < NV; ++j) {
        v[j][0] = __fmul_rn(__fmul_rn(x[j].x, scale), w[j].x);
        v[j][1] = __fmul_rn(__fmul_rn(x[j].y, scale), w[j].y);
        v[j][2] = __fmul_rn(__fmul_rn(x[j].z, scale), w[j].z);
        v[j][3] = __fmul_rn(__fmul_rn(x[j].w, scale), w[j].w);
        if (norm_out)
            reinterpret_cast<float4 *>(norm_out)[tid + T * j] = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
    }
    if (q_out) wave_quantize_q8k_multi<NV>(v, q_out + (size_t)wave * kQ8KBytes, (T / 64) * kQ8KBytes, lane);
}

}  // namespace q38
