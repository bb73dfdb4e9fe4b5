/* Q8_K activation quantiser, row argmax and greedy acceptance on gfx950. */
#include "q38_device.h"

namespace q38 {

/* One wavefront per 256-element block, four elements per lane.
 * Restates q38_quantize_q8_k (src/qwen38/qwen38_quant.c:50-88): the block
 * maximum is the signed value of the FIRST element holding the largest |x|
 * (NaN never wins), inverse = -127/max (IEEE division), quants are
 * round-half-even via the 1.5*2^23 shift and clamped above at 127, sums are
 * per 16 elements, scale = 1/inverse.  An all-zero block stores zeros. */
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *__restrict__ x,
                                                           uint8_t *__restrict__ out,
                                                           uint32_t nblocks)
{
    const int lane = threadIdx.x & 63;
    const uint32_t b = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    const float *src = x + static_cast<size_t>(b) * kQK + 4 * lane;
    const float v[4] = {src[0], src[1], src[2], src[3]};

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
    uint8_t *blk = out + static_cast<size_t>(b) * kQ8KBytes;
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

/* First-maximum selection: NaN never wins, ties go to the lower index.  With
 * a NaN at index 0 the sequential scan keeps index 0 (every comparison with
 * the NaN maximum is false); the final pass applies that rule. */
__device__ __forceinline__ bool better(float va, uint32_t ia, float vb, uint32_t ib)
{
    /* is (va, ia) better than (vb, ib)? */
    if (va != va) return false;
    if (vb != vb) return true;
    return va > vb || (va == vb && ia < ib);
}

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPerThread = 16;
constexpr int kArgmaxChunk = kArgmaxThreads * kArgmaxPerThread;

__device__ __forceinline__ void block_best(float &bv, uint32_t &bi)
{
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ uint32_t si[kArgmaxThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w)
            if (better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    }
}

/* pass 1: grid (chunks, rows); each workgroup reduces 4096 elements */
__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(
    const float *__restrict__ values, uint32_t count, float *__restrict__ pv, uint32_t *__restrict__ pi)
{
    const uint32_t row = blockIdx.y, chunk = blockIdx.x;
    const float *v = values + static_cast<size_t>(row) * count;
    float bv = __builtin_nanf("");
    uint32_t bi = 0xffffffffu;
    const uint32_t base = chunk * kArgmaxChunk;
    for (int i = 0; i < kArgmaxPerThread; ++i) {
        const uint32_t e = base + i * kArgmaxThreads + threadIdx.x;
        if (e < count) {
            const float x = v[e];
            if (better(x, e, bv, bi)) { bv = x; bi = e; }
        }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        pv[static_cast<size_t>(row) * gridDim.x + chunk] = bv;
        pi[static_cast<size_t>(row) * gridDim.x + chunk] = bi;
    }
}

/* pass 2: one workgroup per row over the partials */
__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(
    const float *__restrict__ values, uint32_t count, const float *__restrict__ pv,
    const uint32_t *__restrict__ pi, uint32_t nchunks, uint32_t *__restrict__ out)
{
    const uint32_t row = blockIdx.x;
    float bv = __builtin_nanf("");
    uint32_t bi = 0xffffffffu;
    for (uint32_t c = threadIdx.x; c < nchunks; c += kArgmaxThreads) {
        const float x = pv[static_cast<size_t>(row) * nchunks + c];
        const uint32_t i = pi[static_cast<size_t>(row) * nchunks + c];
        if (better(x, i, bv, bi)) { bv = x; bi = i; }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        const float first = values[static_cast<size_t>(row) * count];
        out[row] = (first != first || bi == 0xffffffffu) ? 0u : bi;
    }
}

/* Greedy acceptance (src/qwen38/qwen38_model.c:1662-1702): the leading
 * rows whose target argmax equals the draft are matched; the first
 * mismatching target becomes `next`; consumed = matched + 1, or all rows. */
__global__ void accept_kernel(uint32_t *__restrict__ result, const uint32_t *__restrict__ targets,
                              const uint32_t *__restrict__ drafts, uint32_t rows)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    uint32_t matched = 0, next = 0;
    while (matched < rows) {
        if (targets[matched] != drafts[matched]) { next = targets[matched]; break; }
        ++matched;
    }
    if (matched == rows) next = drafts[rows - 1];
    const uint32_t consumed = matched < rows ? matched + 1u : rows;
    result[0] = consumed;
    result[1] = matched;
    result[2] = next;
    for (uint32_t i = 0; i < matched; ++i) result[3 + i] = drafts[i];
    if (matched < rows) result[3 + matched] = next;
}

void launch_quantize(const float *x, uint8_t *out, uint32_t nblocks, hipStream_t stream)
{
    hipLaunchKernelGGL(quantize_q8k_kernel, dim3((nblocks + 3) / 4), dim3(256), 0, stream, x, out, nblocks);
}

uint32_t argmax_chunks(uint32_t count) { return (count + kArgmaxChunk - 1) / kArgmaxChunk; }

void launch_argmax(const float *values, uint32_t count, uint32_t rows, float *pv, uint32_t *pi,
                   uint32_t *out, hipStream_t stream)
{
    const uint32_t chunks = argmax_chunks(count);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(chunks, rows), dim3(kArgmaxThreads), 0, stream,
                       values, count, pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(kArgmaxThreads), 0, stream,
                       values, count, pv, pi, chunks, out);
}

void launch_accept(uint32_t *result, const uint32_t *targets, const uint32_t *drafts, uint32_t rows,
                   hipStream_t stream)
{
    hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, stream, result, targets, drafts, rows);
}

}  // namespace q38
