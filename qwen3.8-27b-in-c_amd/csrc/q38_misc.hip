/* Q8_K activation quantiser, row argmax and greedy acceptance on gfx950. */
#include "q38_device.h"
#include "q38_q8k.h"

namespace q38 {

/* One wavefront per 256-element block, four elements per lane
 * (wave_quantize_q8k restates q38_quantize_q8_k).  ALIGNED: x is 16-byte
 * aligned, so each lane reads its four floats with one vector load. */
template <bool ALIGNED>
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *__restrict__ x,
                                                           uint8_t *__restrict__ out,
                                                           uint32_t nblocks)
{
    const int lane = threadIdx.x & 63;
    const uint32_t b = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    const float *src = x + static_cast<size_t>(b) * kQK;
    float v[4];
    if (ALIGNED) {
        const float4 v4 = reinterpret_cast<const float4 *>(src)[lane];
        v[0] = v4.x; v[1] = v4.y; v[2] = v4.z; v[3] = v4.w;
    } else {
        for (int i = 0; i < 4; ++i) v[i] = src[4 * lane + i];
    }
    wave_quantize_q8k(v, out + static_cast<size_t>(b) * kQ8KBytes, lane);
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
    /* every load first (an element past the row re-reads the last one and
     * is not compared), so the thread waits for memory once */
    float x[kArgmaxPerThread];
#pragma unroll
    for (int i = 0; i < kArgmaxPerThread; ++i) {
        const uint32_t e = base + i * kArgmaxThreads + threadIdx.x;
        x[i] = v[e < count ? e : count - 1];
    }
#pragma unroll
    for (int i = 0; i < kArgmaxPerThread; ++i) {
        const uint32_t e = base + i * kArgmaxThreads + threadIdx.x;
        if (e < count && better(x[i], e, bv, bi)) { bv = x[i]; bi = e; }
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
    /* the row's first element (the NaN rule) is read with the partials */
    const float first = values[static_cast<size_t>(row) * count];
    float bv = __builtin_nanf("");
    uint32_t bi = 0xffffffffu;
    for (uint32_t c = threadIdx.x; c < nchunks; c += kArgmaxThreads) {
        const float x = pv[static_cast<size_t>(row) * nchunks + c];
        const uint32_t i = pi[static_cast<size_t>(row) * nchunks + c];
        if (better(x, i, bv, bi)) { bv = x; bi = i; }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) out[row] = (first != first || bi == 0xffffffffu) ? 0u : bi;
}

/* Greedy acceptance (src/qwen38/qwen38_model.c:1662-1702): the leading
 * rows whose target argmax equals the draft are matched; the first
 * mismatching target becomes `next`; consumed = matched + 1, or all rows. */
__global__ void accept_kernel(uint32_t *__restrict__ result, const uint32_t *__restrict__ targets,
                              const uint32_t *__restrict__ drafts, uint32_t rows, const uint32_t *__restrict__ stop)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    /* a draft equal to the stop token ends the rows the reference checks
     * (qwen38_model.c:1640-1649) */
    if (stop) {
        const uint32_t st = *stop;
        for (uint32_t i = 0; i < rows; ++i)
            if (drafts[i] == st) {
                rows = i + 1;
                break;
            }
    }
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
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0)
        hipLaunchKernelGGL(quantize_q8k_kernel<true>, dim3((nblocks + 3) / 4), dim3(256), 0, stream, x, out, nblocks);
    else
        hipLaunchKernelGGL(quantize_q8k_kernel<false>, dim3((nblocks + 3) / 4), dim3(256), 0, stream, x, out, nblocks);
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
                   hipStream_t stream, const uint32_t *stop)
{
    hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, stream, result, targets, drafts, rows, stop);
}

/* dst[0 .. count) = row (*index - 1) of the `rows` rows of src (`stride`
 * floats apart); the index is clamped to 1 .. rows */
__global__ __launch_bounds__(256) void copy_row_kernel(float *__restrict__ dst, const float *__restrict__ src,
                                                       size_t stride, uint32_t count, const uint32_t *__restrict__ index,
                                                       uint32_t rows)
{
    const uint32_t r = min(max(*index, 1u), rows) - 1u;
    const float *row = src + (size_t)r * stride;
    for (uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 4u; i < count; i += gridDim.x * 1024u) {
        if (i + 4u <= count) {
            *reinterpret_cast<float4 *>(dst + i) = *reinterpret_cast<const float4 *>(row + i);
        } else {
            for (uint32_t k = i; k < count; ++k) dst[k] = row[k];
        }
    }
}

void launch_copy_row(float *dst, const float *src, size_t stride, uint32_t count, const uint32_t *index,
                     uint32_t rows, hipStream_t stream)
{
    const uint32_t blocks = (count + 1023u) / 1024u;
    hipLaunchKernelGGL(copy_row_kernel, dim3(blocks < 64u ? blocks : 64u), dim3(256), 0, stream, dst, src, stride,
                       count, index, rows);
}

/* The verify tail after argmax_partial_kernel, in one launch: the argmax of
 * every row from its partials (argmax_final_kernel's selection, one
 * wavefront per row), the greedy acceptance of accept_kernel, and the copy
 * of row consumed - 1 (copy_row_kernel).  Every workgroup reduces the
 * partials of every row (rows x nchunks pairs, a few KB from L2) and runs
 * the acceptance itself, so no workgroup waits for another; workgroup 0
 * writes the targets and the acceptance words, and each workgroup copies
 * its share of the row. */
constexpr uint32_t kTailMaxRows = 8;

__global__ __launch_bounds__(256) void verify_tail_kernel(const float *__restrict__ values, uint32_t count,
                                                          const float *__restrict__ pv, const uint32_t *__restrict__ pi,
                                                          uint32_t nchunks, uint32_t rows,
                                                          uint32_t *__restrict__ targets,
                                                          const uint32_t *__restrict__ drafts,
                                                          const uint32_t *__restrict__ stop,
                                                          uint32_t *__restrict__ result, float *__restrict__ dst)
{
    __shared__ uint32_t tgt[kTailMaxRows];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (uint32_t r = wave; r < rows; r += 4) {
        const float first = values[(size_t)r * count];   /* read with the partials */
        float bv = __builtin_nanf("");
        uint32_t bi = 0xffffffffu;
        for (uint32_t c = lane; c < nchunks; c += 64) {
            const float x = pv[(size_t)r * nchunks + c];
            const uint32_t i = pi[(size_t)r * nchunks + c];
            if (better(x, i, bv, bi)) { bv = x; bi = i; }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const uint32_t oi = __shfl_xor(bi, off, 64);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) tgt[r] = (first != first || bi == 0xffffffffu) ? 0u : bi;
    }
    __syncthreads();
    /* acceptance (src/qwen38/qwen38_model.c:1640-1702), as accept_kernel */
    uint32_t n = rows;
    if (stop) {
        const uint32_t st = *stop;
        for (uint32_t i = 0; i < rows; ++i)
            if (drafts[i] == st) {
                n = i + 1;
                break;
            }
    }
    uint32_t matched = 0, next = 0;
    while (matched < n) {
        if (tgt[matched] != drafts[matched]) { next = tgt[matched]; break; }
        ++matched;
    }
    if (matched == n) next = drafts[n - 1];
    const uint32_t consumed = matched < n ? matched + 1u : n;
    if (blockIdx.x == 0) {
        if (threadIdx.x < rows) targets[threadIdx.x] = tgt[threadIdx.x];
        if (threadIdx.x == 0) {
            result[0] = consumed;
            result[1] = matched;
            result[2] = next;
        }
        if (threadIdx.x < matched) result[3 + threadIdx.x] = drafts[threadIdx.x];
        if (threadIdx.x == 0 && matched < n) result[3 + matched] = next;
    }
    const float *row = values + (size_t)(consumed - 1u) * count;
    for (uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 4u; i < count; i += gridDim.x * 1024u) {
        if (i + 4u <= count) {
            *reinterpret_cast<float4 *>(dst + i) = *reinterpret_cast<const float4 *>(row + i);
        } else {
            for (uint32_t k = i; k < count; ++k) dst[k] = row[k];
        }
    }
}

bool launch_verify_tail(const float *values, uint32_t count, uint32_t rows, float *pv, uint32_t *pi,
                        uint32_t *targets, const uint32_t *drafts, const uint32_t *stop, uint32_t *result, float *dst,
                        hipStream_t stream)
{
    if (rows == 0 || rows > kTailMaxRows || (count & 3u) != 0) return false;
    const uint32_t chunks = argmax_chunks(count);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(chunks, rows), dim3(kArgmaxThreads), 0, stream, values, count, pv,
                       pi);
    const uint32_t blocks = (count + 1023u) / 1024u;
    hipLaunchKernelGGL(verify_tail_kernel, dim3(blocks < 64u ? blocks : 64u), dim3(256), 0, stream, values, count, pv,
                       pi, chunks, rows, targets, drafts, stop, result, dst);
    return true;
}

}  // namespace q38
