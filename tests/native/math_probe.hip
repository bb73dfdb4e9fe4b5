/* Device-math probe for the GPU tests (test infrastructure; not part of
 * libq38hip).  Evaluates the device functions the kernels use
 * (qwen3.8-27b-in-c_amd/csrc/q38_math.h, q38_libm.h, q38_norm.h) on given inputs, and
 * forms an order-independent 64-bit checksum of q38_expf / q38_logf over all
 * 2^32 float inputs that tests/native/libm_check.c also forms on the host
 * with the C library's expf / logf. */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q38_math.h"
#include "q38_norm.h"

namespace {

enum { OP_EXP = 0, OP_LOG = 1, OP_SQRT = 2, OP_DIV = 3, OP_SIGMOID = 4, OP_SILU = 5, OP_SOFTPLUS = 6 };

__device__ float apply(int op, float x, float y)
{
    switch (op) {
    case OP_EXP: return q38_expf(x);
    case OP_LOG: return q38_logf(x);
    case OP_SQRT: return q38::sqrt_rn(x);
    case OP_DIV: return q38::div_rn(x, y);
    case OP_SIGMOID: return q38::sigmoidf_exact(x);
    case OP_SILU: return q38::siluf_exact(x);
    default: return q38::softplusf_exact(x);
    }
}

__global__ void eval_kernel(int op, float *out, const float *x, const float *y, uint64_t n)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = apply(op, x[i], y ? y[i] : 0.0f);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

constexpr int kThreads = 256;
constexpr int kBlocks = 4096;

/* sum over x of mix64((x << 32) | bits(f(x))), NaN results as 0x7fc00000 */
__global__ __launch_bounds__(kThreads) void checksum_kernel(int op, uint64_t *partial)
{
    __shared__ uint64_t red[kThreads];
    uint64_t acc = 0;
    const uint64_t stride = (uint64_t)kBlocks * kThreads;
    for (uint64_t x = (uint64_t)blockIdx.x * kThreads + threadIdx.x; x < (1ull << 32); x += stride) {
        const float v = __uint_as_float((uint32_t)x);
        const float r = op == OP_EXP ? q38_expf(v) : q38_logf(v);
        uint32_t bits = __float_as_uint(r);
        if (r != r) bits = 0x7fc00000u;
        acc += mix64((x << 32) | bits);
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

/* the mean of squares of the RMSNorm (q38_norm.h: parallel double sum,
 * sequential redo near a rounding boundary) over one vector */
__global__ __launch_bounds__(256) void mean_square_kernel(const float *x, int n, float *out)
{
    const float m = q38::block_sum_squares<256>(x, n, q38::MeanPost{(double)n});
    if (threadIdx.x == 0) *out = m;
}

}  // namespace

extern "C" {

/* *out = (float)(sum of x[i]^2 / n) as the kernels' RMSNorm forms it;
 * device pointers, synchronous. */
int probe_mean_square(const float *x, int n, float *out)
{
    if (n <= 0) return 0;
    mean_square_kernel<<<1, 256>>>(x, n, out);
    return hipDeviceSynchronize() == hipSuccess;
}

/* out/x/y are device pointers (y may be null); synchronous. */
int probe_eval(int op, float *out, const float *x, const float *y, uint64_t n)
{
    if (!n) return 1;
    eval_kernel<<<(unsigned)((n + 255) / 256), 256>>>(op, out, x, y, n);
    return hipDeviceSynchronize() == hipSuccess;
}

/* op 0 (expf) or 1 (logf); writes the checksum to *result; synchronous. */
int probe_checksum(int op, uint64_t *result)
{
    if (op != OP_EXP && op != OP_LOG) return 0;
    uint64_t *partial = nullptr;
    if (hipMalloc(&partial, kBlocks * sizeof(uint64_t)) != hipSuccess) return 0;
    checksum_kernel<<<kBlocks, kThreads>>>(op, partial);
    uint64_t host[kBlocks];
    const bool ok = hipMemcpy(host, partial, sizeof(host), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(partial);
    if (!ok) return 0;
    uint64_t sum = 0;
    for (int i = 0; i < kBlocks; ++i) sum += host[i];
    *result = sum;
    return 1;
}

}  // extern "C"
