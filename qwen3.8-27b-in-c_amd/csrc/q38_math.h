/* Scalar fp32 functions of the reference model (src/qwen38/qwen38_model.c),
 * device side, in the reference's operation order: one rounding per
 * operation, correctly rounded division and square root, and the exact
 * expf/logf restatements of q38_libm.h. */
#pragma once

#include "q38_device.h"
#include "q38_libm.h"

namespace q38 {

/* scale = 1 / sqrtf(mean + 1e-6f), qwen38_model.c:432-433 */
__device__ __forceinline__ float rms_scale(float mean)
{
    return div_rn(1.0f, sqrt_rn(__fadd_rn(mean, 1e-6f)));
}

__device__ __forceinline__ float sigmoidf_exact(float v)   /* :437-440 */
{
    return div_rn(1.0f, __fadd_rn(1.0f, q38_expf(-v)));
}

__device__ __forceinline__ float siluf_exact(float v)      /* :442-445 */
{
    return div_rn(v, __fadd_rn(1.0f, q38_expf(-v)));
}

__device__ __forceinline__ float softplusf_exact(float v)  /* :551-555 */
{
    if (v > 20.0f) return v;
    return q38_logf(__fadd_rn(1.0f, q38_expf(v)));
}

}  // namespace q38
