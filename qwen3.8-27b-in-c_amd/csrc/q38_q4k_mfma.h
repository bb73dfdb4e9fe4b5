/* fp16 matrix-core building blocks of the Q4_K x Q8_K kernels
 * (q38_tiled32.hip, q38_wide.hip): 4-bit quants times their 6-bit sub-block
 * scale as exact fp16, int8 activations as exact fp16, and the buffer
 * resource of the raw loads. */
#pragma once

#include "q38_device.h"

namespace q38 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef short short2v __attribute__((ext_vector_type(2)));

constexpr int kRows16 = 16;
constexpr int kBlockBytes = 144;
constexpr int kTileBlock = kRows16 * kBlockBytes;   /* 2304 bytes: one block of a 16-row tile */
constexpr uint32_t kRawBuffer = 0x00020000u;        /* raw 32-bit buffer resource (gfx9) */

__device__ __forceinline__ half2v h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

/* fp16 pair (n, n) for the byte n of w that `sel` picks (sel = 0x07000700
 * + k * 0x00010001 for byte k): (1024 + n) - 1024 */
__device__ __forceinline__ half2v pair_byte(uint32_t w, uint32_t sel)
{
    const half2v v = h2(__builtin_amdgcn_perm(0x64646464u, w, sel));
    return v - (half2v){(_Float16)1024.0f, (_Float16)1024.0f};
}

struct Scale {
    half2v sl, nl, sh16, nh;
};

/* the 8 quants of one dword as fp16 sc * q, element order per half
 * u = 0, 2, 1, 3 (the activations use the same order) */
__device__ __forceinline__ half8 dequant(uint32_t wd, const Scale &s, uint32_t kMask, uint32_t kMaskHi,
                                         uint32_t kMagic)
{
    const uint32_t w8 = wd >> 8;
    const half2v b0 = __builtin_elementwise_fma(h2((wd & kMask) | kMagic), s.sl, s.nl);
    const half2v b1 = __builtin_elementwise_fma(h2((w8 & kMask) | kMagic), s.sl, s.nl);
    const half2v b2 = __builtin_elementwise_fma(h2((wd & kMaskHi) | kMagic), s.sh16, s.nh);
    const half2v b3 = __builtin_elementwise_fma(h2((w8 & kMaskHi) | kMagic), s.sh16, s.nh);
    half8 v;
    v[0] = b0[0]; v[1] = b0[1]; v[2] = b1[0]; v[3] = b1[1];
    v[4] = b2[0]; v[5] = b2[1]; v[6] = b3[0]; v[7] = b3[1];
    return v;
}

/* 8 int8 activations (4 low-nibble elements, 4 high) as fp16 */
__device__ __forceinline__ half8 act8(uint32_t lo, uint32_t hi)
{
    const half2v k1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t ua = lo ^ 0x80808080u, ub = hi ^ 0x80808080u;
    const half2v a02 = h2(__builtin_amdgcn_perm(0x64646464u, ua, 0x04020400u)) + k1152;
    const half2v a13 = h2(__builtin_amdgcn_perm(0x64646464u, ua, 0x04030401u)) + k1152;
    const half2v b02 = h2(__builtin_amdgcn_perm(0x64646464u, ub, 0x04020400u)) + k1152;
    const half2v b13 = h2(__builtin_amdgcn_perm(0x64646464u, ub, 0x04030401u)) + k1152;
    half8 v;
    v[0] = a02[0]; v[1] = a02[1]; v[2] = a13[0]; v[3] = a13[1];
    v[4] = b02[0]; v[5] = b02[1]; v[6] = b13[0]; v[7] = b13[1];
    return v;
}

}  // namespace
}  // namespace q38
