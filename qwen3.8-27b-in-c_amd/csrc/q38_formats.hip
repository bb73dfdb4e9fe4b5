/* GEMV / small-M GEMM, float-input GEMV and row decode for the remaining
 * GGUF matrix formats of the reference model (src/qwen38/qwen38_model.c:
 * 172-189): Q2_K, Q3_K, Q5_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S,
 * IQ4_XS, IQ4_NL, IQ1_S against Q8_K activations, and F32, F16, BF16, Q8_0
 * (plus the K-quants and IQ4_NL) against fp32 activations.
 *
 * Q8_K path.  Each of the reference's AVX2 kernels (qwen38_quant.c:510-1253,
 * 1636-1725) keeps eight fp32 lanes per row; for every super-block, lane l
 * gets d * W[l], where W[l] is the exact integer sum over bytes 4l..4l+3 of
 * each 32-element group, each group-half scaled by its integer sub-block
 * scale.  Here eight GPU lanes own a row's eight accumulator lanes (a
 * wavefront holds eight rows): each decodes the four weights of each group
 * it needs into a packed int8 dword (grid value and sign folded in),
 * multiplies with v_dot4_i32_i8 against the activation dword, scales, and
 * runs its fmaf chain.  The eight lanes then add in the reference's tree
 * ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)); Q2_K and Q5_K add their
 * scalar min chain, IQ1_S 0.125 times its scalar correction sum, and IQ4_NL
 * applies one fp32 scale per 32-element group (eight FMAs per block).
 *
 * Float path (q38_dot_row, :2768-2810): one thread per row runs the row's
 * single fmaf chain in the reference's element order; the weight
 * expression of every element is rounded as the reference rounds it.
 *
 * Row decode (q38_tensor_row_f32, :3185-3223): F32 copied, F16 / BF16
 * converted; otherwise each element is the float dot of its block with a
 * unit vector, which is the element's weight expression (a -0 result
 * becoming +0 through the +0 accumulator), or NaN when another weight of
 * the block is not finite (its product with 0 is NaN; written with the bit
 * pattern x86 gives, 0xffc00000).
 */
#include "q38_device.h"
#include "q38_kernels.h"
#include "q38_iq_grids.inc"

namespace q38 {

namespace {

/* ---- codebooks, expanded at compile time --------------------------------- */

#define Q38_IQ2_LEVEL(i) ((i) == 0 ? 8u : (i) == 1 ? 25u : 43u)
#define Q38_IQ2_BYTE(c, k) Q38_IQ2_LEVEL(((c) >> (2 * (k))) & 3)
#define Q38_IQ2_HALF(c, h) \
    (Q38_IQ2_BYTE(c, 4 * (h)) | Q38_IQ2_BYTE(c, 4 * (h) + 1) << 8 | Q38_IQ2_BYTE(c, 4 * (h) + 2) << 16 | \
     Q38_IQ2_BYTE(c, 4 * (h) + 3) << 24)
#define Q38_IQ2_ENTRY(c) Q38_IQ2_HALF(c, 0), Q38_IQ2_HALF(c, 1),
#define Q38_IQ3XXS_LEVEL(i) ((i) == 7 ? 62u : 8u * (i) + 4u)
#define Q38_IQ3XXS_ENTRY(c) \
    (Q38_IQ3XXS_LEVEL((c) & 7) | Q38_IQ3XXS_LEVEL(((c) >> 3) & 7) << 8 | Q38_IQ3XXS_LEVEL(((c) >> 6) & 7) << 16 | \
     Q38_IQ3XXS_LEVEL(((c) >> 9) & 7) << 24),
#define Q38_IQ3S_LEVEL(i) (2u * (i) + 1u)
#define Q38_IQ3S_ENTRY(c) \
    (Q38_IQ3S_LEVEL((c) & 7) | Q38_IQ3S_LEVEL(((c) >> 3) & 7) << 8 | Q38_IQ3S_LEVEL(((c) >> 6) & 7) << 16 | \
     Q38_IQ3S_LEVEL(((c) >> 9) & 7) << 24),

/* IQ2 grids: entry e, elements 4h..4h+3 at [2e + h]; IQ3 grids: entry e at [e] */
__device__ const uint32_t g_iq2xxs[512] = {Q38_IQ2XXS_CODES(Q38_IQ2_ENTRY)};
__device__ const uint32_t g_iq2xs[1024] = {Q38_IQ2XS_CODES(Q38_IQ2_ENTRY)};
__device__ const uint32_t g_iq2s[2048] = {Q38_IQ2S_CODES(Q38_IQ2_ENTRY)};
__device__ const uint32_t g_iq3xxs[256] = {Q38_IQ3XXS_CODES(Q38_IQ3XXS_ENTRY)};
__device__ const uint32_t g_iq3s[512] = {Q38_IQ3S_CODES(Q38_IQ3S_ENTRY)};

constexpr int8_t kIq4nl[16] = {Q38_IQ4NL_VALUES};
constexpr uint32_t pack4(int a, int b, int c, int d)
{
    return (uint32_t)(uint8_t)a | (uint32_t)(uint8_t)b << 8 | (uint32_t)(uint8_t)c << 16 | (uint32_t)(uint8_t)d << 24;
}
constexpr uint32_t kIq4nlT0 = pack4(kIq4nl[0], kIq4nl[1], kIq4nl[2], kIq4nl[3]);
constexpr uint32_t kIq4nlT1 = pack4(kIq4nl[4], kIq4nl[5], kIq4nl[6], kIq4nl[7]);
constexpr uint32_t kIq4nlT2 = pack4(kIq4nl[8], kIq4nl[9], kIq4nl[10], kIq4nl[11]);
constexpr uint32_t kIq4nlT3 = pack4(kIq4nl[12], kIq4nl[13], kIq4nl[14], kIq4nl[15]);

/* GGML type ids (include/qwen38/qwen38_gguf.h:29-52) */
enum : int {
    kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ2K = 10, kQ3K = 11, kQ5K = 13,
    kIQ2XXS = 16, kIQ2XS = 17, kIQ3XXS = 18, kIQ1S = 19, kIQ4NL = 20, kIQ3S = 21, kIQ2S = 22, kIQ4XS = 23,
    kBF16 = 30
};

__device__ __forceinline__ uint32_t ld16(const uint8_t *p)
{
    return (uint32_t)p[0] | (uint32_t)p[1] << 8;
}
/* 4 bytes at a 2-byte aligned address */
__device__ __forceinline__ uint32_t ld32u(const uint8_t *p)
{
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    return (uint32_t)h[0] | (uint32_t)h[1] << 16;
}
__device__ __forceinline__ uint32_t ld32a(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

/* bytes of 0xff where bit k of `bits` (k < 4) is set */
__device__ __forceinline__ uint32_t byte_mask4(uint32_t bits)
{
    return ((bits & 15u) * 0x00204081u & 0x01010101u) * 0xffu;
}

/* negate the bytes selected by mask (values 1..127, so no byte borrows) */
__device__ __forceinline__ uint32_t negate_bytes(uint32_t v, uint32_t mask)
{
    return (v ^ mask) + (mask & 0x01010101u);
}

/* IQ2/IQ3 sign byte of a 7-bit index: even parity in bit 7 (ksigns_iq2xs) */
__device__ __forceinline__ uint32_t sign_byte(uint32_t index)
{
    index &= 127u;
    return index | (uint32_t)(__popc(index) & 1) << 7;
}

/* nibbles (one per byte) through the IQ4_NL table */
__device__ __forceinline__ uint32_t iq4nl_bytes(uint32_t nib)
{
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4nlT1, kIq4nlT0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4nlT3, kIq4nlT2, sel);
    const uint32_t high = ((nib >> 3) & 0x01010101u) * 0xffu;
    return (hi & high) | (lo & ~high);
}

__device__ __forceinline__ void k4_scale_min(int i, const uint8_t *p, int &sc, int &m)
{
    if (i < 4) {
        sc = p[i] & 63;
        m = p[i + 4] & 63;
    } else {
        sc = (p[i + 4] & 15) | ((p[i - 4] >> 6) << 4);
        m = (p[i + 4] >> 4) | ((p[i] >> 6) << 4);
    }
}

/* ---- Q8_K path: one lane's share of a super-block ------------------------- */

/* The lane's packed weights q[g] (elements 32g + 4l .. +3) and integer
 * scales s[g] of the eight groups, the block's scale factor before the
 * activation scale, and (Q2_K, Q5_K: dmin; IQ1_S: unused) the second
 * factor.  IQ4_NL keeps its eight group scales in gd[]. */
struct LaneBlock {
    uint32_t q[8];
    int s[8];
    float d, dmin;
    float gd[8];
};

template <int T>
__device__ __forceinline__ uint32_t block_bytes()
{
    switch (T) {
    case kQ2K: return 84;
    case kQ3K: return 110;
    case kQ5K: return 176;
    case kIQ2XXS: return 66;
    case kIQ2XS: return 74;
    case kIQ2S: return 82;
    case kIQ3XXS: return 98;
    case kIQ3S: return 110;
    case kIQ4XS: return 136;
    case kIQ4NL: return 144;
    default: return 50;   /* IQ1_S */
    }
}

template <int T>
__device__ __forceinline__ void decode_lane(const uint8_t *blk, int l, const uint32_t *iq1s_grid, LaneBlock &b)
{
    const int hi = l >= 4;
    if constexpr (T == kQ2K) {
        /* qwen38_quant.c:510-585 */
        const uint32_t d0 = ld32a(blk + 16 + 4 * l), d1 = ld32a(blk + 48 + 4 * l);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            b.q[g] = ((g < 4 ? d0 : d1) >> (2 * (g & 3))) & 0x03030303u;
            b.s[g] = blk[2 * g + hi] & 15;
        }
        b.d = f16_to_f32(ld16(blk + 80));
        b.dmin = f16_to_f32(ld16(blk + 82));
    } else if constexpr (T == kQ3K) {
        /* :587-662; scales :319-329 */
        const uint32_t hm = ld32u(blk + 4 * l);
        const uint32_t d0 = ld32u(blk + 32 + 4 * l), d1 = ld32u(blk + 64 + 4 * l);
        const uint8_t *sc = blk + 96;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t low = ((g < 4 ? d0 : d1) >> (2 * (g & 3))) & 0x03030303u;
            const uint32_t absent = ~(hm >> g) & 0x01010101u;
            b.q[g] = low + absent * 0xfcu;   /* minus 4 where the high bit is clear */
            const int i = 2 * g + hi;
            const int lo4 = i < 8 ? sc[i] & 15 : sc[i - 8] >> 4;
            const int hi2 = (sc[8 + i % 4] >> (2 * (i / 4))) & 3;
            b.s[g] = (lo4 | hi2 << 4) - 32;
        }
        b.d = f16_to_f32(ld16(blk + 108));
    } else if constexpr (T == kQ5K) {
        /* :1636-1725 */
        const uint32_t qh = ld32a(blk + 16 + 4 * l);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t qs = ld32a(blk + 48 + 32 * c + 4 * l);
            b.q[2 * c] = (qs & 0x0f0f0f0fu) + (((qh >> (2 * c)) & 0x01010101u) << 4);
            b.q[2 * c + 1] = ((qs >> 4) & 0x0f0f0f0fu) + (((qh >> (2 * c + 1)) & 0x01010101u) << 4);
            int sc0, m0, sc1, m1;
            k4_scale_min(2 * c, blk + 4, sc0, m0);
            k4_scale_min(2 * c + 1, blk + 4, sc1, m1);
            b.s[2 * c] = sc0;
            b.s[2 * c + 1] = sc1;
        }
        b.d = f16_to_f32(ld16(blk));
        b.dmin = f16_to_f32(ld16(blk + 2));
    } else if constexpr (T == kIQ2XXS) {
        /* :758-822 */
        const int sec = l >> 1, half = l & 1;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint8_t *codes = blk + 2 + 8 * g;
            const uint32_t meta = ld32u(codes + 4);
            const uint32_t grid = g_iq2xxs[2 * codes[sec] + half];
            const uint32_t signs = sign_byte(meta >> (7 * sec)) >> (4 * half);
            b.q[g] = negate_bytes(grid, byte_mask4(signs));
            b.s[g] = 1 + 2 * (int)(meta >> 28);
        }
        b.d = 0.125f * f16_to_f32(ld16(blk));
    } else if constexpr (T == kIQ2XS) {
        /* :824-893 */
        const int sec = l >> 1, half = l & 1;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t code = ld16(blk + 2 + 8 * g + 2 * sec);
            const uint32_t grid = g_iq2xs[2 * (code & 511u) + half];
            b.q[g] = negate_bytes(grid, byte_mask4(sign_byte(code >> 9) >> (4 * half)));
            const uint32_t sc = blk[66 + g];
            b.s[g] = 1 + 2 * (int)(hi ? sc >> 4 : sc & 15u);
        }
        b.d = 0.125f * f16_to_f32(ld16(blk));
    } else if constexpr (T == kIQ2S) {
        /* :664-756 */
        const int sec = l >> 1, half = l & 1;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t index = blk[2 + 4 * g + sec] | (((uint32_t)blk[66 + g] << (8 - 2 * sec)) & 0x300u);
            const uint32_t grid = g_iq2s[2 * index + half];
            b.q[g] = negate_bytes(grid, byte_mask4((uint32_t)blk[34 + 4 * g + sec] >> (4 * half)));
            const uint32_t sc = blk[74 + g];
            b.s[g] = 1 + 2 * (int)(hi ? sc >> 4 : sc & 15u);
        }
        b.d = 0.125f * f16_to_f32(ld16(blk));
    } else if constexpr (T == kIQ3XXS) {
        /* :895-976 */
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t packed = ld32u(blk + 66 + 4 * g);
            const uint32_t grid = g_iq3xxs[blk[2 + 8 * g + l]];
            const uint32_t signs = sign_byte(packed >> (7 * (l >> 1))) >> (4 * (l & 1));
            b.q[g] = negate_bytes(grid, byte_mask4(signs));
            b.s[g] = 1 + 2 * (int)(packed >> 28);
        }
        b.d = 0.25f * f16_to_f32(ld16(blk));
    } else if constexpr (T == kIQ3S) {
        /* :978-1061 */
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t index = blk[2 + 8 * g + l] | (((uint32_t)(blk[66 + g] >> l) & 1u) << 8);
            const uint32_t signs = (uint32_t)blk[74 + 4 * g + (l >> 1)] >> (4 * (l & 1));
            b.q[g] = negate_bytes(g_iq3s[index], byte_mask4(signs));
            b.s[g] = 1 + 2 * (int)((blk[106 + g / 2] >> (4 * (g & 1))) & 15u);
        }
        b.d = f16_to_f32(ld16(blk));
    } else if constexpr (T == kIQ4XS) {
        /* :1063-1127 */
        const uint32_t scale_high = ld16(blk + 2);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t qs = ld32a(blk + 8 + 16 * g + 4 * (l & 3));
            b.q[g] = iq4nl_bytes(hi ? qs >> 4 : qs);
            const int scale = (int)((blk[4 + g / 2] >> (4 * (g & 1))) & 15u) | (int)(((scale_high >> (2 * g)) & 3u) << 4);
            b.s[g] = scale - 32;
        }
        b.d = f16_to_f32(ld16(blk));
    } else if constexpr (T == kIQ4NL) {
        /* :1129-1175: eight 18-byte blocks */
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t qs = ld32u(blk + 18 * g + 2 + 4 * (l & 3));
            b.q[g] = iq4nl_bytes(hi ? qs >> 4 : qs);
            b.s[g] = 1;
            b.gd[g] = f16_to_f32(ld16(blk + 18 * g));
        }
    } else {
        /* IQ1_S, :1177-1253 */
        const int sec = l >> 1, half = l & 1;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t high = ld16(blk + 34 + 2 * g);
            const uint32_t index = blk[2 + 4 * g + sec] | (((high >> (3 * sec)) & 7u) << 8);
            b.q[g] = iq1s_grid[2 * index + half];
            b.s[g] = 1 + 2 * (int)((high >> 12) & 7u);
        }
        b.d = f16_to_f32(ld16(blk));
    }
}

/* the block's integer min (Q2_K, Q5_K) or correction (IQ1_S) term for one
 * token's Q8_K block */
template <int T>
__device__ __forceinline__ int block_extra(const uint8_t *blk, const uint8_t *xb)
{
    const int16_t *sums = reinterpret_cast<const int16_t *>(xb + 260);
    int extra = 0;
    if constexpr (T == kQ2K) {
#pragma unroll
        for (int i = 0; i < 16; ++i) extra += (blk[i] >> 4) * sums[i];
    } else if constexpr (T == kQ5K) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            int sc0, m0, sc1, m1;
            k4_scale_min(2 * c, blk + 4, sc0, m0);
            k4_scale_min(2 * c + 1, blk + 4, sc1, m1);
            extra += m0 * (sums[4 * c] + sums[4 * c + 1]) + m1 * (sums[4 * c + 2] + sums[4 * c + 3]);
        }
    } else if constexpr (T == kIQ1S) {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t high = ld16(blk + 34 + 2 * g);
            const int scale = 1 + 2 * (int)((high >> 12) & 7u);
            extra += (high & 0x8000u ? -scale : scale) * (sums[2 * g] + sums[2 * g + 1]);
        }
    }
    return extra;
}

template <int T>
constexpr bool has_extra()
{
    return T == kQ2K || T == kQ5K || T == kIQ1S;
}

/* y[t * ldy + row] for t < MT: eight rows per wavefront, eight lanes per row */
template <int T, int MT>
__global__ __launch_bounds__(256) void gemv_format_kernel(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                          float *__restrict__ y, uint32_t ldy, uint32_t rows,
                                                          uint32_t nb, const uint32_t *__restrict__ iq1s_grid)
{
    const int lane = threadIdx.x & 63, l = lane & 7;
    const uint32_t row = (blockIdx.x * 256u + threadIdx.x) >> 3;
    const uint32_t r = row < rows ? row : rows - 1;
    const uint32_t bytes = block_bytes<T>();
    const uint8_t *wr = w + (size_t)r * nb * bytes;
    float acc[MT], scalar[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = scalar[t] = 0.0f;

    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = wr + (size_t)b * bytes;
        LaneBlock lb;
        decode_lane<T>(blk, l, iq1s_grid, lb);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint8_t *xb = x + ((size_t)t * nb + b) * kQ8KBytes;
            const float xs = *reinterpret_cast<const float *>(xb);
            const uint32_t *aq = reinterpret_cast<const uint32_t *>(xb + 4);
            if constexpr (T == kIQ4NL) {
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    const int wg = dot4z((int)lb.q[g], (int)aq[8 * g + l]);
                    acc[t] = __builtin_fmaf(__fmul_rn(lb.gd[g], xs), (float)wg, acc[t]);
                }
            } else {
                int wsum = 0;
#pragma unroll
                for (int g = 0; g < 8; ++g) wsum += lb.s[g] * dot4z((int)lb.q[g], (int)aq[8 * g + l]);
                const float d = __fmul_rn(lb.d, xs);
                acc[t] = __builtin_fmaf(d, (float)wsum, acc[t]);
                if constexpr (T == kQ2K || T == kQ5K) {
                    const float dmin = __fmul_rn(lb.dmin, xs);
                    scalar[t] = __builtin_fmaf(-dmin, (float)block_extra<T>(blk, xb), scalar[t]);
                } else if constexpr (T == kIQ1S) {
                    scalar[t] = __fadd_rn(scalar[t], __fmul_rn(d, (float)block_extra<T>(blk, xb)));
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        /* ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)), qwen38_quant.c:303-310 */
        float v = __fadd_rn(acc[t], __shfl_xor(acc[t], 4, 64));
        v = __fadd_rn(v, __shfl_xor(v, 2, 64));
        v = __fadd_rn(v, __shfl_xor(v, 1, 64));
        if constexpr (T == kIQ1S) v = __fadd_rn(v, __fmul_rn(0.125f, scalar[t]));
        else if constexpr (has_extra<T>()) v = __fadd_rn(v, scalar[t]);
        if (l == 0 && row < rows) y[(size_t)t * ldy + row] = v;
    }
}

template <int T, int MT>
void launch_format_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t nb,
                         const void *grid, hipStream_t stream)
{
    hipLaunchKernelGGL((gemv_format_kernel<T, MT>), dim3((rows + 31) / 32), dim3(256), 0, stream, w, x, y, ldy, rows,
                       nb, static_cast<const uint32_t *>(grid));
}

template <int T>
void launch_format_m(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t nb,
                     const void *grid, hipStream_t stream)
{
    switch (m) {
    case 1: launch_format_typed<T, 1>(w, x, y, ldy, rows, nb, grid, stream); break;
    case 2: launch_format_typed<T, 2>(w, x, y, ldy, rows, nb, grid, stream); break;
    case 3: launch_format_typed<T, 3>(w, x, y, ldy, rows, nb, grid, stream); break;
    case 4: launch_format_typed<T, 4>(w, x, y, ldy, rows, nb, grid, stream); break;
    case 5: launch_format_typed<T, 5>(w, x, y, ldy, rows, nb, grid, stream); break;
    case 6: launch_format_typed<T, 6>(w, x, y, ldy, rows, nb, grid, stream); break;
    case 7: launch_format_typed<T, 7>(w, x, y, ldy, rows, nb, grid, stream); break;
    default: launch_format_typed<T, 8>(w, x, y, ldy, rows, nb, grid, stream); break;
    }
}

/* ---- float path ------------------------------------------------------------ */

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }

/* The chain over one row for MT tokens: total_t = fmaf(w_e, x_t[e], total_t)
 * for every element e in the reference's order. */
template <int T, int MT>
__device__ __forceinline__ void float_chain(const uint8_t *row, const float *x, uint32_t width, float *total)
{
    auto step = [&](float wv, uint32_t e) {
#pragma unroll
        for (int t = 0; t < MT; ++t) total[t] = __builtin_fmaf(wv, x[(size_t)t * width + e], total[t]);
    };
    if constexpr (T == kF32) {
        for (uint32_t e = 0; e < width; ++e) step(*reinterpret_cast<const float *>(row + 4 * (size_t)e), e);
    } else if constexpr (T == kF16) {
        for (uint32_t e = 0; e < width; ++e) step(f16_to_f32(ld16(row + 2 * (size_t)e)), e);
    } else if constexpr (T == kBF16) {
        for (uint32_t e = 0; e < width; ++e) step(bf16_to_f32(ld16(row + 2 * (size_t)e)), e);
    } else if constexpr (T == kQ8_0) {
        /* :496-507 */
        for (uint32_t base = 0; base < width; base += 32, row += 34) {
            const float d = f16_to_f32(ld16(row));
            for (int i = 0; i < 32; ++i) step(__fmul_rn(d, (float)(int8_t)row[2 + i]), base + i);
        }
    } else if constexpr (T == kIQ4NL) {
        /* :2796-2807 */
        for (uint32_t base = 0; base < width; base += 32, row += 18) {
            const float d = f16_to_f32(ld16(row));
            for (int j = 0; j < 16; ++j) {
                step(__fmul_rn(d, (float)kIq4nl[row[2 + j] & 15]), base + j);
                step(__fmul_rn(d, (float)kIq4nl[row[2 + j] >> 4]), base + 16 + j);
            }
        }
    } else if constexpr (T == kQ2K) {
        /* :331-362 */
        for (uint32_t base = 0; base < width; base += 256, row += 84) {
            const float d = f16_to_f32(ld16(row + 80)), dmin = f16_to_f32(ld16(row + 82));
            for (int i = 0; i < 16; ++i) {
                const float scale = __fmul_rn(d, (float)(row[i] & 15)), minimum = __fmul_rn(dmin, (float)(row[i] >> 4));
                const int half = i / 8, field = (i % 8) / 2, part = i % 2;
                for (int j = 0; j < 16; ++j) {
                    const int q = (row[16 + 32 * half + 16 * part + j] >> (2 * field)) & 3;
                    step(__fsub_rn(__fmul_rn(scale, (float)q), minimum), base + 16 * i + j);
                }
            }
        }
    } else if constexpr (T == kQ3K) {
        /* :364-394 */
        for (uint32_t base = 0; base < width; base += 256, row += 110) {
            const float d = f16_to_f32(ld16(row + 108));
            const uint8_t *sc = row + 96;
            for (int g = 0; g < 8; ++g) {
                const int half = g / 4, field = g % 4;
                for (int j = 0; j < 32; ++j) {
                    const int i = 2 * g + j / 16;
                    const int s = ((i < 8 ? sc[i] & 15 : sc[i - 8] >> 4) | (((sc[8 + i % 4] >> (2 * (i / 4))) & 3) << 4)) - 32;
                    const int q = ((row[32 + 32 * half + j] >> (2 * field)) & 3) - ((row[j] >> g) & 1 ? 0 : 4);
                    step(__fmul_rn(__fmul_rn(d, (float)s), (float)q), base + 32 * g + j);
                }
            }
        }
    } else if constexpr (T == kQ4K || T == kQ5K) {
        /* :396-464 */
        constexpr bool five = T == kQ5K;
        for (uint32_t base = 0; base < width; base += 256, row += five ? 176 : 144) {
            const float d = f16_to_f32(ld16(row)), dmin = f16_to_f32(ld16(row + 2));
            const uint8_t *qh = row + 16, *qs = row + (five ? 48 : 16);
            for (int c = 0; c < 4; ++c) {
                int sc0, m0, sc1, m1;
                k4_scale_min(2 * c, row + 4, sc0, m0);
                k4_scale_min(2 * c + 1, row + 4, sc1, m1);
                const float d0 = __fmul_rn(d, (float)sc0), mm0 = __fmul_rn(dmin, (float)m0);
                const float d1 = __fmul_rn(d, (float)sc1), mm1 = __fmul_rn(dmin, (float)m1);
                for (int i = 0; i < 32; ++i) {
                    const int q = (qs[32 * c + i] & 15) + (five && ((qh[i] >> (2 * c)) & 1) ? 16 : 0);
                    step(__fsub_rn(__fmul_rn(d0, (float)q), mm0), base + 64 * c + i);
                }
                for (int i = 0; i < 32; ++i) {
                    const int q = (qs[32 * c + i] >> 4) + (five && ((qh[i] >> (2 * c + 1)) & 1) ? 16 : 0);
                    step(__fsub_rn(__fmul_rn(d1, (float)q), mm1), base + 64 * c + 32 + i);
                }
            }
        }
    } else {
        /* Q6_K, :466-494 */
        for (uint32_t base = 0; base < width; base += 256, row += 210) {
            const float d = f16_to_f32(ld16(row + 208));
            const int8_t *scales = reinterpret_cast<const int8_t *>(row + 192);
            for (int half = 0; half < 2; ++half) {
                const uint8_t *ql = row + 64 * half, *qh = row + 128 + 32 * half;
                const int8_t *sc = scales + 8 * half;
                for (int i = 0; i < 32; ++i) {
                    const int q[4] = {((ql[i] & 15) | ((qh[i] & 3) << 4)) - 32,
                                      ((ql[i + 32] & 15) | (((qh[i] >> 2) & 3) << 4)) - 32,
                                      ((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32,
                                      ((ql[i + 32] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        step(__fmul_rn(__fmul_rn(d, (float)sc[i / 16 + 2 * k]), (float)q[k]),
                             base + 128 * half + 32 * k + i);
                }
            }
        }
    }
}

template <int T, int MT>
__global__ __launch_bounds__(256) void gemv_float_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                         float *__restrict__ y, uint32_t ldy, uint32_t rows,
                                                         uint32_t width, uint64_t row_bytes)
{
    const uint32_t row = blockIdx.x * 256u + threadIdx.x;
    if (row >= rows) return;
    float total[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) total[t] = 0.0f;
    float_chain<T, MT>(w + row * row_bytes, x, width, total);
#pragma unroll
    for (int t = 0; t < MT; ++t) y[(size_t)t * ldy + row] = total[t];
}

template <int T>
void launch_float_m(int m, const uint8_t *w, const float *x, float *y, uint32_t ldy, uint32_t rows, uint32_t width,
                    uint64_t row_bytes, hipStream_t stream)
{
    const dim3 grid((rows + 255) / 256), block(256);
    switch (m) {
    case 1: hipLaunchKernelGGL((gemv_float_kernel<T, 1>), grid, block, 0, stream, w, x, y, ldy, rows, width, row_bytes); break;
    case 2: hipLaunchKernelGGL((gemv_float_kernel<T, 2>), grid, block, 0, stream, w, x, y, ldy, rows, width, row_bytes); break;
    case 3: hipLaunchKernelGGL((gemv_float_kernel<T, 3>), grid, block, 0, stream, w, x, y, ldy, rows, width, row_bytes); break;
    default: hipLaunchKernelGGL((gemv_float_kernel<T, 4>), grid, block, 0, stream, w, x, y, ldy, rows, width, row_bytes); break;
    }
}

/* ---- row decode ------------------------------------------------------------ */

/* The weight expression of element i of a block (the first operand of its
 * fmaf in the float dot), i < elements per block. */
template <int T>
__device__ __forceinline__ float element_weight(const uint8_t *blk, int i)
{
    if constexpr (T == kQ8_0) {
        return __fmul_rn(f16_to_f32(ld16(blk)), (float)(int8_t)blk[2 + i]);
    } else if constexpr (T == kIQ4NL) {
        const uint32_t byte = blk[2 + (i & 15)];
        return __fmul_rn(f16_to_f32(ld16(blk)), (float)kIq4nl[i < 16 ? byte & 15 : byte >> 4]);
    } else if constexpr (T == kQ2K) {
        const int s = i / 16, j = i % 16, half = s / 8, field = (s % 8) / 2, part = s % 2;
        const float scale = __fmul_rn(f16_to_f32(ld16(blk + 80)), (float)(blk[s] & 15));
        const float minimum = __fmul_rn(f16_to_f32(ld16(blk + 82)), (float)(blk[s] >> 4));
        const int q = (blk[16 + 32 * half + 16 * part + j] >> (2 * field)) & 3;
        return __fsub_rn(__fmul_rn(scale, (float)q), minimum);
    } else if constexpr (T == kQ3K) {
        const int g = i / 32, j = i % 32, half = g / 4, field = g % 4, si = 2 * g + j / 16;
        const uint8_t *sc = blk + 96;
        const int s = ((si < 8 ? sc[si] & 15 : sc[si - 8] >> 4) | (((sc[8 + si % 4] >> (2 * (si / 4))) & 3) << 4)) - 32;
        const int q = ((blk[32 + 32 * half + j] >> (2 * field)) & 3) - ((blk[j] >> g) & 1 ? 0 : 4);
        return __fmul_rn(__fmul_rn(f16_to_f32(ld16(blk + 108)), (float)s), (float)q);
    } else if constexpr (T == kQ4K || T == kQ5K) {
        constexpr bool five = T == kQ5K;
        const int c = i / 64, upper = (i % 64) / 32, j = i % 32;
        int sc, m;
        k4_scale_min(2 * c + upper, blk + 4, sc, m);
        const uint8_t byte = blk[(five ? 48 : 16) + 32 * c + j];
        int q = upper ? byte >> 4 : byte & 15;
        if (five && ((blk[16 + j] >> (2 * c + upper)) & 1)) q += 16;
        const float dd = __fmul_rn(f16_to_f32(ld16(blk)), (float)sc);
        const float mm = __fmul_rn(f16_to_f32(ld16(blk + 2)), (float)m);
        return __fsub_rn(__fmul_rn(dd, (float)q), mm);
    } else {
        /* Q6_K: element 128 half + 32 k + i0 */
        const int half = i / 128, k = (i % 128) / 32, i0 = i % 32;
        const uint8_t *ql = blk + 64 * half, *qh = blk + 128 + 32 * half;
        const uint8_t lowb = ql[i0 + (k & 1) * 32];
        const int q = ((k < 2 ? lowb & 15 : lowb >> 4) | (((qh[i0] >> (2 * k)) & 3) << 4)) - 32;
        const float ds = __fmul_rn(f16_to_f32(ld16(blk + 208)), (float)reinterpret_cast<const int8_t *>(blk + 192)[8 * half + i0 / 16 + 2 * k]);
        return __fmul_rn(ds, (float)q);
    }
}

/* rows[r] of the matrix into out[r * width ..]; the row index of output row
 * r is ids[r] (a token id) when ids is set, else first + r.  One workgroup
 * per (block, output row); E threads = elements per block. */
template <int T, int E>
__global__ __launch_bounds__(256) void row_decode_kernel(const uint8_t *__restrict__ w, const uint32_t *__restrict__ ids,
                                                         uint32_t first, uint32_t limit, float *__restrict__ out,
                                                         uint32_t width, uint64_t row_bytes, uint32_t block_bytes)
{
    __shared__ int bad[256 / 64];
    const uint32_t b = blockIdx.x, r = blockIdx.y;
    uint32_t src = ids ? ids[r] : first + r;
    if (src >= limit) src = limit - 1;
    const uint8_t *blk = w + src * row_bytes + (size_t)b * block_bytes;
    const int i = threadIdx.x;
    float v = 0.0f;
    bool nonfinite = false;
    if (i < E) {
        v = element_weight<T>(blk, i);
        nonfinite = !__builtin_isfinite(v);
    }
    /* non-finite weights in the block: any other one makes this element NaN */
    const unsigned long long ballot = __ballot(nonfinite);
    if ((threadIdx.x & 63) == 0) bad[threadIdx.x >> 6] = __popcll(ballot);
    __syncthreads();
    if (i >= E) return;
    int count = 0;
    for (int k = 0; k < (E + 63) / 64; ++k) count += bad[k];
    /* inf * 0 on the x86 host the reference runs on gives the "indefinite"
     * quiet NaN, sign bit set */
    if (count - (nonfinite ? 1 : 0) > 0) v = __uint_as_float(0xffc00000u);
    else v = __fadd_rn(v, 0.0f);
    out[(size_t)r * width + (size_t)b * E + i] = v;
}

/* F32 / F16 / BF16 rows: copied or converted element by element */
template <int T>
__global__ __launch_bounds__(256) void row_convert_kernel(const uint8_t *__restrict__ w, const uint32_t *__restrict__ ids,
                                                          uint32_t first, uint32_t limit, float *__restrict__ out,
                                                          uint32_t width, uint64_t row_bytes)
{
    const uint32_t r = blockIdx.y, e = blockIdx.x * 256u + threadIdx.x;
    if (e >= width) return;
    uint32_t src = ids ? ids[r] : first + r;
    if (src >= limit) src = limit - 1;
    const uint8_t *row = w + src * row_bytes;
    float v;
    if constexpr (T == kF32) v = reinterpret_cast<const float *>(row)[e];
    else if constexpr (T == kF16) v = f16_to_f32(ld16(row + 2 * (size_t)e));
    else v = bf16_to_f32(ld16(row + 2 * (size_t)e));
    out[(size_t)r * width + e] = v;
}

__global__ __launch_bounds__(256) void fill_kernel(float *__restrict__ out, uint64_t count, float value)
{
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < count) out[i] = value;
}

}  // namespace

/* ---- host side --------------------------------------------------------------- */

void launch_fill_f32(float *out, uint64_t count, float value, hipStream_t stream)
{
    if (!count) return;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream, out, count, value);
}

bool format_block_shape(int type, uint32_t *elements, uint32_t *bytes)
{
    uint32_t e = 256, b = 0;
    switch (type) {
    case kF32: e = 1; b = 4; break;
    case kF16: case kBF16: e = 1; b = 2; break;
    case kQ4_0: e = 32; b = 18; break;
    case kQ4_1: e = 32; b = 20; break;
    case kQ5_0: e = 32; b = 22; break;
    case kQ5_1: e = 32; b = 24; break;
    case kQ8_0: e = 32; b = 34; break;
    case kIQ4NL: e = 32; b = 18; break;
    case kQ2K: b = 84; break;
    case kQ3K: b = 110; break;
    case kQ4K: b = 144; break;
    case kQ5K: b = 176; break;
    case kQ6K: b = 210; break;
    case kIQ2XXS: b = 66; break;
    case kIQ2XS: b = 74; break;
    case kIQ2S: b = 82; break;
    case kIQ3XXS: b = 98; break;
    case kIQ3S: b = 110; break;
    case kIQ4XS: b = 136; break;
    case kIQ1S: b = 50; break;
    case kIQ1M: b = 56; break;
    default: return false;
    }
    *elements = e;
    *bytes = b;
    return true;
}

bool format_takes_q8k(int type)
{
    switch (type) {
    case kQ2K: case kQ3K: case kQ4K: case kQ5K: case kQ6K: case kIQ2XXS: case kIQ2XS: case kIQ2S: case kIQ3XXS:
    case kIQ3S: case kIQ4XS: case kIQ4NL: case kIQ1S: case kIQ1M: return true;
    default: return false;
    }
}

bool launch_gemm_format(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                        uint32_t nb, const void *grid, hipStream_t stream)
{
    if (m < 1 || m > 8 || ldy < rows || !rows || !nb) return false;
    switch (type) {
    case kQ2K: launch_format_m<kQ2K>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kQ3K: launch_format_m<kQ3K>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kQ5K: launch_format_m<kQ5K>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ2XXS: launch_format_m<kIQ2XXS>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ2XS: launch_format_m<kIQ2XS>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ2S: launch_format_m<kIQ2S>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ3XXS: launch_format_m<kIQ3XXS>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ3S: launch_format_m<kIQ3S>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ4XS: launch_format_m<kIQ4XS>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ4NL: launch_format_m<kIQ4NL>(m, w, x, y, ldy, rows, nb, grid, stream); return true;
    case kIQ1S:
        if (!grid) return false;
        launch_format_m<kIQ1S>(m, w, x, y, ldy, rows, nb, grid, stream);
        return true;
    default: return false;
    }
}

bool launch_gemm_float(int type, int m, const uint8_t *w, const float *x, float *y, uint32_t ldy, uint32_t rows,
                       uint32_t width, hipStream_t stream)
{
    uint32_t e = 0, b = 0;
    if (m < 1 || m > 4 || ldy < rows || !rows || !format_block_shape(type, &e, &b) || width % e) return false;
    const uint64_t row_bytes = (uint64_t)width / e * b;
    switch (type) {
    case kF32: launch_float_m<kF32>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kF16: launch_float_m<kF16>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kBF16: launch_float_m<kBF16>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kQ8_0: launch_float_m<kQ8_0>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kIQ4NL: launch_float_m<kIQ4NL>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kQ2K: launch_float_m<kQ2K>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kQ3K: launch_float_m<kQ3K>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kQ4K: launch_float_m<kQ4K>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kQ5K: launch_float_m<kQ5K>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    case kQ6K: launch_float_m<kQ6K>(m, w, x, y, ldy, rows, width, row_bytes, stream); return true;
    default: return false;
    }
}

bool format_row_decodable(int type)
{
    switch (type) {
    case kF32: case kF16: case kBF16: case kQ8_0: case kIQ4NL: case kQ2K: case kQ3K: case kQ4K: case kQ5K: case kQ6K:
        return true;
    default: return false;
    }
}

bool launch_row_decode(int type, const uint8_t *w, const uint32_t *ids, uint32_t first, uint32_t count,
                       uint32_t limit, float *out, uint32_t width, hipStream_t stream)
{
    uint32_t e = 0, b = 0;
    if (!count || !limit || !format_block_shape(type, &e, &b) || width % e || !format_row_decodable(type))
        return false;
    const uint64_t row_bytes = (uint64_t)width / e * b;
    if (e == 1) {
        const dim3 grid((width + 255) / 256, count);
        switch (type) {
        case kF32: hipLaunchKernelGGL(row_convert_kernel<kF32>, grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes); break;
        case kF16: hipLaunchKernelGGL(row_convert_kernel<kF16>, grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes); break;
        default: hipLaunchKernelGGL(row_convert_kernel<kBF16>, grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes); break;
        }
        return true;
    }
    const dim3 grid(width / e, count);
    switch (type) {
    case kQ8_0: hipLaunchKernelGGL((row_decode_kernel<kQ8_0, 32>), grid, dim3(64), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    case kIQ4NL: hipLaunchKernelGGL((row_decode_kernel<kIQ4NL, 32>), grid, dim3(64), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    case kQ2K: hipLaunchKernelGGL((row_decode_kernel<kQ2K, 256>), grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    case kQ3K: hipLaunchKernelGGL((row_decode_kernel<kQ3K, 256>), grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    case kQ4K: hipLaunchKernelGGL((row_decode_kernel<kQ4K, 256>), grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    case kQ5K: hipLaunchKernelGGL((row_decode_kernel<kQ5K, 256>), grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    default: hipLaunchKernelGGL((row_decode_kernel<kQ6K, 256>), grid, dim3(256), 0, stream, w, ids, first, limit, out, width, row_bytes, b); break;
    }
    return true;
}

}  // namespace q38
