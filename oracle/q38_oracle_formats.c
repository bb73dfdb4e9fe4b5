/* CPU oracle for the remaining GGUF matrix formats -- TEST INFRASTRUCTURE
 * ONLY (see q38_oracle.h).
 *
 * Q8_K path (q38_tensor_gemv_q8_k, src/qwen38/qwen38_quant.c:2833-2922):
 * Q2_K, Q3_K, Q5_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS, IQ4_NL
 * and IQ1_S.  Every one of the reference's AVX2 kernels
 * (:510-1253, :1636-1725) forms, per super-block, eight exact int32 lanes:
 * lane l sums the products of bytes 4l..4l+3 of each 32-element group g,
 * each group-half scaled by an integer sub-block scale.  The oracle states
 * each format by what it decodes to -- integer weights q[256] (grid value
 * and sign folded in) and one integer scale per 16 elements -- and forms
 * the lanes from that:
 *     W[l] = sum_g sum_t s16[2g + (l >= 4)] * q[32g + 4l + t] * a[32g + 4l + t].
 * The fp32 part is then the format's own: lane FMAs d * W[l] in block order
 * and the 8-lane tree, plus Q2_K / Q5_K's scalar min chain, IQ1_S's scalar
 * correction sum, and IQ4_NL's per-group scale (eight lane FMAs per block).
 *
 * Float path (q38_dot_row, :2768-2810): F32, F16, BF16, Q8_0 and the float
 * K-quant / IQ4_NL dots (:331-507), one sequential fmaf chain per row in the
 * reference's element order; and the row decode of q38_tensor_row_f32
 * (:3185-3223).
 */
#include "q38_oracle.h"

#include <math.h>
#include <string.h>

#include "../qwen3.8-27b-in-c_amd/csrc/q38_iq_grids.inc"

static uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }
static uint32_t ld32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

static const int8_t iq4nl_values[16] = {Q38_IQ4NL_VALUES};

#define CODE(c) c,
static const uint16_t iq2xxs_codes[256] = {Q38_IQ2XXS_CODES(CODE)};
static const uint16_t iq2xs_codes[512] = {Q38_IQ2XS_CODES(CODE)};
static const uint16_t iq2s_codes[1024] = {Q38_IQ2S_CODES(CODE)};
static const uint16_t iq3xxs_codes[256] = {Q38_IQ3XXS_CODES(CODE)};
static const uint16_t iq3s_codes[512] = {Q38_IQ3S_CODES(CODE)};
#undef CODE

static int iq2_level(uint16_t code, int k)
{
    static const int levels[3] = {8, 25, 43};
    return levels[(code >> (2 * k)) & 3];
}

static int iq3xxs_level(uint16_t code, int k)
{
    static const int levels[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    return levels[(code >> (3 * k)) & 7];
}

static int iq3s_level(uint16_t code, int k) { return 1 + 2 * ((code >> (3 * k)) & 7); }

/* the IQ2/IQ3 sign byte of a 7-bit index: even parity in bit 7 (ksigns_iq2xs) */
static int sign_byte(uint32_t index)
{
    index &= 127u;
    int parity = 0;
    for (uint32_t v = index; v; v >>= 1) parity ^= (int)(v & 1u);
    return (int)(index | (uint32_t)parity << 7);
}

uint32_t orc_format_block_bytes(uint32_t type)
{
    switch (type) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_Q2_K: return 84;
    case ORC_Q3_K: return 110;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ2_XXS: return 66;
    case ORC_IQ2_XS: return 74;
    case ORC_IQ2_S: return 82;
    case ORC_IQ3_XXS: return 98;
    case ORC_IQ3_S: return 110;
    case ORC_IQ4_XS: return 136;
    case ORC_IQ4_NL: return 18;
    case ORC_IQ1_S: return 50;
    case ORC_IQ1_M: return 56;
    default: return 0;
    }
}

uint32_t orc_format_block_elements(uint32_t type)
{
    switch (type) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q8_0: case ORC_IQ4_NL: return 32;
    default: return orc_format_block_bytes(type) ? 256 : 0;
    }
}

/* ---- Q8_K path: decode to integer weights and 16-element scales ---------- */

static void q3k_scales(const uint8_t *packed, int s[16])
{
    /* src/qwen38/qwen38_quant.c:319-329: 4 low bits from bytes 0..7 (low
     * nibble for scales 0..7, high nibble for 8..15), 2 high bits from
     * bytes 8..11, minus 32 */
    for (int i = 0; i < 16; ++i) {
        const int low = i < 8 ? packed[i] & 15 : packed[i - 8] >> 4;
        const int high = (packed[8 + i % 4] >> (2 * (i / 4))) & 3;
        s[i] = (low | high << 4) - 32;
    }
}

static void k4_scale_min(int i, const uint8_t *p, int *sc, int *m)
{
    /* :131-143 */
    if (i < 4) {
        *sc = p[i] & 63;
        *m = p[i + 4] & 63;
    } else {
        *sc = (p[i + 4] & 15) | ((p[i - 4] >> 6) << 4);
        *m = (p[i + 4] >> 4) | ((p[i] >> 6) << 4);
    }
}

/* Integer form of one super-block: q[256], s16[16], plus the block's
 * integer min / correction term where the format has one (Q2_K, Q5_K: the
 * min sum; IQ1_S: the signed-scale correction), in *extra. */
static int decode_q8k_block(uint32_t type, const uint8_t *blk, const OrcQ8K *a, int q[256], int s16[16],
                            int *extra)
{
    *extra = 0;
    switch (type) {
    case ORC_Q2_K: {      /* :510-585 */
        const uint8_t *scales = blk, *qs = blk + 16;
        for (int g = 0; g < 8; ++g) {
            const int half = g / 4, field = g % 4;
            for (int j = 0; j < 32; ++j) q[32 * g + j] = (qs[32 * half + j] >> (2 * field)) & 3;
        }
        for (int i = 0; i < 16; ++i) {
            s16[i] = scales[i] & 15;
            *extra += (scales[i] >> 4) * a->sums[i];
        }
        return 1;
    }
    case ORC_Q3_K: {      /* :587-662 */
        const uint8_t *hmask = blk, *qs = blk + 32;
        q3k_scales(blk + 96, s16);
        for (int g = 0; g < 8; ++g) {
            const int half = g / 4, field = g % 4;
            for (int j = 0; j < 32; ++j)
                q[32 * g + j] = ((qs[32 * half + j] >> (2 * field)) & 3) - ((hmask[j] >> g) & 1 ? 0 : 4);
        }
        return 1;
    }
    case ORC_Q5_K: {      /* :1636-1725 */
        const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
        for (int c = 0; c < 4; ++c) {
            int sc0, m0, sc1, m1;
            k4_scale_min(2 * c, scales, &sc0, &m0);
            k4_scale_min(2 * c + 1, scales, &sc1, &m1);
            for (int j = 0; j < 32; ++j) {
                q[64 * c + j] = (qs[32 * c + j] & 15) + (((qh[j] >> (2 * c)) & 1) << 4);
                q[64 * c + 32 + j] = (qs[32 * c + j] >> 4) + (((qh[j] >> (2 * c + 1)) & 1) << 4);
            }
            s16[4 * c] = s16[4 * c + 1] = sc0;
            s16[4 * c + 2] = s16[4 * c + 3] = sc1;
            *extra += m0 * (a->sums[4 * c] + a->sums[4 * c + 1]) + m1 * (a->sums[4 * c + 2] + a->sums[4 * c + 3]);
        }
        return 1;
    }
    case ORC_IQ2_XXS: {   /* :758-822 */
        for (int g = 0; g < 8; ++g) {
            const uint8_t *codes = blk + 2 + 8 * g;
            const uint32_t meta = ld32(codes + 4);
            for (int j = 0; j < 32; ++j) {
                const int s = j / 8, k = j % 8;
                const int sign = (sign_byte(meta >> (7 * s)) >> k) & 1;
                const int v = iq2_level(iq2xxs_codes[codes[s]], k);
                q[32 * g + j] = sign ? -v : v;
            }
            s16[2 * g] = s16[2 * g + 1] = 1 + 2 * (int)(meta >> 28);
        }
        return 1;
    }
    case ORC_IQ2_XS: {    /* :824-893 */
        const uint8_t *scales = blk + 66;
        for (int g = 0; g < 8; ++g) {
            for (int j = 0; j < 32; ++j) {
                const int s = j / 8, k = j % 8;
                const uint16_t code = ld16(blk + 2 + 8 * g + 2 * s);
                const int sign = (sign_byte(code >> 9) >> k) & 1;
                const int v = iq2_level(iq2xs_codes[code & 511u], k);
                q[32 * g + j] = sign ? -v : v;
            }
            s16[2 * g] = 1 + 2 * (scales[g] & 15);
            s16[2 * g + 1] = 1 + 2 * (scales[g] >> 4);
        }
        return 1;
    }
    case ORC_IQ2_S: {     /* :664-756 */
        const uint8_t *idx = blk + 2, *signs = blk + 34, *qh = blk + 66, *scales = blk + 74;
        for (int g = 0; g < 8; ++g) {
            for (int j = 0; j < 32; ++j) {
                const int s = j / 8, k = j % 8;
                const uint32_t index = idx[4 * g + s] | (((uint32_t)qh[g] << (8 - 2 * s)) & 0x300u);
                const int v = iq2_level(iq2s_codes[index], k);
                q[32 * g + j] = (signs[4 * g + s] >> k) & 1 ? -v : v;
            }
            s16[2 * g] = 1 + 2 * (scales[g] & 15);
            s16[2 * g + 1] = 1 + 2 * (scales[g] >> 4);
        }
        return 1;
    }
    case ORC_IQ3_XXS: {   /* :895-976 */
        for (int g = 0; g < 8; ++g) {
            const uint32_t packed = ld32(blk + 66 + 4 * g);
            for (int j = 0; j < 32; ++j) {
                const int sign = (sign_byte(packed >> (7 * (j / 8))) >> (j % 8)) & 1;
                const int v = iq3xxs_level(iq3xxs_codes[blk[2 + 8 * g + j / 4]], j % 4);
                q[32 * g + j] = sign ? -v : v;
            }
            s16[2 * g] = s16[2 * g + 1] = 1 + 2 * (int)(packed >> 28);
        }
        return 1;
    }
    case ORC_IQ3_S: {     /* :978-1061 */
        const uint8_t *idx = blk + 2, *qh = blk + 66, *signs = blk + 74, *scales = blk + 106;
        for (int g = 0; g < 8; ++g) {
            for (int j = 0; j < 32; ++j) {
                const int k = j / 4;
                const uint32_t index = idx[8 * g + k] | (((uint32_t)(qh[g] >> k) & 1u) << 8);
                const int v = iq3s_level(iq3s_codes[index], j % 4);
                q[32 * g + j] = (signs[4 * g + j / 8] >> (j % 8)) & 1 ? -v : v;
            }
            s16[2 * g] = s16[2 * g + 1] = 1 + 2 * ((scales[g / 2] >> (4 * (g % 2))) & 15);
        }
        return 1;
    }
    case ORC_IQ4_XS: {    /* :1063-1127 */
        const uint16_t scale_high = ld16(blk + 2);
        const uint8_t *scale_low = blk + 4, *qs = blk + 8;
        for (int g = 0; g < 8; ++g) {
            for (int j = 0; j < 16; ++j) {
                q[32 * g + j] = iq4nl_values[qs[16 * g + j] & 15];
                q[32 * g + 16 + j] = iq4nl_values[qs[16 * g + j] >> 4];
            }
            const int scale = ((scale_low[g / 2] >> (4 * (g % 2))) & 15) | (((scale_high >> (2 * g)) & 3) << 4);
            s16[2 * g] = s16[2 * g + 1] = scale - 32;
        }
        return 1;
    }
    case ORC_IQ4_NL: {    /* :1129-1175, per group: 2-byte scale + 16 bytes */
        for (int g = 0; g < 8; ++g) {
            const uint8_t *qs = blk + 18 * g + 2;
            for (int j = 0; j < 16; ++j) {
                q[32 * g + j] = iq4nl_values[qs[j] & 15];
                q[32 * g + 16 + j] = iq4nl_values[qs[j] >> 4];
            }
            s16[2 * g] = s16[2 * g + 1] = 1;
        }
        return 1;
    }
    case ORC_IQ1_S: {     /* :1177-1253 */
        const uint8_t *idx = blk + 2;
        for (int g = 0; g < 8; ++g) {
            const uint16_t high = ld16(blk + 34 + 2 * g);
            for (int s = 0; s < 4; ++s) {
                int8_t grid[8];
                orc_iq1m_grid_entry(idx[4 * g + s] | (((uint32_t)(high >> (3 * s)) & 7u) << 8), grid);
                for (int k = 0; k < 8; ++k) q[32 * g + 8 * s + k] = grid[k];
            }
            const int scale = 1 + 2 * ((high >> 12) & 7);
            s16[2 * g] = s16[2 * g + 1] = scale;
            *extra += scale * (high & 0x8000u ? -1 : 1) * (a->sums[2 * g] + a->sums[2 * g + 1]);
        }
        return 1;
    }
    default:
        return 0;
    }
}

/* the eight lanes of one group range [g0, g1) */
static void lanes(const int q[256], const int s16[16], const OrcQ8K *a, int g0, int g1, int32_t w[8])
{
    for (int l = 0; l < 8; ++l) {
        int32_t sum = 0;
        for (int g = g0; g < g1; ++g) {
            int32_t dot = 0;
            for (int t = 0; t < 4; ++t) dot += q[32 * g + 4 * l + t] * a->quants[32 * g + 4 * l + t];
            sum += s16[2 * g + (l >= 4)] * dot;
        }
        w[l] = sum;
    }
}

int orc_format_block_lanes(uint32_t type, const uint8_t *block, const OrcQ8K *input, int32_t w[8], int32_t *extra)
{
    int q[256], s16[16];
    if (!decode_q8k_block(type, block, input, q, s16, extra)) return 0;
    lanes(q, s16, input, 0, 8, w);
    return 1;
}

int orc_format_block_decode(uint32_t type, const uint8_t *block, int32_t q[256], int32_t s16[16])
{
    static const OrcQ8K zero;
    int qi[256], si[16], extra;
    if (!decode_q8k_block(type, block, &zero, qi, si, &extra)) return 0;
    for (int i = 0; i < 256; ++i) q[i] = qi[i];
    for (int i = 0; i < 16; ++i) s16[i] = si[i];
    return 1;
}

static float sum8(const float v[8])
{
    /* src/qwen38/qwen38_quant.c:303-310 */
    const float s0 = v[0] + v[4], s1 = v[1] + v[5];
    const float s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s2) + (s1 + s3);
}

static float block_scale(uint32_t type, const uint8_t *blk)
{
    switch (type) {
    case ORC_Q2_K: return orc_f16_to_f32(ld16(blk + 80));
    case ORC_Q3_K: return orc_f16_to_f32(ld16(blk + 108));
    case ORC_IQ2_XXS: case ORC_IQ2_XS: case ORC_IQ2_S: return 0.125f * orc_f16_to_f32(ld16(blk));
    case ORC_IQ3_XXS: return 0.25f * orc_f16_to_f32(ld16(blk));
    default: return orc_f16_to_f32(ld16(blk));
    }
}

float orc_format_dot_q8_k(uint32_t type, const uint8_t *row, const OrcQ8K *input, uint64_t blocks)
{
    const uint32_t bytes = orc_format_block_bytes(type) * (type == ORC_IQ4_NL ? 8u : 1u);
    float acc[8] = {0}, scalar = 0.0f;
    int q[256], s16[16], extra;
    int32_t w[8];
    for (uint64_t b = 0; b < blocks; ++b, row += bytes) {
        const OrcQ8K *a = input + b;
        decode_q8k_block(type, row, a, q, s16, &extra);
        if (type == ORC_IQ4_NL) {
            for (int g = 0; g < 8; ++g) {
                const float d = orc_f16_to_f32(ld16(row + 18 * g)) * a->scale;
                lanes(q, s16, a, g, g + 1, w);
                for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)w[l], acc[l]);
            }
            continue;
        }
        lanes(q, s16, a, 0, 8, w);
        const float d = block_scale(type, row) * a->scale;
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)w[l], acc[l]);
        if (type == ORC_Q2_K || type == ORC_Q5_K) {
            const float dmin = orc_f16_to_f32(ld16(row + (type == ORC_Q2_K ? 82 : 2))) * a->scale;
            scalar = fmaf(-dmin, (float)extra, scalar);
        } else if (type == ORC_IQ1_S) {
            const float product = d * (float)extra;
            scalar = scalar + product;
        }
    }
    if (type == ORC_IQ1_S) {
        const float corr = 0.125f * scalar;
        return sum8(acc) + corr;
    }
    return sum8(acc) + scalar;
}

/* ---- float path ----------------------------------------------------------- */

static float bf16_to_f32(uint16_t bits)
{
    const uint32_t wide = (uint32_t)bits << 16;
    float out;
    memcpy(&out, &wide, 4);
    return out;
}

/* One chain over a row of `length` elements; :331-507 and :2768-2810.  The
 * weight expressions are rounded as the reference rounds them (products
 * and the subtraction of the min, then one fmaf each). */
float orc_format_dot_f32(uint32_t type, const uint8_t *row, const float *x, uint64_t length)
{
    float total = 0.0f;
    switch (type) {
    case ORC_F32:
        for (uint64_t i = 0; i < length; ++i) {
            float w;
            memcpy(&w, row + 4 * i, 4);
            total = fmaf(w, x[i], total);
        }
        return total;
    case ORC_F16:
        for (uint64_t i = 0; i < length; ++i) total = fmaf(orc_f16_to_f32(ld16(row + 2 * i)), x[i], total);
        return total;
    case ORC_BF16:
        for (uint64_t i = 0; i < length; ++i) total = fmaf(bf16_to_f32(ld16(row + 2 * i)), x[i], total);
        return total;
    case ORC_Q8_0:
        for (uint64_t base = 0; base < length; base += 32, row += 34) {
            const float d = orc_f16_to_f32(ld16(row));
            for (int i = 0; i < 32; ++i) {
                const float w = d * (float)(int8_t)row[2 + i];
                total = fmaf(w, x[base + i], total);
            }
        }
        return total;
    case ORC_IQ4_NL:
        for (uint64_t base = 0; base < length; base += 32, row += 18) {
            const float d = orc_f16_to_f32(ld16(row));
            for (int j = 0; j < 16; ++j) {
                const float w0 = d * (float)iq4nl_values[row[2 + j] & 15];
                total = fmaf(w0, x[base + j], total);
                const float w1 = d * (float)iq4nl_values[row[2 + j] >> 4];
                total = fmaf(w1, x[base + 16 + j], total);
            }
        }
        return total;
    case ORC_Q2_K:
        for (uint64_t base = 0; base < length; base += 256, row += 84) {
            const float d = orc_f16_to_f32(ld16(row + 80)), dmin = orc_f16_to_f32(ld16(row + 82));
            for (int i = 0; i < 16; ++i) {   /* elements 16i .. 16i+15, scale byte i */
                const float scale = d * (float)(row[i] & 15), minimum = dmin * (float)(row[i] >> 4);
                const int half = i / 8, field = (i % 8) / 2, part = i % 2;
                for (int lane = 0; lane < 16; ++lane) {
                    const int q = (row[16 + 32 * half + 16 * part + lane] >> (2 * field)) & 3;
                    const float sq = scale * (float)q;
                    total = fmaf(sq - minimum, x[base + 16 * i + lane], total);
                }
            }
        }
        return total;
    case ORC_Q3_K:
        for (uint64_t base = 0; base < length; base += 256, row += 110) {
            int s[16];
            q3k_scales(row + 96, s);
            const float d = orc_f16_to_f32(ld16(row + 108));
            for (int g = 0; g < 8; ++g) {
                const int half = g / 4, field = g % 4;
                for (int j = 0; j < 32; ++j) {
                    const int q = ((row[32 + 32 * half + j] >> (2 * field)) & 3) - ((row[j] >> g) & 1 ? 0 : 4);
                    const float ds = d * (float)s[2 * g + j / 16];
                    total = fmaf(ds * (float)q, x[base + 32 * g + j], total);
                }
            }
        }
        return total;
    case ORC_Q4_K:
    case ORC_Q5_K: {
        const int five = type == ORC_Q5_K;
        const uint32_t bytes = five ? 176 : 144;
        for (uint64_t base = 0; base < length; base += 256, row += bytes) {
            const float d = orc_f16_to_f32(ld16(row)), dmin = orc_f16_to_f32(ld16(row + 2));
            const uint8_t *qh = row + 16, *qs = row + (five ? 48 : 16);
            for (int c = 0; c < 4; ++c) {
                int sc0, m0, sc1, m1;
                k4_scale_min(2 * c, row + 4, &sc0, &m0);
                k4_scale_min(2 * c + 1, row + 4, &sc1, &m1);
                const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
                const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
                for (int i = 0; i < 32; ++i) {
                    const int q = (qs[32 * c + i] & 15) + (five && ((qh[i] >> (2 * c)) & 1) ? 16 : 0);
                    const float dq = d0 * (float)q;
                    total = fmaf(dq - mm0, x[base + 64 * c + i], total);
                }
                for (int i = 0; i < 32; ++i) {
                    const int q = (qs[32 * c + i] >> 4) + (five && ((qh[i] >> (2 * c + 1)) & 1) ? 16 : 0);
                    const float dq = d1 * (float)q;
                    total = fmaf(dq - mm1, x[base + 64 * c + 32 + i], total);
                }
            }
        }
        return total;
    }
    case ORC_Q6_K:
        for (uint64_t base = 0; base < length; base += 256, row += 210) {
            const float d = orc_f16_to_f32(ld16(row + 208));
            const int8_t *scales = (const int8_t *)(row + 192);
            for (int half = 0; half < 2; ++half) {
                const uint8_t *ql = row + 64 * half, *qh = row + 128 + 32 * half;
                const int8_t *sc = scales + 8 * half;
                for (int i = 0; i < 32; ++i) {
                    const int q[4] = {((ql[i] & 15) | ((qh[i] & 3) << 4)) - 32,
                                      ((ql[i + 32] & 15) | (((qh[i] >> 2) & 3) << 4)) - 32,
                                      ((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32,
                                      ((ql[i + 32] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32};
                    for (int k = 0; k < 4; ++k) {
                        const float ds = d * (float)sc[i / 16 + 2 * k];
                        total = fmaf(ds * (float)q[k], x[base + 128 * half + 32 * k + i], total);
                    }
                }
            }
        }
        return total;
    default:
        return NAN;
    }
}

int orc_format_gemv_f32(float *output, const float *input, uint64_t width, uint32_t type, const uint8_t *data,
                        uint64_t rows)
{
    const uint32_t e = orc_format_block_elements(type), b = orc_format_block_bytes(type);
    if (!output || !input || !data || !e || width % e) return 0;
    const uint64_t row_bytes = width / e * b;
    for (uint64_t r = 0; r < rows; ++r) output[r] = orc_format_dot_f32(type, data + r * row_bytes, input, width);
    return 1;
}

int orc_format_gemv_q8_k(float *output, const OrcQ8K *input, uint64_t width, uint32_t type, const uint8_t *data,
                         uint64_t rows)
{
    const uint32_t b = orc_format_block_bytes(type) * (type == ORC_IQ4_NL ? 8u : 1u);
    if (!output || !input || !data || width % ORC_QK) return 0;
    if (type == ORC_Q4_K || type == ORC_Q6_K || type == ORC_IQ1_M)
        return orc_gemv_q8_k(output, input, width, type, data, rows);
    if (orc_format_block_elements(type) != 256 && type != ORC_IQ4_NL) return 0;
    const uint64_t blocks = width / ORC_QK;
    for (uint64_t r = 0; r < rows; ++r)
        output[r] = orc_format_dot_q8_k(type, data + r * blocks * b, input, blocks);
    return 1;
}

/* q38_tensor_row_f32 (:3185-3223): F32 copied, F16 / BF16 converted, every
 * other element the float dot of its block with a unit vector. */
int orc_format_row_f32(float *output, uint32_t type, const uint8_t *data, uint64_t width, uint64_t row)
{
    const uint32_t e = orc_format_block_elements(type), b = orc_format_block_bytes(type);
    if (!output || !data || !e || width % e) return 0;
    const uint8_t *src = data + row * (width / e * b);
    if (type == ORC_F32) {
        memcpy(output, src, (size_t)width * 4);
        return 1;
    }
    if (type == ORC_F16 || type == ORC_BF16) {
        for (uint64_t i = 0; i < width; ++i)
            output[i] = type == ORC_F16 ? orc_f16_to_f32(ld16(src + 2 * i)) : bf16_to_f32(ld16(src + 2 * i));
        return 1;
    }
    float basis[256] = {0};
    for (uint64_t base = 0; base < width; base += e) {
        for (uint32_t i = 0; i < e; ++i) {
            basis[i] = 1.0f;
            output[base + i] = orc_format_dot_f32(type, src + base / e * b, basis, e);
            basis[i] = 0.0f;
        }
    }
    return 1;
}
