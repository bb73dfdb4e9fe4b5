/* CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.
 * See q38_oracle.h.  Loaded by tests/, smoke() and bench.py's cpu_baseline
 * leg; never by the product library.
 *
 * Reference files cited below are relative to the reference repository root
 * (shyringo/qwen3.8-27b-in-c).
 */
#include "q38_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../qwen3.8-27b-in-c_amd/csrc/q38_iq1m_grid.inc"

static uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }

/* Exact IEEE binary16 -> binary32; src/qwen38/qwen38_quant.c:90-122 (the
 * portable branch; the F16C branch computes the same exact conversion). */
float orc_f16_to_f32(uint16_t value)
{
    const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    const uint32_t exponent = (value >> 10) & 31u;
    uint32_t mantissa = value & 1023u;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            int e = 113; /* 127 - 14 */
            while (!(mantissa & 0x400u)) { mantissa <<= 1; --e; }
            bits = sign | (uint32_t)e << 23 | (mantissa & 0x3ffu) << 13;
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | mantissa << 13;
    } else {
        bits = sign | (exponent + 112u) << 23 | mantissa << 13;
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* Round-half-even via the 1.5*2^23 shift; src/qwen38/qwen38_quant.c:42-48. */
int orc_nearest_int(float value)
{
    volatile float shifted = value + 12582912.0f;
    float s = shifted;
    uint32_t bits;
    memcpy(&bits, &s, 4);
    return (int)(bits & 0x007fffffu) - 0x00400000;
}

/* Q8_K activation quantizer; src/qwen38/qwen38_quant.c:50-88.  The block
 * maximum is the signed value of the first element with the largest |x|
 * (strict >), the inverse scale is -127/max, and the stored scale is
 * 1/inverse. */
int orc_quantize_q8_k(OrcQ8K *output, const float *input, uint64_t length)
{
    if (!output || !input || length % ORC_QK) return 0;
    for (uint64_t b = 0; b < length / ORC_QK; ++b) {
        const float *x = input + b * ORC_QK;
        OrcQ8K *q = output + b;
        float maximum = 0.0f, amax = 0.0f;
        for (int i = 0; i < ORC_QK; ++i) {
            const float a = fabsf(x[i]);
            if (a > amax) { amax = a; maximum = x[i]; }
        }
        if (amax == 0.0f) {
            memset(q, 0, sizeof(*q));
            continue;
        }
        const float inv = -127.0f / maximum;
        for (int i = 0; i < ORC_QK; ++i) {
            volatile float product = inv * x[i];
            int v = orc_nearest_int(product);
            if (v > 127) v = 127;
            q->quants[i] = (int8_t)v;
        }
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += q->quants[g * 16 + i];
            q->sums[g] = (int16_t)s;
        }
        q->scale = 1.0f / inv;
    }
    return 1;
}

uint32_t orc_block_bytes(uint32_t type)
{
    switch (type) {
    case ORC_Q4_K: return 144;
    case ORC_Q6_K: return 210;
    case ORC_IQ1_M: return 56;
    default: return 0;
    }
}

/* 6-bit scale/min unpacking; src/qwen38/qwen38_quant.c:131-143. */
static void scale_min_k4(int i, const uint8_t *p, int *sc, int *m)
{
    if (i < 4) {
        *sc = p[i] & 63;
        *m = p[i + 4] & 63;
    } else {
        *sc = (p[i + 4] & 15) | ((p[i - 4] >> 6) << 4);
        *m = (p[i + 4] >> 4) | ((p[i] >> 6) << 4);
    }
}

/* Q4_K integer lanes, as the AVX2 kernel forms them
 * (src/qwen38/qwen38_quant.c:1564-1620): eight 32-bit lanes, lane l owning
 * bytes 4l..4l+3 of each 32-byte nibble chunk, scaled per sub-block, plus
 * four min lanes M[i] = m[2i](s[4i]+s[4i+1]) + m[2i+1](s[4i+2]+s[4i+3]). */
static void q4k_ints(const uint8_t *blk, const OrcQ8K *a, int32_t ints[12])
{
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    for (int l = 0; l < 8; ++l) ints[l] = 0;
    for (int c = 0; c < 4; ++c) {
        int sc0, m0, sc1, m1;
        scale_min_k4(2 * c, scales, &sc0, &m0);
        scale_min_k4(2 * c + 1, scales, &sc1, &m1);
        for (int l = 0; l < 8; ++l) {
            int dot0 = 0, dot1 = 0;
            for (int t = 0; t < 4; ++t) {
                const int byte = qs[32 * c + 4 * l + t];
                dot0 += (byte & 15) * a->quants[64 * c + 4 * l + t];
                dot1 += (byte >> 4) * a->quants[64 * c + 32 + 4 * l + t];
            }
            ints[l] += dot0 * sc0 + dot1 * sc1;
        }
        const int p0 = (int16_t)(a->sums[4 * c] + a->sums[4 * c + 1]);
        const int p1 = (int16_t)(a->sums[4 * c + 2] + a->sums[4 * c + 3]);
        ints[8 + c] = m0 * p0 + m1 * p1;
    }
}

/* IQ1_M integer sums; src/qwen38/qwen38_quant.c:1388-1544 (the portable
 * loop, :1490-1522, which the AVX2 lanes sum to the same integers). */
static void iq1m_ints(const uint8_t *blk, const OrcQ8K *a, int32_t ints[2])
{
    const uint8_t *idx = blk, *qh = blk + 32, *sc = blk + 48;
    int weighted = 0, correction = 0;
    for (int g = 0; g < 8; ++g) {
        int dot[2] = {0, 0}, cdot[2] = {0, 0};
        for (int s = 0; s < 4; ++s) {
            const uint8_t h = qh[2 * g + s / 2];
            const uint32_t gi = idx[4 * g + s] | (((uint32_t)h << (8 - 4 * (s % 2))) & 0x700u);
            const int delta = (h & (s % 2 ? 0x80 : 0x08)) ? -1 : 1;
            int8_t grid[8];
            orc_iq1m_grid_entry(gi, grid);
            for (int k = 0; k < 8; ++k) {
                const int av = a->quants[32 * g + 8 * s + k];
                dot[s / 2] += av * grid[k];
                cdot[s / 2] += av * delta;
            }
        }
        const uint16_t packed = ld16(sc + (g / 2) * 2);
        const int shift = 6 * (g % 2);
        const int s0 = 1 + 2 * ((packed >> shift) & 7);
        const int s1 = 1 + 2 * ((packed >> (shift + 3)) & 7);
        weighted += s0 * dot[0] + s1 * dot[1];
        correction += s0 * cdot[0] + s1 * cdot[1];
    }
    ints[0] = weighted;
    ints[1] = correction;
}

/* Q6_K integer lanes of the AVX2 kernel (src/qwen38/qwen38_quant.c:1727-1814):
 * lane l holds sum over halves h, quarters j, bytes t of
 * scale[8h+2j+(l>=4)] * q_j[4l+t] * a[128h+32j+4l+t] (q unsigned 0..63),
 * minus the offset lane 32*(s[2l]*scale[2l] + s[2l+1]*scale[2l+1]). */
static void q6k_ints(const uint8_t *blk, const OrcQ8K *a, int32_t ints[8])
{
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *scales = (const int8_t *)(blk + 192);
    for (int l = 0; l < 8; ++l) {
        int w = 0;
        for (int h = 0; h < 2; ++h) {
            for (int j = 0; j < 4; ++j) {
                int dot = 0;
                for (int t = 0; t < 4; ++t) {
                    const int i = 4 * l + t;
                    const uint8_t low = ql[64 * h + (j & 1) * 32 + i];
                    const int lo4 = (j < 2) ? (low & 15) : (low >> 4);
                    const int hi2 = (qh[32 * h + i] >> (2 * j)) & 3;
                    dot += (lo4 | hi2 << 4) * a->quants[128 * h + 32 * j + i];
                }
                w += scales[8 * h + 2 * j + (l >= 4)] * dot;
            }
        }
        const int offset = 32 * (a->sums[2 * l] * scales[2 * l] +
                                 a->sums[2 * l + 1] * scales[2 * l + 1]);
        ints[l] = w - offset;
    }
}

int orc_block_ints(uint32_t type, const uint8_t *block, const OrcQ8K *input,
                   int32_t ints[12])
{
    switch (type) {
    case ORC_Q4_K: q4k_ints(block, input, ints); return 12;
    case ORC_IQ1_M: iq1m_ints(block, input, ints); return 2;
    case ORC_Q6_K: q6k_ints(block, input, ints); return 8;
    default: return 0;
    }
}

/* _mm256 8-lane horizontal sum; src/qwen38/qwen38_quant.c:303-310. */
static float sum8(const float v[8])
{
    const float s0 = v[0] + v[4], s1 = v[1] + v[5];
    const float s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s2) + (s1 + s3);
}

/* Row dot products with the fp32 accumulation order of the AVX2 kernels:
 * Q4_K src/qwen38/qwen38_quant.c:1546-1634 (lane FMAs, then sum8 + min tree),
 * IQ1_M :1388-1544 (scalar total += d*(w + 0.125f*c)),
 * Q6_K :1727-1833 (lane FMAs, then sum8). */
float orc_dot_q8_k(uint32_t type, const uint8_t *row, const OrcQ8K *input,
                   uint64_t blocks)
{
    const uint32_t bytes = orc_block_bytes(type);
    float acc[8] = {0}, accm[4] = {0}, total = 0.0f;
    int32_t ints[12];
    for (uint64_t b = 0; b < blocks; ++b, row += bytes) {
        const OrcQ8K *a = input + b;
        orc_block_ints(type, row, a, ints);
        if (type == ORC_Q4_K) {
            const float d = orc_f16_to_f32(ld16(row)) * a->scale;
            const float dmin = orc_f16_to_f32(ld16(row + 2)) * a->scale;
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)ints[l], acc[l]);
            for (int i = 0; i < 4; ++i) accm[i] = fmaf(-dmin, (float)ints[8 + i], accm[i]);
        } else if (type == ORC_Q6_K) {
            const float d = orc_f16_to_f32(ld16(row + 208)) * a->scale;
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)ints[l], acc[l]);
        } else {
            const uint8_t *sc = row + 48;
            const uint16_t bits = (uint16_t)((ld16(sc) >> 12) | ((ld16(sc + 2) >> 8) & 0x00f0u) |
                                             ((ld16(sc + 4) >> 4) & 0x0f00u) | (ld16(sc + 6) & 0xf000u));
            const float d = orc_f16_to_f32(bits) * a->scale;
            volatile float corr = 0.125f * (float)ints[1];
            volatile float inner = (float)ints[0] + corr;
            volatile float term = d * inner;
            total = total + term;
        }
    }
    if (type == ORC_Q4_K) {
        const float m = (accm[0] + accm[2]) + (accm[1] + accm[3]);
        return sum8(acc) + m;
    }
    if (type == ORC_Q6_K) return sum8(acc);
    return total;
}

/* Row-parallel GEMV dispatch; src/qwen38/qwen38_quant.c:2833-2922. */
int orc_gemv_q8_k(float *output, const OrcQ8K *input, uint64_t input_length,
                  uint32_t type, const uint8_t *data, uint64_t rows)
{
    const uint32_t bytes = orc_block_bytes(type);
    if (!output || !input || !data || !bytes || input_length % ORC_QK) return 0;
    const uint64_t blocks = input_length / ORC_QK;
    for (uint64_t r = 0; r < rows; ++r)
        output[r] = orc_dot_q8_k(type, data + r * blocks * bytes, input, blocks);
    return 1;
}

/* Batch-major GEMM; src/qwen38/qwen38_quant.c:2950-3169.  Its 4-token tiles
 * are bit-identical to the per-token GEMV (tests/unit/test_qwen38_quant.c:
 * 637-684), so the oracle evaluates each token with the GEMV kernel. */
int orc_gemm_q8_k(float *output, const OrcQ8K *input, uint32_t batch,
                  uint64_t input_length, uint32_t type, const uint8_t *data,
                  uint64_t rows)
{
    if (!batch) return 0;
    const uint64_t blocks = input_length / ORC_QK;
    for (uint32_t t = 0; t < batch; ++t)
        if (!orc_gemv_q8_k(output + (uint64_t)t * rows, input + (uint64_t)t * blocks,
                           input_length, type, data, rows)) return 0;
    return 1;
}

/* Dequantised row via unit-basis dots (src/qwen38/qwen38_quant.c:3186-3223
 * with q38_dot_q4_k :396-426): element = (d*sc)*q - dmin*m in fp32, a -0.0
 * result becomes +0.0 through the fmaf with a +0 accumulator. */
int orc_row_f32(float *output, uint32_t type, const uint8_t *data,
                uint64_t width, uint64_t row)
{
    if (type != ORC_Q4_K || width % ORC_QK) return 0;
    const uint64_t blocks = width / ORC_QK;
    const uint8_t *blk = data + row * blocks * 144u;
    for (uint64_t b = 0; b < blocks; ++b, blk += 144) {
        const float d = orc_f16_to_f32(ld16(blk));
        const float dmin = orc_f16_to_f32(ld16(blk + 2));
        for (int c = 0; c < 4; ++c) {
            int sc0, m0, sc1, m1;
            scale_min_k4(2 * c, blk + 4, &sc0, &m0);
            scale_min_k4(2 * c + 1, blk + 4, &sc1, &m1);
            const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
            const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
            for (int i = 0; i < 32; ++i) {
                const uint8_t q = blk[16 + 32 * c + i];
                volatile float p0 = d0 * (float)(q & 15);
                volatile float p1 = d1 * (float)(q >> 4);
                output[b * 256 + 64 * c + i] = (p0 - mm0) + 0.0f;
                output[b * 256 + 64 * c + 32 + i] = (p1 - mm1) + 0.0f;
            }
        }
    }
    return 1;
}

/* First index of the maximum; src/qwen38/qwen38_model.c:1228-1239. */
uint32_t orc_argmax(const float *values, uint32_t count)
{
    uint32_t best = 0;
    float maximum = values[0];
    for (uint32_t i = 1; i < count; ++i) {
        if (values[i] > maximum) { maximum = values[i]; best = i; }
    }
    return best;
}

/* Greedy acceptance; src/qwen38/qwen38_model.c:1662-1702. */
uint32_t orc_accept(const float *batch_logits, uint32_t rows, uint32_t count,
                    const uint32_t *drafts, uint32_t *matched_out,
                    uint32_t *next_out, uint32_t *accepted)
{
    uint32_t matched = 0, next = 0;
    while (matched < rows) {
        const uint32_t target = orc_argmax(batch_logits + (uint64_t)matched * count, count);
        if (target != drafts[matched]) { next = target; break; }
        ++matched;
    }
    if (matched == rows) next = drafts[rows - 1];
    const uint32_t consumed = matched < rows ? matched + 1u : rows;
    for (uint32_t i = 0; i < matched; ++i) accepted[i] = drafts[i];
    if (matched < rows) accepted[matched] = next;
    *matched_out = matched;
    *next_out = next;
    return consumed;
}

void orc_iq1m_grid_entry(uint32_t index, int8_t out[8])
{
    const uint16_t code = q38_iq1m_grid_codes[index & 2047u];
    for (int k = 0; k < 8; ++k) out[k] = (int8_t)(((code >> (2 * k)) & 3) - 1);
}

/* RMS norm with a double-precision sum of float squares;
 * src/qwen38/qwen38_model.c:426-435. */
static void rmsnorm(float *out, const float *in, const float *w, int n)
{
    double sum = 0.0;
    for (int i = 0; i < n; ++i) {
        volatile float sq = in[i] * in[i];
        sum += (double)sq;
    }
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + 1e-6f);
    for (int i = 0; i < n; ++i) {
        volatile float t = in[i] * scale;
        out[i] = t * w[i];
    }
}

/* RoPE on dims 0..63 of each 256-wide head with the iterative theta;
 * src/qwen38/qwen38_model.c:697-713. */
static void rope(float *values, int heads, uint32_t position)
{
    const float theta_scale = powf(10000000.0f, -2.0f / 64.0f);
    for (int h = 0; h < heads; ++h) {
        float *v = values + h * 256;
        float theta = (float)position;
        for (int p = 0; p < 32; ++p) {
            const float c = cosf(theta), s = sinf(theta);
            const float x0 = v[p], x1 = v[p + 32];
            volatile float a0 = x0 * c, a1 = x1 * s, b0 = x0 * s, b1 = x1 * c;
            v[p] = a0 - a1;
            v[p + 32] = b0 + b1;
            theta *= theta_scale;
        }
    }
}

static float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

/* Full-attention decode core; src/qwen38/qwen38_model.c:816-885.  GQA 6:1
 * over 4 KV heads of 256, scores as an fmaf chain times 1/16, softmax with a
 * sequential denominator, output as an fmaf chain over positions, gated by
 * sigmoid.  The caches hold rows [0, position] of one layer. */
void orc_attention_decode(float *attention, const float *q_and_gate,
                          const float *key, const float *value,
                          float *key_cache, float *value_cache,
                          const float *q_norm, const float *k_norm,
                          uint32_t position)
{
    static float q[24 * 256], gate[24 * 256], k[1024];
    static float scores[1u << 20];
    for (int h = 0; h < 24; ++h) {
        memcpy(q + h * 256, q_and_gate + h * 512, 256 * sizeof(float));
        memcpy(gate + h * 256, q_and_gate + h * 512 + 256, 256 * sizeof(float));
        rmsnorm(q + h * 256, q + h * 256, q_norm, 256);
    }
    memcpy(k, key, sizeof(k));
    for (int h = 0; h < 4; ++h) rmsnorm(k + h * 256, k + h * 256, k_norm, 256);
    rope(q, 24, position);
    rope(k, 4, position);
    memcpy(key_cache + (uint64_t)position * 1024, k, 1024 * sizeof(float));
    memcpy(value_cache + (uint64_t)position * 1024, value, 1024 * sizeof(float));
    for (int h = 0; h < 24; ++h) {
        const int kv = h / 6;
        const float *qh = q + h * 256;
        float maximum = -INFINITY;
        for (uint32_t p = 0; p <= position; ++p) {
            const float *kr = key_cache + (uint64_t)p * 1024 + kv * 256;
            float s = 0.0f;
            for (int i = 0; i < 256; ++i) s = fmaf(qh[i], kr[i], s);
            s *= 1.0f / sqrtf(256.0f);
            scores[p] = s;
            if (s > maximum) maximum = s;
        }
        float den = 0.0f;
        for (uint32_t p = 0; p <= position; ++p) {
            scores[p] = expf(scores[p] - maximum);
            den += scores[p];
        }
        float *out = attention + h * 256;
        memset(out, 0, 256 * sizeof(float));
        for (uint32_t p = 0; p <= position; ++p) {
            const float *vr = value_cache + (uint64_t)p * 1024 + kv * 256;
            const float prob = scores[p] / den;
            for (int i = 0; i < 256; ++i) out[i] = fmaf(prob, vr[i], out[i]);
        }
        const float *g = gate + h * 256;
        for (int i = 0; i < 256; ++i) out[i] *= sigmoidf_ref(g[i]);
    }
}

/* ---- token sampler ------------------------------------------------------ */

typedef struct {
    uint32_t id;
    float logit;
} OrcCandidate;

/* higher logit first, lower id among equal logits (no NaN reaches here) */
static int candidate_order(const void *pa, const void *pb)
{
    const OrcCandidate *a = (const OrcCandidate *)pa, *b = (const OrcCandidate *)pb;
    if (a->logit != b->logit) return a->logit > b->logit ? -1 : 1;
    return a->id < b->id ? -1 : (a->id > b->id);
}

/* qwen38_sampler.c:38-46: the presence penalty is one fp32 subtraction */
static float penalised(const float *logits, const uint8_t *presence,
                       uint32_t presence_size, float penalty, uint32_t id)
{
    if (penalty == 0.0f || !presence || id >= presence_size || !presence[id])
        return logits[id];
    return logits[id] - penalty;
}

/* Restated by what it selects rather than by the reference's loops:
 *  - greedy (temperature <= 0 or top_k <= 1, :55): the first maximum of the
 *    adjusted logits, NaN never winning, except that a NaN at index 0 makes
 *    every comparison of the reference's strict > scan false (:57-60) and
 *    index 0 is kept;
 *  - sampling: the count = min(top_k, vocab) best adjusted logits that lie
 *    above -FLT_MAX, ordered by (logit descending, id ascending) and padded
 *    with (id 0, -FLT_MAX) -- the list the insertion of :74-83 leaves, found
 *    here by sorting.  With a NaN among the logits no such order exists and
 *    the list depends on where the NaN falls in the insertion sequence, so
 *    that sequence is stated as it is (a NaN fails every comparison and
 *    enters the last slot);
 *  - then :84-115 in fp32, sequential sums, expf of the C library, one
 *    xorshift64* draw (:12-20) as (double)(r >> 11) * 2^-53. */
int orc_sample(uint32_t *token, uint64_t *state, const float *logits,
               uint32_t vocab, float temperature, float top_p,
               float penalty, uint32_t top_k, const uint8_t *presence,
               uint32_t presence_size)
{
    if (!token || !state || !logits || vocab == 0) return 0;
    if (temperature <= 0.0f || top_k <= 1) {
        uint32_t best = 0;
        float best_value = penalised(logits, presence, presence_size, penalty, 0);
        if (!isnan(best_value)) {
            for (uint32_t id = 1; id < vocab; ++id) {
                const float v = penalised(logits, presence, presence_size, penalty, id);
                if (!isnan(v) && v > best_value) { best = id; best_value = v; }
            }
        }
        *token = best;
        return 1;
    }
    const uint32_t count = top_k < vocab ? top_k : vocab;
    OrcCandidate *all = (OrcCandidate *)malloc((size_t)vocab * sizeof(*all));
    float *prob = (float *)malloc((size_t)count * sizeof(float));
    if (!all || !prob) { free(all); free(prob); return 0; }
    int any_nan = 0;
    uint32_t eligible = 0;
    for (uint32_t id = 0; id < vocab; ++id) {
        const float v = penalised(logits, presence, presence_size, penalty, id);
        any_nan |= isnan(v);
        if (v > -FLT_MAX) { all[eligible].id = id; all[eligible].logit = v; ++eligible; }
    }
    OrcCandidate *list = all;   /* count entries */
    if (any_nan) {
        list = (OrcCandidate *)malloc((size_t)count * sizeof(*list));
        if (!list) { free(all); free(prob); return 0; }
        for (uint32_t i = 0; i < count; ++i) { list[i].id = 0; list[i].logit = -FLT_MAX; }
        for (uint32_t id = 0; id < vocab; ++id) {
            const float v = penalised(logits, presence, presence_size, penalty, id);
            /* a NaN on either side fails <=, so it enters */
            if (v <= list[count - 1].logit) continue;
            uint32_t at = count - 1;
            for (; at > 0 && v > list[at - 1].logit; --at) list[at] = list[at - 1];
            list[at].id = id;
            list[at].logit = v;
        }
    } else {
        qsort(all, eligible, sizeof(*all), candidate_order);
        for (uint32_t i = eligible; i < count; ++i) { all[i].id = 0; all[i].logit = -FLT_MAX; }
    }
    float total = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        prob[i] = expf((list[i].logit - list[0].logit) / temperature);
        total += prob[i];
    }
    const float keep = top_p > 0.0f && top_p < 1.0f ? top_p : 1.0f;
    uint32_t retained = count;
    float cumulative = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        cumulative += prob[i] / total;
        if (cumulative >= keep) { retained = i + 1; break; }
    }
    float retained_total = 0.0f;
    for (uint32_t i = 0; i < retained; ++i) retained_total += prob[i];
    uint64_t r = *state;
    r ^= r >> 12;
    r ^= r << 25;
    r ^= r >> 27;
    *state = r;
    const double unit = (double)((r * UINT64_C(2685821657736338717)) >> 11) * 0x1.0p-53;
    const float target = (float)unit * retained_total;
    uint32_t selected = list[retained - 1].id;
    float running = 0.0f;
    for (uint32_t i = 0; i < retained; ++i) {
        running += prob[i];
        if (target < running) { selected = list[i].id; break; }
    }
    if (list != all) free(list);
    free(all);
    free(prob);
    *token = selected;
    return 1;
}
