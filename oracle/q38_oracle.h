/* CPU oracle for the decode hot path of the Qwen3.8 engine.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (libq38hip.so) never links, calls or falls back to it.
 *
 * It restates, in plain C, the reference's x86 AVX2 build of the kernels
 * (the build the reference ships with -march=native on AVX2 hosts,
 * GNUmakefile:24).  Integer block sums are restated exactly; fp32 results
 * follow the reference's AVX2 lane order so they are bit-identical.
 * Every function cites the reference lines it follows.
 */
#ifndef Q38_ORACLE_H
#define Q38_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 256

/* Same layout as Q38Q8KBlock (include/qwen38/qwen38_quant.h:14-18). */
typedef struct {
    float scale;
    int8_t quants[ORC_QK];
    int16_t sums[ORC_QK / 16];
} OrcQ8K;

/* GGML type ids (include/qwen38/qwen38_gguf.h:29-52) */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13,
    ORC_Q6_K = 14, ORC_IQ2_XXS = 16, ORC_IQ2_XS = 17, ORC_IQ3_XXS = 18, ORC_IQ1_S = 19, ORC_IQ4_NL = 20,
    ORC_IQ3_S = 21, ORC_IQ2_S = 22, ORC_IQ4_XS = 23, ORC_IQ1_M = 29, ORC_BF16 = 30
};

float orc_f16_to_f32(uint16_t value);
int orc_nearest_int(float value);
int orc_quantize_q8_k(OrcQ8K *output, const float *input, uint64_t length);

uint32_t orc_block_bytes(uint32_t type);

/* Integer part of one 256-element super-block against one Q8_K block.
 * Q4_K: ints[0..7] = per-lane weighted sums W[l], ints[8..11] = min sums M[i].
 * IQ1_M: ints[0] = weighted, ints[1] = correction.
 * Q6_K: ints[0..7] = per-lane (weighted - offset).  Returns the count. */
int orc_block_ints(uint32_t type, const uint8_t *block, const OrcQ8K *input,
                   int32_t ints[12]);

float orc_dot_q8_k(uint32_t type, const uint8_t *row, const OrcQ8K *input,
                   uint64_t blocks);
int orc_gemv_q8_k(float *output, const OrcQ8K *input, uint64_t input_length,
                  uint32_t type, const uint8_t *data, uint64_t rows);
int orc_gemm_q8_k(float *output, const OrcQ8K *input, uint32_t batch,
                  uint64_t input_length, uint32_t type, const uint8_t *data,
                  uint64_t rows);
int orc_row_f32(float *output, uint32_t type, const uint8_t *data,
                uint64_t width, uint64_t row);

uint32_t orc_argmax(const float *values, uint32_t count);
/* Greedy acceptance of a verify batch (qwen38_model.c:1662-1702).  batch rows
 * of count logits; drafts[0..rows).  Returns consumed, writes matched,
 * next and the accepted token list (consumed entries). */
uint32_t orc_accept(const float *batch_logits, uint32_t rows, uint32_t count,
                    const uint32_t *drafts, uint32_t *matched, uint32_t *next,
                    uint32_t *accepted);

void orc_iq1m_grid_entry(uint32_t index, int8_t out[8]);

/* Full-attention decode core for one layer (qwen38_model.c:816-885): q_and_gate
 * [24][512], key/value [1024] for the new position, caches [ctx][1024] fp32.
 * Writes the new K/V row at position and the gated attention output [6144]. */
void orc_attention_decode(float *attention, const float *q_and_gate,
                          const float *key, const float *value,
                          float *key_cache, float *value_cache,
                          const float *q_norm, const float *k_norm,
                          uint32_t position);

/* ---- q38_oracle_formats.c: every matrix format of the reference model ---- */

/* Bytes and elements of one GGUF block of `type` (IQ4_NL: 18 / 32); 0 if
 * the format is not one the reference model accepts. */
uint32_t orc_format_block_bytes(uint32_t type);
uint32_t orc_format_block_elements(uint32_t type);
/* Q8_K path, one super-block (Q2_K .. IQ1_S except Q4_K, Q6_K, IQ1_M):
 * the eight int32 lanes of the AVX2 kernels and the block's integer min /
 * correction term (Q2_K, Q5_K, IQ1_S; else 0).  IQ4_NL: the 144 bytes of
 * eight 32-element blocks. */
int orc_format_block_lanes(uint32_t type, const uint8_t *block, const OrcQ8K *input, int32_t w[8],
                           int32_t *extra);
/* The integer weights q[256] (grid value and sign included) and the
 * integer scale of every 16 elements, s16[16], of one super-block. */
int orc_format_block_decode(uint32_t type, const uint8_t *block, int32_t q[256], int32_t s16[16]);
float orc_format_dot_q8_k(uint32_t type, const uint8_t *row, const OrcQ8K *input, uint64_t blocks);
int orc_format_gemv_q8_k(float *output, const OrcQ8K *input, uint64_t width, uint32_t type,
                         const uint8_t *data, uint64_t rows);
/* Float path (q38_dot_row): F32, F16, BF16, Q8_0, IQ4_NL and the K-quants
 * against fp32 input, one fmaf chain per row. */
float orc_format_dot_f32(uint32_t type, const uint8_t *row, const float *x, uint64_t length);
int orc_format_gemv_f32(float *output, const float *input, uint64_t width, uint32_t type,
                        const uint8_t *data, uint64_t rows);
/* q38_tensor_row_f32: row `row` of a [rows][width] matrix as fp32. */
int orc_format_row_f32(float *output, uint32_t type, const uint8_t *data, uint64_t width, uint64_t row);

/* Token sampler (src/qwen38/qwen38_sampler.c:51-119): the token drawn from
 * `logits` [vocab] with the Q38Sampler fields as arguments; *state is the
 * xorshift64* state, advanced by one step on the sampling path.  presence
 * may be NULL.  Returns 0 on bad arguments, as the reference does. */
int orc_sample(uint32_t *token, uint64_t *state, const float *logits,
               uint32_t vocab, float temperature, float top_p,
               float presence_penalty, uint32_t top_k,
               const uint8_t *presence, uint32_t presence_size);

#ifdef __cplusplus
}
#endif

#endif
