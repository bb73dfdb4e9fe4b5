/* libq38hip: MI355X (gfx950) kernels for the Qwen3.8 decode hot path.
 *
 * C ABI only: plain pointers and sizes.  Two families of entry points:
 *
 *  1. Drop-in replacements for the reference kernel ABI
 *     (include/qwen38/qwen38_quant.h:20-49 of shyringo/qwen3.8-27b-in-c):
 *     same names, same argument meaning, same 1/0 return convention.  They
 *     take HOST pointers, stage them through HBM and run the HIP kernels.
 *
 *  2. Device-resident variants (q38hip_*): every pointer, including
 *     tensor->data, is a device pointer; work is enqueued on `stream`
 *     (a hipStream_t; NULL means the legacy default stream) and the call
 *     returns without synchronising.  Return 1 on success, 0 on an argument
 *     error (message via q38hip_last_error()).
 *
 * Results are bit-identical to the reference's x86 AVX2 CPU kernels on the
 * same inputs: integer block sums exactly, fp32 outputs in the reference's
 * lane order.
 */
#ifndef Q38HIP_H
#define Q38HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout-compatible with Q38Q8KBlock (include/qwen38/qwen38_quant.h:14-18). */
#define Q38_Q8_K_BLOCK_SIZE 256
typedef struct {
    float scale;
    int8_t quants[Q38_Q8_K_BLOCK_SIZE];
    int16_t sums[Q38_Q8_K_BLOCK_SIZE / 16];
} Q38Q8KBlock;

/* Layout-compatible with Q38GGUFString / Q38GGUFTensor
 * (include/qwen38/qwen38_gguf.h:57-77).  shape[0] = input width,
 * shape[1] = output rows, type = GGML type id (Q4_K 12, Q6_K 14, IQ1_M 29). */
typedef struct {
    const char *data;
    uint64_t length;
} Q38GGUFString;

typedef struct {
    Q38GGUFString name;
    uint32_t n_dims;
    uint64_t shape[8];
    uint32_t type;
    uint64_t offset;
    uint64_t nbytes;
    const uint8_t *data;
    void *iq1_s_repack;
} Q38GGUFTensor;

/* Layout-compatible with Q38GGUFMeta / Q38GGUF
 * (include/qwen38/qwen38_gguf.h:59-90): the reference's mapped GGUF file,
 * which q38_prepare_iq1_s_repacks takes. */
typedef struct {
    Q38GGUFString key;
    uint32_t type;
    uint32_t array_type;
    uint64_t count;
    const uint8_t *data;
    uint64_t data_size;
} Q38GGUFMeta;

typedef struct {
    int fd;
    const uint8_t *mapping;
    uint64_t mapping_size;
    uint32_t version;
    uint32_t alignment;
    uint64_t data_offset;
    uint64_t tensor_count;
    uint64_t metadata_count;
    Q38GGUFTensor *tensors;
    Q38GGUFMeta *metadata;
} Q38GGUF;

/* ---- 1. reference kernel ABI, host pointers ------------------------------ */

/* replaces q38_f16_to_f32, include/qwen38/qwen38_quant.h:20 */
float q38_f16_to_f32(uint16_t value);

/* replaces q38_quantize_q8_k, include/qwen38/qwen38_quant.h:24-25 */
int q38_quantize_q8_k(Q38Q8KBlock *output, const float *input,
                      uint64_t length);

/* replaces q38_tensor_row_f32, include/qwen38/qwen38_quant.h:27-28: row
 * `row` as fp32 (F32 copied, F16 / BF16 converted, Q8_0, IQ4_NL and
 * Q2_K..Q6_K decoded; other types give NaN, as in the reference) */
int q38_tensor_row_f32(float *output, const Q38GGUFTensor *tensor,
                       uint64_t row);

/* replaces q38_tensor_dot_row_f32, include/qwen38/qwen38_quant.h:30-31:
 * one row's float dot; returns 1 only for a finite result */
int q38_tensor_dot_row_f32(float *output, const float *input,
                           const Q38GGUFTensor *tensor, uint64_t row);

/* replaces q38_tensor_gemv_f32, include/qwen38/qwen38_quant.h:34-35: fp32
 * input (F32, F16, BF16, Q8_0, IQ4_NL, Q2_K..Q6_K; NaN rows for the other
 * types, as in the reference) */
int q38_tensor_gemv_f32(float *output, const float *input,
                        const Q38GGUFTensor *tensor);

/* replaces q38_tensor_gemm_f32, include/qwen38/qwen38_quant.h:44-46;
 * batch-major output, any batch_size >= 1 */
int q38_tensor_gemm_f32(float *output, const float *input,
                        uint32_t batch_size, uint64_t input_length,
                        const Q38GGUFTensor *tensor);

/* replaces q38_tensor_gemv_q8_k, include/qwen38/qwen38_quant.h:38-40
 * (every Q8_K-path format: Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ1_S, IQ1_M,
 * IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_NL, IQ4_XS) */
int q38_tensor_gemv_q8_k(float *output, const Q38Q8KBlock *input,
                         uint64_t input_length,
                         const Q38GGUFTensor *tensor);

/* replaces q38_tensor_gemm_q8_k, include/qwen38/qwen38_quant.h:48-50;
 * output is batch-major, output[token * rows + row]; any batch_size >= 1 */
int q38_tensor_gemm_q8_k(float *output, const Q38Q8KBlock *input,
                         uint32_t batch_size, uint64_t input_length,
                         const Q38GGUFTensor *tensor);

/* replace q38_prepare_iq1_s_repacks / q38_release_iq1_s_repacks,
 * include/qwen38/qwen38_quant.h:54-55 (argument: the caller's Q38GGUF).
 * The GPU kernels read IQ1_S blocks as stored, so no view is built:
 * prepare returns 1 for a non-NULL argument and changes nothing. */
int q38_prepare_iq1_s_repacks(Q38GGUF *gguf);
void q38_release_iq1_s_repacks(Q38GGUF *gguf);

/* ---- 2. device-resident variants ---------------------------------------- */

/* Device form of q38_quantize_q8_k (src/qwen38/qwen38_quant.c:50-88):
 * `rows` independent fp32 rows of `length` elements each. */
int q38hip_quantize_q8_k(Q38Q8KBlock *output, const float *input,
                         uint64_t length, uint32_t rows, void *stream);

/* Device form of q38_tensor_gemm_q8_k (src/qwen38/qwen38_quant.c:2950-3169);
 * batch_size = 1 is q38_tensor_gemv_q8_k (:2833-2922).  Any batch_size >= 1:
 * the kernels take up to 8 tokens per launch, and larger batches run as
 * consecutive launches over token chunks (every token's outputs are
 * independent of the rest of the batch, so the bits are those of one call). */
int q38hip_gemm_q8_k(float *output, const Q38Q8KBlock *input,
                     uint32_t batch_size, uint64_t input_length,
                     const Q38GGUFTensor *tensor, void *stream);

/* Device form of q38_tensor_gemm_f32 (src/qwen38/qwen38_quant.c:2924-2948):
 * input is batch_size rows of input_length fp32 values; batch_size = 1 is
 * q38_tensor_gemv_f32 (:2812-2831).  Each output is the row's single fmaf
 * chain in the reference's element order (q38_dot_row, :2768-2810). */
int q38hip_gemm_f32(float *output, const float *input, uint32_t batch_size,
                    uint64_t input_length, const Q38GGUFTensor *tensor,
                    void *stream);

/* Device form of q38_tensor_row_f32 (src/qwen38/qwen38_quant.c:3185-3223)
 * for rows first_row .. first_row + row_count - 1: output[r * width + e]. */
int q38hip_row_f32(float *output, const Q38GGUFTensor *tensor,
                   uint64_t first_row, uint32_t row_count, void *stream);

/* Row-wise first-maximum index (q38_argmax, src/qwen38/qwen38_model.c:
 * 1228-1239) of `rows` rows of `count` floats; index_out[rows].  Partial
 * maxima go to a per-device scratch buffer that the library grows on demand
 * (after synchronising the device): calls that overlap on one device race. */
int q38hip_argmax(uint32_t *index_out, const float *values, uint32_t count,
                  uint32_t rows, void *stream);

/* No counterpart in the reference: q38hip_argmax for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  It allocates nothing: the partial
 * maxima go to a fixed 64 KiB array in the library's device memory instead
 * of the growable scratch, so ceil(count / 4096) * rows must be at most 8192
 * (248320-wide rows: up to 134 rows); larger calls return 0 with a message.
 * Every call on one device shares that array, so calls that overlap on one
 * device (on any streams) race.  Results are those of q38hip_argmax. */
int q38hip_argmax_noalloc(uint32_t *index_out, const float *values, uint32_t count,
                          uint32_t rows, void *stream);

/* Device form of q38_sample (src/qwen38/qwen38_sampler.c:51-119): the
 * token drawn from `logits` (vocabulary_size floats, device memory) into
 * *token (a device word).  The sampler's fields
 * (include/qwen38/qwen38_sampler.h:10-18) come as arguments: *state is the
 * xorshift64* state in HOST memory, read at the call and advanced before it
 * returns exactly as q38_sample advances it (one step when temperature > 0
 * and top_k > 1, none otherwise); presence, when not NULL, is presence_size
 * bytes of DEVICE memory (nonzero = token observed).  Token and state are
 * those of q38_sample on the same logits, bit for bit, NaN and infinite
 * logits included.  Limits: vocabulary_size <= 2^20 and, when sampling,
 * min(top_k, vocabulary_size) <= 1024; beyond them the call returns 0 with
 * a message.  Working memory is a per-device buffer (2 MiB, allocated on
 * the first call on a device): calls that overlap on one device race. */
int q38hip_sample(uint32_t *token, uint64_t *state, const float *logits, uint32_t vocabulary_size,
                  float temperature, float top_p, float presence_penalty, uint32_t top_k,
                  const uint8_t *presence, uint32_t presence_size, void *stream);

/* Greedy acceptance of a verify batch (src/qwen38/qwen38_model.c:1662-1702):
 * targets[rows] are the per-row argmaxes, drafts[rows] the draft ids.
 * result[0] = consumed, result[1] = matched, result[2] = next,
 * result[3 .. 3+consumed) = accepted tokens.  result needs rows + 3 words. */
int q38hip_accept(uint32_t *result, const uint32_t *targets,
                  const uint32_t *drafts, uint32_t rows, void *stream);

/* Library extension (no counterpart in the reference): the 16-row tiled
 * layout of a Q4_K matrix that the model engine keeps beside the GGUF
 * layout for its GEMVs and GEMMs.  Tile k holds rows 16k..16k+15 as
 * [block][row][144 bytes]; the last tile is zero-padded.
 * q38hip_tiled_q4k_bytes: size of the tiled copy of `rows` rows of
 * `input_length` elements.  q38hip_repack_q4k_tiles: write it from the
 * row-major matrix (both in device memory). */
uint64_t q38hip_tiled_q4k_bytes(uint32_t rows, uint64_t input_length);
int q38hip_repack_q4k_tiles(void *tiled, const void *q4k_rows, uint32_t rows,
                            uint64_t input_length, void *stream);

/* q38hip_gemm_q8_k over a tiled Q4_K copy: output[t * rows + r] for
 * t < batch_size (at least 1: one launch for one token or a prefill batch,
 * else launches of 2..8 tokens), input_length 5120, 6144, 10240 or 17408.
 * The results are those of q38hip_gemm_q8_k bit for bit. */
int q38hip_gemm_q8_k_tiled(float *output, const Q38Q8KBlock *input,
                           uint32_t batch_size, uint64_t input_length,
                           const void *tiled, uint32_t rows, void *stream);

/* Library extension: the same 16-row tiled copy for IQ1_M
 * ([tile = row / 16][block][row % 16][56 bytes], rows past the last zero),
 * which the engine keeps beside the row-major blocks.
 * q38hip_tiled_iq1m_bytes: its size (0 for a bad shape);
 * q38hip_repack_iq1m_tiles: write it from the row-major matrix (both in
 * device memory, the copy 8-byte aligned); q38hip_gemm_q8_k_iq1m_tiled:
 * q38hip_gemm_q8_k over it for batch_size 1..8 (output[t * rows + r]),
 * input_length 5120, 6144, 10240 or 17408, bit for bit q38hip_gemm_q8_k's
 * results. */
uint64_t q38hip_tiled_iq1m_bytes(uint32_t rows, uint64_t input_length);
int q38hip_repack_iq1m_tiles(void *tiled, const void *iq1m_rows, uint32_t rows,
                             uint64_t input_length, void *stream);
int q38hip_gemm_q8_k_iq1m_tiled(float *output, const Q38Q8KBlock *input,
                                uint32_t batch_size, uint64_t input_length,
                                const void *tiled, uint32_t rows, void *stream);

/* Library extension: the full-attention decode core of one layer on the
 * device, for kernel-level use and tests.  It is the reference's static
 * q38_full_core (src/qwen38/qwen38_model.c:816-885) for `rows` consecutive
 * positions position .. position + rows - 1, row t seeing positions
 * 0 .. position + t (q38_batch_full_attention, :1089-1119): per-head RMS
 * norms of q and k (q_norm, k_norm: 256 floats), RoPE, the K/V cache write
 * of each row, scores, softmax and the sigmoid-gated output.
 *   q_and_gate: row t at t * in_stride floats, 24 heads x (256 q | 256 gate);
 *   key, value: row t at t * in_stride floats, 1024 each;
 *   key_cache: [context_length][1024] fp32 (one layer); value_cache:
 *     channel-major [1024][pitch] fp32 with pitch = context_length rounded
 *     up to a multiple of 32 (position p of channel e at e * pitch + p);
 *     positions before `position` already filled, positions position ..
 *     position + rows - 1 are written;
 *   attention: [rows][6144] gated output; attention_q8k (optional, may be
 *     NULL): its Q8_K blocks [rows][24], the input of the output projection.
 * All pointers are device pointers.  position + rows <= context_length <= 524256.
 * Allocates and frees its working buffers (the RoPE table of the context,
 * the scores) and synchronises `stream` before returning. */
int q38hip_attention_rows(float *attention, Q38Q8KBlock *attention_q8k, const float *q_and_gate,
                          const float *key, const float *value, uint64_t in_stride,
                          const float *q_norm, const float *k_norm, float *key_cache,
                          float *value_cache, uint32_t context_length, uint32_t position,
                          uint32_t rows, void *stream);

/* Last argument error of the calling thread ("" when none). */
const char *q38hip_last_error(void);

/* Synchronise the device; returns 1 when no HIP error is pending. */
int q38hip_synchronize(void);

#ifdef __cplusplus
}
#endif

#endif
