/* libq38hip model ABI: the reference engine's model API on one MI355X.
 *
 * Same names, signatures, argument meaning, ownership and 1/0 (NULL) return
 * convention as include/qwen38/qwen38_model.h:10-50 of
 * shyringo/qwen3.8-27b-in-c, so the reference's CLI, server and probes link
 * against libq38hip.so unchanged.  The GGUF weights are uploaded to HBM at
 * open; every call runs on one HIP stream owned by the model and returns
 * after its results are on the host.  Returned logits pointers are owned by
 * the model (pinned host memory) and are overwritten by the next call, as in
 * the reference.  Not reentrant: one caller thread per model.
 *
 * Supported checkpoints: the Qwen3.8-27B "qwen35" contract
 * (src/qwen38/qwen38_model.c:196-319) with every matrix type the reference
 * accepts (q38_matrix_type_supported, qwen38_model.c:172-189): the Q8_K
 * path types Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS,
 * IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS and IQ4_NL, and the float-input types F32,
 * F16, BF16 and Q8_0; F32 norm / conv / ssm vectors.  The token embedding
 * may be any of these; for a type the reference's row decode has no case for
 * (qwen38_quant.c:2768-2810: the IQ types but IQ4_NL) its rows are NaN, as
 * in the reference.  Other types are rejected at open with a message.
 */
#ifndef Q38MODEL_H
#define Q38MODEL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct Q38Model Q38Model;

/* qwen38_model.h:12 (open + upload to HBM; NULL on failure, and for a
 * context_length above 524256 positions) */
Q38Model *q38_model_open_gguf(const char *path, uint32_t context_length);
/* qwen38_model.h:13 */
int q38_model_attach_mtp_gguf(Q38Model *model, const char *path);
/* qwen38_model.h:14-15 */
void q38_model_close(Q38Model *model);
void q38_model_reset(Q38Model *model);

/* qwen38_model.h:19-20: one token through the model; *logits = 248320 floats */
int q38_model_forward_token(Q38Model *model, uint32_t token_id, const float **logits);

/* qwen38_model.h:24-25: layer-major prompt evaluation, logits of the last token */
int q38_model_prefill(Q38Model *model, const uint32_t *tokens, uint32_t token_count, const float **logits);

/* qwen38_model.h:29-31: MTP head (enable before the first target token) */
int q38_model_enable_mtp(Q38Model *model);
int q38_model_mtp_forward(Q38Model *model, uint32_t token_id, const float **logits);

/* qwen38_model.h:37-41: draft up to draft_count MTP tokens, verify them in
 * one batch, greedy acceptance; accepted_tokens needs draft_count entries.
 * Any draft_count from 1 to context_length - position, as the reference:
 * up to 8 the step runs as captured HIP graphs with one verify batch, above
 * 8 the verify runs in 8-row chunks (the same results) */
int q38_model_speculative_greedy(Q38Model *model, uint32_t token_id, uint32_t stop_token, uint32_t draft_count,
                                 uint32_t *accepted_tokens, uint32_t *accepted_count, const float **next_logits);

/* qwen38_model.h:45-46: hidden state after the first layer_count blocks */
int q38_model_forward_token_layers(Q38Model *model, uint32_t token_id, uint32_t layer_count, float *hidden_out);

/* Library extension (no counterpart in the reference): q38_sample
 * (src/qwen38/qwen38_sampler.c:51-119) on the device over the logits that
 * the model's last forward_token / prefill / mtp_forward /
 * speculative_greedy call returned (their copy in HBM; 0 when the last call
 * returned none or failed).  The arguments are the Q38Sampler fields
 * (include/qwen38/qwen38_sampler.h:10-18): *state is the xorshift64* state,
 * advanced as q38_sample advances it; presence is the caller's HOST array
 * of presence_size bytes, as the reference CLI keeps it, copied to the
 * device when presence_penalty is nonzero.  *token and *state are those of
 * q38_sample on the same logits, bit for bit.  Sampling calls take at most
 * 1024 candidates (min(top_k, vocabulary)); beyond that the call returns 0. */
int q38hip_model_sample(Q38Model *model, uint64_t *state, float temperature, float top_p, float presence_penalty,
                        uint32_t top_k, const uint8_t *presence, uint32_t presence_size, uint32_t *token);

/* Library extension: q38_model_forward_token(token_id) followed by
 * q38hip_model_sample, without downloading the logits (the reference CLI's
 * generation step, src/cli/qwen38_main.c:545-553 and the forward that
 * follows it, in one call).  The logits stay in HBM, where a following
 * q38hip_model_sample can sample them again. */
int q38hip_model_forward_sample(Q38Model *model, uint32_t token_id, uint64_t *state, float temperature, float top_p,
                                float presence_penalty, uint32_t top_k, const uint8_t *presence,
                                uint32_t presence_size, uint32_t *next_token);

/* Library extension for measurement (no counterpart in the reference): the
 * device time of one block of the target model over `rows` (1..8) verify
 * rows, as the speculative verify runs it, at positions position ..
 * position + rows - 1 of the current cache.  `layer` is 0..63 (every fourth,
 * 3, 7, .., a full-attention block).  The block is captured as a HIP graph
 * and replayed `repeats` times between two events on the model's stream;
 * *block_us is the mean time of one replay.  *tail_us is the same for the
 * verify tail of a `rows`-row batch: the argmax of `rows` logits rows,
 * the greedy acceptance and the gather of the returned logits row.  The
 * call leaves the model's position, state slots and logits as they were
 * (it writes only cache entries at and after `position`, which the next
 * token overwrites before any read).  0 on bad arguments. */
int q38hip_model_time_block(Q38Model *model, uint32_t layer, uint32_t rows, uint32_t repeats, float *block_us,
                            float *tail_us);

/* qwen38_model.h:48-50 */
uint32_t q38_model_vocab_size(const Q38Model *model);
uint32_t q38_model_position(const Q38Model *model);
uint32_t q38_model_context_length(const Q38Model *model);

#ifdef __cplusplus
}
#endif

#endif
