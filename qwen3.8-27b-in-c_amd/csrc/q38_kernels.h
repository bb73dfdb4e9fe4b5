/* Host-side launchers of the gfx950 kernels (enqueue only; no synchronisation). */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q38 {

/* state slots of each recurrent layer: one more than the largest batch */
constexpr uint32_t kRecurrentStateSlots = 9;

/* q38_gemm.hip: y[m][rows] = W (rows x nblk*256, GGUF type) . x (m Q8_K rows);
 * m <= 8.  `grid` is the device IQ1_M codebook: 2048 x 8 int8 grid values,
 * followed by the one-token kernel's 4096 x 8 table of 8 g + delta (q38_abi.hip). */
bool launch_gemm(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t rows, uint32_t nblk,
                 const void *grid, hipStream_t stream);
/* lane-chain kernel for 2..4 tokens; false when it does not apply */
bool launch_gemv_lanes(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                       uint32_t nb, hipStream_t stream);
/* Q4_K matrices in the 16-row tiled layout (q38_tiled.hip): bytes of the
 * tiled copy, the repack from row-major, and the matrix-core GEMM for 2..8
 * tokens (false when the width or token count is not supported) */
size_t tiled_q4k_bytes(uint32_t rows, uint32_t nb);
bool launch_repack_q4k_tiles(uint8_t *dst, const uint8_t *src, uint32_t rows, uint32_t nb, hipStream_t stream);
/* IQ1_M x Q8_K for prefill batches (any token count, 256 rows x 64 tokens
 * per workgroup; false for unsupported widths) */
bool launch_gemm_iq1m_wide(uint32_t tokens, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, const void *grid, hipStream_t stream);
/* IQ1_M x Q8_K for 1..8 tokens on the matrix cores (row-major blocks) */
bool launch_gemm_iq1m_mfma(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, const void *grid, hipStream_t stream);
/* the same over a 16-row tiled copy ([tile = row / 16][block][row % 16][56
 * bytes], rows past the last zero), made by launch_repack_iq1m_tiles into
 * tiled_iq1m_bytes(rows, nb) bytes (8-byte aligned) */
bool launch_gemm_iq1m_tiled(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                            uint32_t nb, const void *grid, hipStream_t stream);
size_t tiled_iq1m_bytes(uint32_t rows, uint32_t nb);
bool launch_repack_iq1m_tiles(uint8_t *dst, const uint8_t *src, uint32_t rows, uint32_t nb, hipStream_t stream);
bool launch_gemm_q4k_tiled(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, hipStream_t stream);
/* one token over the 16-row Q4_K tiled copy (q38_q4k_gemv.hip): y[row] for
 * widths of 20, 24, 40 or 68 blocks; false otherwise */
bool launch_gemv_q4k_tiled(const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t rows, uint32_t nb,
                           hipStream_t stream);
/* same product, 32 weight rows per wavefront (v_mfma_f32_32x32x16_f16) */
bool launch_gemm_q4k_t32(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                         uint32_t nb, hipStream_t stream);
/* q38_mm16.hip: the same product for 2..4 tokens on 20-block matrices of
 * kMm16MinRows .. 36864 rows, 16 rows per wavefront
 * (v_mfma_f32_16x16x32_f16); false for unsupported shapes */
constexpr uint32_t kMm16MinRows = 32768;
bool launch_gemm_q4k_mm16(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                          uint32_t nb, hipStream_t stream);
/* q38_wide.hip: the same product for any token count (the prefill batch),
 * 64 rows x 64 tokens per workgroup; false for unsupported shapes.
 * launch_gemm_q4k_tiled takes it from kWideMinTokens tokens on. */
constexpr int kWideMinTokens = 9;
bool launch_gemm_q4k_wide(uint32_t tokens, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy,
                          uint32_t rows, uint32_t nb, hipStream_t stream);
/* same with the token rows of y `ldy` floats apart (ldy >= rows) */
bool launch_gemm_ld(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                    uint32_t nblk, const void *grid, hipStream_t stream);

/* q38_formats.hip: every other matrix format of the reference model.
 * format_block_shape: elements and bytes of one GGUF block of any type the
 * GGUF reader sizes (q38_ggml_block_elements / _bytes,
 * src/io/qwen38_gguf.c:129-184; false otherwise).  format_takes_q8k: the GEMV takes Q8_K
 * activations (else fp32).  launch_gemm_format: y[t * ldy + row] for t < m
 * (1..8) against Q8_K activations, for Q2_K, Q3_K, Q5_K, IQ2_XXS, IQ2_XS,
 * IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS, IQ4_NL and IQ1_S (`grid`: the IQ1_M/IQ1_S
 * codebook as 2048 x 8 int8); false for other types.  launch_gemm_float:
 * the same against fp32 activations x[t * width + e] (m 1..4) for F32, F16,
 * BF16, Q8_0, IQ4_NL and Q2_K..Q6_K.  launch_row_decode: rows of such a
 * matrix as fp32 (q38_tensor_row_f32), output row r from matrix row ids[r]
 * (clamped below `limit`) or first + r. */
bool format_block_shape(int type, uint32_t *elements, uint32_t *bytes);
bool format_takes_q8k(int type);
bool format_row_decodable(int type);
bool launch_gemm_format(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                        uint32_t nb, const void *grid, hipStream_t stream);
bool launch_gemm_float(int type, int m, const uint8_t *w, const float *x, float *y, uint32_t ldy, uint32_t rows,
                       uint32_t width, hipStream_t stream);
bool launch_row_decode(int type, const uint8_t *w, const uint32_t *ids, uint32_t first, uint32_t count,
                       uint32_t limit, float *out, uint32_t width, hipStream_t stream);
/* out[0 .. count) = value */
void launch_fill_f32(float *out, uint64_t count, float value, hipStream_t stream);

/* q38_abi.hip: record an argument error for q38hip_last_error(); returns 0 */
int abi_fail(const char *message);

/* q38_misc.hip */
void launch_quantize(const float *x, uint8_t *out, uint32_t nblocks, hipStream_t stream);
uint32_t argmax_chunks(uint32_t count);
void launch_argmax(const float *values, uint32_t count, uint32_t rows, float *pv, uint32_t *pi, uint32_t *out,
                   hipStream_t stream);
/* result[0] = rows consumed, [1] = drafts matched, [2] = next token,
 * [3 ..] = accepted tokens, over `rows` rows, or over the rows up to the
 * first draft equal to *stop when stop is not null */
void launch_accept(uint32_t *result, const uint32_t *targets, const uint32_t *drafts, uint32_t rows,
                   hipStream_t stream, const uint32_t *stop = nullptr);
/* dst[0 .. count) = row (*index - 1) of the `rows` rows of src, `stride`
 * floats apart (index clamped to 1 .. rows) */
void launch_copy_row(float *dst, const float *src, size_t stride, uint32_t count, const uint32_t *index,
                     uint32_t rows, hipStream_t stream);
/* The verify tail of a speculative transaction (rows <= 8): the argmax of
 * each of `rows` rows of `count` values into targets, the greedy acceptance
 * of the drafts into result (3 + rows words, as launch_accept) and the copy
 * of row consumed - 1 into dst; two launches.  count must be a multiple of
 * 4; false for unsupported shapes. */
bool launch_verify_tail(const float *values, uint32_t count, uint32_t rows, float *pv, uint32_t *pi,
                        uint32_t *targets, const uint32_t *drafts, const uint32_t *stop, uint32_t *result, float *dst,
                        hipStream_t stream);

/* q38_sample.hip: q38_sample (qwen38_sampler.c:51-119) on a device logits
 * row; *token_out is a device word written on `stream`.  *state is the
 * caller's xorshift64* state in host memory: a sampling call (temperature
 * > 0 and top_k > 1) draws once from it, and launch_sample advances it as
 * q38_sample does.  presence is a device byte per token or null.
 * check_sample names what a call exceeds (at most kMaxSampleTopK
 * candidates, kMaxSampleVocab logits), or null; launch_sample returns false
 * for such calls.  `scratch` holds sample_scratch_bytes(vocab, top_k)
 * bytes. */
constexpr uint32_t kMaxSampleTopK = 1024;
constexpr uint32_t kMaxSampleVocab = 1u << 20;
constexpr uint32_t kMaxSampleChunks = 256;
size_t sample_scratch_bytes(uint32_t vocab, uint32_t top_k);
const char *check_sample(uint32_t vocab, float temperature, uint32_t top_k);
bool launch_sample(uint32_t *token_out, uint64_t *state, const float *logits, uint32_t vocab, const uint8_t *presence,
                   uint32_t presence_size, float temperature, float top_p, float presence_penalty, uint32_t top_k,
                   void *scratch, hipStream_t stream);

/* q38_model.hip.  Rows of a batch are contiguous; q_out receives Q8_K blocks. */
void launch_norm_quant(float *norm_out, long long norm_stride, uint8_t *q_out, int q_stride_blocks, float *hidden,
                       long long in_stride, const float *branch, const float *weight, int rows, hipStream_t stream);
void launch_add(float *hidden, const float *branch, long long n, hipStream_t stream);
/* row t of gate and up starts at t * stride floats; f_out (optional) gets
 * the fp32 rows before quantisation, row t at t * 17408 */
void launch_swiglu_quant(uint8_t *q_out, const float *gate, const float *up, long long stride, int rows,
                         hipStream_t stream, float *f_out = nullptr);
void launch_embed_q4k(float *out, const uint8_t *w, const uint32_t *tokens, int count, int width, uint32_t vocab,
                      hipStream_t stream);
/* gated DeltaNet core of one row: conv + SiLU + q/k L2 norm + beta/alpha,
 * then the state update; the per-head norm, z gate and Q8_K run over all rows */
/* Recurrent state lives in kRecurrentStateSlots slots per layer, `slot_stride`
 * floats apart: row t of a batch reads slot (*slot + t) and writes slot
 * (*slot + t + 1), both mod kRecurrentStateSlots, so the state after any
 * prefix of the batch stays available. */
/* last_only: write only the state after the last row (slot *slot + rows),
 * for prefill batches of any length */
void launch_deltanet_prep(float *qkv, long long ld, int beta_off, int alpha_off, float *conv_state,
                          long long slot_stride, const uint32_t *slot, int rows, const float *conv_w,
                          const float *ssm_a, const float *ssm_dt, bool last_only, hipStream_t stream);
void launch_deltanet_state(float *attn, float *delta_state, long long slot_stride, const uint32_t *slot, int rows,
                           const float *qkv, long long ld, int beta_off, int alpha_off, float query_scale,
                           bool last_only, hipStream_t stream);
/* the prep of a prefill batch, all rows in parallel: prepared q/k/v, beta
 * and alpha of row t go to out + t * ld (qkv untouched); the conv state
 * after the batch goes to slot *slot + rows */
void launch_deltanet_prep_rows(float *out, const float *qkv, long long ld, int beta_off, int alpha_off,
                               float *conv_state, long long slot_stride, const uint32_t *slot, int rows,
                               const float *conv_w, const float *ssm_a, const float *ssm_dt, hipStream_t stream);
/* launch_deltanet_prep + launch_deltanet_state in one kernel (1..8 rows;
 * false otherwise); q/k/v, beta and alpha in qkv stay untransformed */
bool launch_deltanet_fused(float *attn, float *delta_state, long long slot_stride, const uint32_t *slot, int rows,
                           const float *qkv, long long ld, int beta_off, int alpha_off, float query_scale,
                           float *conv_state, long long conv_stride, const float *conv_w, const float *ssm_a,
                           const float *ssm_dt, hipStream_t stream);
void launch_deltanet_out_quant(float *attn, uint8_t *q_out, const float *z, long long z_stride, const float *ssm_norm,
                               int rows, hipStream_t stream);
/* full attention over `rows` rows at positions *position + t: prep (norms,
 * RoPE, K/V write), scores, softmax, V + gate, Q8_K of the output.
 * key_cache of one layer: [context][1024] fp32; value_cache: channel-major
 * [1024][value_pitch(context)] fp32 (position p of channel e at
 * e * value_pitch + p), so each chain of the weighted sum reads consecutive
 * positions.  configure_attention(context) sets the kernels up for a
 * context length on the current device; false for a context above
 * kMaxAttentionContext (a layer's value block is addressed with 31-bit byte
 * offsets). */
constexpr uint32_t kMaxAttentionContext = 524256;
__host__ __device__ inline uint32_t value_pitch(uint32_t context) { return (context + 31) & ~31u; }
bool configure_attention(int context);
/* host: the RoPE cos/sin table of positions [0, context), 64 floats each */
void rope_table_host(float *table, uint32_t context);
void launch_attention(float *attn, uint8_t *q_out, float *q_buf, const float *q_and_gate, const float *key,
                      const float *value, long long in_stride, const float *q_norm, const float *k_norm,
                      const float *rope, float *key_cache, float *value_cache, float *scores, int context,
                      const uint32_t *position, int rows, hipStream_t stream);
/* K-norm, RoPE and K/V cache write of `rows` rows without the query side */
void launch_kv_write(const float *key, const float *value, long long in_stride, const float *k_norm,
                     const float *rope, float *key_cache, float *value_cache, int context, const uint32_t *position,
                     int rows, hipStream_t stream);

}  // namespace q38
