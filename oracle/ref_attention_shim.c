/* TEST INFRASTRUCTURE ONLY (never linked into the product).
 *
 * Compiles the reference's own engine source, src/qwen38/qwen38_model.c,
 * found through the include path oracle/Makefile passes, into
 * oracle/_ref/libq38ref.so, and exports one entry into its static
 * full-attention core q38_full_core (src/qwen38/qwen38_model.c:816-885):
 * per-head q/k RMS norms, RoPE, the K/V cache write at `position`, scores,
 * softmax and the gated output of one decode row of a full-attention layer
 * (layer 3, full-attention index 0).  The caches are caller-owned
 * [context_length][1024] fp32 arrays and are updated in place, as the
 * reference updates its own.  Nothing in the reference is changed: the shim
 * only fills the Q38Model fields that q38_full_core reads. */
#include "qwen38_model.c"

int q38ref_full_core(float *attention, const float *q_and_gate, float *key, const float *value,
                     float *key_cache, float *value_cache, uint32_t context_length,
                     const float *q_norm, const float *k_norm, uint32_t position)
{
    if (!attention || !q_and_gate || !key || !value || !key_cache || !value_cache || !q_norm || !k_norm ||
        position >= context_length)
        return 0;
    Q38GGUFTensor qn, kn;
    memset(&qn, 0, sizeof(qn));
    memset(&kn, 0, sizeof(kn));
    qn.n_dims = kn.n_dims = 1;
    qn.shape[0] = kn.shape[0] = Q38_ATTN_HEAD_DIM;
    qn.type = kn.type = Q38_GGML_F32;
    qn.data = (const uint8_t *)q_norm;
    kn.data = (const uint8_t *)k_norm;
    Q38Model *model = (Q38Model *)calloc(1, sizeof(*model));
    float *q = (float *)calloc(Q38_ATTN_Q_DIM, sizeof(float));
    float *gate = (float *)calloc(Q38_ATTN_Q_DIM, sizeof(float));
    float *scores = (float *)calloc((size_t)Q38_ATTN_HEADS * context_length, sizeof(float));
    int ok = 0;
    if (model && q && gate && scores) {
        model->layers[3].attention.full.q_norm = &qn;
        model->layers[3].attention.full.k_norm = &kn;
        model->context_length = context_length;
        model->key_cache = key_cache;
        model->value_cache = value_cache;
        model->scratch.q = q;
        model->scratch.gate = gate;
        model->scratch.scores = scores;
        ok = q38_full_core(model, 3, q_and_gate, key, value, attention, position);
    }
    free(scores);
    free(gate);
    free(q);
    free(model);
    return ok;
}
