/* Deterministic synthetic Qwen3.8-27B GGUF writer (random-init weights).
 *
 * Writes the 65-block "qwen35" GGUF that the reference engine's loader accepts
 * (metadata and tensor contract of src/qwen38/qwen38_model.c:196-319 and
 * src/io/qwen38_gguf.c:263-370): 64 layers (every fourth a full-attention
 * layer, the rest DeltaNet), the MTP block 64 with its nextn.* tensors, a Q4_K
 * token embedding and a Q6_K LM head.  Layer matrices are Q4_K ("q4km") or
 * IQ1_M ("iq1m").
 *
 * Every byte is a pure function of (seed, tensor index, position): a
 * splitmix64 hash of a counter, so the file is identical on every host and
 * thread count.  Block scales are chosen so that the effective weights have
 * mean ~0 and standard deviation ~1/sqrt(fan_in), which keeps 64 random layers
 * finite:
 *   Q4_K  w = d*sc*q - dmin*m with dmin = 8d and m = round(15 sc / 16), so
 *         each 32-element sub-block is centred (q uniform 0..15);
 *   Q6_K  w = d*sc*(q-32), sc uniform int8;
 *   IQ1_M w = d*(2s+1)*(grid +- 1/8), grid values in {-1,0,1}.
 *
 * Two more variants exercise the speculative path, whose drafts random
 * weights almost never get accepted:
 *   accept      the Q4_K_M layout without the MTP block (64 blocks), with an
 *               LM head whose rows 2.. are all-zero blocks, so every logit
 *               but the first two is exactly zero and the greedy token is 0,
 *               1 or 2: MTP drafts and the target agree about a third of the
 *               time;
 *   accept_mtp  the matching separate MTP checkpoint (q38_model_attach_mtp_gguf):
 *               65-block metadata, token_embd, the same LM head and block 64
 *               with its nextn.* tensors.
 * A third accepts every draft:
 *   accept_all  the 65-block Q4_K_M file whose LM head rows all hold the
 *               bytes of row 0: every logit of a row is the same value (a
 *               function of the hidden state), so the target's and the MTP
 *               head's greedy token is always 0 and every draft is accepted.
 * A tensor's bytes depend on its place in the full 65-block Q4_K_M list, so
 * tensors shared between variants are byte-identical.
 *
 * The mixed variant exercises every other matrix format the reference model
 * accepts: the layer matrices cycle through Q2_K, Q3_K, Q5_K, IQ2_XXS,
 * IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS, IQ4_NL, IQ1_S, Q4_K, Q6_K and
 * IQ1_M; the small DeltaNet alpha / beta and attention K / V matrices cycle
 * through Q8_0, F16, BF16 and F32, as do the FFN down, attention output and
 * DeltaNet output matrices of a few layers (so every producer of a float
 * projection input is used); the token embedding is Q8_0 and the LM head
 * Q5_K.  Random bytes with each format's fp16 scales set to a size that
 * gives weights of standard deviation ~1/sqrt(fan_in) (the constants below
 * are the standard deviation of a block's weights at scale 1); Q2_K and Q5_K
 * mins are set to centre their sub-blocks as for Q4_K.
 *
 * Usage: q38_synth_gguf OUT.gguf SEED q4km|iq1m|accept|accept_mtp|accept_all|mixed
 *        (OUT.gguf "-": print the file size only)
 */
#define _GNU_SOURCE
#include <fcntl.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

enum {
    F32 = 0, F16 = 1, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ2_XXS = 16, IQ2_XS = 17,
    IQ3_XXS = 18, IQ1_S = 19, IQ4_NL = 20, IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23, IQ1_M = 29, BF16 = 30
};
enum { HIDDEN = 5120, FFN = 17408, VOCAB = 248320, LAYERS = 64 };

static uint64_t mix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static uint64_t hash3(uint64_t seed, uint64_t tensor, uint64_t counter)
{
    return mix64(mix64(seed ^ (tensor * 0xd1b54a32d192ed03ull)) ^ counter);
}

/* uniform in [0, 1) from the top 53 bits */
static double unit(uint64_t h) { return (double)(h >> 11) * 0x1p-53; }

/* IEEE binary16, round to nearest even (finite, |x| < 65504) */
static uint16_t f32_to_f16(float value)
{
    uint32_t x;
    memcpy(&x, &value, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x >= 0x477fe000u) return (uint16_t)(sign | 0x7c00u);          /* overflow */
    if (x < 0x38800000u) {                                           /* subnormal half */
        if (x < 0x33000000u) return (uint16_t)sign;                  /* < 2^-25 -> 0 */
        const uint32_t e = x >> 23, m = (x & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;                              /* 14..24 */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((x >> 13) - (112u << 10));
    const uint32_t rem = x & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return (uint16_t)(sign | h);
}

typedef struct {
    char name[64];
    uint32_t n_dims;
    uint64_t shape[2];
    uint32_t type;
    uint64_t offset;
    uint64_t nbytes;
    int kind;      /* 0 matrix, 1 norm weight, 2 conv, 3 dt bias, 4 ssm_a */
    int live_rows; /* > 0: only the first live_rows rows are non-zero */
    int same_rows; /* every row holds the bytes of row 0 */
    int written;   /* part of the output file */
    uint64_t id;   /* seed index: place in the full tensor list */
} Tensor;

static Tensor tensors[1024];
static int tensor_count;

/* bytes and elements of one block */
static uint64_t block_bytes(uint32_t type)
{
    switch (type) {
    case Q4_K: return 144;
    case Q6_K: return 210;
    case IQ1_M: return 56;
    case Q2_K: return 84;
    case Q3_K: return 110;
    case Q5_K: return 176;
    case IQ2_XXS: return 66;
    case IQ2_XS: return 74;
    case IQ2_S: return 82;
    case IQ3_XXS: return 98;
    case IQ3_S: return 110;
    case IQ4_XS: return 136;
    case IQ4_NL: return 18;
    case IQ1_S: return 50;
    case Q8_0: return 34;
    case F16: case BF16: return 2;
    default: return 4;
    }
}

static uint64_t block_elements(uint32_t type)
{
    switch (type) {
    case F32: case F16: case BF16: return 1;
    case Q8_0: case IQ4_NL: return 32;
    default: return 256;
    }
}

/* matrix formats of the mixed variant */
static const uint32_t q8k_cycle[14] = {Q2_K, Q3_K, Q5_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS,
                                       IQ3_S, IQ4_XS, IQ4_NL, IQ1_S, Q4_K, Q6_K, IQ1_M};
static const uint32_t float_cycle[4] = {Q8_0, F16, BF16, F32};
static int mixed_variant;
static int mixed_counter;

/* the type of the next layer matrix of `rows` rows in the mixed variant */
static uint32_t mixed_type(const char *suffix, int layer)
{
    const int small = strstr(suffix, "ssm_alpha") || strstr(suffix, "ssm_beta") || strstr(suffix, "attn_k.") ||
                      strstr(suffix, "attn_v.");
    /* float-input projections fed by every producer: SwiGLU (ffn_down),
     * attention (attn_output), DeltaNet (ssm_out), the MTP input (eh_proj) */
    const int float_big = (strstr(suffix, "ffn_down") && (layer == 5 || layer == 40)) ||
                          (strstr(suffix, "attn_output") && layer == 7) || (strstr(suffix, "ssm_out") && layer == 9) ||
                          strstr(suffix, "eh_proj");
    if (small || float_big) return float_cycle[(mixed_counter++ + layer) % 4];
    return q8k_cycle[mixed_counter++ % 14];
}

static void add(const char *name, uint64_t width, uint64_t rows, uint32_t type, int kind)
{
    Tensor *t = &tensors[tensor_count];
    memset(t, 0, sizeof(*t));
    t->id = (uint64_t)tensor_count++;
    t->written = 1;
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->n_dims = rows ? 2 : 1;
    t->shape[0] = width;
    t->shape[1] = rows ? rows : 1;
    t->type = type;
    t->kind = kind;
    const uint64_t elements = width * (rows ? rows : 1);
    t->nbytes = elements / block_elements(type) * block_bytes(type);
}

static void add_layer(int layer, uint32_t m)
{
    char name[64];
#define T(suffix, w, r, type, kind) \
    do { \
        snprintf(name, sizeof(name), "blk.%d.%s", layer, suffix); \
        add(name, w, r, mixed_variant && !(kind) ? mixed_type(suffix, layer) : (uint32_t)(type), kind); \
    } while (0)
    T("attn_norm.weight", HIDDEN, 0, F32, 1);
    T("post_attention_norm.weight", HIDDEN, 0, F32, 1);
    T("ffn_gate.weight", HIDDEN, FFN, m, 0);
    T("ffn_up.weight", HIDDEN, FFN, m, 0);
    T("ffn_down.weight", FFN, HIDDEN, m, 0);
    if ((layer + 1) % 4 == 0 || layer == LAYERS) {
        T("attn_q.weight", HIDDEN, 12288, m, 0);
        T("attn_k.weight", HIDDEN, 1024, m, 0);
        T("attn_v.weight", HIDDEN, 1024, m, 0);
        T("attn_output.weight", 6144, HIDDEN, m, 0);
        T("attn_q_norm.weight", 256, 0, F32, 1);
        T("attn_k_norm.weight", 256, 0, F32, 1);
    } else {
        T("attn_qkv.weight", HIDDEN, 10240, m, 0);
        T("attn_gate.weight", HIDDEN, 6144, m, 0);
        T("ssm_alpha.weight", HIDDEN, 48, m, 0);
        T("ssm_beta.weight", HIDDEN, 48, m, 0);
        T("ssm_conv1d.weight", 4, 10240, F32, 2);
        T("ssm_dt.bias", 48, 0, F32, 3);
        T("ssm_a", 48, 0, F32, 4);
        T("ssm_norm.weight", 128, 0, F32, 1);
        T("ssm_out.weight", 6144, HIDDEN, m, 0);
    }
    if (layer == LAYERS) {
        T("nextn.eh_proj.weight", 2 * HIDDEN, HIDDEN, m, 0);
        T("nextn.enorm.weight", HIDDEN, 0, F32, 1);
        T("nextn.hnorm.weight", HIDDEN, 0, F32, 1);
        T("nextn.shared_head_norm.weight", HIDDEN, 0, F32, 1);
    }
#undef T
}

/* ---- block generators ---------------------------------------------------- */

static void fill_words(uint8_t *out, uint64_t bytes, uint64_t seed, uint64_t tid, uint64_t counter)
{
    for (uint64_t i = 0; i < bytes; i += 8) {
        const uint64_t h = hash3(seed, tid, counter + i / 8);
        memcpy(out + i, &h, bytes - i < 8 ? bytes - i : 8);
    }
}

static void q4k_block(uint8_t *b, uint64_t seed, uint64_t tid, uint64_t index, double base)
{
    fill_words(b, 144, seed, tid, index * 32);
    const uint64_t h = hash3(seed, tid, index * 32 + 30);
    const float d = (float)(base * (0.5 + unit(h)));
    const uint16_t dh = f32_to_f16(d), mh = f32_to_f16(8.0f * d);
    memcpy(b, &dh, 2);
    memcpy(b + 2, &mh, 2);
    /* 6-bit scales sc[j] from the random bytes, mins m[j] = round(15 sc / 16) */
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = b[4 + j] & 63;
        mn[j] = (uint8_t)((15 * sc[j] + 8) / 16);
    }
    uint8_t *s = b + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

static void q6k_block(uint8_t *b, uint64_t seed, uint64_t tid, uint64_t index, double base)
{
    fill_words(b, 210, seed, tid, index * 32);
    const uint64_t h = hash3(seed, tid, index * 32 + 30);
    const uint16_t dh = f32_to_f16((float)(base * (0.5 + unit(h))));
    memcpy(b + 208, &dh, 2);
}

static void iq1m_block(uint8_t *b, uint64_t seed, uint64_t tid, uint64_t index, double base)
{
    fill_words(b, 56, seed, tid, index * 8);
    const uint64_t h = hash3(seed, tid, index * 8 + 7);
    const uint16_t dh = f32_to_f16((float)(base * (0.5 + unit(h))));
    for (int i = 0; i < 4; ++i) {
        uint16_t v;
        memcpy(&v, b + 48 + 2 * i, 2);
        v = (uint16_t)((v & 0x0fffu) | (((dh >> (4 * i)) & 15u) << 12));
        memcpy(b + 48 + 2 * i, &v, 2);
    }
}

/* store half h at b + offset */
static void put_half(uint8_t *b, int offset, float value)
{
    const uint16_t h = f32_to_f16(value);
    memcpy(b + offset, &h, 2);
}

/* a block of one of the other formats: random bytes, fp16 scale fields set
 * to base * (0.5 + u) / unit_std */
static void other_block(uint32_t type, uint8_t *b, uint64_t seed, uint64_t tid, uint64_t index, double base)
{
    const uint64_t bytes = block_bytes(type);
    fill_words(b, bytes, seed, tid, index * 32);
    const float d = (float)(base * (0.5 + unit(hash3(seed, tid, index * 32 + 30))));
    switch (type) {
    case Q2_K: {
        /* w = d sc q - dmin m, q in 0..3: m = round(3 sc / 4), dmin = 2d centres it */
        for (int i = 0; i < 16; ++i) {
            const int sc = b[i] & 15;
            b[i] = (uint8_t)(sc | ((3 * sc + 2) / 4) << 4);
        }
        put_half(b, 80, d / 9.8f);
        put_half(b, 82, 2.0f * d / 9.8f);
        break;
    }
    case Q3_K: put_half(b, 108, d / 43.0f); break;
    case Q5_K: {
        /* q in 0..31: m = round(31 sc / 32), dmin = 16 d */
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = b[4 + j] & 63;
            mn[j] = (uint8_t)((31 * sc[j] + 16) / 32);
        }
        uint8_t *s = b + 4;
        for (int j = 0; j < 4; ++j) {
            s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
        }
        put_half(b, 0, d / 336.0f);
        put_half(b, 2, 16.0f * d / 336.0f);
        break;
    }
    case IQ2_XXS: case IQ2_XS: case IQ2_S: put_half(b, 0, d / 67.0f); break;
    case IQ3_XXS: put_half(b, 0, d / 172.0f); break;
    case IQ3_S: put_half(b, 0, d / 170.0f); break;
    case IQ4_XS: put_half(b, 0, d / 1245.0f); break;
    case IQ4_NL: put_half(b, 0, d / 67.0f); break;
    case IQ1_S: put_half(b, 0, d / 7.5f); break;
    case Q8_0: put_half(b, 0, d / 74.0f); break;
    default: break;
    }
}

static float f32_value(const Tensor *t, uint64_t seed, uint64_t tid, uint64_t i)
{
    const double u = unit(hash3(seed, tid, i));
    switch (t->kind) {
    case 1: return (float)(0.9 + 0.2 * u);            /* norm weights */
    case 2: return (float)(1.2 * u - 0.6);            /* conv taps */
    case 3: return (float)(2.0 * u - 1.0);            /* dt bias */
    case 4: return (float)(-(0.05 + 0.95 * u));       /* ssm_a < 0 */
    default: return 0.0f;
    }
}

/* Fill bytes [begin, end) of tensor t (block aligned for quantised types). */
static void generate(const Tensor *t, uint64_t seed, uint64_t tid, uint64_t begin, uint64_t end, uint8_t *out)
{
    if (t->kind == 0 && (t->type == F32 || t->type == F16 || t->type == BF16)) {
        /* dense matrix: uniform weights of standard deviation 1/sqrt(fan_in) */
        const uint64_t size = t->type == F32 ? 4 : 2;
        const double a = sqrt(3.0 / (double)t->shape[0]);
        for (uint64_t i = begin / size; i < end / size; ++i) {
            const float v = (float)(a * (2.0 * unit(hash3(seed, tid, i)) - 1.0));
            uint8_t *dst = out + (i * size - begin);
            if (t->type == F32) {
                memcpy(dst, &v, 4);
            } else if (t->type == F16) {
                const uint16_t h = f32_to_f16(v);
                memcpy(dst, &h, 2);
            } else {
                uint32_t x;
                memcpy(&x, &v, 4);
                const uint16_t h = (uint16_t)(x >> 16);
                memcpy(dst, &h, 2);
            }
        }
        return;
    }
    if (t->type == F32) {
        for (uint64_t i = begin / 4; i < end / 4; ++i) {
            const float v = f32_value(t, seed, tid, i);
            memcpy(out + (i * 4 - begin), &v, 4);
        }
        return;
    }
    const uint64_t bb = block_bytes(t->type);
    const double fan_in = (double)t->shape[0];
    const uint64_t live_end = t->live_rows > 0 ? (uint64_t)t->live_rows * (t->shape[0] / 256) * bb : UINT64_MAX;
    for (uint64_t off = begin; off < end; off += bb) {
        const uint64_t index = t->same_rows ? off / bb % (t->shape[0] / 256) : off / bb;
        uint8_t *b = out + (off - begin);
        if (off >= live_end) {
            memset(b, 0, bb);          /* zero block: d = 0, every weight 0 */
            continue;
        }
        if (t->type == Q4_K) q4k_block(b, seed, tid, index, 1.0 / (168.0 * sqrt(fan_in)));
        else if (t->type == Q6_K) q6k_block(b, seed, tid, index, 1.0 / (1367.0 * sqrt(fan_in)));
        else if (t->type == IQ1_M) iq1m_block(b, seed, tid, index, 1.0 / (7.5 * sqrt(fan_in)));
        else other_block(t->type, b, seed, tid, index, 1.0 / sqrt(fan_in));
    }
}

/* ---- GGUF header ---------------------------------------------------------- */

typedef struct { uint8_t *p; size_t n, cap; } Buf;

static void put(Buf *b, const void *data, size_t n)
{
    if (b->n + n > b->cap) {
        b->cap = (b->n + n) * 2;
        b->p = realloc(b->p, b->cap);
    }
    memcpy(b->p + b->n, data, n);
    b->n += n;
}
static void put_u32(Buf *b, uint32_t v) { put(b, &v, 4); }
static void put_u64(Buf *b, uint64_t v) { put(b, &v, 8); }
static void put_str(Buf *b, const char *s) { put_u64(b, strlen(s)); put(b, s, strlen(s)); }
static void meta_u32(Buf *b, const char *key, uint32_t v) { put_str(b, key); put_u32(b, 4); put_u32(b, v); }
static void meta_str(Buf *b, const char *key, const char *v) { put_str(b, key); put_u32(b, 8); put_str(b, v); }

/* ---- tokenizer metadata ----------------------------------------------------- *
 * A byte-level BPE vocabulary of VOCAB entries that the reference's tokenizer
 * (src/qwen38/qwen38_tokenizer.c:171-205) loads, so the reference CLI and
 * server can run on the synthetic model: ids 0..255 are the 256 byte symbols
 * of the GPT-2 byte map (every byte string encodes), ids 256..260 the results
 * of the five merges below, the chat-template tokens at SPECIAL0.. (control
 * tokens, type 3, and the think tags, type 4), every other id "w<id>".  The
 * end-of-sequence token is <|im_end|>. */
enum { SPECIAL0 = 248310, EOS_ID = SPECIAL0 + 2 };
static const char *const kMerges[5][2] = {{"h", "e"}, {"l", "l"}, {"\xc4\xa0", "t"}, {"t", "h"}, {"i", "n"}};
static const char *const kSpecials[5] = {"<|endoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "</think>"};

/* UTF-8 of the byte map's code point for byte b (33..126, 161..172 and
 * 174..255 map to themselves, the rest to 256, 257, ... in byte order) */
static int byte_symbol(int b, char *out)
{
    int cp = b, extra = 0;
    const int direct = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
    if (!direct) {
        for (int c = 0; c < b; ++c)
            if (!((c >= 33 && c <= 126) || (c >= 161 && c <= 172) || (c >= 174 && c <= 255))) ++extra;
        cp = 256 + extra;
    }
    if (cp < 0x80) {
        out[0] = (char)cp;
        out[1] = 0;
        return 1;
    }
    out[0] = (char)(0xc0 | (cp >> 6));
    out[1] = (char)(0x80 | (cp & 0x3f));
    out[2] = 0;
    return 2;
}

static void put_tokenizer(Buf *h)
{
    char text[32];
    meta_str(h, "tokenizer.ggml.model", "gpt2");
    meta_str(h, "tokenizer.ggml.pre", "qwen2");
    put_str(h, "tokenizer.ggml.tokens");
    put_u32(h, 9);
    put_u32(h, 8);
    put_u64(h, VOCAB);
    for (int id = 0; id < VOCAB; ++id) {
        if (id < 256) {
            byte_symbol(id, text);
        } else if (id < 261) {
            snprintf(text, sizeof(text), "%s%s", kMerges[id - 256][0], kMerges[id - 256][1]);
        } else if (id >= SPECIAL0 && id < SPECIAL0 + 5) {
            snprintf(text, sizeof(text), "%s", kSpecials[id - SPECIAL0]);
        } else {
            snprintf(text, sizeof(text), "w%d", id);
        }
        put_str(h, text);
    }
    put_str(h, "tokenizer.ggml.token_type");
    put_u32(h, 9);
    put_u32(h, 5);
    put_u64(h, VOCAB);
    for (int id = 0; id < VOCAB; ++id) {
        const int32_t type = id >= SPECIAL0 && id < SPECIAL0 + 3 ? 3 : id >= SPECIAL0 + 3 && id < SPECIAL0 + 5 ? 4 : 1;
        put(h, &type, 4);
    }
    put_str(h, "tokenizer.ggml.merges");
    put_u32(h, 9);
    put_u32(h, 8);
    put_u64(h, 5);
    for (int i = 0; i < 5; ++i) {
        snprintf(text, sizeof(text), "%s %s", kMerges[i][0], kMerges[i][1]);
        put_str(h, text);
    }
    meta_u32(h, "tokenizer.ggml.eos_token_id", EOS_ID);
}

int main(int argc, char **argv)
{
    const char *variant = argc == 4 ? argv[3] : "";
    const int accept = strcmp(variant, "accept") == 0, accept_mtp = strcmp(variant, "accept_mtp") == 0;
    const int accept_all = strcmp(variant, "accept_all") == 0;
    mixed_variant = strcmp(variant, "mixed") == 0;
    if (argc != 4 || (strcmp(variant, "q4km") && strcmp(variant, "iq1m") && !accept && !accept_mtp && !accept_all &&
                      !mixed_variant)) {
        fprintf(stderr, "usage: %s OUT.gguf SEED q4km|iq1m|accept|accept_mtp|accept_all|mixed\n", argv[0]);
        return 2;
    }
    const uint64_t seed = strtoull(argv[2], NULL, 0);
    const uint32_t m = strcmp(variant, "iq1m") == 0 ? IQ1_M : Q4_K;

    add("token_embd.weight", HIDDEN, VOCAB, mixed_variant ? Q8_0 : Q4_K, 0);
    add("output_norm.weight", HIDDEN, 0, F32, 1);
    add("output.weight", HIDDEN, VOCAB, mixed_variant ? Q5_K : Q6_K, 0);
    const int first_mtp_tensor = tensor_count;
    for (int layer = 0; layer <= LAYERS; ++layer) add_layer(layer, m);
    int mtp_begin = first_mtp_tensor;
    while (mtp_begin < tensor_count && strncmp(tensors[mtp_begin].name, "blk.64.", 7) != 0) ++mtp_begin;
    if (accept_all) tensors[2].same_rows = 1;
    if (accept || accept_mtp) {
        tensors[2].live_rows = 2;
        for (int i = 0; i < tensor_count; ++i) {
            const int mtp_part = i == 0 || i == 2 || i >= mtp_begin;
            tensors[i].written = accept ? i < mtp_begin : mtp_part;
        }
    }
    /* the written tensors, in list order */
    int kept = 0;
    for (int i = 0; i < tensor_count; ++i)
        if (tensors[i].written) tensors[kept++] = tensors[i];
    tensor_count = kept;
    const uint32_t block_count = accept ? LAYERS : LAYERS + 1;

    uint64_t offset = 0;
    for (int i = 0; i < tensor_count; ++i) {
        tensors[i].offset = offset;
        offset = (offset + tensors[i].nbytes + 31) & ~31ull;
    }
    const uint64_t data_bytes = offset;

    Buf h = {0};
    put_u32(&h, 0x46554747u);
    put_u32(&h, 3);
    put_u64(&h, (uint64_t)tensor_count);
    put_u64(&h, 14 + 6);
    put_str(&h, "general.architecture"); put_u32(&h, 8); put_str(&h, "qwen35");
    meta_u32(&h, "general.alignment", 32);
    meta_u32(&h, "qwen35.block_count", block_count);
    meta_u32(&h, "qwen35.nextn_predict_layers", block_count == LAYERS + 1 ? 1 : 0);
    meta_u32(&h, "qwen35.embedding_length", HIDDEN);
    meta_u32(&h, "qwen35.feed_forward_length", FFN);
    meta_u32(&h, "qwen35.attention.head_count", 24);
    meta_u32(&h, "qwen35.attention.head_count_kv", 4);
    meta_u32(&h, "qwen35.full_attention_interval", 4);
    meta_u32(&h, "qwen35.ssm.state_size", 128);
    meta_u32(&h, "qwen35.ssm.group_count", 16);
    meta_u32(&h, "qwen35.ssm.time_step_rank", 48);
    meta_u32(&h, "qwen35.ssm.inner_size", 6144);
    meta_u32(&h, "general.file_type", m == Q4_K ? 15u : 31u);
    put_tokenizer(&h);
    for (int i = 0; i < tensor_count; ++i) {
        const Tensor *t = &tensors[i];
        put_str(&h, t->name);
        put_u32(&h, t->n_dims);
        for (uint32_t d = 0; d < t->n_dims; ++d) put_u64(&h, t->shape[d]);
        put_u32(&h, t->type);
        put_u64(&h, t->offset);
    }
    const uint64_t data_start = (h.n + 31) & ~31ull;
    while (h.n < data_start) put(&h, "", 1);
    if (strcmp(argv[1], "-") == 0) {
        /* size only: the file this seed and variant would produce */
        printf("%llu\n", (unsigned long long)(data_start + data_bytes));
        return 0;
    }

    const int fd = open(argv[1], O_CREAT | O_TRUNC | O_WRONLY, 0644);
    if (fd < 0) { perror(argv[1]); return 1; }
    if (ftruncate(fd, (off_t)(data_start + data_bytes)) != 0) { perror("ftruncate"); return 1; }
    if (pwrite(fd, h.p, h.n, 0) != (ssize_t)h.n) { perror("pwrite"); return 1; }

    /* work items: 4 MiB slices of every tensor, block aligned */
    const uint64_t slice = 4u << 20;
    int failed = 0;
    uint64_t written = 0, next_report = data_bytes / 10;
    for (int i = 0; i < tensor_count; ++i) {
        const Tensor *t = &tensors[i];
        const uint64_t unit_bytes = block_bytes(t->type);
        const uint64_t step = slice / unit_bytes * unit_bytes;
        const int64_t slices = (int64_t)((t->nbytes + step - 1) / step);
#pragma omp parallel for schedule(dynamic, 1) reduction(| : failed)
        for (int64_t s = 0; s < slices; ++s) {
            const uint64_t begin = (uint64_t)s * step;
            const uint64_t end = begin + step < t->nbytes ? begin + step : t->nbytes;
            uint8_t *buffer = malloc(end - begin);
            generate(t, seed, t->id, begin, end, buffer);
            if (pwrite(fd, buffer, end - begin, (off_t)(data_start + t->offset + begin)) != (ssize_t)(end - begin))
                failed |= 1;
            free(buffer);
        }
        written += t->nbytes;
        if (written >= next_report) {
            printf("  %3d%% (%d/%d tensors)\n", (int)(100 * written / data_bytes), i + 1, tensor_count);
            fflush(stdout);
            next_report += data_bytes / 10;
        }
    }
    if (close(fd) != 0 || failed) { fprintf(stderr, "write failed\n"); return 1; }
    printf("wrote %s: %d tensors, %llu bytes\n", argv[1], tensor_count,
           (unsigned long long)(data_start + data_bytes));
    return 0;
}
