/* Qwen3.8-27B decode engine on one MI355X: GGUF reader, HBM-resident weights
 * and state, and the model ABI of include/q38model.h.
 *
 * The control flow restates src/qwen38/qwen38_model.c (forward_token
 * :1494-1517, prefill :1519-1560, MTP :1562-1612, speculative greedy
 * :1614-1714, batch evaluation :1121-1294); every arithmetic step runs in the
 * HIP kernels of q38_gemm.hip, q38_misc.hip and q38_model.hip on the model's
 * stream.  Rows of a batch are independent in every GEMM, and the recurrent /
 * KV-cache cores run row by row in token order, so a batch of M rows gives
 * the same bits as M single-token steps (the reference's own invariant).
 */
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <initializer_list>
#include <string>
#include <map>
#include <unordered_map>
#include <vector>

#include "q38_kernels.h"
#include "q38model.h"

namespace q38 {
const void *iq1m_grid_for_current_device();
}

namespace {

constexpr uint32_t kHidden = 5120, kFFN = 17408, kLayers = 64, kTotalLayers = 65;
constexpr uint32_t kRecurrent = 48, kFullLayers = 17;
constexpr uint32_t kQKV = 10240, kLinV = 6144, kVHeads = 48, kHeadDim = 128;
constexpr uint32_t kQGDim = 12288, kQDim = 6144, kKVDim = 1024, kAttnHeads = 24;
constexpr uint32_t kVocab = 248320;
constexpr uint32_t kBatch = 8;           /* rows per batched decode step (verify, catch-up) */
/* rows of one prefill batch: the prompt runs through all blocks in batches
 * of up to this many tokens (fewer at long contexts, where the attention
 * scores of a batch take rows x 24 x context floats).  Larger batches give
 * the 5120-row projections more workgroups and read each layer's weights
 * fewer times (IQ1_M 4096-token prompt on MI355X: 512-token batches 0.662 s,
 * 2048 0.566 s, one batch 0.547 s) */
constexpr uint32_t kPrefillRows = 4096;
constexpr size_t kPrefillScoresBytes = (size_t)4 << 30;
constexpr uint32_t kQ8KBytes = 292;

/* device parameter blocks of kParamWords words: [0] position of row 0 of
 * the step, [1 + r] current state slot of recurrent layer r */
constexpr uint32_t kParamWords = 64;
/* word of the verify parameter block holding the stop token */
constexpr uint32_t kParamStopWord = kParamWords - 1;
enum : uint32_t { kParamTarget = 0, kParamCatchup = 1, kParamDraft0 = 2, kParamSets = 2 + kBatch };

enum : uint32_t { F32 = 0, Q4_K = 12, Q6_K = 14, IQ1_M = 29 };

bool report(const char *what)
{
    fprintf(stderr, "qwen38: %s\n", what);
    return false;
}

bool hip_ok(hipError_t e, const char *what)
{
    if (e == hipSuccess) return true;
    fprintf(stderr, "qwen38: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

/* ---- GGUF reader (format v2/v3) ------------------------------------------ */

/* elements and bytes per block of the GGML types (the GGUF format's own
 * constants; src/io/qwen38_gguf.c:129-185 lists the same) */
/* every kernel launch of a step is checked once, at the step's end; an
 * error left by the caller's own HIP work before the call is not ours */
bool launches_ok() { return hip_ok(hipGetLastError(), "kernel launch"); }
void begin_call() { (void)hipGetLastError(); }

void ggml_block(uint32_t type, uint32_t *elements, uint32_t *bytes)
{
    uint32_t e = 0, b = 0;
    switch (type) {
    case 0: e = 1; b = 4; break;                    /* F32 */
    case 1: case 30: e = 1; b = 2; break;           /* F16, BF16 */
    case 2: e = 32; b = 18; break;                  /* Q4_0 */
    case 3: e = 32; b = 20; break;                  /* Q4_1 */
    case 6: e = 32; b = 22; break;                  /* Q5_0 */
    case 7: e = 32; b = 24; break;                  /* Q5_1 */
    case 8: e = 32; b = 34; break;                  /* Q8_0 */
    case 20: e = 32; b = 18; break;                 /* IQ4_NL */
    case 10: e = 256; b = 84; break;                /* Q2_K */
    case 11: e = 256; b = 110; break;               /* Q3_K */
    case 12: e = 256; b = 144; break;               /* Q4_K */
    case 13: e = 256; b = 176; break;               /* Q5_K */
    case 14: e = 256; b = 210; break;               /* Q6_K */
    case 16: e = 256; b = 66; break;                /* IQ2_XXS */
    case 17: e = 256; b = 74; break;                /* IQ2_XS */
    case 18: e = 256; b = 98; break;                /* IQ3_XXS */
    case 19: e = 256; b = 50; break;                /* IQ1_S */
    case 21: e = 256; b = 110; break;               /* IQ3_S */
    case 22: e = 256; b = 82; break;                /* IQ2_S */
    case 23: e = 256; b = 136; break;               /* IQ4_XS */
    case 29: e = 256; b = 56; break;                /* IQ1_M */
    default: break;
    }
    *elements = e;
    *bytes = b;
}

struct TensorInfo {
    uint32_t n_dims = 0;
    uint64_t shape[8] = {0};
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t nbytes = 0;
    uint64_t device_offset = 0;   /* placement in the HBM copy (plan_layout) */
};

struct MetaValue {
    uint32_t type = 0;
    uint32_t u32 = 0;
    std::string str;
};

struct GGUFFile {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint64_t data_offset = 0;
    uint64_t data_bytes = 0;
    uint64_t device_bytes = 0;   /* size of the HBM copy (plan_layout) */
    std::unordered_map<std::string, TensorInfo> tensors;
    std::unordered_map<std::string, MetaValue> meta;

    ~GGUFFile() { close(); }
    void close()
    {
        if (map) munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0) ::close(fd);
        map = nullptr;
        fd = -1;
    }

    struct Reader {
        const uint8_t *p, *end;
        bool failed = false;
        bool take(uint64_t n, const uint8_t **out)
        {
            if (failed || (uint64_t)(end - p) < n) return !(failed = true);
            *out = p;
            p += n;
            return true;
        }
        uint32_t u32()
        {
            const uint8_t *q;
            uint32_t v = 0;
            if (take(4, &q)) memcpy(&v, q, 4);
            return v;
        }
        uint64_t u64()
        {
            const uint8_t *q;
            uint64_t v = 0;
            if (take(8, &q)) memcpy(&v, q, 8);
            return v;
        }
        bool str(std::string *s)
        {
            const uint64_t n = u64();
            const uint8_t *q;
            if (!take(n, &q)) return false;
            if (s) s->assign(reinterpret_cast<const char *>(q), n);
            return true;
        }
        bool skip_value(uint32_t type, uint64_t count)
        {
            static const uint8_t sizes[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
            if (type > 12 || type == 9) return !(failed = true);
            if (type == 8) {
                for (uint64_t i = 0; i < count; ++i)
                    if (!str(nullptr)) return false;
                return true;
            }
            const uint8_t *q;
            if (count > UINT64_MAX / sizes[type]) return !(failed = true);
            return take(count * sizes[type], &q);
        }
    };

    bool open(const char *path)
    {
        fd = ::open(path, O_RDONLY);
        if (fd < 0) {
            perror(path);
            return false;
        }
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size < 24) return report("invalid GGUF file size");
        size = (uint64_t)st.st_size;
        void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) return report("mmap of the GGUF file failed");
        map = static_cast<const uint8_t *>(m);
        Reader r{map, map + size};
        const uint32_t magic = r.u32();
        const uint32_t version = r.u32();
        const uint64_t n_tensors = r.u64();
        const uint64_t n_meta = r.u64();
        if (magic != 0x46554747u || version < 2 || version > 3 || n_tensors == 0)
            return report("unsupported or corrupt GGUF header");
        for (uint64_t i = 0; i < n_meta; ++i) {
            std::string key;
            MetaValue v;
            if (!r.str(&key)) return report("malformed GGUF metadata");
            v.type = r.u32();
            if (r.failed || v.type > 12) return report("malformed GGUF metadata");
            if (v.type == 8) {
                if (!r.str(&v.str)) return report("malformed GGUF metadata");
            } else if (v.type == 9) {
                const uint32_t at = r.u32();
                const uint64_t count = r.u64();
                if (at == 9 || !r.skip_value(at, count)) return report("malformed GGUF metadata");
            } else if (v.type == 4) {
                v.u32 = r.u32();
            } else if (!r.skip_value(v.type, 1)) {
                return report("malformed GGUF metadata");
            }
            meta[key] = v;
        }
        for (uint64_t i = 0; i < n_tensors; ++i) {
            std::string name;
            TensorInfo t;
            if (!r.str(&name)) return report("malformed GGUF tensor table");
            t.n_dims = r.u32();
            if (r.failed || t.n_dims == 0 || t.n_dims > 8) return report("malformed GGUF tensor table");
            uint64_t elements = 1;
            for (uint32_t d = 0; d < t.n_dims; ++d) {
                t.shape[d] = r.u64();
                if (!t.shape[d] || elements > UINT64_MAX / t.shape[d]) return report("malformed GGUF tensor table");
                elements *= t.shape[d];
            }
            t.type = r.u32();
            t.offset = r.u64();
            uint32_t be, bb;
            ggml_block(t.type, &be, &bb);
            if (r.failed || !be || t.shape[0] % be || elements % be || elements / be > UINT64_MAX / bb)
                return report("malformed GGUF tensor table");
            t.nbytes = elements / be * bb;
            tensors[name] = t;
        }
        uint64_t alignment = 32;
        auto a = meta.find("general.alignment");
        if (a != meta.end() && a->second.type == 4) {
            alignment = a->second.u32;
            if (!alignment || (alignment & (alignment - 1))) return report("invalid GGUF alignment");
        }
        const uint64_t end = (uint64_t)(r.p - map);
        data_offset = (end + alignment - 1) & ~(alignment - 1);
        if (data_offset > size) return report("GGUF tensor data begins past end of file");
        data_bytes = size - data_offset;
        for (auto &kv : tensors) {
            const TensorInfo &t = kv.second;
            if (t.offset > data_bytes || t.nbytes > data_bytes - t.offset)
                return report(("tensor outside GGUF file: " + kv.first).c_str());
        }
        return true;
    }

    bool u32_is(const char *key, uint32_t want) const
    {
        auto it = meta.find(key);
        return it != meta.end() && it->second.type == 4 && it->second.u32 == want;
    }
    bool get_u32(const char *key, uint32_t *out) const
    {
        auto it = meta.find(key);
        if (it == meta.end() || it->second.type != 4) return false;
        *out = it->second.u32;
        return true;
    }
    bool str_is(const char *key, const char *want) const
    {
        auto it = meta.find(key);
        return it != meta.end() && it->second.type == 8 && it->second.str == want;
    }
};

/* ---- device-resident model ------------------------------------------------ */

struct DevTensor {
    uint32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t width = 0, rows = 0;
    const uint8_t *data = nullptr;
    /* Q4_K matrices: 16-row tiled copy used for 2..8-token GEMMs (may be
     * null); for a group member, its rows inside its run's tiled copy */
    const uint8_t *tiled = nullptr;
    const float *f32() const { return reinterpret_cast<const float *>(data); }
};

/* Projections of one input whose output rows are concatenated: row t of
 * the result holds member i at columns first[i] .. first[i] + rows - 1, and
 * rows are `width` floats apart.  Runs of members that sit back to back in
 * HBM with one type and row width are computed by one GEMM. */
struct Group {
    DevTensor part[4];
    uint32_t first[4] = {0};
    int n = 0;
    uint32_t width = 0;
};

struct Layer {
    bool full = false;
    DevTensor attn_norm, post_norm, ffn_gate, ffn_up, ffn_down;
    DevTensor qkv, z, alpha, beta, conv, dt, a, ssm_norm, ssm_out;   /* DeltaNet */
    DevTensor q, k, v, out, q_norm, k_norm;                          /* full attention */
    Group ffn_in;   /* gate | up */
    Group mix_in;   /* DeltaNet: qkv | z | beta | alpha; full attention: q+gate | k | v */
};

void make_group(Group *g, std::initializer_list<const DevTensor *> parts)
{
    g->n = 0;
    g->width = 0;
    for (const DevTensor *t : parts) {
        g->part[g->n] = *t;
        g->first[g->n++] = g->width;
        g->width += (uint32_t)t->rows;
    }
}

/* q38_matrix_type_supported (qwen38_model.c:172-189): the Q8_K-path formats
 * and F32, F16, BF16, Q8_0 */
bool matrix_type_ok(uint32_t t) { return q38::format_takes_q8k((int)t) || t == 0 || t == 1 || t == 8 || t == 30; }

/* projections of these types take the fp32 input (q38_project,
 * qwen38_model.c:598-605) */
bool float_input(const DevTensor &t) { return !q38::format_takes_q8k((int)t.type); }

}  // namespace

struct Q38Model {
    GGUFFile gguf, mtp_gguf;
    void *weights = nullptr, *mtp_weights = nullptr;
    void *tiled_weights = nullptr, *tiled_mtp = nullptr;   /* tiled copies (target layers, MTP block) */
    DevTensor embedding, output_norm, output, mtp_embedding, mtp_output;
    DevTensor eh_proj, enorm, hnorm, shared_head_norm;
    Layer layers[kTotalLayers];
    uint32_t context_length = 0, position = 0, mtp_position = 0;
    bool mtp_weights_loaded = false, mtp_enabled = false;
    uint32_t ck_position = 0, ck_mtp_position = 0;

    hipStream_t stream = nullptr;
    /* second stream (default priority) for the logits download, which then
     * overlaps the MTP catch-up on `stream` */
    hipStream_t copy_stream = nullptr;
    hipEvent_t logits_ready = nullptr;
    const void *grid = nullptr;
    /* state */
    /* recurrent state: kRecurrentStateSlots slots of [48 layers][...]; layer r's
     * current slot is slot_host[r] (mirrored in params[1 + r]) */
    float *conv_state = nullptr, *delta_state = nullptr, *key_cache = nullptr, *value_cache = nullptr;
    float *mtp_hidden = nullptr, *ck_mtp_hidden = nullptr;
    uint32_t slot_host[kRecurrent] = {0}, ck_slot[kRecurrent] = {0};
    float *rope = nullptr;
    /* scratch of scratch_rows rows (the larger of kBatch and the prefill batch) */
    uint32_t prefill_rows = kBatch, scratch_rows = kBatch;
    /* wide0 holds a group's concatenated outputs: up to 2 * kFFN floats per row */
    float *hidden = nullptr, *norm = nullptr, *branch = nullptr, *wide0 = nullptr;
    float *qbuf = nullptr, *attn = nullptr;
    float *scores = nullptr, *logits = nullptr, *target_norm = nullptr;
    float *prep = nullptr;   /* prepared DeltaNet inputs of a prefill batch */
    /* fp32 inputs of the projections whose matrices take them (F32, F16,
     * BF16, Q8_0): scratch_rows rows of up to kFFN floats, allocated only
     * when the checkpoint has such a matrix */
    float *fin = nullptr;
    bool float_inputs = false;
    /* output-norm rows of a verify longer than kBatch rows (grown on demand) */
    float *long_norm = nullptr;
    uint32_t long_norm_rows = 0;
    uint8_t *q8k = nullptr;
    /* params[0] = position of row 0 of the current step, params[1 + r] = slot of recurrent layer r */
    uint32_t *tokens = nullptr, *params = nullptr, *targets = nullptr, *drafts = nullptr, *accept = nullptr;
    /* one allocation: drafts [0, 16), targets [16, 32), accept [32, 48),
     * sampled token [48] */
    uint32_t *words = nullptr, *sampled = nullptr;
    float *argmax_pv = nullptr;
    /* the logits row a speculative call returns, gathered on the device */
    float *logits_stage = nullptr;
    uint32_t *argmax_pi = nullptr;
    /* device sampling: the row of the logits the last call returned (valid
     * until the next call), a device copy of the sampler's presence bytes
     * and the sampler's candidate lists */
    const float *last_logits = nullptr;
    uint8_t *presence = nullptr, *sample_scratch = nullptr;
    /* host side */
    float *host_logits = nullptr;
    uint32_t *host_words = nullptr;
    uint32_t *host_params = nullptr;   /* pinned staging of the device parameter blocks */
    uint32_t *host_sampled = nullptr;  /* pinned word of a sampled token */
    float query_scale = 0.0f;
    bool pending_branch = false;   /* m->branch holds an FFN output not yet added to m->hidden */
    /* instantiated HIP graphs of the step sequences, by key; `seen` marks
     * keys that already ran once without capture */
    std::map<uint64_t, hipGraphExec_t> graphs;
    std::map<uint64_t, bool> seen;
    bool graphs_enabled = true;
};

namespace {

bool bind_tensor(const GGUFFile &f, const uint8_t *base, const std::string &name, DevTensor *out)
{
    auto it = f.tensors.find(name);
    if (it == f.tensors.end()) {
        fprintf(stderr, "qwen38: missing tensor %s\n", name.c_str());
        return false;
    }
    const TensorInfo &t = it->second;
    out->type = t.type;
    out->n_dims = t.n_dims;
    out->width = t.shape[0];
    out->rows = t.n_dims > 1 ? t.shape[1] : 0;
    out->data = base + t.device_offset;
    return true;
}

/* q38_expect_tensor (qwen38_model.c:190-207) */
bool expect(const DevTensor &t, const std::string &name, uint64_t width, uint64_t rows, bool f32_only)
{
    const uint32_t dims = rows ? 2u : 1u;
    const bool shape_ok = t.n_dims == dims && t.width == width && (!rows || t.rows == rows);
    const bool type_ok = f32_only ? t.type == F32 : matrix_type_ok(t.type);
    if (shape_ok && type_ok) return true;
    fprintf(stderr, "qwen38: incompatible tensor %s; expected %s[%llu", name.c_str(), f32_only ? "F32 " : "",
            (unsigned long long)width);
    if (rows) fprintf(stderr, ",%llu", (unsigned long long)rows);
    fprintf(stderr, "]%s\n", f32_only ? "" : " of a supported matrix type");
    return false;
}

bool bind_layer(Layer *L, const GGUFFile &f, const uint8_t *base, int layer)
{
    const std::string p = "blk." + std::to_string(layer) + ".";
    L->full = (layer + 1) % 4 == 0 || layer == (int)kLayers;
    int ok = bind_tensor(f, base, p + "attn_norm.weight", &L->attn_norm) &&
              bind_tensor(f, base, p + "post_attention_norm.weight", &L->post_norm) &&
              bind_tensor(f, base, p + "ffn_gate.weight", &L->ffn_gate) && bind_tensor(f, base, p + "ffn_up.weight", &L->ffn_up) &&
              bind_tensor(f, base, p + "ffn_down.weight", &L->ffn_down);
    if (!ok) return false;
    ok = (int)expect(L->attn_norm, p + "attn_norm.weight", kHidden, 0, true) &
         (int)expect(L->post_norm, p + "post_attention_norm.weight", kHidden, 0, true) &
         (int)expect(L->ffn_gate, p + "ffn_gate.weight", kHidden, kFFN, false) &
         (int)expect(L->ffn_up, p + "ffn_up.weight", kHidden, kFFN, false) &
         (int)expect(L->ffn_down, p + "ffn_down.weight", kFFN, kHidden, false);
    if (L->full) {
        if (!(bind_tensor(f, base, p + "attn_q.weight", &L->q) && bind_tensor(f, base, p + "attn_k.weight", &L->k) &&
              bind_tensor(f, base, p + "attn_v.weight", &L->v) && bind_tensor(f, base, p + "attn_output.weight", &L->out) &&
              bind_tensor(f, base, p + "attn_q_norm.weight", &L->q_norm) &&
              bind_tensor(f, base, p + "attn_k_norm.weight", &L->k_norm)))
            return false;
        ok &= (int)expect(L->q, p + "attn_q.weight", kHidden, kQGDim, false) &
              (int)expect(L->k, p + "attn_k.weight", kHidden, kKVDim, false) &
              (int)expect(L->v, p + "attn_v.weight", kHidden, kKVDim, false) &
              (int)expect(L->out, p + "attn_output.weight", kQDim, kHidden, false) &
              (int)expect(L->q_norm, p + "attn_q_norm.weight", 256, 0, true) &
              (int)expect(L->k_norm, p + "attn_k_norm.weight", 256, 0, true);
    } else {
        if (!(bind_tensor(f, base, p + "attn_qkv.weight", &L->qkv) && bind_tensor(f, base, p + "attn_gate.weight", &L->z) &&
              bind_tensor(f, base, p + "ssm_alpha.weight", &L->alpha) && bind_tensor(f, base, p + "ssm_beta.weight", &L->beta) &&
              bind_tensor(f, base, p + "ssm_conv1d.weight", &L->conv) && bind_tensor(f, base, p + "ssm_dt.bias", &L->dt) &&
              bind_tensor(f, base, p + "ssm_a", &L->a) && bind_tensor(f, base, p + "ssm_norm.weight", &L->ssm_norm) &&
              bind_tensor(f, base, p + "ssm_out.weight", &L->ssm_out)))
            return false;
        ok &= (int)expect(L->qkv, p + "attn_qkv.weight", kHidden, kQKV, false) &
              (int)expect(L->z, p + "attn_gate.weight", kHidden, kLinV, false) &
              (int)expect(L->alpha, p + "ssm_alpha.weight", kHidden, kVHeads, false) &
              (int)expect(L->beta, p + "ssm_beta.weight", kHidden, kVHeads, false) &
              (int)expect(L->conv, p + "ssm_conv1d.weight", 4, kQKV, true) &
              (int)expect(L->dt, p + "ssm_dt.bias", kVHeads, 0, true) & (int)expect(L->a, p + "ssm_a", kVHeads, 0, true) &
              (int)expect(L->ssm_norm, p + "ssm_norm.weight", kHeadDim, 0, true) &
              (int)expect(L->ssm_out, p + "ssm_out.weight", kLinV, kHidden, false);
    }
    make_group(&L->ffn_in, {&L->ffn_gate, &L->ffn_up});
    if (L->full) make_group(&L->mix_in, {&L->q, &L->k, &L->v});
    else make_group(&L->mix_in, {&L->qkv, &L->z, &L->beta, &L->alpha});
    return ok;
}

/* Projections that read the same input.  Their tensors are placed back to
 * back in HBM, so members of one type and width form a single matrix whose
 * output rows are the members' rows in this order. */
const char *const kFusionGroups[][4] = {
    {"ffn_gate.weight", "ffn_up.weight", nullptr, nullptr},
    {"attn_qkv.weight", "attn_gate.weight", "ssm_beta.weight", "ssm_alpha.weight"},
    {"attn_q.weight", "attn_k.weight", "attn_v.weight", nullptr},
};

uint64_t align256(uint64_t v) { return (v + 255) & ~(uint64_t)255; }

/* Device placement of every tensor: the fusion groups of each block first
 * (a member directly after the previous one when both have the same type and
 * row width, else 256-byte aligned), then all other tensors 256-byte aligned
 * in file order. */
void plan_layout(GGUFFile &f)
{
    uint64_t at = 0;
    std::map<std::string, bool> placed;
    for (uint32_t layer = 0; layer < kTotalLayers; ++layer) {
        const std::string p = "blk." + std::to_string(layer) + ".";
        for (const auto &group : kFusionGroups) {
            const TensorInfo *prev = nullptr;
            for (const char *member : group) {
                if (!member) break;
                auto it = f.tensors.find(p + member);
                if (it == f.tensors.end()) continue;
                TensorInfo &t = it->second;
                if (!prev || prev->type != t.type || prev->shape[0] != t.shape[0]) at = align256(at);
                t.device_offset = at;
                at += t.nbytes;
                placed[it->first] = true;
                prev = &t;
            }
        }
    }
    std::vector<std::pair<uint64_t, TensorInfo *>> rest;
    for (auto &kv : f.tensors)
        if (!placed.count(kv.first)) rest.emplace_back(kv.second.offset, &kv.second);
    std::sort(rest.begin(), rest.end(),
              [](const std::pair<uint64_t, TensorInfo *> &a, const std::pair<uint64_t, TensorInfo *> &b) {
                  return a.first < b.first;
              });
    for (auto &r : rest) {
        at = align256(at);
        r.second->device_offset = at;
        at += r.second->nbytes;
    }
    f.device_bytes = at;
}

/* Read the tensor-data region of a GGUF file sequentially through two pinned
 * staging buffers and copy each tensor's bytes to its planned place in one
 * HBM allocation. */
bool upload(GGUFFile &f, void **device)
{
    plan_layout(f);
    if (!hip_ok(hipMalloc(device, f.device_bytes ? f.device_bytes : 1), "weight allocation")) return false;
    std::vector<const TensorInfo *> order;
    for (const auto &kv : f.tensors) order.push_back(&kv.second);
    std::sort(order.begin(), order.end(),
              [](const TensorInfo *a, const TensorInfo *b) { return a->offset < b->offset; });
    const size_t chunk = 256u << 20;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t s = nullptr;
    bool ok = hip_ok(hipHostMalloc(&stage[0], chunk), "pinned staging") &&
              hip_ok(hipHostMalloc(&stage[1], chunk), "pinned staging") &&
              hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "upload stream") &&
              hip_ok(hipEventCreate(&done[0]), "event") && hip_ok(hipEventCreate(&done[1]), "event");
    size_t first = 0;   /* first tensor that may overlap the current chunk */
    uint64_t off = 0;
    for (int i = 0; ok && off < f.data_bytes; ++i, off += chunk) {
        const size_t n = (size_t)std::min<uint64_t>(chunk, f.data_bytes - off);
        const int b = i & 1;
        ok = hip_ok(hipEventSynchronize(done[b]), "upload wait");
        uint64_t got = 0;
        while (ok && got < n) {
            const ssize_t r = pread(f.fd, static_cast<uint8_t *>(stage[b]) + got, n - got,
                                    (off_t)(f.data_offset + off + got));
            if (r <= 0) ok = report("reading GGUF tensor data failed");
            else got += (uint64_t)r;
        }
        while (first < order.size() && order[first]->offset + order[first]->nbytes <= off) ++first;
        for (size_t k = first; ok && k < order.size() && order[k]->offset < off + n; ++k) {
            const TensorInfo &t = *order[k];
            const uint64_t lo = std::max<uint64_t>(t.offset, off), hi = std::min<uint64_t>(t.offset + t.nbytes, off + n);
            if (lo >= hi) continue;
            ok = hip_ok(hipMemcpyAsync(static_cast<uint8_t *>(*device) + t.device_offset + (lo - t.offset),
                                       static_cast<uint8_t *>(stage[b]) + (lo - off), hi - lo,
                                       hipMemcpyHostToDevice, s),
                        "weight upload");
        }
        ok = ok && hip_ok(hipEventRecord(done[b], s), "event");
    }
    if (s) ok = hip_ok(hipStreamSynchronize(s), "upload") && ok;
    for (int b = 0; b < 2; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (stage[b]) (void)hipHostFree(stage[b]);
    }
    if (s) (void)hipStreamDestroy(s);
    return ok;
}

template <typename T>
bool dalloc(T **p, size_t count)
{
    return hip_ok(hipMalloc(reinterpret_cast<void **>(p), count * sizeof(T) + 256), "device allocation");
}

template <typename T>
void dfree(T *&p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

size_t conv_count() { return (size_t)kRecurrent * kQKV * 3; }
size_t delta_count() { return (size_t)kRecurrent * kVHeads * kHeadDim * kHeadDim; }
size_t kv_count(uint32_t ctx) { return (size_t)kFullLayers * ctx * kKVDim; }
/* the value cache is channel-major per layer: [1024][value_pitch(ctx)] */
size_t value_layer_floats(uint32_t ctx) { return (size_t)kKVDim * q38::value_pitch(ctx); }

bool validate_base(Q38Model *m)
{
    const GGUFFile &f = m->gguf;
    uint32_t blocks = 0, nextn = 0;
    const bool ok = f.get_u32("qwen35.block_count", &blocks) && f.get_u32("qwen35.nextn_predict_layers", &nextn) &&
                    ((blocks == kLayers && nextn == 0) || (blocks == kTotalLayers && nextn == 1)) &&
                    f.str_is("general.architecture", "qwen35") && f.u32_is("qwen35.embedding_length", kHidden) &&
                    f.u32_is("qwen35.feed_forward_length", kFFN) && f.u32_is("qwen35.attention.head_count", 24) &&
                    f.u32_is("qwen35.attention.head_count_kv", 4) &&
                    f.u32_is("qwen35.full_attention_interval", 4) && f.u32_is("qwen35.ssm.state_size", 128) &&
                    f.u32_is("qwen35.ssm.group_count", 16) && f.u32_is("qwen35.ssm.time_step_rank", 48) &&
                    f.u32_is("qwen35.ssm.inner_size", kLinV);
    if (!ok) return report("checkpoint metadata is not Qwen3.8-27B");
    return true;
}

bool bind_mtp(Q38Model *m, const GGUFFile &f, const uint8_t *base)
{
    const bool meta_ok = f.str_is("general.architecture", "qwen35") && f.u32_is("qwen35.block_count", kTotalLayers) &&
                         f.u32_is("qwen35.nextn_predict_layers", 1) && f.u32_is("qwen35.embedding_length", kHidden) &&
                         f.u32_is("qwen35.feed_forward_length", kFFN);
    if (!meta_ok) return report("MTP checkpoint metadata is not Qwen3.8-27B");
    if (!bind_tensor(f, base, "token_embd.weight", &m->mtp_embedding) || !bind_tensor(f, base, "output.weight", &m->mtp_output) ||
        !bind_layer(&m->layers[kLayers], f, base, kLayers) ||
        !bind_tensor(f, base, "blk.64.nextn.eh_proj.weight", &m->eh_proj) ||
        !bind_tensor(f, base, "blk.64.nextn.enorm.weight", &m->enorm) ||
        !bind_tensor(f, base, "blk.64.nextn.hnorm.weight", &m->hnorm) ||
        !bind_tensor(f, base, "blk.64.nextn.shared_head_norm.weight", &m->shared_head_norm))
        return false;
    bool ok = expect(m->mtp_embedding, "token_embd.weight", kHidden, kVocab, false) &&
              expect(m->mtp_output, "output.weight", kHidden, kVocab, false) &&
              expect(m->eh_proj, "blk.64.nextn.eh_proj.weight", 2 * kHidden, kHidden, false) &&
              expect(m->enorm, "blk.64.nextn.enorm.weight", kHidden, 0, true) &&
              expect(m->hnorm, "blk.64.nextn.hnorm.weight", kHidden, 0, true) &&
              expect(m->shared_head_norm, "blk.64.nextn.shared_head_norm.weight", kHidden, 0, true);
    if (ok) m->mtp_weights_loaded = true;
    return ok;
}

void release(Q38Model *m)
{
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    float **fbufs[] = {&m->conv_state, &m->delta_state, &m->key_cache, &m->value_cache, &m->mtp_hidden,
                       &m->ck_mtp_hidden, &m->rope, &m->hidden, &m->norm,
                       &m->branch, &m->wide0, &m->qbuf, &m->attn, &m->scores, &m->logits, &m->target_norm,
                       &m->argmax_pv, &m->long_norm, &m->prep, &m->fin, &m->logits_stage};
    for (float **p : fbufs) dfree(*p);
    uint32_t **ubufs[] = {&m->tokens, &m->params, &m->words, &m->argmax_pi};
    for (uint32_t **p : ubufs) dfree(*p);
    dfree(m->q8k);
    dfree(m->presence);
    dfree(m->sample_scratch);
    if (m->weights) (void)hipFree(m->weights);
    if (m->mtp_weights) (void)hipFree(m->mtp_weights);
    if (m->tiled_weights) (void)hipFree(m->tiled_weights);
    if (m->tiled_mtp) (void)hipFree(m->tiled_mtp);
    if (m->host_logits) (void)hipHostFree(m->host_logits);
    if (m->host_words) (void)hipHostFree(m->host_words);
    if (m->host_params) (void)hipHostFree(m->host_params);
    if (m->host_sampled) (void)hipHostFree(m->host_sampled);
    for (auto &g : m->graphs) (void)hipGraphExecDestroy(g.second);
    if (m->copy_stream) (void)hipStreamSynchronize(m->copy_stream);
    if (m->logits_ready) (void)hipEventDestroy(m->logits_ready);
    if (m->copy_stream) (void)hipStreamDestroy(m->copy_stream);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

bool allocate_state(Q38Model *m)
{
    const uint32_t ctx = m->context_length;
    const size_t by_scores = kPrefillScoresBytes / ((size_t)kAttnHeads * ctx * sizeof(float));
    m->prefill_rows = (uint32_t)std::max<size_t>(kBatch, std::min<size_t>(kPrefillRows, by_scores));
    m->scratch_rows = std::max(kBatch, m->prefill_rows);
    const uint32_t B = m->scratch_rows;
    const size_t slots = q38::kRecurrentStateSlots;
    bool ok = dalloc(&m->conv_state, slots * conv_count()) && dalloc(&m->delta_state, slots * delta_count()) &&
              dalloc(&m->key_cache, kv_count(ctx)) && dalloc(&m->value_cache, kFullLayers * value_layer_floats(ctx)) &&
              dalloc(&m->mtp_hidden, kHidden) && dalloc(&m->rope, (size_t)ctx * 64) &&
              dalloc(&m->hidden, (size_t)B * kHidden) && dalloc(&m->norm, (size_t)kBatch * 2 * kHidden) &&
              dalloc(&m->branch, (size_t)B * kHidden) && dalloc(&m->wide0, (size_t)B * 2 * kFFN) &&
              dalloc(&m->qbuf, (size_t)B * kQDim) && dalloc(&m->attn, (size_t)B * kLinV) &&
              dalloc(&m->prep, (size_t)B * 2 * kFFN) &&
              dalloc(&m->scores, (size_t)B * kAttnHeads * ctx) &&
              dalloc(&m->logits, (size_t)kBatch * kVocab) && dalloc(&m->logits_stage, kVocab) &&
              dalloc(&m->target_norm, (size_t)B * kHidden) &&
              dalloc(&m->q8k, (size_t)B * (kFFN / 256) * kQ8KBytes) && dalloc(&m->tokens, B) &&
              dalloc(&m->params, (size_t)kParamSets * kParamWords) && dalloc(&m->words, 64) &&
              dalloc(&m->argmax_pv, (size_t)kBatch * q38::argmax_chunks(kVocab)) &&
              dalloc(&m->argmax_pi, (size_t)kBatch * q38::argmax_chunks(kVocab)) &&
              dalloc(&m->presence, kVocab) &&
              dalloc(&m->sample_scratch, q38::sample_scratch_bytes(kVocab, q38::kMaxSampleTopK)) &&
              hip_ok(hipHostMalloc(reinterpret_cast<void **>(&m->host_sampled), 16 * sizeof(uint32_t)),
                     "pinned token") &&
              hip_ok(hipHostMalloc(reinterpret_cast<void **>(&m->host_logits), kVocab * sizeof(float)),
                     "pinned logits") &&
              hip_ok(hipHostMalloc(reinterpret_cast<void **>(&m->host_words), ((size_t)B + 128) * sizeof(uint32_t)),
                     "pinned ids") &&
              hip_ok(hipHostMalloc(reinterpret_cast<void **>(&m->host_params),
                                   (size_t)kParamSets * kParamWords * sizeof(uint32_t)), "pinned parameters");
    if (!ok) return false;
    m->drafts = m->words;
    m->targets = m->words + 16;
    m->accept = m->words + 32;
    m->sampled = m->words + 48;
    std::vector<float> table((size_t)ctx * 64);
    q38::rope_table_host(table.data(), ctx);
    m->query_scale = 1.0f / sqrtf(128.0f);
    return hip_ok(hipMemcpy(m->rope, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice),
                  "rope table upload");
}

/* whether a projection of the loaded blocks takes fp32 input (an F32, F16,
 * BF16 or Q8_0 matrix); if so, allocate their input rows m->fin.  Captured
 * step graphs are dropped when this changes what the steps compute. */
bool setup_float_inputs(Q38Model *m)
{
    bool any = float_input(m->output);
    const uint32_t last = m->mtp_weights_loaded ? kLayers + 1 : kLayers;
    for (uint32_t l = 0; l < last; ++l) {
        const Layer &L = m->layers[l];
        const DevTensor *mats[] = {&L.ffn_gate, &L.ffn_up, &L.ffn_down};
        for (const DevTensor *t : mats) any = any || float_input(*t);
        if (L.full) {
            any = any || float_input(L.q) || float_input(L.k) || float_input(L.v) || float_input(L.out);
        } else {
            any = any || float_input(L.qkv) || float_input(L.z) || float_input(L.alpha) || float_input(L.beta) ||
                  float_input(L.ssm_out);
        }
    }
    if (m->mtp_weights_loaded) any = any || float_input(m->eh_proj) || float_input(m->mtp_output);
    if (!any || m->float_inputs) return true;
    if (!dalloc(&m->fin, (size_t)m->scratch_rows * kFFN)) return false;
    m->float_inputs = true;
    for (auto &g : m->graphs) (void)hipGraphExecDestroy(g.second);
    m->graphs.clear();
    m->seen.clear();
    return true;
}

/* zero the recurrent state (slot 0 of every layer becomes current), KV
 * caches and MTP hidden (q38_model_reset) */
bool clear_state(Q38Model *m)
{
    hipStream_t s = m->stream;
    for (uint32_t r = 0; r < kRecurrent; ++r) m->slot_host[r] = 0;
    return hip_ok(hipMemsetAsync(m->conv_state, 0, conv_count() * sizeof(float), s), "reset") &&
           hip_ok(hipMemsetAsync(m->delta_state, 0, delta_count() * sizeof(float), s), "reset") &&
           hip_ok(hipMemsetAsync(m->key_cache, 0, kv_count(m->context_length) * sizeof(float), s), "reset") &&
           hip_ok(hipMemsetAsync(m->value_cache, 0, kFullLayers * value_layer_floats(m->context_length) * sizeof(float), s),
                  "reset") &&
           hip_ok(hipMemsetAsync(m->mtp_hidden, 0, kHidden * sizeof(float), s), "reset") &&
           hip_ok(hipStreamSynchronize(s), "reset");
}

/* ---- layer trace (QWEN38_TRACE_LAYERS, as src/qwen38/qwen38_model.c:556-591) */

/* read on every call (a step's launches are recorded once per graph, so a
 * change reaches graph-replayed steps only when they are recorded) */
bool trace_enabled()
{
    const char *v = getenv("QWEN38_TRACE_LAYERS");
    return v && v[0] && strcmp(v, "0") != 0;
}

/* same line format as the reference's q38_trace_vector; synchronises the
 * stream, so it is only for correctness probes */
void trace(Q38Model *m, const char *name, int layer, const float *device, uint64_t length)
{
    if (!trace_enabled()) return;
    std::vector<float> v(length);
    if (hipMemcpyAsync(v.data(), device, length * sizeof(float), hipMemcpyDeviceToHost, m->stream) != hipSuccess ||
        hipStreamSynchronize(m->stream) != hipSuccess)
        return;
    float sum = 0.0f;
    double sum_abs = 0.0;
    for (uint64_t i = 0; i < length; ++i) {
        sum += v[i];
        sum_abs += fabsf(v[i]);
    }
    fprintf(stderr, "trace %s%d sum=%.9g abs=%.9g first=%.9g,%.9g,%.9g last=%.9g,%.9g,%.9g\n", name, layer, sum,
            sum_abs, v[0], v[1], v[2], v[length - 3], v[length - 2], v[length - 1]);
    /* QWEN38_TRACE_DIR: also write the whole vector as raw float32 */
    if (const char *dir = getenv("QWEN38_TRACE_DIR")) {
        const std::string path = std::string(dir) + "/" + name + std::to_string(layer) + ".f32";
        if (FILE *f = fopen(path.c_str(), "wb")) {
            fwrite(v.data(), sizeof(float), length, f);
            fclose(f);
        }
    }
}

/* ---- step building blocks -------------------------------------------------- */

/* Where a step reads its parameter block and its input token ids (device). */
struct Step {
    const uint32_t *params;
    const uint32_t *tokens;
};

Step step_of(Q38Model *m, uint32_t param_set, const uint32_t *tokens)
{
    return Step{m->params + (size_t)param_set * kParamWords, tokens};
}

/* GEMM over `count` Q8_K rows already in m->q8k (starting at block
 * `first_block`) */
/* row-major GEMM of `count` Q8_K rows at x: launches of up to kBatch
 * tokens (every token's outputs are independent of the batch) */
bool gemm_rows(Q38Model *m, const DevTensor &w, uint32_t count, const uint8_t *x, float *out, uint32_t ldy,
               uint32_t rows, const uint8_t *wdata)
{
    const uint32_t nb = (uint32_t)(w.width / 256);
    if (w.type == IQ1_M && count >= (uint32_t)q38::kWideMinTokens &&
        q38::launch_gemm_iq1m_wide(count, wdata, x, out, ldy, rows, nb, m->grid, m->stream))
        return true;
    /* Q4_K, Q6_K and IQ1_M have their own kernel families; the other Q8_K
     * formats run the generic lane-chain kernel */
    const bool tuned = w.type == Q4_K || w.type == Q6_K || w.type == IQ1_M;
    for (uint32_t t0 = 0; t0 < count; t0 += kBatch) {
        const uint32_t n = std::min(kBatch, count - t0);
        const uint8_t *xt = x + (size_t)t0 * nb * kQ8KBytes;
        const bool ok = tuned ? q38::launch_gemm_ld((int)w.type, (int)n, wdata, xt, out + (size_t)t0 * ldy, ldy, rows,
                                                   nb, m->grid, m->stream)
                              : q38::launch_gemm_format((int)w.type, (int)n, wdata, xt, out + (size_t)t0 * ldy, ldy,
                                                        rows, nb, m->grid, m->stream);
        if (!ok) return report("unsupported GEMM configuration");
    }
    return true;
}

/* a float-input matrix (F32, F16, BF16, Q8_0) over `count` fp32 rows at xf,
 * rows w.width floats apart (q38_tensor_gemv_f32 per row) */
bool gemm_float(Q38Model *m, const DevTensor &w, uint32_t count, const float *xf, float *out, uint32_t ldy,
                uint32_t rows, const uint8_t *wdata)
{
    if (!xf) return report("float-input projection without its fp32 input");
    for (uint32_t t0 = 0; t0 < count; t0 += 4) {
        const uint32_t n = std::min<uint32_t>(4, count - t0);
        if (!q38::launch_gemm_float((int)w.type, (int)n, wdata, xf + (size_t)t0 * w.width, out + (size_t)t0 * ldy, ldy,
                                    rows, (uint32_t)w.width, m->stream))
            return report("unsupported float GEMM configuration");
    }
    return true;
}

/* the tiled copy's kernel where there is one: Q4_K for any row count
 * (one row, 2..8 rows and prefill batches), IQ1_M for 1..8 rows (prefill
 * batches keep the row-major blocks); false when none ran */
bool gemm_tiled(Q38Model *m, const DevTensor &w, uint32_t count, const uint8_t *x, float *out, uint32_t ldy,
                uint32_t rows)
{
    if (!w.tiled) return false;
    const uint32_t nb = (uint32_t)(w.width / 256);
    if (w.type == Q4_K)
        return count >= 1 && q38::launch_gemm_q4k_tiled((int)count, w.tiled, x, out, ldy, rows, nb, m->stream);
    if (w.type == IQ1_M)
        return count >= 1 && count <= kBatch &&
               q38::launch_gemm_iq1m_tiled((int)count, w.tiled, x, out, ldy, rows, nb, m->grid, m->stream);
    return false;
}

/* one projection: Q8_K rows from m->q8k (starting at block first_block), or
 * for a float-input matrix the fp32 rows at xf */
bool gemm_q(Q38Model *m, const DevTensor &w, uint32_t count, float *out, size_t first_block = 0,
            const float *xf = nullptr)
{
    if (float_input(w)) return gemm_float(m, w, count, xf, out, (uint32_t)w.rows, (uint32_t)w.rows, w.data);
    if (gemm_tiled(m, w, count, m->q8k + first_block * kQ8KBytes, out, (uint32_t)w.rows, (uint32_t)w.rows))
        return true;
    return gemm_rows(m, w, count, m->q8k + first_block * kQ8KBytes, out, (uint32_t)w.rows, (uint32_t)w.rows,
                     w.data);
}

uint64_t row_bytes(const DevTensor &t)
{
    uint32_t e = 0, b = 0;
    ggml_block(t.type, &e, &b);
    return t.width / e * b;
}

/* runs of members [lo, hi) of g that form one matrix (same type and width,
 * back to back in HBM): f(first member, end member, total rows) */
template <typename F>
void for_runs(const Group &g, int lo, int hi, F f)
{
    for (int i = lo; i < hi;) {
        const DevTensor &a = g.part[i];
        uint64_t rows = a.rows;
        int j = i + 1;
        while (j < hi && g.part[j].type == a.type && g.part[j].width == a.width &&
               g.part[j].data == a.data + rows * row_bytes(a)) {
            rows += g.part[j].rows;
            ++j;
        }
        f(i, j, rows);
        i = j;
    }
}

/* Build 16-row tiled copies of the Q4_K GEMM matrices of blocks
 * [first, last) (plus eh_proj when `with_eh`) in one allocation: every run
 * of a fusion group, the down projection and the attention / DeltaNet
 * output projection.  A group member whose first row inside its run is a
 * multiple of 16 gets a pointer to its own tiles. */
bool build_tiled(Q38Model *m, uint32_t first, uint32_t last, bool with_eh, void **mem)
{
    struct Job {
        const uint8_t *src;
        uint32_t rows, nb, type;
        std::vector<std::pair<DevTensor *, uint64_t>> targets;   /* tensor, first tile */
    };
    std::vector<Job> jobs;
    auto supported = [](const DevTensor &t) {
        const uint64_t nb = t.width / 256;
        return (t.type == Q4_K || t.type == IQ1_M) && t.data && (nb == 20 || nb == 24 || nb == 40 || nb == 68);
    };
    /* bytes of one block of a 16-row tile, and of the whole copy */
    auto tile_block = [](uint32_t type) -> size_t { return type == IQ1_M ? 16 * 56 : 2304; };
    auto tiled_bytes = [](const Job &j) {
        return j.type == IQ1_M ? q38::tiled_iq1m_bytes(j.rows, j.nb) : q38::tiled_q4k_bytes(j.rows, j.nb);
    };
    auto add_group = [&](Group &g) {
        for_runs(g, 0, g.n, [&](int i, int j, uint64_t rows) {
            if (!supported(g.part[i])) return;
            Job job{g.part[i].data, (uint32_t)rows, (uint32_t)(g.part[i].width / 256), g.part[i].type, {}};
            uint64_t row = 0;
            for (int k = i; k < j; ++k) {
                if (row % 16 == 0) job.targets.emplace_back(&g.part[k], row / 16);
                row += g.part[k].rows;
            }
            jobs.push_back(job);
        });
    };
    auto add_one = [&](DevTensor &t) {
        if (supported(t))
            jobs.push_back(Job{t.data, (uint32_t)t.rows, (uint32_t)(t.width / 256), t.type, {{&t, 0}}});
    };
    for (uint32_t l = first; l < last; ++l) {
        Layer &L = m->layers[l];
        add_group(L.ffn_in);
        add_group(L.mix_in);
        add_one(L.ffn_down);
        add_one(L.full ? L.out : L.ssm_out);
    }
    if (with_eh) add_one(m->eh_proj);
    size_t total = 0;
    std::vector<size_t> offsets;
    for (const Job &j : jobs) {
        offsets.push_back(total);
        total += align256(tiled_bytes(j));
    }
    if (!total) return true;
    if (!hip_ok(hipMalloc(mem, total), "tiled weight allocation")) return false;
    uint8_t *base = static_cast<uint8_t *>(*mem);
    for (size_t k = 0; k < jobs.size(); ++k) {
        const Job &j = jobs[k];
        uint8_t *dst = base + offsets[k];
        const bool ok = j.type == IQ1_M ? q38::launch_repack_iq1m_tiles(dst, j.src, j.rows, j.nb, m->stream)
                                        : q38::launch_repack_q4k_tiles(dst, j.src, j.rows, j.nb, m->stream);
        if (!ok) return report("tiled repack failed");
        for (const auto &t : j.targets) t.first->tiled = dst + t.second * j.nb * tile_block(j.type);
    }
    return hip_ok(hipStreamSynchronize(m->stream), "tiled repack");
}

/* members [lo, hi) of group g over `count` Q8_K rows in m->q8k; row t of
 * member i lands at out + t * ldy + first[i] - first[lo].  Two or more rows
 * use the tiled copy where there is one. */
bool gemm_group(Q38Model *m, const Group &g, int lo, int hi, uint32_t count, float *out, uint32_t ldy,
                const float *xf = nullptr)
{
    bool ok = true;
    for_runs(g, lo, hi, [&](int i, int, uint64_t rows) {
        const DevTensor &a = g.part[i];
        float *y = out + (g.first[i] - g.first[lo]);
        if (float_input(a)) {
            if (!gemm_float(m, a, count, xf, y, ldy, (uint32_t)rows, a.data)) ok = false;
            return;
        }
        if (gemm_tiled(m, a, count, m->q8k, y, ldy, (uint32_t)rows)) return;
        if (!gemm_rows(m, a, count, m->q8k, y, ldy, (uint32_t)rows, a.data)) ok = false;
    });
    return ok;
}

/* host staging of a parameter block: position of row 0 and the current
 * state slot of every recurrent layer */
void write_params(Q38Model *m, uint32_t set, uint32_t position)
{
    uint32_t *p = m->host_params + (size_t)set * kParamWords;
    p[0] = position;
    for (uint32_t r = 0; r < kRecurrent; ++r) p[1 + r] = m->slot_host[r];
}

/* copy all staged parameter blocks to the device (ordered on the stream) */
bool flush_params(Q38Model *m)
{
    return hip_ok(hipMemcpyAsync(m->params, m->host_params, (size_t)kParamSets * kParamWords * sizeof(uint32_t),
                                 hipMemcpyHostToDevice, m->stream),
                  "parameter upload");
}

/* after `rows` rows ran through recurrent layers 0..layers-1 */
void advance_slots(Q38Model *m, uint32_t rows, uint32_t layers = kLayers)
{
    for (uint32_t layer = 0; layer < layers; ++layer) {
        if ((layer + 1) % 4 == 0) continue;
        const uint32_t r = layer - (layer + 1) / 4;
        m->slot_host[r] = (m->slot_host[r] + rows) % q38::kRecurrentStateSlots;
    }
}

/* token embedding rows of `count` token ids into m->hidden
 * (q38_tensor_row_f32 of token_embd): the Q4_K kernel, the generic row
 * decode, or NaN rows for a type the reference's row decode has no case for */
void embed(Q38Model *m, const DevTensor &table, const uint32_t *tokens, uint32_t count)
{
    if (table.type == Q4_K) {
        q38::launch_embed_q4k(m->hidden, table.data, tokens, (int)count, kHidden, kVocab, m->stream);
    } else if (!q38::launch_row_decode((int)table.type, table.data, tokens, 0, count, kVocab, m->hidden, kHidden,
                                       m->stream)) {
        q38::launch_fill_f32(m->hidden, (uint64_t)count * kHidden, __builtin_nanf(""), m->stream);
    }
}

/* apply a pending FFN residual add to m->hidden */
void flush_branch(Q38Model *m, uint32_t count)
{
    if (m->pending_branch) q38::launch_add(m->hidden, m->branch, (long long)count * kHidden, m->stream);
    m->pending_branch = false;
}

/* RMSNorm of the rows of m->hidden (after adding the pending FFN branch of
 * the previous block, if any) into Q8_K rows of m->q8k, and the fp32 rows
 * into norm_out (m->fin by default when float-input matrices need them) */
void norm_hidden(Q38Model *m, const DevTensor &weight, uint32_t count, float *norm_out = nullptr)
{
    if (!norm_out && m->float_inputs) norm_out = m->fin;
    q38::launch_norm_quant(norm_out, kHidden, m->q8k, kHidden / 256, m->hidden, kHidden,
                           m->pending_branch ? m->branch : nullptr, weight.f32(), (int)count, m->stream);
    m->pending_branch = false;
}

/* attention mixer of a full-attention layer over `count` rows at positions
 * params[0] + t (q38_batch_full_attention, qwen38_model.c:1089-1119); input
 * Q8_K rows in m->q8k, output rows in m->branch */
bool full_attention_rows(Q38Model *m, const Step &s, int layer, uint32_t count)
{
    const Layer &L = m->layers[layer];
    const int full_index = layer / 4;
    const size_t kv_off = (size_t)full_index * m->context_length * kKVDim;
    const size_t v_off = (size_t)full_index * value_layer_floats(m->context_length);
    /* per row: q+gate [12288] | k [1024] | v [1024] */
    const Group &g = L.mix_in;
    if (!gemm_group(m, g, 0, 3, count, m->wide0, g.width, m->fin)) return false;
    q38::launch_attention(m->attn, m->q8k, m->qbuf, m->wide0, m->wide0 + g.first[1], m->wide0 + g.first[2], g.width,
                          L.q_norm.f32(), L.k_norm.f32(), m->rope, m->key_cache + kv_off, m->value_cache + v_off,
                          m->scores, (int)m->context_length, s.params, (int)count, m->stream);
    if (count == 1 && trace_enabled()) {
        uint32_t pos = 0;
        (void)hipMemcpy(&pos, s.params, 4, hipMemcpyDeviceToHost);
        trace(m, "Qcur_full-", layer, m->wide0, kQGDim);
        trace(m, "Kcur-", layer, m->key_cache + kv_off + (size_t)pos * kKVDim, kKVDim);
        trace(m, "Vcur-", layer, m->wide0 + g.first[2], kKVDim);
        trace(m, "attn_gated-", layer, m->attn, kQDim);
    }
    if (!gemm_q(m, L.out, count, m->branch, 0, m->attn)) return false;
    if (count == 1) trace(m, "attn_output-", layer, m->branch, kHidden);
    return true;
}

/* DeltaNet mixer (q38_batch_linear_attention, qwen38_model.c:1062-1087) */
bool linear_attention_rows(Q38Model *m, const Step &s, int layer, uint32_t count)
{
    const Layer &L = m->layers[layer];
    const int r = layer - (layer + 1) / 4;
    /* per row: qkv [10240] | z [6144] | beta [48] | alpha [48] */
    const Group &g = L.mix_in;
    const uint32_t ld = g.width;
    if (!gemm_group(m, g, 0, 4, count, m->wide0, ld, m->fin)) return false;
    const bool tr = count == 1 && trace_enabled();
    if (tr) {
        trace(m, "dn_qkv_proj-", layer, m->wide0, kQKV);
        trace(m, "dn_z-", layer, m->wide0 + g.first[1], kLinV);
        trace(m, "dn_beta_proj-", layer, m->wide0 + g.first[2], kVHeads);
        trace(m, "dn_alpha_proj-", layer, m->wide0 + g.first[3], kVHeads);
    }
    float *conv = m->conv_state + (size_t)r * kQKV * 3;
    float *delta = m->delta_state + (size_t)r * kVHeads * kHeadDim * kHeadDim;
    if (count > kBatch) {
        /* a prefill batch: the prep of all rows in parallel into m->prep,
         * then the state update keeping only the state after the last row */
        q38::launch_deltanet_prep_rows(m->prep, m->wide0, ld, (int)g.first[2], (int)g.first[3], conv,
                                       (long long)conv_count(), s.params + 1 + r, (int)count, L.conv.f32(),
                                       L.a.f32(), L.dt.f32(), m->stream);
        q38::launch_deltanet_state(m->attn, delta, (long long)delta_count(), s.params + 1 + r, (int)count, m->prep,
                                   ld, (int)g.first[2], (int)g.first[3], m->query_scale, true, m->stream);
    } else if (tr) {
        /* the layer trace prints the prepared q/k/v: separate kernels */
        const bool last_only = false;
        q38::launch_deltanet_prep(m->wide0, ld, (int)g.first[2], (int)g.first[3], conv, (long long)conv_count(),
                                  s.params + 1 + r, (int)count, L.conv.f32(), L.a.f32(), L.dt.f32(), last_only,
                                  m->stream);
        trace(m, "dn_qkv-", layer, m->wide0, kQKV);
        trace(m, "dn_beta-", layer, m->wide0 + g.first[2], kVHeads);
        trace(m, "dn_alpha-", layer, m->wide0 + g.first[3], kVHeads);
        q38::launch_deltanet_state(m->attn, delta, (long long)delta_count(), s.params + 1 + r, (int)count, m->wide0,
                                   ld, (int)g.first[2], (int)g.first[3], m->query_scale, last_only, m->stream);
    } else if (!q38::launch_deltanet_fused(m->attn, delta, (long long)delta_count(), s.params + 1 + r, (int)count,
                                           m->wide0, ld, (int)g.first[2], (int)g.first[3], m->query_scale, conv,
                                           (long long)conv_count(), L.conv.f32(), L.a.f32(), L.dt.f32(),
                                           m->stream)) {
        return report("unsupported DeltaNet batch");
    }
    if (tr) trace(m, "dn_core-", layer, m->attn, kLinV);
    q38::launch_deltanet_out_quant(m->attn, m->q8k, m->wide0 + g.first[1], ld, L.ssm_norm.f32(), (int)count,
                                   m->stream);
    if (tr) trace(m, "dn_gated-", layer, m->attn, kLinV);
    return gemm_q(m, L.ssm_out, count, m->branch, 0, m->attn);
}

/* one transformer block over `count` rows of m->hidden
 * (q38_layer_forward / q38_batch_layer, qwen38_model.c:955-984, 1121-1155).
 * The FFN's residual add is left pending in m->branch and fused into the
 * next RMSNorm. */
bool layer_rows(Q38Model *m, const Step &s, int layer, uint32_t count)
{
    const Layer &L = m->layers[layer];
    norm_hidden(m, L.attn_norm, count);
    if (!(L.full ? full_attention_rows(m, s, layer, count) : linear_attention_rows(m, s, layer, count))) return false;
    if (count == 1) trace(m, "attention_branch-", layer, m->branch, kHidden);
    m->pending_branch = true;
    norm_hidden(m, L.post_norm, count);
    if (count == 1) trace(m, "attn_residual-", layer, m->hidden, kHidden);
    const Group &g = L.ffn_in;   /* per row: gate [17408] | up [17408] */
    if (!gemm_group(m, g, 0, 2, count, m->wide0, g.width, m->fin)) return false;
    q38::launch_swiglu_quant(m->q8k, m->wide0, m->wide0 + g.first[1], g.width, (int)count, m->stream,
                             m->float_inputs ? m->fin : nullptr);
    if (!gemm_q(m, L.ffn_down, count, m->branch, 0, m->fin)) return false;
    m->pending_branch = true;
    if (count == 1 && trace_enabled()) {
        trace(m, "ffn_out-", layer, m->branch, kHidden);
        flush_branch(m, count);
        if (layer < (int)kLayers) trace(m, "l_out-", layer, m->hidden, kHidden);
    }
    return true;
}

/* Target model over `count` (<= scratch_rows) tokens at positions params[0] + t:
 * all 64 blocks, the output norm into m->target_norm and, if `logit_rows`,
 * the LM head of the last `logit_rows` rows into m->logits
 * (q38_batch_target_eval, qwen38_model.c:1241-1266).  Enqueue only: the
 * caller advances the host-side state (slots, position). */
bool target_rows(Q38Model *m, const Step &s, uint32_t count, uint32_t logit_rows)
{
    embed(m, m->embedding, s.tokens, count);
    m->pending_branch = false;
    if (count == 1) trace(m, "model.input_embed", -1, m->hidden, kHidden);
    for (uint32_t layer = 0; layer < kLayers; ++layer)
        if (!layer_rows(m, s, (int)layer, count)) return false;
    norm_hidden(m, m->output_norm, count, m->target_norm);
    if (logit_rows && !gemm_q(m, m->output, logit_rows, m->logits, (size_t)(count - logit_rows) * (kHidden / 256),
                              m->target_norm + (size_t)(count - logit_rows) * kHidden))
        return false;
    return launches_ok();
}

/* KV-cache rows of the MTP block for `count` tokens at positions
 * params[0] + t: eh_proj over [enorm(embedding) | hnorm(previous hidden)],
 * attn_norm, K and V projections and the k-norm / RoPE / cache write
 * (q38_mtp_catchup, qwen38_model.c:1268-1294), then the MTP hidden becomes
 * target_norm[count - 1].  The rest of the reference's catch-up block
 * (queries, attention output, FFN) is computed there and never read, so it
 * is not computed here.  Enqueue only. */
bool mtp_catchup(Q38Model *m, const Step &s, uint32_t count, const float *prev0 = nullptr,
                 const uint32_t *last_row = nullptr)
{
    if (!prev0) prev0 = m->mtp_hidden;
    const Layer &L = m->layers[kLayers];
    constexpr int kHB = kHidden / 256;   /* Q8_K blocks per hidden row */
    embed(m, m->mtp_embedding, s.tokens, count);
    /* Q8_K rows of 2*kHidden: [enorm(e_t) | hnorm(prev_t)], prev_0 = MTP hidden,
     * prev_t = target_norm[t-1] (and the same fp32 rows in m->fin when the
     * projection takes them) */
    float *f = m->float_inputs ? m->fin : nullptr;
    q38::launch_norm_quant(f, 2 * kHidden, m->q8k, 2 * kHB, m->hidden, kHidden, nullptr, m->enorm.f32(), (int)count,
                           m->stream);
    q38::launch_norm_quant(f ? f + kHidden : nullptr, 2 * kHidden, m->q8k + kHB * kQ8KBytes, 2 * kHB,
                           const_cast<float *>(prev0), kHidden, nullptr, m->hnorm.f32(), 1, m->stream);
    if (count > 1)
        q38::launch_norm_quant(f ? f + 3 * kHidden : nullptr, 2 * kHidden, m->q8k + 3 * kHB * kQ8KBytes, 2 * kHB,
                               m->target_norm, kHidden, nullptr, m->hnorm.f32(), (int)count - 1, m->stream);
    if (!gemm_q(m, m->eh_proj, count, m->hidden, 0, m->fin)) return false;
    m->pending_branch = false;
    norm_hidden(m, L.attn_norm, count);
    /* k | v members of the block's q+gate | k | v group, rows 2048 apart */
    const Group &g = L.mix_in;
    const uint32_t ld = g.first[2] + (uint32_t)g.part[2].rows - g.first[1];
    if (!gemm_group(m, g, 1, 3, count, m->wide0, ld, m->fin)) return false;
    const size_t kv_off = (size_t)(kLayers / 4) * m->context_length * kKVDim;
    const size_t v_off = (size_t)(kLayers / 4) * value_layer_floats(m->context_length);
    q38::launch_kv_write(m->wide0, m->wide0 + (g.first[2] - g.first[1]), ld, L.k_norm.f32(), m->rope,
                         m->key_cache + kv_off, m->value_cache + v_off, (int)m->context_length, s.params,
                         (int)count, m->stream);
    /* the MTP hidden state continues from the last row (or from row
     * *last_row - 1, read on the device) */
    if (last_row) {
        q38::launch_copy_row(m->mtp_hidden, m->target_norm, kHidden, kHidden, last_row, count, m->stream);
        return launches_ok();
    }
    return launches_ok() &&
           hip_ok(hipMemcpyAsync(m->mtp_hidden, m->target_norm + (size_t)(count - 1) * kHidden,
                                 kHidden * sizeof(float), hipMemcpyDeviceToDevice, m->stream),
                  "mtp hidden");
}

/* one MTP draft step for token s.tokens[0] at position params[0]
 * (q38_model_mtp_forward, qwen38_model.c:1588-1612; the block is
 * q38_mtp_layer_forward :932-953): logits into m->logits, MTP hidden updated.
 * Enqueue only. */
bool mtp_step(Q38Model *m, const Step &s)
{
    constexpr int kHB = kHidden / 256;
    embed(m, m->mtp_embedding, s.tokens, 1);
    float *f = m->float_inputs ? m->fin : nullptr;
    q38::launch_norm_quant(f, 2 * kHidden, m->q8k, 2 * kHB, m->hidden, kHidden, nullptr, m->enorm.f32(), 1, m->stream);
    q38::launch_norm_quant(f ? f + kHidden : nullptr, 2 * kHidden, m->q8k + kHB * kQ8KBytes, 2 * kHB, m->mtp_hidden,
                           kHidden, nullptr, m->hnorm.f32(), 1, m->stream);
    if (!gemm_q(m, m->eh_proj, 1, m->hidden, 0, m->fin)) return false;
    m->pending_branch = false;
    if (!layer_rows(m, s, (int)kLayers, 1)) return false;
    /* mtp hidden = shared_head_norm(hidden + branch), and its Q8_K rows */
    q38::launch_norm_quant(m->mtp_hidden, kHidden, m->q8k, kHB, m->hidden, kHidden,
                           m->pending_branch ? m->branch : nullptr, m->shared_head_norm.f32(), 1, m->stream);
    m->pending_branch = false;
    return gemm_q(m, m->mtp_output, 1, m->logits, 0, m->mtp_hidden) && launches_ok();
}

/* ---- graphs ------------------------------------------------------------------ */

enum : uint32_t { kGraphTarget = 1, kGraphDraft = 3, kGraphCatchup = 4, kGraphTransaction = 5 };

uint64_t graph_key(uint32_t kind, uint32_t a, uint32_t b = 0) { return ((uint64_t)kind << 32) | (a << 16) | b; }

/* Run the enqueue-only sequence `body` on the model's stream: the first
 * time eagerly, from the second time on as a HIP graph captured then and
 * replayed afterwards (the parameter blocks and token ids it reads are in
 * device memory, so one graph serves every position).  Graphs are off while
 * tracing or when QWEN38_NO_GRAPHS is set. */
template <typename Body>
bool run_step(Q38Model *m, uint64_t key, Body raw_body)
{
    auto body = [&] { return raw_body() && launches_ok(); };
    if (!m->graphs_enabled || trace_enabled()) return body();
    auto it = m->graphs.find(key);
    if (it != m->graphs.end()) return hip_ok(hipGraphLaunch(it->second, m->stream), "graph launch");
    if (!m->seen[key]) {
        m->seen[key] = true;
        return body();
    }
    hipGraph_t graph = nullptr;
    if (!hip_ok(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal), "graph capture")) return false;
    const bool ok = body();
    const bool ended = hip_ok(hipStreamEndCapture(m->stream, &graph), "graph capture");
    if (!ok || !ended) {
        if (graph) (void)hipGraphDestroy(graph);
        return false;
    }
    hipGraphExec_t exec = nullptr;
    const bool inst = hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate");
    (void)hipGraphDestroy(graph);
    if (!inst) return false;
    m->graphs[key] = exec;
    return hip_ok(hipGraphLaunch(exec, m->stream), "graph launch");
}

/* token ids through the pinned staging (count <= scratch_rows) */
bool upload_tokens(Q38Model *m, const uint32_t *tokens, uint32_t count, uint32_t *device)
{
    if (count > m->scratch_rows) return report("token batch larger than the scratch");
    for (uint32_t i = 0; i < count; ++i) {
        if (tokens[i] >= kVocab) return report("token id out of range");
        m->host_words[i] = tokens[i];
    }
    return hip_ok(hipMemcpyAsync(device, m->host_words, count * sizeof(uint32_t), hipMemcpyHostToDevice, m->stream),
                  "token upload");
}

bool logits_to_host(Q38Model *m, const float *device_row)
{
    m->last_logits = device_row;
    return hip_ok(hipMemcpyAsync(m->host_logits, device_row, kVocab * sizeof(float), hipMemcpyDeviceToHost,
                                 m->stream),
                  "logits download") &&
           hip_ok(hipStreamSynchronize(m->stream), "logits download");
}

/* q38_checkpoint_state (qwen38_model.c:1200-1210): the recurrent state is
 * not copied, only its slot indices are remembered; the slots a verify
 * batch writes are the ones after the current one, so the checkpointed
 * state stays intact. */
bool checkpoint(Q38Model *m)
{
    m->ck_position = m->position;
    m->ck_mtp_position = m->mtp_position;
    for (uint32_t r = 0; r < kRecurrent; ++r) m->ck_slot[r] = m->slot_host[r];
    return hip_ok(hipMemcpyAsync(m->ck_mtp_hidden, m->mtp_hidden, kHidden * sizeof(float), hipMemcpyDeviceToDevice,
                                 m->stream), "checkpoint");
}

/* target state after the first `rows` rows of the batch that followed the
 * checkpoint (rows = 0 restores the checkpoint itself) */
void restore_target(Q38Model *m, uint32_t rows = 0)
{
    m->position = m->ck_position + rows;
    for (uint32_t r = 0; r < kRecurrent; ++r)
        m->slot_host[r] = (m->ck_slot[r] + rows) % q38::kRecurrentStateSlots;
}

bool restore_mtp(Q38Model *m)
{
    m->mtp_position = m->ck_mtp_position;
    return hip_ok(hipMemcpyAsync(m->mtp_hidden, m->ck_mtp_hidden, kHidden * sizeof(float), hipMemcpyDeviceToDevice,
                                 m->stream), "restore");
}

bool download_words(Q38Model *m, uint32_t *host, const uint32_t *device, uint32_t count)
{
    return hip_ok(hipMemcpyAsync(host, device, count * sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream),
                  "id download") &&
           hip_ok(hipStreamSynchronize(m->stream), "id download");
}

/* q38_model_speculative_greedy for draft counts above kBatch
 * (qwen38_model.c:1614-1714), in steps of at most kBatch rows:
 *  - drafts in groups of kBatch MTP steps (the same per-step graphs as the
 *    short path), each group's last draft feeding the next group, until
 *    draft_count drafts or the stop token;
 *  - the verify rows [token, d0 .. d_{n-2}] in chunks of kBatch rows, the
 *    acceptance checked after each chunk.  A chunk runs only when every row
 *    before it was accepted, so the state the result needs (after `consumed`
 *    rows) is always in one of the slots the last chunk wrote, and the
 *    checkpoint's slot may be reused once a whole chunk is accepted.  Rows
 *    after the first rejected one are never needed (the reference replays
 *    only the consumed rows), so they are not computed;
 *  - the MTP catch-up over the consumed rows in chunks, each chunk's first
 *    previous hidden state being the last output-norm row of the chunk
 *    before it.
 * Every row's arithmetic is that of the one-batch evaluation (rows are
 * independent in the GEMMs, the recurrent and KV-cache cores run in token
 * order), so results are the reference's.  Eager launches with host waits
 * between chunks; the short path keeps one graph per step. */
bool speculative_chunked(Q38Model *m, uint32_t token, uint32_t stop_token, uint32_t k, std::vector<uint32_t> *accepted,
                         const float **next_row)
{
    std::vector<uint32_t> drafts;
    drafts.reserve(k);
    uint32_t input = token;
    bool stopped = false;
    while (drafts.size() < k && !stopped) {
        const uint32_t g = (uint32_t)drafts.size(), n = std::min(kBatch, k - g);
        for (uint32_t i = 0; i < n; ++i) write_params(m, kParamDraft0 + i, m->ck_mtp_position + g + i);
        if (!upload_tokens(m, &input, 1, m->drafts) || !flush_params(m)) return false;
        for (uint32_t i = 0; i < n; ++i) {
            const Step s = step_of(m, kParamDraft0 + i, m->drafts + i);
            if (!run_step(m, graph_key(kGraphDraft, i, 0), [&] {
                    if (!mtp_step(m, s)) return false;
                    q38::launch_argmax(m->logits, kVocab, 1, m->argmax_pv, m->argmax_pi, m->drafts + i + 1, m->stream);
                    return true;
                }))
                return false;
        }
        uint32_t *hw = m->host_words + 64;
        if (!download_words(m, hw, m->drafts + 1, n)) return false;
        for (uint32_t i = 0; i < n && !stopped; ++i) {
            drafts.push_back(hw[i]);
            stopped = hw[i] == stop_token;
        }
        input = drafts.back();
    }
    const uint32_t n_rows = (uint32_t)drafts.size();
    if (m->long_norm_rows < n_rows) {
        dfree(m->long_norm);
        m->long_norm_rows = 0;
        if (!dalloc(&m->long_norm, (size_t)n_rows * kHidden)) return false;
        m->long_norm_rows = n_rows;
    }
    std::vector<uint32_t> inputs(n_rows);
    inputs[0] = token;
    for (uint32_t i = 1; i < n_rows; ++i) inputs[i] = drafts[i - 1];
    float *saved_norm = m->target_norm;
    uint32_t matched = 0, next = 0;
    bool ok = true, mismatch = false;
    uint32_t last_chunk = 0;
    for (uint32_t c0 = 0; ok && c0 < n_rows && !mismatch; c0 += kBatch) {
        const uint32_t rows = std::min(kBatch, n_rows - c0);
        last_chunk = c0;
        write_params(m, kParamTarget, m->ck_position + c0);
        m->target_norm = m->long_norm + (size_t)c0 * kHidden;
        ok = upload_tokens(m, inputs.data() + c0, rows, m->tokens) && flush_params(m) &&
             target_rows(m, step_of(m, kParamTarget, m->tokens), rows, rows);
        if (ok) {
            q38::launch_argmax(m->logits, kVocab, rows, m->argmax_pv, m->argmax_pi, m->targets, m->stream);
            ok = download_words(m, m->host_words + 64, m->targets, rows);
        }
        for (uint32_t t = 0; ok && t < rows && !mismatch; ++t) {
            const uint32_t target = m->host_words[64 + t];
            if (target != drafts[c0 + t]) {
                next = target;
                mismatch = true;
            } else {
                ++matched;
            }
        }
        /* the rows of this chunk advanced the recurrent slots */
        if (ok) advance_slots(m, rows);
    }
    const uint32_t consumed = mismatch ? matched + 1 : n_rows;
    restore_target(m, consumed);
    ok = ok && restore_mtp(m);
    for (uint32_t c0 = 0; ok && c0 < consumed; c0 += kBatch) {
        const uint32_t rows = std::min(kBatch, consumed - c0);
        write_params(m, kParamCatchup, m->ck_mtp_position + c0);
        m->target_norm = m->long_norm + (size_t)c0 * kHidden;
        ok = upload_tokens(m, inputs.data() + c0, rows, m->tokens) && flush_params(m) &&
             mtp_catchup(m, step_of(m, kParamCatchup, m->tokens), rows) &&
             hip_ok(hipStreamSynchronize(m->stream), "catch-up");
    }
    m->target_norm = saved_norm;
    if (!ok) return false;
    accepted->assign(drafts.begin(), drafts.begin() + matched);
    if (mismatch) accepted->push_back(next);
    *next_row = m->logits + (size_t)(consumed - 1 - last_chunk) * kVocab;
    m->mtp_position = m->ck_mtp_position + consumed;
    return true;
}

}  // namespace

namespace {

/* q38_model_forward_token without the logits download: the logits of the
 * token are in m->logits row 0 when it returns true */
bool forward_device(Q38Model *m, uint32_t token)
{
    m->last_logits = nullptr;
    write_params(m, kParamTarget, m->position);
    if (!upload_tokens(m, &token, 1, m->tokens) || !flush_params(m)) return false;
    const Step s = step_of(m, kParamTarget, m->tokens);
    const bool mtp = m->mtp_enabled;
    const bool ok = run_step(m, graph_key(kGraphTarget, 1, mtp), [&] {
        /* q38_model_forward_token (qwen38_model.c:1494-1517): the normed final
         * hidden becomes the MTP input when MTP is enabled */
        return target_rows(m, s, 1, 1) &&
               (!mtp || hip_ok(hipMemcpyAsync(m->mtp_hidden, m->target_norm, kHidden * sizeof(float),
                                              hipMemcpyDeviceToDevice, m->stream), "mtp hidden"));
    });
    if (!ok) return false;
    advance_slots(m, 1);
    ++m->position;
    m->last_logits = m->logits;
    return true;
}

/* the Q38Sampler fields (include/qwen38/qwen38_sampler.h:10-18) */
struct SampleArgs {
    uint64_t *state;
    float temperature, top_p, presence_penalty;
    uint32_t top_k;
    const uint8_t *presence;
    uint32_t presence_size;
};

/* q38_sample (qwen38_sampler.c:51-119) over the device logits row `row`;
 * the caller's host presence bytes are copied to the device when the
 * penalty applies (tokens at or above presence_size are never penalised,
 * nor are ids beyond the vocabulary ever read) */
bool sample_row(Q38Model *m, const float *row, const SampleArgs &a, uint32_t *token)
{
    if (const char *why = q38::check_sample(kVocab, a.temperature, a.top_k)) {
        fprintf(stderr, "qwen38: sampler: %s\n", why);
        return false;
    }
    const uint8_t *presence = nullptr;
    uint32_t presence_size = 0;
    if (a.presence_penalty != 0.0f && a.presence && a.presence_size) {
        presence_size = std::min(a.presence_size, kVocab);
        if (!hip_ok(hipMemcpyAsync(m->presence, a.presence, presence_size, hipMemcpyHostToDevice, m->stream),
                    "presence upload"))
            return false;
        presence = m->presence;
    }
    if (!q38::launch_sample(m->sampled, a.state, row, kVocab, presence, presence_size, a.temperature, a.top_p,
                            a.presence_penalty, a.top_k, m->sample_scratch, m->stream)) {
        fprintf(stderr, "qwen38: sampler launch failed\n");
        return false;
    }
    if (!hip_ok(hipMemcpyAsync(m->host_sampled, m->sampled, sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream),
                "token download") ||
        !hip_ok(hipStreamSynchronize(m->stream), "token download"))
        return false;
    *token = m->host_sampled[0];
    return true;
}

}  // namespace

extern "C" {

Q38Model *q38_model_open_gguf(const char *path, uint32_t context_length)
{
    if (!path || context_length == 0) return nullptr;
    if (context_length > q38::kMaxAttentionContext) {
        report("context length above 524256 positions");
        return nullptr;
    }
    Q38Model *m = new Q38Model();
    m->context_length = context_length;
    bool ok = m->gguf.open(path) && validate_base(m) &&
              hip_ok(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "stream") &&
              hip_ok(hipStreamCreateWithFlags(&m->copy_stream, hipStreamNonBlocking), "stream") &&
              hip_ok(hipEventCreateWithFlags(&m->logits_ready, hipEventDisableTiming), "event");
    ok = ok && (m->grid = q38::iq1m_grid_for_current_device()) != nullptr;
    ok = ok && upload(m->gguf, &m->weights);
    const uint8_t *base = static_cast<const uint8_t *>(m->weights);
    ok = ok && bind_tensor(m->gguf, base, "token_embd.weight", &m->embedding) &&
         bind_tensor(m->gguf, base, "output_norm.weight", &m->output_norm) && bind_tensor(m->gguf, base, "output.weight", &m->output);
    for (uint32_t layer = 0; ok && layer < kLayers; ++layer) ok = bind_layer(&m->layers[layer], m->gguf, base, (int)layer);
    ok = ok && expect(m->embedding, "token_embd.weight", kHidden, kVocab, false) &&
         expect(m->output_norm, "output_norm.weight", kHidden, 0, true) &&
         expect(m->output, "output.weight", kHidden, kVocab, false);
    uint32_t blocks = 0;
    if (ok && m->gguf.get_u32("qwen35.block_count", &blocks) && blocks == kTotalLayers)
        ok = bind_mtp(m, m->gguf, base);
    ok = ok && build_tiled(m, 0, kLayers, false, &m->tiled_weights) &&
         (!m->mtp_weights_loaded || build_tiled(m, kLayers, kLayers + 1, true, &m->tiled_mtp));
    ok = ok && allocate_state(m) && clear_state(m) && setup_float_inputs(m);
    if (ok && !q38::configure_attention((int)context_length)) ok = report("attention kernel configuration failed");
    if (const char *v = getenv("QWEN38_NO_GRAPHS")) m->graphs_enabled = !(v[0] && strcmp(v, "0") != 0);
    if (!ok) {
        release(m);
        return nullptr;
    }
    return m;
}

int q38_model_attach_mtp_gguf(Q38Model *m, const char *path)
{
    if (!m || !path || m->position != 0 || m->mtp_position != 0 || m->mtp_enabled || m->mtp_weights_loaded ||
        m->mtp_gguf.fd >= 0)
        return 0;
    const bool ok = m->mtp_gguf.open(path) && upload(m->mtp_gguf, &m->mtp_weights) &&
                    bind_mtp(m, m->mtp_gguf, static_cast<const uint8_t *>(m->mtp_weights)) &&
                    build_tiled(m, kLayers, kLayers + 1, true, &m->tiled_mtp) && setup_float_inputs(m);
    if (!ok) {
        m->layers[kLayers] = Layer();
        m->mtp_embedding = m->mtp_output = m->eh_proj = m->enorm = m->hnorm = m->shared_head_norm = DevTensor();
        m->mtp_weights_loaded = false;
        if (m->mtp_weights) (void)hipFree(m->mtp_weights);
        m->mtp_weights = nullptr;
        if (m->tiled_mtp) (void)hipFree(m->tiled_mtp);
        m->tiled_mtp = nullptr;
        m->mtp_gguf.close();
        return 0;
    }
    return 1;
}

void q38_model_close(Q38Model *m) { release(m); }

void q38_model_reset(Q38Model *m)
{
    if (!m) return;
    (void)clear_state(m);
    m->position = 0;
    m->mtp_position = 0;
    m->last_logits = nullptr;
}

int q38_model_forward_token(Q38Model *m, uint32_t token, const float **logits)
{
    begin_call();
    if (!m || !logits || token >= kVocab || m->position >= m->context_length) return 0;
    if (!forward_device(m, token) || !logits_to_host(m, m->logits)) return 0;
    *logits = m->host_logits;
    return 1;
}

int q38hip_model_sample(Q38Model *m, uint64_t *state, float temperature, float top_p, float presence_penalty,
                        uint32_t top_k, const uint8_t *presence, uint32_t presence_size, uint32_t *token)
{
    begin_call();
    if (!m || !state || !token || !m->last_logits) return 0;
    return sample_row(m, m->last_logits, {state, temperature, top_p, presence_penalty, top_k, presence, presence_size},
                      token) ? 1 : 0;
}

int q38hip_model_forward_sample(Q38Model *m, uint32_t token_id, uint64_t *state, float temperature, float top_p,
                                float presence_penalty, uint32_t top_k, const uint8_t *presence,
                                uint32_t presence_size, uint32_t *next_token)
{
    begin_call();
    if (!m || !state || !next_token || token_id >= kVocab || m->position >= m->context_length) return 0;
    if (!forward_device(m, token_id)) return 0;
    return sample_row(m, m->logits, {state, temperature, top_p, presence_penalty, top_k, presence, presence_size},
                      next_token) ? 1 : 0;
}

int q38_model_forward_token_layers(Q38Model *m, uint32_t token, uint32_t layer_count, float *hidden_out)
{
    begin_call();
    if (!m || !hidden_out || token >= kVocab || layer_count > kLayers || m->position >= m->context_length) return 0;
    m->last_logits = nullptr;
    write_params(m, kParamTarget, m->position);
    if (!upload_tokens(m, &token, 1, m->tokens) || !flush_params(m)) return 0;
    const Step s = step_of(m, kParamTarget, m->tokens);
    embed(m, m->embedding, s.tokens, 1);
    trace(m, "model.input_embed", -1, m->hidden, kHidden);
    m->pending_branch = false;
    for (uint32_t layer = 0; layer < layer_count; ++layer)
        if (!layer_rows(m, s, (int)layer, 1)) return 0;
    flush_branch(m, 1);
    if (!launches_ok() || !hip_ok(hipMemcpyAsync(hidden_out, m->hidden, kHidden * sizeof(float), hipMemcpyDeviceToHost, m->stream),
                "hidden download") ||
        !hip_ok(hipStreamSynchronize(m->stream), "hidden download"))
        return 0;
    advance_slots(m, 1, layer_count);
    ++m->position;
    return 1;
}

int q38_model_prefill(Q38Model *m, const uint32_t *tokens, uint32_t count, const float **logits)
{
    begin_call();
    if (!m || !tokens || !count || !logits || count > m->context_length - m->position) return 0;
    for (uint32_t i = 0; i < count; ++i)
        if (tokens[i] >= kVocab) return 0;
    m->last_logits = nullptr;
    const uint32_t base = m->position;
    /* batches of up to prefill_rows tokens through all blocks
     * (q38_model_prefill, qwen38_model.c:1519-1560): every row's arithmetic
     * is independent of the batching, and state advances in token order */
    for (uint32_t done = 0; done < count; done += m->prefill_rows) {
        const uint32_t n = std::min(m->prefill_rows, count - done);
        const bool last = done + n == count;
        write_params(m, kParamTarget, base + done);
        write_params(m, kParamCatchup, base + done);
        if (!upload_tokens(m, tokens + done, n, m->tokens) || !flush_params(m)) return 0;
        const Step st = step_of(m, kParamTarget, m->tokens);
        if (!target_rows(m, st, n, last ? 1 : 0)) return 0;
        if (m->mtp_enabled && !mtp_catchup(m, step_of(m, kParamCatchup, m->tokens), n)) return 0;
        /* the pinned staging is rewritten by the next chunk */
        if (!hip_ok(hipStreamSynchronize(m->stream), "prefill")) return 0;
        advance_slots(m, n);
        if (m->mtp_enabled) m->mtp_position = base + done + n;
    }
    if (!logits_to_host(m, m->logits)) return 0;
    m->position = base + count;
    *logits = m->host_logits;
    return 1;
}

int q38_model_enable_mtp(Q38Model *m)
{
    if (!m || m->position != 0 || m->mtp_position != 0) return 0;
    if (!m->mtp_weights_loaded) {
        fprintf(stderr, "qwen38: MTP weights are unavailable; attach the MTP GGUF first\n");
        return 0;
    }
    if (!m->ck_mtp_hidden && !dalloc(&m->ck_mtp_hidden, kHidden)) return 0;
    m->mtp_enabled = true;
    return 1;
}

int q38_model_mtp_forward(Q38Model *m, uint32_t token, const float **logits)
{
    begin_call();
    if (!m || !m->mtp_enabled || !logits || token >= kVocab || m->mtp_position >= m->context_length) return 0;
    m->last_logits = nullptr;
    write_params(m, kParamDraft0, m->mtp_position);
    if (!upload_tokens(m, &token, 1, m->drafts) || !flush_params(m)) return 0;
    const Step s = step_of(m, kParamDraft0, m->drafts);
    if (!run_step(m, graph_key(kGraphDraft, 0, 1), [&] { return mtp_step(m, s); }) ||
        !logits_to_host(m, m->logits))
        return 0;
    ++m->mtp_position;
    *logits = m->host_logits;
    return 1;
}

/* q38_model_speculative_greedy (qwen38_model.c:1614-1714).
 *
 * Device-side chain: m->drafts[0] = token; MTP step i embeds m->drafts[i]
 * and its argmax becomes m->drafts[i + 1], so the verify rows
 * [token, d0 .. d_{n-2}] are m->drafts[0 .. n) without a round trip.  All
 * `draft_count` drafts run; if one equals stop_token the reference stops
 * there (n = its index + 1), and the extra drafts only wrote MTP cache
 * entries beyond the positions catch-up rewrites, which are overwritten
 * before they are read.  The verify batch runs over all drafts too; the
 * acceptance is decided over its first n rows exactly as the reference
 * does over its n (rows are independent, row t only sees rows < t). */
int q38_model_speculative_greedy(Q38Model *m, uint32_t token, uint32_t stop_token, uint32_t draft_count,
                                 uint32_t *accepted_tokens, uint32_t *accepted_count, const float **next_logits)
{
    begin_call();
    if (!m || !m->mtp_enabled || !accepted_tokens || !accepted_count || !next_logits || token >= kVocab ||
        draft_count == 0 || m->position != m->mtp_position || draft_count > m->context_length - m->position)
        return 0;
    const uint32_t k = draft_count;
    m->last_logits = nullptr;
    if (!checkpoint(m)) return 0;
    if (k > kBatch) {
        std::vector<uint32_t> accepted;
        const float *row = nullptr;
        if (!speculative_chunked(m, token, stop_token, k, &accepted, &row) || !logits_to_host(m, row)) {
            m->last_logits = nullptr;
            restore_target(m);
            (void)restore_mtp(m);
            (void)hipStreamSynchronize(m->stream);
            return 0;
        }
        for (size_t i = 0; i < accepted.size(); ++i) accepted_tokens[i] = accepted[i];
        *accepted_count = (uint32_t)accepted.size();
        *next_logits = m->host_logits;
        return 1;
    }
    for (uint32_t i = 0; i < k; ++i) write_params(m, kParamDraft0 + i, m->ck_mtp_position + i);
    write_params(m, kParamTarget, m->ck_position);
    write_params(m, kParamCatchup, m->ck_mtp_position);
    m->host_params[(size_t)kParamTarget * kParamWords + kParamStopWord] = stop_token;
    if (!upload_tokens(m, &token, 1, m->drafts) || !flush_params(m)) return 0;

    /* one graph per draft count: the k MTP drafts (draft i + 1 is the argmax
     * of draft i's logits), the verify rows m->drafts[0 .. k) with their
     * per-row argmax into m->targets, the device acceptance (rows up to the
     * first draft equal to the stop token, as the reference checks), the
     * returned logits row (row consumed - 1) gathered into m->logits_stage,
     * and the MTP catch-up.
     *
     * On a rejection the reference restores its checkpoint and replays the
     * consumed rows (qwen38_model.c:1684-1691).  Every row of the verify
     * batch computed exactly what the replay would (rows are independent in
     * the GEMMs and the recurrent state advanced row by row), so the state
     * after the consumed rows is already in slot checkpoint + consumed, their
     * K/V entries are in the caches, and the last consumed row's logits are
     * row consumed - 1 of the batch; entries of the rejected rows are never
     * read before being overwritten.  The MTP catch-up runs over all k rows
     * from the checkpointed MTP hidden state (rows past the consumed ones
     * only write MTP cache entries past the positions the next drafts
     * rewrite before reading them) and continues the MTP hidden state from
     * row consumed - 1, read on the device: one host wait per call. */
    const Step sv = step_of(m, kParamTarget, m->drafts);
    const Step sc = step_of(m, kParamCatchup, m->drafts);
    const uint32_t *stop = m->params + (size_t)kParamTarget * kParamWords + kParamStopWord;
    uint32_t *hw = m->host_words;
    bool ok = run_step(m, graph_key(kGraphTransaction, k), [&] {
                  for (uint32_t i = 0; i < k; ++i) {
                      if (!mtp_step(m, step_of(m, kParamDraft0 + i, m->drafts + i))) return false;
                      q38::launch_argmax(m->logits, kVocab, 1, m->argmax_pv, m->argmax_pi, m->drafts + i + 1,
                                         m->stream);
                  }
                  if (!target_rows(m, sv, k, k) ||
                      !q38::launch_verify_tail(m->logits, kVocab, k, m->argmax_pv, m->argmax_pi, m->targets,
                                               m->drafts + 1, stop, m->accept, m->logits_stage, m->stream))
                      return false;
                  return mtp_catchup(m, sc, k, m->ck_mtp_hidden, m->accept);
              }) &&
         /* then the acceptance words and the logits row: host words [64..)
          * mirror m->words (drafts at 64, targets at 80, acceptance at 96) */
         hip_ok(hipMemcpyAsync(hw + 64, m->words, 48 * sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream),
                "acceptance") &&
         hip_ok(hipMemcpyAsync(m->host_logits, m->logits_stage, kVocab * sizeof(float), hipMemcpyDeviceToHost,
                               m->stream), "logits download") &&
         hip_ok(hipStreamSynchronize(m->stream), "catch-up");
    if (!ok) {
        restore_target(m);
        (void)restore_mtp(m);
        (void)hipStreamSynchronize(m->stream);
        return 0;
    }
    const uint32_t consumed = hw[96];
    if (consumed == 0 || consumed > k) {
        restore_target(m);
        (void)restore_mtp(m);
        (void)hipStreamSynchronize(m->stream);
        return report("acceptance result out of range");
    }
    uint32_t accepted[kBatch];
    for (uint32_t i = 0; i < consumed; ++i) accepted[i] = hw[99 + i];
    restore_target(m, consumed);
    m->mtp_position = m->ck_mtp_position + consumed;
    m->last_logits = m->logits + (size_t)(consumed - 1) * kVocab;
    for (uint32_t i = 0; i < consumed; ++i) accepted_tokens[i] = accepted[i];
    *accepted_count = consumed;
    *next_logits = m->host_logits;
    return 1;
}

/* Device time of one block over `rows` verify rows and of the verify tail
 * (argmax, acceptance, row gather), each captured once as a graph and
 * replayed `repeats` times between two events on the model's stream.  The
 * block reads the hidden rows left in the scratch (their values do not
 * change the work) and runs at positions position .. position + rows - 1;
 * nothing the next call reads is changed: position and slots stay, the
 * recurrent slots after the current one and the cache entries at and after
 * `position` are rewritten by the next step before they are read. */
int q38hip_model_time_block(Q38Model *m, uint32_t layer, uint32_t rows, uint32_t repeats, float *block_us,
                            float *tail_us)
{
    begin_call();
    if (!m || layer >= kLayers || rows == 0 || rows > kBatch || repeats == 0 || !block_us || !tail_us ||
        rows > m->context_length - m->position)
        return 0;
    write_params(m, kParamTarget, m->position);
    m->host_params[(size_t)kParamTarget * kParamWords + kParamStopWord] = 0xFFFFFFFFu;
    const uint32_t zeros[kBatch] = {0};
    if (!upload_tokens(m, zeros, rows, m->tokens) ||
        !hip_ok(hipMemcpyAsync(m->drafts + 1, m->tokens, rows * sizeof(uint32_t), hipMemcpyDeviceToDevice,
                               m->stream), "time block") ||
        !flush_params(m) || !hip_ok(hipStreamSynchronize(m->stream), "time block"))
        return 0;
    const Step s = step_of(m, kParamTarget, m->tokens);
    const uint32_t *stop = m->params + (size_t)kParamTarget * kParamWords + kParamStopWord;
    auto block = [&] {
        m->pending_branch = false;
        const bool ok = layer_rows(m, s, (int)layer, rows);
        m->pending_branch = false;
        return ok;
    };
    auto tail = [&] {
        return q38::launch_verify_tail(m->logits, kVocab, rows, m->argmax_pv, m->argmax_pi, m->targets, m->drafts + 1,
                                       stop, m->accept, m->logits_stage, m->stream);
    };
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool ok = hip_ok(hipEventCreate(&e0), "event") && hip_ok(hipEventCreate(&e1), "event");
    float *outs[2] = {block_us, tail_us};
    for (int part = 0; ok && part < 2; ++part) {
        /* one eager run (first-use allocations and module loads), then the graph */
        ok = (part == 0 ? block() : tail()) && launches_ok();
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        ok = ok && hip_ok(hipStreamSynchronize(m->stream), "time block") &&
             hip_ok(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal), "graph capture");
        if (ok) {
            const bool body = (part == 0 ? block() : tail()) && launches_ok();
            ok = hip_ok(hipStreamEndCapture(m->stream, &graph), "graph capture") && body;
        }
        ok = ok && hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate");
        if (graph) (void)hipGraphDestroy(graph);
        /* warm replays, then the timed ones */
        for (uint32_t i = 0; ok && i < 3; ++i) ok = hip_ok(hipGraphLaunch(exec, m->stream), "graph launch");
        ok = ok && hip_ok(hipEventRecord(e0, m->stream), "event");
        for (uint32_t i = 0; ok && i < repeats; ++i) ok = hip_ok(hipGraphLaunch(exec, m->stream), "graph launch");
        ok = ok && hip_ok(hipEventRecord(e1, m->stream), "event") && hip_ok(hipEventSynchronize(e1), "event");
        float ms = 0.0f;
        ok = ok && hip_ok(hipEventElapsedTime(&ms, e0, e1), "event");
        if (ok) *outs[part] = ms * 1e3f / (float)repeats;
        if (exec) (void)hipGraphExecDestroy(exec);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return ok ? 1 : 0;
}

uint32_t q38_model_vocab_size(const Q38Model *m) { return m ? kVocab : 0; }
uint32_t q38_model_position(const Q38Model *m) { return m ? m->position : 0; }
uint32_t q38_model_context_length(const Q38Model *m) { return m ? m->context_length : 0; }

}  // extern "C"
