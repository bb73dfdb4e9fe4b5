/* Token sampler on the device: q38_sample (src/qwen38/qwen38_sampler.c:51-119)
 * over a logits row that stays in HBM, so sampled decoding needs no logits
 * download.
 *
 * The reference's arithmetic, step by step:
 *  - adjusted logit = logit - presence_penalty for observed tokens
 *    (:38-46), plain fp32 subtraction;
 *  - temperature <= 0 or top_k <= 1: the first maximum of the adjusted
 *    logits by a strict > scan from index 0 (:55-63), so NaN never wins
 *    unless it is at index 0, where it stays;
 *  - otherwise the top count = min(top_k, vocabulary) candidates by
 *    insertion (:64-82): a candidate enters with a logit above the current
 *    last one (initially -FLT_MAX, id 0), equal logits keep the lower id
 *    first, so the list is the count largest logits above -FLT_MAX ordered
 *    by (logit descending, id ascending), padded with (0, -FLT_MAX); then
 *    p_i = expf((l_i - l_0) / T) with a sequential fp32 total, the
 *    smallest prefix whose sequential cumulative p_i / total reaches top_p
 *    (top_p outside (0, 1) means 1), its sequential total, one
 *    xorshift64* draw (:12-20) as (double)(r >> 11) * 2^-53, the target
 *    (float)unit * retained_total and the first candidate whose running
 *    sum exceeds it (:84-115).
 *
 * Device method: each workgroup selects the count best candidates of a
 * 4096-logit chunk (count rounds of a workgroup-wide best-of with the
 * reference's order); one workgroup merges the chunks' lists the same way
 * and one thread runs the probability arithmetic (expf is the C library's
 * function restated in q38_libm.h, division correctly rounded).  With a NaN
 * among the adjusted logits the insertion order matters (a NaN enters the
 * last slot), so then that thread runs the reference's insertion loop
 * itself, over the whole row.
 */
#include <cfloat>

#include "q38_device.h"
#include "q38_kernels.h"
#include "q38_libm.h"

namespace q38 {

namespace {

constexpr int kSampleThreads = 256;
constexpr int kSamplePerThread = 16;
constexpr int kSampleChunk = kSampleThreads * kSamplePerThread;
static_assert((size_t)kMaxSampleChunks * kSampleChunk >= kMaxSampleVocab, "chunk table");
constexpr uint32_t kNone = 0xffffffffu;

__device__ __forceinline__ float adjusted_logit(const float *logits, const uint8_t *presence, uint32_t presence_size,
                                                float penalty, uint32_t id)
{
    const float v = logits[id];
    if (penalty == 0.0f || !presence || id >= presence_size || !presence[id]) return v;
    return __fsub_rn(v, penalty);
}

/* does (va, ia) come before (vb, ib)?  higher logit first, lower id among
 * equal logits; (x, kNone) is an empty slot and comes last */
__device__ __forceinline__ bool ahead(float va, uint32_t ia, float vb, uint32_t ib)
{
    if (ia == kNone) return false;
    if (ib == kNone) return true;
    return va > vb || (va == vb && ia < ib);
}

/* the workgroup's best (value, id) among the threads' candidates, returned
 * to every thread */
__device__ void block_best(float &bv, uint32_t &bi)
{
    __shared__ float sv[kSampleThreads / 64];
    __shared__ uint32_t si[kSampleThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        if (ahead(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int w = 1; w < kSampleThreads / 64; ++w)
        if (ahead(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
}

/* pass 1: the `count` best eligible logits of each 4096-logit chunk, in
 * order, then empty slots.  Greedy (count 1): every non-NaN logit is
 * eligible; sampling: logits above -FLT_MAX (a NaN sets the chunk's flag). */
__global__ __launch_bounds__(kSampleThreads) void sample_select_kernel(
    const float *__restrict__ logits, uint32_t vocab, const uint8_t *__restrict__ presence, uint32_t presence_size,
    float penalty, uint32_t count, int greedy, float *__restrict__ cand_v, uint32_t *__restrict__ cand_i,
    uint32_t *__restrict__ nan_flags)
{
    const uint32_t chunk = blockIdx.x;
    float v[kSamplePerThread];
    uint32_t live = 0;   /* bit i: element i is eligible and not yet taken */
    bool nan_seen = false;
#pragma unroll
    for (int i = 0; i < kSamplePerThread; ++i) {
        const uint32_t id = chunk * kSampleChunk + i * kSampleThreads + threadIdx.x;
        v[i] = 0.0f;
        if (id < vocab) {
            v[i] = adjusted_logit(logits, presence, presence_size, penalty, id);
            const bool nan = v[i] != v[i];
            nan_seen |= nan;
            const bool eligible = greedy ? !nan : v[i] > -FLT_MAX;
            if (eligible) live |= 1u << i;
        }
    }
    const bool any_nan = __syncthreads_or(nan_seen);
    if (threadIdx.x == 0) nan_flags[chunk] = any_nan ? 1u : 0u;
    for (uint32_t r = 0; r < count; ++r) {
        float bv = 0.0f;
        uint32_t bi = kNone, slot = 0;
#pragma unroll
        for (int i = 0; i < kSamplePerThread; ++i) {
            const uint32_t id = chunk * kSampleChunk + i * kSampleThreads + threadIdx.x;
            if (((live >> i) & 1u) && ahead(v[i], id, bv, bi)) { bv = v[i]; bi = id; slot = i; }
        }
        const uint32_t mine = bi;
        block_best(bv, bi);
        if (threadIdx.x == 0) {
            cand_v[(size_t)chunk * count + r] = bv;
            cand_i[(size_t)chunk * count + r] = bi;
        }
        if (bi == kNone) {
            for (uint32_t q = r + 1 + threadIdx.x; q < count; q += kSampleThreads) cand_i[(size_t)chunk * count + q] = kNone;
            break;
        }
        if (mine == bi) live &= ~(1u << slot);
    }
}

/* xorshift64* (qwen38_sampler.c:12-20); the host advances the caller's
 * state the same way (one step per sampling call) */
__device__ __forceinline__ uint64_t next_random(uint64_t &state)
{
    uint64_t value = state;
    value ^= value >> 12;
    value ^= value << 25;
    value ^= value >> 27;
    state = value;
    return value * 2685821657736338717ull;
}

/* pass 2, one workgroup: merge the chunks' lists, then the probabilities,
 * top-p and the draw in one thread.  cl/ci hold count entries in LDS. */
__global__ __launch_bounds__(kSampleThreads) void sample_final_kernel(
    const float *__restrict__ logits, uint32_t vocab, const uint8_t *__restrict__ presence, uint32_t presence_size,
    float penalty, float temperature, float top_p, uint32_t count, int greedy, uint32_t nchunks,
    const float *__restrict__ cand_v, const uint32_t *__restrict__ cand_i, const uint32_t *__restrict__ nan_flags,
    uint64_t state, uint32_t *__restrict__ token_out)
{
    __shared__ float cl[kMaxSampleTopK];
    __shared__ uint32_t ci[kMaxSampleTopK];
    __shared__ float prob[kMaxSampleTopK];
    bool nan_seen = false;
    for (uint32_t c = threadIdx.x; c < nchunks; c += kSampleThreads) nan_seen |= nan_flags[c] != 0u;
    const bool any_nan = __syncthreads_or(nan_seen);

    if (greedy) {
        /* the best of the chunks' winners; a NaN at index 0 keeps index 0
         * (the scan's every comparison with it is false), as does a row
         * with no non-NaN logit */
        float bv = 0.0f;
        uint32_t bi = kNone;
        for (uint32_t c = threadIdx.x; c < nchunks; c += kSampleThreads)
            if (ahead(cand_v[c], cand_i[c], bv, bi)) { bv = cand_v[c]; bi = cand_i[c]; }
        block_best(bv, bi);
        if (threadIdx.x == 0) {
            const float first = adjusted_logit(logits, presence, presence_size, penalty, 0);
            token_out[0] = (bi == kNone || first != first) ? 0u : bi;
        }
        return;
    }

    if (any_nan) {
        /* the reference's insertion loop (qwen38_sampler.c:64-82) */
        if (threadIdx.x == 0) {
            for (uint32_t i = 0; i < count; ++i) { ci[i] = 0; cl[i] = -FLT_MAX; }
            for (uint32_t id = 0; id < vocab; ++id) {
                const float logit = adjusted_logit(logits, presence, presence_size, penalty, id);
                if (logit <= cl[count - 1]) continue;
                uint32_t slot = count - 1;
                while (slot > 0 && logit > cl[slot - 1]) {
                    cl[slot] = cl[slot - 1];
                    ci[slot] = ci[slot - 1];
                    --slot;
                }
                ci[slot] = id;
                cl[slot] = logit;
            }
        }
    } else {
        /* merge of the chunks' sorted lists: count rounds of best-of over
         * the list heads (a chunk is its ids / 4096) */
        __shared__ uint32_t head[kMaxSampleChunks];
        for (uint32_t c = threadIdx.x; c < nchunks; c += kSampleThreads) head[c] = 0;
        __syncthreads();
        for (uint32_t r = 0; r < count; ++r) {
            float bv = 0.0f;
            uint32_t bi = kNone;
            for (uint32_t c = threadIdx.x; c < nchunks; c += kSampleThreads) {
                const uint32_t h = head[c];
                if (h < count && ahead(cand_v[(size_t)c * count + h], cand_i[(size_t)c * count + h], bv, bi)) {
                    bv = cand_v[(size_t)c * count + h];
                    bi = cand_i[(size_t)c * count + h];
                }
            }
            block_best(bv, bi);
            if (threadIdx.x == 0) {
                ci[r] = bi == kNone ? 0u : bi;
                cl[r] = bi == kNone ? -FLT_MAX : bv;
                if (bi != kNone) ++head[bi / kSampleChunk];
            }
            __syncthreads();
        }
    }
    __syncthreads();
    if (threadIdx.x != 0) return;

    /* qwen38_sampler.c:84-115 */
    float total = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        prob[i] = q38_expf(div_rn(__fsub_rn(cl[i], cl[0]), temperature));
        total = __fadd_rn(total, prob[i]);
    }
    float cumulative = 0.0f;
    uint32_t retained = count;
    const float p = top_p > 0.0f && top_p < 1.0f ? top_p : 1.0f;
    for (uint32_t i = 0; i < count; ++i) {
        cumulative = __fadd_rn(cumulative, div_rn(prob[i], total));
        if (cumulative >= p) {
            retained = i + 1;
            break;
        }
    }
    float retained_total = 0.0f;
    for (uint32_t i = 0; i < retained; ++i) retained_total = __fadd_rn(retained_total, prob[i]);
    const double unit = (double)(next_random(state) >> 11) * 0x1.0p-53;
    const float target = __fmul_rn((float)unit, retained_total);
    float running = 0.0f;
    uint32_t selected = ci[retained - 1];
    for (uint32_t i = 0; i < retained; ++i) {
        running = __fadd_rn(running, prob[i]);
        if (target < running) {
            selected = ci[i];
            break;
        }
    }
    token_out[0] = selected;
}

}  // namespace

size_t sample_scratch_bytes(uint32_t vocab, uint32_t top_k)
{
    const size_t chunks = (vocab + kSampleChunk - 1) / kSampleChunk;
    const size_t count = top_k < 1 ? 1 : (top_k < vocab ? top_k : vocab);
    return chunks * count * (sizeof(float) + sizeof(uint32_t)) + chunks * sizeof(uint32_t);
}

const char *check_sample(uint32_t vocab, float temperature, uint32_t top_k)
{
    if (!vocab) return "empty vocabulary";
    if (vocab > kMaxSampleVocab) return "vocabulary above 2^20 tokens";
    const bool greedy = temperature <= 0.0f || top_k <= 1;
    if (!greedy && (top_k < vocab ? top_k : vocab) > kMaxSampleTopK)
        return "more than 1024 sampling candidates (min(top_k, vocabulary))";
    return nullptr;
}

bool launch_sample(uint32_t *token_out, uint64_t *state, const float *logits, uint32_t vocab, const uint8_t *presence,
                   uint32_t presence_size, float temperature, float top_p, float presence_penalty, uint32_t top_k,
                   void *scratch, hipStream_t stream)
{
    if (!token_out || !state || !logits || !scratch || check_sample(vocab, temperature, top_k)) return false;
    /* qwen38_sampler.c:55 */
    const int greedy = temperature <= 0.0f || top_k <= 1;
    const uint32_t count = greedy ? 1u : (top_k < vocab ? top_k : vocab);
    const uint32_t chunks = (vocab + kSampleChunk - 1) / kSampleChunk;
    float *cand_v = static_cast<float *>(scratch);
    uint32_t *cand_i = reinterpret_cast<uint32_t *>(cand_v + (size_t)chunks * count);
    uint32_t *flags = cand_i + (size_t)chunks * count;
    hipLaunchKernelGGL(sample_select_kernel, dim3(chunks), dim3(kSampleThreads), 0, stream, logits, vocab, presence,
                       presence_size, presence_penalty, count, greedy, cand_v, cand_i, flags);
    hipLaunchKernelGGL(sample_final_kernel, dim3(1), dim3(kSampleThreads), 0, stream, logits, vocab, presence,
                       presence_size, presence_penalty, temperature, top_p, count, greedy, chunks, cand_v, cand_i,
                       flags, *state, token_out);
    if (hipGetLastError() != hipSuccess) return false;
    /* the kernel drew from the state as it was; a sampling call advances
     * the caller's copy by one step (q38_random, qwen38_sampler.c:105) */
    if (!greedy) {
        uint64_t s = *state;
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        *state = s;
    }
    return true;
}

}  // namespace q38
