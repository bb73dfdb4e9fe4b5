/* C ABI of the full-attention decode core (declared in include/q38hip.h):
 * the kernels the engine runs for a full-attention block, callable on their
 * own for kernel-level parity tests and external callers. */
#include <hip/hip_runtime.h>

#include <vector>

#include "q38hip.h"
#include "q38_kernels.h"

namespace {

constexpr uint32_t kQGDim = 12288, kQDim = 6144, kKVDim = 1024, kHeads = 24;

struct Buffers {
    std::vector<void *> owned;
    ~Buffers()
    {
        for (void *p : owned) (void)hipFree(p);
    }
    template <typename T>
    T *get(size_t count)
    {
        void *p = nullptr;
        if (hipMalloc(&p, count * sizeof(T)) != hipSuccess) return nullptr;
        owned.push_back(p);
        return static_cast<T *>(p);
    }
};

}  // namespace

extern "C" int q38hip_attention_rows(float *attention, Q38Q8KBlock *attention_q8k, const float *q_and_gate,
                                     const float *key, const float *value, uint64_t in_stride, const float *q_norm,
                                     const float *k_norm, float *key_cache, float *value_cache,
                                     uint32_t context_length, uint32_t position, uint32_t rows, void *stream)
{
    if (!attention || !q_and_gate || !key || !value || !q_norm || !k_norm || !key_cache || !value_cache || !rows ||
        !context_length)
        return q38::abi_fail("bad attention arguments");
    if (in_stride < kKVDim || (rows > 1 && in_stride < kQGDim)) return q38::abi_fail("row stride too small");
    if ((uint64_t)position + rows > context_length) return q38::abi_fail("position + rows beyond the context");
    if (context_length > q38::kMaxAttentionContext) return q38::abi_fail("context length above 524256 positions");
    hipStream_t s = static_cast<hipStream_t>(stream);
    /* drain the caller's earlier work on the stream: the buffers below are
     * released before return */
    if (hipStreamSynchronize(s) != hipSuccess) return q38::abi_fail("stream synchronisation failed");
    Buffers buf;
    float *rope = buf.get<float>((size_t)context_length * 64);
    float *q_buf = buf.get<float>((size_t)rows * kQDim);
    float *scores = buf.get<float>((size_t)rows * kHeads * context_length);
    uint8_t *q_out = attention_q8k ? reinterpret_cast<uint8_t *>(attention_q8k)
                                   : buf.get<uint8_t>((size_t)rows * kHeads * sizeof(Q38Q8KBlock));
    uint32_t *pos = buf.get<uint32_t>(1);
    if (!rope || !q_buf || !scores || !q_out || !pos) return q38::abi_fail("device allocation failed");
    std::vector<float> table((size_t)context_length * 64);
    q38::rope_table_host(table.data(), context_length);
    if (hipMemcpyAsync(rope, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(pos, &position, sizeof(position), hipMemcpyHostToDevice, s) != hipSuccess ||
        !q38::configure_attention((int)context_length))
        return q38::abi_fail("attention set-up failed");
    q38::launch_attention(attention, q_out, q_buf, q_and_gate, key, value, (long long)in_stride, q_norm, k_norm, rope,
                          key_cache, value_cache, scores, (int)context_length, pos, (int)rows, s);
    const hipError_t launched = hipGetLastError();
    const hipError_t done = hipStreamSynchronize(s);
    if (launched != hipSuccess || done != hipSuccess) return q38::abi_fail("attention kernels failed");
    return 1;
}
