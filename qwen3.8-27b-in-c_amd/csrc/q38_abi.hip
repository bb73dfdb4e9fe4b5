/* C ABI of libq38hip (declared in include/q38hip.h). */
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "q38hip.h"
#include "q38_device.h"
#include "q38_iq1m_grid.inc"
#include "q38_kernels.h"

/* Fixed partials buffer of q38hip_argmax_noalloc: kNoAllocPairs partial
 * maxima (fp32 values, then uint32 indices), 64 KiB on every device the
 * library runs on, held until the process ends.  Host code never uses the
 * array's name as an address: it uses the per-device address that
 * hipGetSymbolAddress returns (g_scratch_ptr below). */
constexpr size_t kNoAllocPairs = 8192;
static __device__ __align__(256) uint32_t scratch[2 * kNoAllocPairs];

namespace {

thread_local std::string g_error;

int fail(const char *message)
{
    g_error = message;
    return 0;
}

/* Per-device constant state: the IQ1_M codebook as 2048 x 8 int8 values
 * (the form the GEMM kernel stages into LDS), a growable argmax
 * partials buffer and the sampler's candidate lists (allocated once, at the
 * largest size the sampler accepts). */
struct DeviceState {
    int8_t *grid = nullptr;
    float *argmax_values = nullptr;
    uint32_t *argmax_index = nullptr;
    size_t argmax_capacity = 0;
    void *sample_scratch = nullptr;
};

std::mutex g_mutex;
std::vector<DeviceState> g_devices;

std::vector<uint32_t *> g_scratch_ptr;

/* device address of `scratch` on the current device, looked up once per
 * device (nullptr on failure) */
uint32_t *noalloc_scratch()
{
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_mutex);
    if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_ptr[device] = static_cast<uint32_t *>(ptr);
    }
    return g_scratch_ptr[device];
}

DeviceState *device_state()
{
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_mutex);
    if ((int)g_devices.size() <= device) g_devices.resize(device + 1);
    DeviceState &s = g_devices[device];
    if (!s.grid) {
        /* 2048 entries of 8 ternary values, then the 4096-entry signed
         * table of the one-token IQ1_M kernel: entry i + 2048 h holds the
         * bytes 8 g + (h ? -1 : 1) of entry i */
        static int8_t host[(2048 + 4096) * 8];
        for (int e = 0; e < 2048; ++e) {
            const uint32_t code = q38_iq1m_grid_codes[e];
            for (int k = 0; k < 8; ++k) {
                const int g = (int)((code >> (2 * k)) & 3u) - 1;
                host[8 * e + k] = (int8_t)g;
                host[8 * (2048 + e) + k] = (int8_t)(8 * g + 1);
                host[8 * (4096 + e) + k] = (int8_t)(8 * g - 1);
            }
        }
        if (hipMalloc(&s.grid, sizeof(host)) != hipSuccess) return nullptr;
        if (hipMemcpy(s.grid, host, sizeof(host), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    }
    return &s;
}

/* the Q8_K-path matrix formats (q38_matrix_type_q8_k, src/qwen38/qwen38_model.c:172-182) */
bool supported_type(uint32_t type) { return q38::format_takes_q8k((int)type); }

/* bytes of `length` elements of `type` (0 for unknown types) */
uint64_t span_bytes(uint32_t type, uint64_t length)
{
    uint32_t e = 0, b = 0;
    if (!q38::format_block_shape((int)type, &e, &b) || length % e) return 0;
    return length / e * b;
}

/* types with a dedicated kernel family (the decode path's formats) */
bool tuned_type(uint32_t type) { return type == q38::kQ4K || type == q38::kQ6K || type == q38::kIQ1M; }

/* Argument checks of q38_tensor_gemm_q8_k (src/qwen38/qwen38_quant.c:2950-2974). */
int check_gemm(const void *output, const void *input, uint32_t batch, uint64_t input_length,
               const Q38GGUFTensor *tensor)
{
    if (!output || !input || !batch || !tensor) return fail("null argument");
    if (tensor->n_dims != 2) return fail("tensor must be 2-D");
    if (tensor->shape[0] != input_length) return fail("tensor width differs from input length");
    if (input_length % Q38_Q8_K_BLOCK_SIZE) return fail("input length is not a multiple of 256");
    if (!supported_type(tensor->type))
        return fail("tensor type is not a Q8_K-path format (Q2_K..Q6_K, IQ1_S, IQ1_M, IQ2_*, IQ3_*, IQ4_*)");
    if (!tensor->data) return fail("tensor has no data");
    if (tensor->shape[1] == 0 || tensor->shape[1] > 0xffffffffull) return fail("bad row count");
    if (input_length / 256 > 0xffffffffull) return fail("input too long");
    return 1;
}

/* tokens of the next launch when `left` tokens remain: at most 8, and never
 * leaving fewer than `min_tokens` for the launch after it */
uint32_t token_chunk(uint32_t left, uint32_t min_tokens)
{
    uint32_t n = left < 8 ? left : 8;
    if (left > n && left - n < min_tokens) n = left - min_tokens;
    return n;
}

struct DeviceBuffer {
    void *ptr = nullptr;
    explicit DeviceBuffer(size_t bytes)
    {
        if (bytes && hipMalloc(&ptr, bytes) != hipSuccess) ptr = nullptr;
    }
    ~DeviceBuffer()
    {
        if (ptr) (void)hipFree(ptr);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
};

}  // namespace

namespace q38 {
/* record an argument error for q38hip_last_error(); returns 0 */
int abi_fail(const char *message) { return fail(message); }

/* device IQ1_M codebook of the current device (uploaded on first use) */
const void *iq1m_grid_for_current_device()
{
    DeviceState *s = device_state();
    return s ? s->grid : nullptr;
}
}  // namespace q38

extern "C" {

const char *q38hip_last_error(void) { return g_error.c_str(); }

int q38hip_synchronize(void)
{
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 1;
}

float q38_f16_to_f32(uint16_t value)
{
    const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    const uint32_t exponent = (value >> 10) & 31u;
    uint32_t mantissa = value & 1023u;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            uint32_t e = 113;
            while (!(mantissa & 0x400u)) { mantissa <<= 1; --e; }
            bits = sign | e << 23 | (mantissa & 0x3ffu) << 13;
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | mantissa << 13;
    } else {
        bits = sign | (exponent + 112u) << 23 | mantissa << 13;
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

int q38hip_quantize_q8_k(Q38Q8KBlock *output, const float *input, uint64_t length, uint32_t rows,
                         void *stream)
{
    if (!output || !input) return fail("null argument");
    if (length % Q38_Q8_K_BLOCK_SIZE) return fail("length is not a multiple of 256");
    const uint64_t blocks = length / Q38_Q8_K_BLOCK_SIZE * rows;
    if (blocks == 0) return 1;
    if (blocks > 0xffffffffull / 4) return fail("input too long");
    q38::launch_quantize(input, reinterpret_cast<uint8_t *>(output), (uint32_t)blocks,
                         static_cast<hipStream_t>(stream));
    return 1;
}

int q38hip_gemm_q8_k(float *output, const Q38Q8KBlock *input, uint32_t batch_size, uint64_t input_length,
                     const Q38GGUFTensor *tensor, void *stream)
{
    if (!check_gemm(output, input, batch_size, input_length, tensor)) return 0;
    DeviceState *state = device_state();
    if (!state) return fail("device initialisation failed");
    /* Any batch size, as the reference (qwen38_quant.c:2950-2956): the
     * kernels take up to 8 tokens per launch and every token's row results
     * are independent of the others in the batch, so consecutive launches
     * over token chunks give the same bits as one. */
    const uint32_t rows = (uint32_t)tensor->shape[1], nb = (uint32_t)(input_length / 256);
    /* IQ1_M prefill batches: one launch of the 256 x 64 matrix-core tiles */
    if (tensor->type == q38::kIQ1M && batch_size >= (uint32_t)q38::kWideMinTokens &&
        q38::launch_gemm_iq1m_wide(batch_size, tensor->data, reinterpret_cast<const uint8_t *>(input), output, rows,
                                   rows, nb, state->grid, static_cast<hipStream_t>(stream)))
        return 1;
    for (uint32_t t0 = 0; t0 < batch_size;) {
        const uint32_t n = token_chunk(batch_size - t0, 1);
        const uint8_t *x = reinterpret_cast<const uint8_t *>(input) + (size_t)t0 * nb * sizeof(Q38Q8KBlock);
        const bool ok = tuned_type(tensor->type)
                            ? q38::launch_gemm((int)tensor->type, (int)n, tensor->data, x, output + (size_t)t0 * rows,
                                               rows, nb, state->grid, static_cast<hipStream_t>(stream))
                            : q38::launch_gemm_format((int)tensor->type, (int)n, tensor->data, x,
                                                      output + (size_t)t0 * rows, rows, rows, nb, state->grid,
                                                      static_cast<hipStream_t>(stream));
        if (!ok) return fail("unsupported GEMM configuration");
        t0 += n;
    }
    return 1;
}

int q38hip_gemm_f32(float *output, const float *input, uint32_t batch_size, uint64_t input_length,
                    const Q38GGUFTensor *tensor, void *stream)
{
    /* argument checks of q38_tensor_gemm_f32 (qwen38_quant.c:2928-2936) */
    if (!output || !input || !batch_size || !tensor || tensor->n_dims != 2 || tensor->shape[0] != input_length)
        return fail("bad float GEMM arguments");
    if (!span_bytes(tensor->type, input_length) || !input_length) return fail("unsupported tensor type or width");
    if (!tensor->data) return fail("tensor has no data");
    if (tensor->shape[1] == 0 || tensor->shape[1] > 0xffffffffull || input_length > 0xffffffffull)
        return fail("bad tensor shape");
    if (!device_state()) return fail("device initialisation failed");
    const uint32_t rows = (uint32_t)tensor->shape[1];
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (!q38::format_row_decodable((int)tensor->type)) {
        /* the reference's float dot has no case for this type: NaN rows */
        q38::launch_fill_f32(output, (uint64_t)batch_size * rows, __builtin_nanf(""), s);
        return 1;
    }
    for (uint32_t t0 = 0; t0 < batch_size;) {
        const uint32_t n = std::min<uint32_t>(4, batch_size - t0);
        if (!q38::launch_gemm_float((int)tensor->type, (int)n, tensor->data, input + (size_t)t0 * input_length,
                                    output + (size_t)t0 * rows, rows, rows, (uint32_t)input_length, s))
            return fail("unsupported float GEMM configuration");
        t0 += n;
    }
    return 1;
}

int q38hip_row_f32(float *output, const Q38GGUFTensor *tensor, uint64_t first_row, uint32_t row_count, void *stream)
{
    /* argument checks of q38_tensor_row_f32 (qwen38_quant.c:3185-3194) */
    if (!output || !tensor || tensor->n_dims != 2 || !row_count || first_row >= tensor->shape[1] ||
        row_count > tensor->shape[1] - first_row)
        return fail("bad row arguments");
    const uint64_t width = tensor->shape[0];
    if (!span_bytes(tensor->type, width) || width > 0xffffffffull || tensor->shape[1] > 0xffffffffull)
        return fail("unsupported tensor type or width");
    if (!tensor->data) return fail("tensor has no data");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (!q38::format_row_decodable((int)tensor->type)) {
        q38::launch_fill_f32(output, (uint64_t)row_count * width, __builtin_nanf(""), s);
        return 1;
    }
    return q38::launch_row_decode((int)tensor->type, tensor->data, nullptr, (uint32_t)first_row, row_count,
                                  (uint32_t)tensor->shape[1], output, (uint32_t)width, s)
               ? 1
               : fail("row decode launch failed");
}

uint64_t q38hip_tiled_q4k_bytes(uint32_t rows, uint64_t input_length)
{
    if (!rows || !input_length || input_length % Q38_Q8_K_BLOCK_SIZE || input_length / 256 > 0xffffffffull) return 0;
    return q38::tiled_q4k_bytes(rows, (uint32_t)(input_length / 256));
}

int q38hip_repack_q4k_tiles(void *tiled, const void *q4k_rows, uint32_t rows, uint64_t input_length, void *stream)
{
    if (!tiled || !q4k_rows || !rows) return fail("null argument");
    if (!input_length || input_length % Q38_Q8_K_BLOCK_SIZE || input_length / 256 > 0xffffffffull)
        return fail("input length is not a positive multiple of 256");
    if (!device_state()) return fail("device initialisation failed");
    return q38::launch_repack_q4k_tiles(static_cast<uint8_t *>(tiled), static_cast<const uint8_t *>(q4k_rows), rows,
                                        (uint32_t)(input_length / 256), static_cast<hipStream_t>(stream))
               ? 1
               : fail("repack launch failed (tiled copy must be 16-byte aligned)");
}

uint64_t q38hip_tiled_iq1m_bytes(uint32_t rows, uint64_t input_length)
{
    if (!rows || !input_length || input_length % Q38_Q8_K_BLOCK_SIZE || input_length / 256 > 0xffffffffull) return 0;
    return q38::tiled_iq1m_bytes(rows, (uint32_t)(input_length / 256));
}

int q38hip_repack_iq1m_tiles(void *tiled, const void *iq1m_rows, uint32_t rows, uint64_t input_length, void *stream)
{
    if (!tiled || !iq1m_rows || !rows) return fail("null argument");
    if (!input_length || input_length % Q38_Q8_K_BLOCK_SIZE || input_length / 256 > 0xffffffffull)
        return fail("input length is not a positive multiple of 256");
    if (!device_state()) return fail("device initialisation failed");
    return q38::launch_repack_iq1m_tiles(static_cast<uint8_t *>(tiled), static_cast<const uint8_t *>(iq1m_rows),
                                         rows, (uint32_t)(input_length / 256), static_cast<hipStream_t>(stream))
               ? 1
               : fail("repack launch failed (tiled copy must be 8-byte aligned)");
}

int q38hip_gemm_q8_k_iq1m_tiled(float *output, const Q38Q8KBlock *input, uint32_t batch_size, uint64_t input_length,
                                const void *tiled, uint32_t rows, void *stream)
{
    if (!output || !input || !tiled || !rows) return fail("null argument");
    if (batch_size < 1 || batch_size > 8) return fail("batch_size must be 1..8");
    DeviceState *state = device_state();
    if (!state) return fail("device initialisation failed");
    if (input_length % Q38_Q8_K_BLOCK_SIZE) return fail("input length is not a multiple of 256");
    return q38::launch_gemm_iq1m_tiled((int)batch_size, static_cast<const uint8_t *>(tiled),
                                       reinterpret_cast<const uint8_t *>(input), output, rows, rows,
                                       (uint32_t)(input_length / 256), state->grid, static_cast<hipStream_t>(stream))
               ? 1
               : fail("unsupported tiled GEMM shape (input_length 5120, 6144, 10240 or 17408)");
}

int q38hip_gemm_q8_k_tiled(float *output, const Q38Q8KBlock *input, uint32_t batch_size, uint64_t input_length,
                           const void *tiled, uint32_t rows, void *stream)
{
    if (!output || !input || !tiled || !rows) return fail("null argument");
    if (batch_size < 1) return fail("batch_size must be at least 1");
    if (!device_state()) return fail("device initialisation failed");
    if (input_length % Q38_Q8_K_BLOCK_SIZE) return fail("input length is not a multiple of 256");
    const uint32_t nb = (uint32_t)(input_length / 256);
    /* one launch for one token or from kWideMinTokens tokens on, else
     * launches of 2..8 tokens (see q38hip_gemm_q8_k) */
    for (uint32_t t0 = 0; t0 < batch_size;) {
        const uint32_t left = batch_size - t0;
        const uint32_t n = left == 1 || left >= (uint32_t)q38::kWideMinTokens ? left : token_chunk(left, 2);
        if (!q38::launch_gemm_q4k_tiled((int)n, static_cast<const uint8_t *>(tiled),
                                        reinterpret_cast<const uint8_t *>(input) + (size_t)t0 * nb * sizeof(Q38Q8KBlock),
                                        output + (size_t)t0 * rows, rows, rows, nb, static_cast<hipStream_t>(stream)))
            return fail("unsupported tiled GEMM shape (input_length 5120, 6144, 10240 or 17408)");
        t0 += n;
    }
    return 1;
}

int q38hip_argmax(uint32_t *index_out, const float *values, uint32_t count, uint32_t rows, void *stream)
{
    if (!index_out || !values || !count || !rows) return fail("bad argmax arguments");
    DeviceState *state = device_state();
    if (!state) return fail("device initialisation failed");
    const size_t need = (size_t)q38::argmax_chunks(count) * rows;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        if (state->argmax_capacity < need) {
            /* launches enqueued earlier (on any stream) may still read the
             * old scratch: let them finish before it is released */
            if (state->argmax_values && hipDeviceSynchronize() != hipSuccess)
                return fail("device synchronisation failed");
            if (state->argmax_values) (void)hipFree(state->argmax_values);
            if (state->argmax_index) (void)hipFree(state->argmax_index);
            state->argmax_values = nullptr;
            state->argmax_index = nullptr;
            state->argmax_capacity = 0;
            if (hipMalloc(&state->argmax_values, need * sizeof(float)) != hipSuccess ||
                hipMalloc(&state->argmax_index, need * sizeof(uint32_t)) != hipSuccess)
                return fail("argmax scratch allocation failed");
            state->argmax_capacity = need;
        }
    }
    q38::launch_argmax(values, count, rows, state->argmax_values, state->argmax_index, index_out,
                       static_cast<hipStream_t>(stream));
    return 1;
}

int q38hip_sample(uint32_t *token, uint64_t *state, const float *logits, uint32_t vocabulary_size,
                  float temperature, float top_p, float presence_penalty, uint32_t top_k,
                  const uint8_t *presence, uint32_t presence_size, void *stream)
{
    if (!token || !state || !logits) return fail("bad sample arguments");
    if (const char *why = q38::check_sample(vocabulary_size, temperature, top_k)) return fail(why);
    DeviceState *dev = device_state();
    if (!dev) return fail("device initialisation failed");
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        if (!dev->sample_scratch &&
            hipMalloc(&dev->sample_scratch, q38::sample_scratch_bytes(q38::kMaxSampleVocab, q38::kMaxSampleTopK)) !=
                hipSuccess) {
            dev->sample_scratch = nullptr;
            return fail("sampler scratch allocation failed");
        }
    }
    if (!q38::launch_sample(token, state, logits, vocabulary_size, presence, presence ? presence_size : 0, temperature,
                            top_p, presence_penalty, top_k, dev->sample_scratch, static_cast<hipStream_t>(stream)))
        return fail("sampler launch failed");
    return 1;
}

int q38hip_argmax_noalloc(uint32_t *index_out, const float *values, uint32_t count, uint32_t rows, void *stream)
{
    if (!index_out || !values || !count || !rows) return fail("bad argmax arguments");
    const size_t need = (size_t)q38::argmax_chunks(count) * rows;
    if (need > kNoAllocPairs)
        return fail("argmax too large for the fixed scratch: ceil(count / 4096) * rows must be at most 8192");
    uint32_t *base = noalloc_scratch();
    if (!base) return fail("scratch address lookup failed");
    /* pass 1 writes every partial that pass 2 reads: nothing to clear */
    q38::launch_argmax(values, count, rows, reinterpret_cast<float *>(base), base + kNoAllocPairs, index_out,
                       static_cast<hipStream_t>(stream));
    return 1;
}

int q38hip_accept(uint32_t *result, const uint32_t *targets, const uint32_t *drafts, uint32_t rows,
                  void *stream)
{
    if (!result || !targets || !drafts || !rows) return fail("bad acceptance arguments");
    q38::launch_accept(result, targets, drafts, rows, static_cast<hipStream_t>(stream));
    return 1;
}

/* ---- host-pointer drop-ins for the reference kernel ABI ------------------ */

int q38_quantize_q8_k(Q38Q8KBlock *output, const float *input, uint64_t length)
{
    if (!output || !input || length % Q38_Q8_K_BLOCK_SIZE) return fail("bad quantize arguments");
    if (length == 0) return 1;
    const uint64_t blocks = length / Q38_Q8_K_BLOCK_SIZE;
    DeviceBuffer din(length * sizeof(float)), dout(blocks * sizeof(Q38Q8KBlock));
    if (!din.ptr || !dout.ptr) return fail("device allocation failed");
    if (hipMemcpy(din.ptr, input, length * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        return fail("copy to device failed");
    if (!q38hip_quantize_q8_k(static_cast<Q38Q8KBlock *>(dout.ptr), static_cast<const float *>(din.ptr),
                              length, 1, nullptr))
        return 0;
    if (hipMemcpy(output, dout.ptr, blocks * sizeof(Q38Q8KBlock), hipMemcpyDeviceToHost) != hipSuccess)
        return fail("copy from device failed");
    return 1;
}

int q38_tensor_gemm_q8_k(float *output, const Q38Q8KBlock *input, uint32_t batch_size,
                         uint64_t input_length, const Q38GGUFTensor *tensor)
{
    if (!check_gemm(output, input, batch_size, input_length, tensor)) return 0;
    const uint64_t rows = tensor->shape[1];
    const uint64_t blocks = input_length / 256;
    const uint64_t wbytes = rows * span_bytes(tensor->type, input_length);
    const uint64_t xbytes = (uint64_t)batch_size * blocks * sizeof(Q38Q8KBlock);
    const uint64_t ybytes = (uint64_t)batch_size * rows * sizeof(float);
    DeviceBuffer dw(wbytes), dx(xbytes), dy(ybytes);
    if (!dw.ptr || !dx.ptr || !dy.ptr) return fail("device allocation failed");
    if (hipMemcpy(dw.ptr, tensor->data, wbytes, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dx.ptr, input, xbytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail("copy to device failed");
    Q38GGUFTensor dev = *tensor;
    dev.data = static_cast<const uint8_t *>(dw.ptr);
    if (!q38hip_gemm_q8_k(static_cast<float *>(dy.ptr), static_cast<const Q38Q8KBlock *>(dx.ptr), batch_size,
                          input_length, &dev, nullptr))
        return 0;
    if (hipMemcpy(output, dy.ptr, ybytes, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("copy from device failed");
    return 1;
}

int q38_tensor_gemv_q8_k(float *output, const Q38Q8KBlock *input, uint64_t input_length,
                         const Q38GGUFTensor *tensor)
{
    return q38_tensor_gemm_q8_k(output, input, 1, input_length, tensor);
}

int q38_tensor_gemm_f32(float *output, const float *input, uint32_t batch_size, uint64_t input_length,
                        const Q38GGUFTensor *tensor)
{
    if (!output || !input || !batch_size || !tensor || tensor->n_dims != 2 || tensor->shape[0] != input_length)
        return fail("bad float GEMM arguments");
    const uint64_t rows = tensor->shape[1];
    const uint64_t wbytes = rows * span_bytes(tensor->type, input_length);
    if (!wbytes || !tensor->data) return fail("unsupported tensor type or width");
    const uint64_t xbytes = (uint64_t)batch_size * input_length * sizeof(float);
    const uint64_t ybytes = (uint64_t)batch_size * rows * sizeof(float);
    DeviceBuffer dw(wbytes), dx(xbytes), dy(ybytes);
    if (!dw.ptr || !dx.ptr || !dy.ptr) return fail("device allocation failed");
    if (hipMemcpy(dw.ptr, tensor->data, wbytes, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dx.ptr, input, xbytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail("copy to device failed");
    Q38GGUFTensor dev = *tensor;
    dev.data = static_cast<const uint8_t *>(dw.ptr);
    if (!q38hip_gemm_f32(static_cast<float *>(dy.ptr), static_cast<const float *>(dx.ptr), batch_size,
                         input_length, &dev, nullptr))
        return 0;
    if (hipMemcpy(output, dy.ptr, ybytes, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("copy from device failed");
    return 1;
}

int q38_tensor_gemv_f32(float *output, const float *input, const Q38GGUFTensor *tensor)
{
    if (!tensor) return fail("bad float GEMV arguments");
    return q38_tensor_gemm_f32(output, input, 1, tensor->shape[0], tensor);
}

int q38_tensor_dot_row_f32(float *output, const float *input, const Q38GGUFTensor *tensor, uint64_t row)
{
    if (!output || !input || !tensor || tensor->n_dims != 2 || row >= tensor->shape[1])
        return fail("bad row dot arguments");
    const uint64_t bytes = span_bytes(tensor->type, tensor->shape[0]);
    if (!bytes || !tensor->data) return fail("unsupported tensor type or width");
    Q38GGUFTensor one = *tensor;
    one.shape[1] = 1;
    one.data = tensor->data + row * bytes;
    if (!q38_tensor_gemv_f32(output, input, &one)) return 0;
    return std::isfinite(*output) ? 1 : 0;
}

int q38_tensor_row_f32(float *output, const Q38GGUFTensor *tensor, uint64_t row)
{
    if (!output || !tensor || tensor->n_dims != 2 || row >= tensor->shape[1]) return fail("bad row arguments");
    const uint64_t width = tensor->shape[0];
    const uint64_t bytes = span_bytes(tensor->type, width);
    if (!bytes || !tensor->data) return fail("unsupported tensor type or width");
    DeviceBuffer dw(bytes), dy(width * sizeof(float));
    if (!dw.ptr || !dy.ptr) return fail("device allocation failed");
    if (hipMemcpy(dw.ptr, tensor->data + row * bytes, bytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail("copy to device failed");
    Q38GGUFTensor dev = *tensor;
    dev.shape[1] = 1;
    dev.data = static_cast<const uint8_t *>(dw.ptr);
    if (!q38hip_row_f32(static_cast<float *>(dy.ptr), &dev, 0, 1, nullptr)) return 0;
    if (hipMemcpy(output, dy.ptr, width * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
        return fail("copy from device failed");
    return 1;
}

/* The GPU kernels read the GGUF blocks as they are, so there is no IQ1_S
 * view to build: both calls succeed and leave every tensor unchanged. */
int q38_prepare_iq1_s_repacks(Q38GGUF *gguf) { return gguf ? 1 : 0; }
void q38_release_iq1_s_repacks(Q38GGUF *gguf) { (void)gguf; }

}  // extern "C"
