/* Decode-step kernels of the Qwen3.8 hybrid model on gfx950: embedding rows,
 * RMS/L2 norms, SwiGLU, residual adds, the gated DeltaNet recurrence and the
 * full-attention KV-cache decode.
 *
 * Every kernel reproduces the reference's fp32 operation order
 * (src/qwen38/qwen38_model.c, compiled with -ffp-contract=off): plain
 * products and sums round separately, fmaf appears only where the reference
 * calls it or uses an FMA intrinsic, transcendentals are the exact restated
 * expf/logf of q38_libm.h, and the double-precision squared sums of the norms
 * reproduce the reference's sequential loop (block_sum_finish, q38_norm.h).
 */
#include <cmath>
#include <mutex>
#include <vector>

#include "q38_device.h"
#include "q38_kernels.h"
#include "q38_libm.h"
#include "q38_math.h"
#include "q38_norm.h"
#include "q38_q8k.h"

namespace q38 {

/* ---- RMSNorm + Q8_K ------------------------------------------------------ */

/* One block of kNormThreads threads per 5120-element row
 * (rmsnorm_quant_row): ten wavefronts of two Q8_K blocks each, so that the
 * per-block reductions of the quantisation run on ten SIMDs. */
constexpr int kNormThreads = 640;
template <int NV, bool ADD>
__global__ __launch_bounds__(kNormThreads) void norm_quant_kernel(float *__restrict__ norm_out, long long norm_stride,
                                                         uint8_t *__restrict__ q_out, int q_stride_blocks,
                                                         float *__restrict__ hidden, long long in_stride,
                                                         const float *__restrict__ branch,
                                                         const float *__restrict__ weight)
{
    const long long row = blockIdx.x;
    rmsnorm_quant_row<kNormThreads, NV, ADD>(norm_out ? norm_out + row * norm_stride : nullptr,
                               q_out ? q_out + (size_t)row * q_stride_blocks * kQ8KBytes : nullptr,
                               hidden + row * in_stride, ADD ? branch + row * in_stride : nullptr, weight);
}

__global__ __launch_bounds__(256) void add_kernel(float *__restrict__ hidden, const float *__restrict__ branch,
                                                  long long n)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) hidden[i] = __fadd_rn(hidden[i], branch[i]);
}

constexpr int kFFNWidth = 17408;

/* SwiGLU then Q8_K: y = silu(gate) * up (q38_swiglu scalar path,
 * qwen38_model.c:532-549), one wavefront per 256-element block; row t of
 * gate and up starts at t * stride (a multiple of 4). */
__global__ __launch_bounds__(256) void swiglu_quant_kernel(uint8_t *__restrict__ q_out, const float *__restrict__ gate,
                                                           const float *__restrict__ up, long long stride, int nblocks,
                                                           float *__restrict__ f_out)
{
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    const int t = b / (kFFNWidth / 256), j = b - t * (kFFNWidth / 256);
    const size_t at = (size_t)t * stride + (size_t)j * 256 + 4 * lane;
    const float4 g = *reinterpret_cast<const float4 *>(gate + at);
    const float4 u = *reinterpret_cast<const float4 *>(up + at);
    const float v[4] = {__fmul_rn(siluf_exact(g.x), u.x), __fmul_rn(siluf_exact(g.y), u.y),
                        __fmul_rn(siluf_exact(g.z), u.z), __fmul_rn(siluf_exact(g.w), u.w)};
    if (f_out) *reinterpret_cast<float4 *>(f_out + (size_t)b * 256 + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
    wave_quantize_q8k(v, q_out + (size_t)b * kQ8KBytes, lane);
}

/* ---- embedding rows ------------------------------------------------------ */

/* Dequantised Q4_K row (q38_tensor_row_f32 -> q38_dot_q4_k with unit
 * vectors, src/qwen38/qwen38_quant.c:396-426, 3186-3223): element 64c+i of a
 * block is (d*sc)*q - dmin*m, plus 0.0f (a -0 result becomes +0).  One block
 * of 256 threads per (token, super-block). */
__global__ __launch_bounds__(256) void embed_q4k_kernel(float *__restrict__ out, const uint8_t *__restrict__ w,
                                                        const uint32_t *__restrict__ tokens, int blocks_per_row,
                                                        uint32_t vocab)
{
    const int t = blockIdx.y;
    const int b = blockIdx.x;
    const uint32_t token = tokens[t];
    if (token >= vocab) return;
    const uint8_t *blk = w + ((size_t)token * blocks_per_row + b) * 144;
    const int e = threadIdx.x;          /* element 0..255 */
    const int c = e >> 6, hi = (e >> 5) & 1, i = e & 31;
    const int j = 2 * c + hi;           /* sub-block */
    const uint8_t *s = blk + 4;
    int sc, m;
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const float d = f16_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = f16_to_f32(blk[2] | (blk[3] << 8));
    const uint8_t qb = blk[16 + 32 * c + i];
    const int q = hi ? (qb >> 4) : (qb & 15);
    const float scaled = __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
    const float v = __fadd_rn(__fsub_rn(scaled, __fmul_rn(dmin, (float)m)), 0.0f);
    out[(size_t)t * blocks_per_row * 256 + (size_t)b * 256 + e] = v;
}

/* ---- gated DeltaNet ------------------------------------------------------ */

constexpr int kQKV = 10240, kQKDim = 2048, kVHeads = 48, kHeadDim = 128, kLinV = 6144;
constexpr uint32_t kStateSlots = kRecurrentStateSlots;

/* Causal conv (4 taps, state of 3 per channel), SiLU, per-head L2 norm of q
 * and k, and the beta / alpha transforms (q38_linear_core,
 * qwen38_model.c:720-757) for `rows` consecutive tokens.  Row t's
 * projections are at qkv + t * ld (q, k, v, then beta at + beta_off and
 * alpha at + alpha_off) and are transformed in place.  Blocks 0..79 each own
 * 128 channels (blocks 0..31 are the 16 q heads and 16 k heads); block 80
 * does beta/alpha.  The conv state before row t is slot (*slot_ptr + t) (mod
 * kStateSlots); each row's shifted state is written to the next slot, and
 * the chain between rows stays in registers.  With `last_only` (a prefill
 * batch, whose intermediate states nothing reads) only the last row's state
 * is written, to slot (*slot_ptr + rows). */
__global__ __launch_bounds__(128) void deltanet_prep_kernel(float *__restrict__ qkv, long long ld, int beta_off,
                                                            int alpha_off, float *__restrict__ conv_state,
                                                            long long slot_stride,
                                                            const uint32_t *__restrict__ slot_ptr, int rows,
                                                            const float *__restrict__ conv_w,
                                                            const float *__restrict__ ssm_a,
                                                            const float *__restrict__ ssm_dt, int last_only)
{
    const int tid = threadIdx.x;
    if (blockIdx.x == kQKV / 128) {
        if (tid < kVHeads) {
            for (int t = 0; t < rows; ++t) {
                float *beta = qkv + (long long)t * ld + beta_off, *alpha = qkv + (long long)t * ld + alpha_off;
                beta[tid] = sigmoidf_exact(beta[tid]);
                alpha[tid] = __fmul_rn(ssm_a[tid], softplusf_exact(__fadd_rn(alpha[tid], ssm_dt[tid])));
            }
        }
        return;
    }
    const int ch = blockIdx.x * 128 + tid;
    const uint32_t slot0 = *slot_ptr;
    const float *st = conv_state + (size_t)(slot0 % kStateSlots) * slot_stride + (size_t)ch * 3;
    const float4 k = reinterpret_cast<const float4 *>(conv_w)[ch];
    float s0 = st[0], s1 = st[1], s2 = st[2];
    __shared__ float head[128];
    for (int t = 0; t < rows; ++t) {
        float *row = qkv + (long long)t * ld;
        const float x = row[ch];
        float value = 0.0f;
        value = __fadd_rn(value, __fmul_rn(s0, k.x));
        value = __fadd_rn(value, __fmul_rn(s1, k.y));
        value = __fadd_rn(value, __fmul_rn(s2, k.z));
        value = __fadd_rn(value, __fmul_rn(x, k.w));
        s0 = s1;
        s1 = s2;
        s2 = x;
        if (!last_only || t == rows - 1) {
            float *st_out = conv_state + (size_t)((slot0 + t + 1) % kStateSlots) * slot_stride + (size_t)ch * 3;
            st_out[0] = s0;
            st_out[1] = s1;
            st_out[2] = s2;
        }
        const float y = siluf_exact(value);
        if (blockIdx.x >= 2 * kQKDim / 128) {
            row[ch] = y;
            continue;
        }
        head[tid] = y;
        __syncthreads();
        const float sum = block_sum_squares<128>(head, 128, FloatPost{});
        const float scale = div_rn(1.0f, fmaxf(sqrt_rn(sum), 1e-6f));
        row[ch] = __fmul_rn(y, scale);
    }
}

/* lane l of each 16-lane row gets lane (l - N) mod 16 of the row (DPP row_ror:N) */
template <int N>
__device__ __forceinline__ float dpp_ror(float v)
{
    return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x120 + N, 0xf, 0xf, false));
}
/* lane l of each quad gets lane CTRL-selected within the quad (DPP quad_perm) */
template <int CTRL>
__device__ __forceinline__ float dpp_quad(float v)
{
    return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), CTRL, 0xf, 0xf, false));
}

constexpr int kScanChunk = 16;

/* Sum of a column's 32 accumulators in the reference's AVX2 reduction order
 * (q38_dot_f32_128, qwen38_model.c:616-637): P_a[j] is the accumulator of
 * vector a = 0..3, element j = 0..7, and the result is ((H0+H1)+(H2+H3))
 * with H[j] = Q[j] + Q[j+4], Q[j] = (P0[j]+P2[j]) + (P1[j]+P3[j]).  A column
 * runs on a 16-lane row: lane l = 8a + j (a = 0, 1) holds P_a[j] in `a` and
 * P_{a+2}[j] in `b`, so the first pair is added inside the lane; each later
 * step adds a lane holding the other operand of the reference's pair (row_ror
 * 8: lane l ^ 8; row_ror 4: lane (l - 4) mod 16, which then holds the value
 * of j ^ 4; the quad permutations: lanes l ^ 1 and l ^ 2).  Lane 0 adds exactly the reference's
 * operand pairs in its order; every other lane adds the same pairs, some
 * with the operands swapped, which rounds to the same float, so every lane
 * of the row ends with the sum. */
__device__ __forceinline__ float avx2_tree16(float a, float b)
{
    float v = __fadd_rn(a, b);                  /* lane 8a + j: P_a[j] + P_{a+2}[j] */
    v = __fadd_rn(v, dpp_ror<8>(v));            /* Q[l % 8] */
    v = __fadd_rn(v, dpp_ror<4>(v));            /* Q[j] + Q[j ^ 4], j = l % 8: H[l % 4] */
    v = __fadd_rn(v, dpp_quad<0xb1>(v));        /* H0 + H1 or H2 + H3 */
    v = __fadd_rn(v, dpp_quad<0x4e>(v));        /* (H0 + H1) + (H2 + H3) */
    return v;
}

/* State update of one value head over a batch of rows
 * (qwen38_model.c:759-783): S *= decay; per column c: pred = dot(S_c, k);
 * delta = (v[c] - pred) * beta; S_c = fma(k, delta, S_c);
 * out[c] = dot(S_c, q) * (1/sqrt(128)).  Columns are independent.  The
 * reference's dots are 32 fixed accumulators P[j] (element j + 32a added in
 * a = 0..3 order) and a tree; here 16 lanes run a column: lane l owns
 * elements l + 32a and l + 16 + 32a, i.e. P[l] and P[l + 16] as two
 * independent fmaf chains, and avx2_tree16 adds them in the reference's
 * order (measured on MI355X against one column per 32 lanes: 4096-token
 * prefill 422 -> 415 ms).  Sixteen columns of one value head per block of
 * 256.  The columns run through `rows` consecutive tokens (row t's prepared
 * q|k|v at qkv + t * ld, beta and alpha at + beta_off / alpha_off, output at
 * out + t * kLinV): the state before row t is slot (*slot_ptr + t), read
 * once, kept in registers, and each row's result is written to the next
 * slot (with `last_only`, only the last row's, to slot *slot_ptr + rows).
 * The block's inputs (k and q of head h % 16, the block's v values, the
 * decay and beta of head h) come through LDS in chunks of kScanChunk rows,
 * the next chunk's global loads in flight while the current one is
 * scanned, so the sequential scan reads only LDS. */
constexpr int kScan16Cols = 16;

__global__ __launch_bounds__(256) void deltanet_state_kernel(float *__restrict__ out, float *__restrict__ state,
                                                              long long slot_stride,
                                                              const uint32_t *__restrict__ slot_ptr, int rows,
                                                              const float *__restrict__ qkv, long long ld,
                                                              int beta_off, int alpha_off, float query_scale,
                                                              int last_only)
{
    __shared__ float kq_s[2][kScanChunk][2 * kHeadDim];   /* [parity][row][k 0..127 | q 0..127] */
    __shared__ float v_s[2][kScanChunk][kScan16Cols];
    __shared__ float ab_s[2][kScanChunk][2];               /* decay = expf(alpha), beta */
    const int tid = threadIdx.x;
    const int col0 = blockIdx.x * kScan16Cols;   /* 0 .. 48*128-1 */
    const int h = col0 >> 7;
    const int c0 = col0 & 127;
    const int cl = tid >> 4, l = tid & 15;
    const int c = c0 + cl;
    const int kh = h % 16;
    const uint32_t slot0 = *slot_ptr;
    const size_t col_off = ((size_t)h * kHeadDim + c) * kHeadDim;
    const float *s = state + (size_t)(slot0 % kStateSlots) * slot_stride + col_off;
    float sv[8];   /* elements 32a + l (a = 0..3), then 32a + l + 16 */
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        sv[a] = s[32 * a + l];
        sv[4 + a] = s[32 * a + l + 16];
    }

    /* thread tid stages element tid of the k|q vector of every row of a
     * chunk, the v value of row tid / 16 and column tid % 16, and threads
     * 0..2R-1 an alpha or beta */
    const int kq_src = tid < kHeadDim ? kQKDim + kh * kHeadDim + tid : kh * kHeadDim + (tid - kHeadDim);
    float kq_r[kScanChunk], v_r = 0.0f, ab_r = 0.0f;
    const int nchunks = (rows + kScanChunk - 1) / kScanChunk;
    auto fetch = [&](int ch) {
        const int r0 = ch * kScanChunk;
#pragma unroll
        for (int i = 0; i < kScanChunk; ++i) {
            const int t = r0 + i < rows ? r0 + i : rows - 1;
            kq_r[i] = qkv[(long long)t * ld + kq_src];
        }
        {
            const int i = tid >> 4;
            const int t = r0 + i < rows ? r0 + i : rows - 1;
            v_r = qkv[(long long)t * ld + 2 * kQKDim + h * kHeadDim + c0 + (tid & 15)];
        }
        if (tid < 2 * kScanChunk) {
            const int i = tid >> 1;
            const int t = r0 + i < rows ? r0 + i : rows - 1;
            ab_r = qkv[(long long)t * ld + ((tid & 1) ? beta_off + h : alpha_off + h)];
        }
    };
    auto stage = [&](int par) {
#pragma unroll
        for (int i = 0; i < kScanChunk; ++i) kq_s[par][i][tid] = kq_r[i];
        v_s[par][tid >> 4][tid & 15] = v_r;
        if (tid < 2 * kScanChunk) ab_s[par][tid >> 1][tid & 1] = (tid & 1) ? ab_r : q38_expf(ab_r);
    };
    struct RowIn {
        float k[8], q[8], v, beta, decay;
    };
    auto read_row = [&](int par, int i) {
        RowIn in;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            in.k[a] = kq_s[par][i][32 * a + l];
            in.k[4 + a] = kq_s[par][i][32 * a + l + 16];
            in.q[a] = kq_s[par][i][kHeadDim + 32 * a + l];
            in.q[4 + a] = kq_s[par][i][kHeadDim + 32 * a + l + 16];
        }
        in.v = v_s[par][i][cl];
        in.beta = ab_s[par][i][1];
        in.decay = ab_s[par][i][0];
        return in;
    };
    fetch(0);
    stage(0);
    __syncthreads();
    for (int ch = 0; ch < nchunks; ++ch) {
        const int par = ch & 1;
        if (ch + 1 < nchunks) fetch(ch + 1);
        const int r0 = ch * kScanChunk;
        const int n = rows - r0 < kScanChunk ? rows - r0 : kScanChunk;
        RowIn cur = read_row(par, 0);
        for (int i = 0; i < n; ++i) {
            const int t = r0 + i;
            const RowIn nxt = read_row(par, i + 1 < n ? i + 1 : i);
#pragma unroll
            for (int e = 0; e < 8; ++e) sv[e] = __fmul_rn(sv[e], cur.decay);
            float pa = 0.0f, pb = 0.0f;
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                pa = __builtin_fmaf(sv[a], cur.k[a], pa);
                pb = __builtin_fmaf(sv[4 + a], cur.k[4 + a], pb);
            }
            const float pred = avx2_tree16(pa, pb);
            const float delta = __fmul_rn(__fsub_rn(cur.v, pred), cur.beta);
            float *s_out = state + (size_t)((slot0 + t + 1) % kStateSlots) * slot_stride + col_off;
            const bool store = !last_only || t == rows - 1;
            float ra = 0.0f, rb = 0.0f;
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                sv[a] = __builtin_fmaf(cur.k[a], delta, sv[a]);
                sv[4 + a] = __builtin_fmaf(cur.k[4 + a], delta, sv[4 + a]);
                if (store) {
                    s_out[32 * a + l] = sv[a];
                    s_out[32 * a + l + 16] = sv[4 + a];
                }
                ra = __builtin_fmaf(sv[a], cur.q[a], ra);
                rb = __builtin_fmaf(sv[4 + a], cur.q[4 + a], rb);
            }
            const float result = avx2_tree16(ra, rb);
            if (l == 0) out[(size_t)t * kLinV + h * kHeadDim + c] = __fmul_rn(result, query_scale);
            cur = nxt;
        }
        if (ch + 1 < nchunks) stage(par ^ 1);
        __syncthreads();
    }
}

/* Prefill form of deltanet_prep_kernel.  The conv of row t reads only the
 * inputs of rows t-3 .. t (the conv state before the batch stands in for
 * rows before the first), so every (channel, row) is independent: block
 * (cb, g) runs channels 128 cb .. 128 cb + 127 over rows kPrepRows g ..,
 * reading the untransformed projections in `qkv` and writing the prepared
 * values to `out` (same row stride and offsets).  The arithmetic per
 * element, including the L2 norm of each q/k head and row (the block's sum
 * over its 128 channels), is deltanet_prep_kernel's.  The blocks of row
 * group 0 write the conv state after the batch to slot *slot_ptr + rows:
 * they are the only readers of slot *slot_ptr, and each thread reads its
 * channel's state before it writes, so the store stays ordered after the
 * read also when rows is a multiple of kStateSlots (the same slot).  Block
 * kQKV / 128 does beta / alpha. */
constexpr int kPrepRows = 8;

__global__ __launch_bounds__(128) void deltanet_prep_rows_kernel(float *__restrict__ out,
                                                                 const float *__restrict__ qkv, long long ld,
                                                                 int beta_off, int alpha_off,
                                                                 float *__restrict__ conv_state,
                                                                 long long slot_stride,
                                                                 const uint32_t *__restrict__ slot_ptr, int rows,
                                                                 const float *__restrict__ conv_w,
                                                                 const float *__restrict__ ssm_a,
                                                                 const float *__restrict__ ssm_dt)
{
    const int tid = threadIdx.x;
    const int t0 = blockIdx.y * kPrepRows;
    const int tn = rows - t0 < kPrepRows ? rows - t0 : kPrepRows;
    if (blockIdx.x == kQKV / 128) {
        if (tid < kVHeads) {
            for (int i = 0; i < tn; ++i) {
                const long long base = (long long)(t0 + i) * ld;
                out[base + beta_off + tid] = sigmoidf_exact(qkv[base + beta_off + tid]);
                out[base + alpha_off + tid] =
                    __fmul_rn(ssm_a[tid], softplusf_exact(__fadd_rn(qkv[base + alpha_off + tid], ssm_dt[tid])));
            }
        }
        return;
    }
    const int ch = blockIdx.x * 128 + tid;
    const uint32_t slot0 = *slot_ptr;
    const float *st = conv_state + (size_t)(slot0 % kStateSlots) * slot_stride + (size_t)ch * 3;
    const float4 k = reinterpret_cast<const float4 *>(conv_w)[ch];
    /* inputs of rows t0 - 3 .. t0 - 1 (the state before the batch for rows < 0) */
    float s0 = t0 >= 3 ? qkv[(long long)(t0 - 3) * ld + ch] : st[t0];
    float s1 = t0 >= 2 ? qkv[(long long)(t0 - 2) * ld + ch] : st[t0 + 1];
    float s2 = t0 >= 1 ? qkv[(long long)(t0 - 1) * ld + ch] : st[2];
    float xs[kPrepRows];
#pragma unroll
    for (int i = 0; i < kPrepRows; ++i) xs[i] = i < tn ? qkv[(long long)(t0 + i) * ld + ch] : 0.0f;
    __shared__ float head[128];
    for (int i = 0; i < tn; ++i) {
        const float x = xs[i];
        float value = 0.0f;
        value = __fadd_rn(value, __fmul_rn(s0, k.x));
        value = __fadd_rn(value, __fmul_rn(s1, k.y));
        value = __fadd_rn(value, __fmul_rn(s2, k.z));
        value = __fadd_rn(value, __fmul_rn(x, k.w));
        s0 = s1;
        s1 = s2;
        s2 = x;
        const float y = siluf_exact(value);
        float *o = out + (long long)(t0 + i) * ld + ch;
        if (blockIdx.x >= 2 * kQKDim / 128) {
            *o = y;
            continue;
        }
        head[tid] = y;
        __syncthreads();
        const float sum = block_sum_squares<128>(head, 128, FloatPost{});
        const float scale = div_rn(1.0f, fmaxf(sqrt_rn(sum), 1e-6f));
        *o = __fmul_rn(y, scale);
    }
    if (t0 == 0) {
        /* the inputs of rows rows-3 .. rows-1; row r < 0 is state entry 3 + r */
        float last[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int r = rows - 3 + j;
            last[j] = r >= 0 ? qkv[(long long)r * ld + ch] : st[3 + r];
        }
        float *so = conv_state + (size_t)((slot0 + rows) % kStateSlots) * slot_stride + (size_t)ch * 3;
        so[0] = last[0];
        so[1] = last[1];
        so[2] = last[2];
    }
}

/* deltanet_prep_kernel and deltanet_state_kernel in one launch, for up to
 * kFusedRows rows.  Block (h, cg) = (blockIdx.x / 8, blockIdx.x % 8) owns
 * the state columns 16cg..16cg+15 of value head h, 16 lanes per column as
 * in deltanet_state_kernel, and first redoes, into LDS, the prep arithmetic
 * of what those columns read: the conv + SiLU + L2 norm of q and k head
 * kh = h % 16 (thread i: q channel i, k channel i - 128), conv + SiLU of its
 * sixteen v channels, and
 * beta / alpha of head h.  Each conv channel's next state slots are written
 * by one block: q/k channels by block (kh, 0), v channels by their owner. */
constexpr int kFusedRows = 8;
constexpr int kFusedCols = 16;   /* state columns per block, 16 lanes each */

__device__ __forceinline__ void conv_silu_rows(float *y_out, int y_stride, const float *qkv, long long ld, int ch,
                                               const float *conv_state, float *conv_out, long long conv_stride,
                                               uint32_t slot0, int rows, const float *conv_w)
{
    const float *st = conv_state + (size_t)(slot0 % kStateSlots) * conv_stride + (size_t)ch * 3;
    const float4 k = reinterpret_cast<const float4 *>(conv_w)[ch];
    float s0 = st[0], s1 = st[1], s2 = st[2];
    float xs[kFusedRows];   /* every row's input in flight at once */
#pragma unroll
    for (int t = 0; t < kFusedRows; ++t) xs[t] = t < rows ? qkv[(long long)t * ld + ch] : 0.0f;
#pragma unroll
    for (int t = 0; t < kFusedRows; ++t) {
        if (t >= rows) break;
        const float x = xs[t];
        float value = 0.0f;
        value = __fadd_rn(value, __fmul_rn(s0, k.x));
        value = __fadd_rn(value, __fmul_rn(s1, k.y));
        value = __fadd_rn(value, __fmul_rn(s2, k.z));
        value = __fadd_rn(value, __fmul_rn(x, k.w));
        s0 = s1;
        s1 = s2;
        s2 = x;
        if (conv_out) {
            float *o = conv_out + (size_t)((slot0 + t + 1) % kStateSlots) * conv_stride + (size_t)ch * 3;
            o[0] = s0;
            o[1] = s1;
            o[2] = s2;
        }
        y_out[t * y_stride] = siluf_exact(value);
    }
}

__global__ __launch_bounds__(256) void deltanet_fused_kernel(float *__restrict__ out, float *__restrict__ state,
                                                             long long slot_stride,
                                                             const uint32_t *__restrict__ slot_ptr, int rows,
                                                             const float *__restrict__ qkv, long long ld,
                                                             int beta_off, int alpha_off, float query_scale,
                                                             float *__restrict__ conv_state, long long conv_stride,
                                                             const float *__restrict__ conv_w,
                                                             const float *__restrict__ ssm_a,
                                                             const float *__restrict__ ssm_dt)
{
    __shared__ float qk_s[kFusedRows][256];   /* SiLU outputs: q of head kh (0..127), k (128..255) */
    __shared__ float v_s[kFusedRows][kFusedCols];
    __shared__ float beta_s[kFusedRows], alpha_s[kFusedRows];   /* beta and decay = expf(alpha) */
    __shared__ double part_s[kFusedRows][4];
    __shared__ float scale_s[kFusedRows][2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int kGroups = kHeadDim / kFusedCols;   /* column groups per head */
    const int h = blockIdx.x / kGroups, cg = blockIdx.x % kGroups, kh = h % 16;
    const int c = cg * kFusedCols + (tid >> 4), l = tid & 15;
    const uint32_t slot0 = *slot_ptr;
    const size_t col_off = ((size_t)h * kHeadDim + c) * kHeadDim;
    const float *s = state + (size_t)(slot0 % kStateSlots) * slot_stride + col_off;
    float sv[8];   /* elements 32a + l (a = 0..3), then 32a + l + 16 */
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        sv[a] = s[32 * a + l];
        sv[4 + a] = s[32 * a + l + 16];
    }
    /* beta / alpha inputs of row tid - 64 (threads 64 .. 64 + rows - 1 use
     * them; the others read a row of the batch too), requested with the
     * state, ahead of the conv */
    const float *brow = qkv + (long long)(tid < 64 ? 0 : (tid - 64 < rows ? tid - 64 : rows - 1)) * ld;
    const float beta_in = brow[beta_off + h], alpha_in = brow[alpha_off + h];
    const float a_h = ssm_a[h], dt_h = ssm_dt[h];

    /* prep (deltanet_prep_kernel, qwen38_model.c:720-757) */
    const int ch = tid < 128 ? kh * kHeadDim + tid : kQKDim + kh * kHeadDim + (tid - 128);
    conv_silu_rows(&qk_s[0][tid], 256, qkv, ld, ch, conv_state, h < 16 && cg == 0 ? conv_state : nullptr,
                   conv_stride, slot0, rows, conv_w);
    if (tid < kFusedCols)
        conv_silu_rows(&v_s[0][tid], kFusedCols, qkv, ld, 2 * kQKDim + h * kHeadDim + cg * kFusedCols + tid,
                       conv_state, conv_state, conv_stride, slot0, rows, conv_w);
    if (tid >= 64 && tid < 64 + rows) {
        beta_s[tid - 64] = sigmoidf_exact(beta_in);
        /* the row's decay expf(alpha), here in parallel rather than on the
         * state update's dependent chain */
        alpha_s[tid - 64] = q38_expf(__fmul_rn(a_h, softplusf_exact(__fadd_rn(alpha_in, dt_h))));
    }
    /* L2 norms of q and k per row: the double sum of squares of each
     * 128-vector as block_sum_finish (two wavefronts each) */
    for (int t = 0; t < rows; ++t) {
        const float y = qk_s[t][tid];
        const double sq = wave_sum((double)__fmul_rn(y, y));
        if (lane == 0) part_s[t][wave] = sq;
    }
    __syncthreads();
    if (tid < 2 * rows) {
        const int t = tid >> 1, g = tid & 1;
        const double total = part_s[t][2 * g] + part_s[t][2 * g + 1];
        const FloatPost post;
        const float lo = post(total * (1.0 - 0x1p-36)), hi = post(total * (1.0 + 0x1p-36));
        float sum = lo;
        if (lo != hi) {
            double seq = 0.0;
            for (int i = 0; i < kHeadDim; ++i) seq += (double)__fmul_rn(qk_s[t][128 * g + i], qk_s[t][128 * g + i]);
            sum = post(seq);
        }
        scale_s[t][g] = div_rn(1.0f, fmaxf(sqrt_rn(sum), 1e-6f));
    }
    __syncthreads();

    /* state update (deltanet_state_kernel's arithmetic and lane layout) */
    for (int t = 0; t < rows; ++t) {
        const float decay = alpha_s[t];
        const float qs = scale_s[t][0], ks = scale_s[t][1];
        float kv[8], qv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int i = 32 * (e & 3) + l + 16 * (e >> 2);
            sv[e] = __fmul_rn(sv[e], decay);
            kv[e] = __fmul_rn(qk_s[t][128 + i], ks);
            qv[e] = __fmul_rn(qk_s[t][i], qs);
        }
        float pa = 0.0f, pb = 0.0f;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            pa = __builtin_fmaf(sv[a], kv[a], pa);
            pb = __builtin_fmaf(sv[4 + a], kv[4 + a], pb);
        }
        const float pred = avx2_tree16(pa, pb);
        const float delta = __fmul_rn(__fsub_rn(v_s[t][tid >> 4], pred), beta_s[t]);
        float *s_out = state + (size_t)((slot0 + t + 1) % kStateSlots) * slot_stride + col_off;
        float ra = 0.0f, rb = 0.0f;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            sv[a] = __builtin_fmaf(kv[a], delta, sv[a]);
            sv[4 + a] = __builtin_fmaf(kv[4 + a], delta, sv[4 + a]);
            s_out[32 * a + l] = sv[a];
            s_out[32 * a + l + 16] = sv[4 + a];
            ra = __builtin_fmaf(sv[a], qv[a], ra);
            rb = __builtin_fmaf(sv[4 + a], qv[4 + a], rb);
        }
        const float result = avx2_tree16(ra, rb);
        if (l == 0) out[(size_t)t * kLinV + h * kHeadDim + c] = __fmul_rn(result, query_scale);
    }
}

/* Per value head: RMSNorm over 128 (ssm_norm weight), then out *= silu(z)
 * (qwen38_model.c:785-791), then Q8_K of the 6144-wide result for the
 * ssm_out projection.  One block of 256 threads per pair of heads (one Q8_K
 * block) and row. */
__global__ __launch_bounds__(256) void deltanet_out_quant_kernel(float *__restrict__ attn, uint8_t *__restrict__ q_out,
                                                                 const float *__restrict__ z, long long z_stride,
                                                                 const float *__restrict__ norm_w)
{
    __shared__ double partial[4];
    __shared__ float mean_s[2];
    __shared__ float ybuf[256];
    const int t = blockIdx.y, pair = blockIdx.x, tid = threadIdx.x;
    const int half = tid >> 7, i = tid & 127;
    const int head = 2 * pair + half;
    float *x = attn + (size_t)t * kLinV + head * kHeadDim;
    const float v = x[i];
    /* the gate and the norm weight do not depend on the sum: loaded (and
     * the gate's SiLU computed) before it, so one memory wait covers all */
    const float w = norm_w[i];
    const float gz = siluf_exact(z[(size_t)t * z_stride + head * kHeadDim + i]);
    double s = (double)__fmul_rn(v, v);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((tid & 63) == 0) partial[tid >> 6] = s;
    __syncthreads();
    if (i == 0) {
        const double total = partial[2 * half] + partial[2 * half + 1];
        const MeanPost post{128.0};
        const float lo = post(total * (1.0 - 0x1p-36)), hi = post(total * (1.0 + 0x1p-36));
        if (lo == hi) {
            mean_s[half] = lo;
        } else {
            double seq = 0.0;
            for (int k = 0; k < kHeadDim; ++k) seq += (double)__fmul_rn(x[k], x[k]);
            mean_s[half] = post(seq);
        }
    }
    __syncthreads();
    const float scale = rms_scale(mean_s[half]);
    const float y = __fmul_rn(__fmul_rn(__fmul_rn(v, scale), w), gz);
    x[i] = y;
    ybuf[tid] = y;
    __syncthreads();
    if (tid < 64) {
        const float q4[4] = {ybuf[4 * tid], ybuf[4 * tid + 1], ybuf[4 * tid + 2], ybuf[4 * tid + 3]};
        wave_quantize_q8k(q4, q_out + ((size_t)t * (kLinV / 256) + pair) * kQ8KBytes, tid);
    }
}

/* ---- full attention ------------------------------------------------------ */

constexpr int kAttnHeads = 24, kKVHeads = 4, kAttnDim = 256, kKVDim = 1024, kQDim = 6144;
constexpr int kScoreChunk = 64;
/* q heads per lane in the score kernel (more heads: fewer wavefronts, more
 * independent chains per lane) */
constexpr int kScoreHeadsPerLane = 6;
/* rows per workgroup of the prompt-batch scores kernel */
constexpr int kScoreRows = 8;
constexpr int kMaxLdsPositions = 32768;   /* softmax weights kept in LDS up to this many positions */
constexpr int kAttnLoadBatch = 32;        /* softmax weights read ahead of the denominator's adds */
constexpr int kSoftmaxPad = 64;           /* LDS floats past the context in the softmax kernel */

/* q / gate split, per-head RMSNorm of q and k (q_norm / k_norm weights),
 * RoPE on dims 0..63 (pairs i, i+32) and the K/V cache write
 * (q38_full_core, qwen38_model.c:816-846; q38_rope :697-713) for row t
 * (blockIdx.y) at position *position_ptr + t; the value row goes into the
 * channel-major value cache (pitch v_pitch).  Blocks 0..23 are q heads,
 * 24..27 k heads, 28 copies v.  `rope` holds cos (32) then sin (32) per
 * position, computed once on the host with the C library.  `block_base` =
 * 24 runs only the K/V part.  Row t of q_and_gate, key and value starts at
 * t * in_stride. */
__global__ __launch_bounds__(256) void attn_prep_kernel(float *__restrict__ q_out, const float *__restrict__ q_and_gate,
                                                        const float *__restrict__ key, const float *__restrict__ value,
                                                        long long in_stride,
                                                        const float *__restrict__ q_norm,
                                                        const float *__restrict__ k_norm,
                                                        const float *__restrict__ rope, float *__restrict__ key_cache,
                                                        float *__restrict__ value_cache, int v_pitch,
                                                        const uint32_t *__restrict__ position_ptr, int block_base)
{
    const int t = blockIdx.y;
    const uint32_t pos = *position_ptr + t;
    const int i = threadIdx.x;
    const int block = blockIdx.x + block_base;
    float *kc = key_cache + (size_t)pos * kKVDim;
    if (block == kAttnHeads + kKVHeads) {
        for (int e = i; e < kKVDim; e += 256) value_cache[(size_t)e * v_pitch + pos] = value[(size_t)t * in_stride + e];
        return;
    }
    const bool is_q = block < kAttnHeads;
    const int h = is_q ? block : block - kAttnHeads;
    const float *src = is_q ? q_and_gate + (size_t)t * in_stride + h * 2 * kAttnDim
                            : key + (size_t)t * in_stride + h * kAttnDim;
    const float *w = is_q ? q_norm : k_norm;
    const float x = src[i];
    /* the norm weight and the RoPE pair do not depend on the sum: loaded
     * before it, so one memory wait covers all */
    const float wi = w[i];
    const int pair = i & 31;
    const float c = i < 64 ? rope[(size_t)pos * 64 + pair] : 0.0f;
    const float s = i < 64 ? rope[(size_t)pos * 64 + 32 + pair] : 0.0f;
    const float mean = block_sum_finish<256>((double)__fmul_rn(x, x), src, kAttnDim, MeanPost{256.0});
    const float scale = rms_scale(mean);
    __shared__ float v[kAttnDim];
    v[i] = __fmul_rn(__fmul_rn(x, scale), wi);
    __syncthreads();
    float y = v[i];
    if (i < 64) {
        const float x0 = v[pair], x1 = v[pair + 32];
        y = i < 32 ? __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s))
                   : __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
    }
    if (is_q) q_out[(size_t)t * kQDim + h * kAttnDim + i] = y;
    else kc[h * kAttnDim + i] = y;
}

/* Attention scores of one row for HPL of the six q heads sharing a KV head,
 * 64 positions per workgroup (one per lane): score = fmaf-chain over the 256
 * dims in order, times 1/16 (qwen38_model.c:854-862).  Each lane reads its K
 * row once for HPL independent chains.  scores is [rows][24][context].
 * Workgroups go to the eight XCDs round-robin; XCD x = blockIdx.x % 8 takes
 * KV head x / 2 and every other position chunk of it (chunk parity x % 2),
 * so the key rows of a KV head are read into two L2s only. */
template <int HPL>
__global__ __launch_bounds__(64) void attn_scores_kernel(float *__restrict__ scores, const float *__restrict__ q,
                                                         const float *__restrict__ key_cache, int context,
                                                         const uint32_t *__restrict__ position_ptr)
{
    constexpr int kGroups = 6 / HPL;   /* head groups per KV head */
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, lane = threadIdx.x;
    const int half_chunks = ((context + kScoreChunk - 1) / kScoreChunk + 1) / 2;
    const int hg = (xcd >> 1) * kGroups + slot % kGroups;
    const int chunk = 2 * ((slot / kGroups) % half_chunks) + (xcd & 1);
    const int t = slot / (kGroups * half_chunks);
    const int kvh = hg / kGroups, h0 = kvh * 6 + (hg % kGroups) * HPL;
    const int n = (int)*position_ptr + t + 1;
    if (chunk * kScoreChunk >= n) return;
    __shared__ float4 qs4[HPL * kAttnDim / 4];
    /* the lane's key row (position p; lanes past n read row n - 1 and store
     * nothing) in two halves of 32 quads, each requested at once; the first
     * half before the q heads are staged */
    const int p = chunk * kScoreChunk + lane;
    const float4 *k4 =
        reinterpret_cast<const float4 *>(key_cache + (size_t)(p < n ? p : n - 1) * kKVDim + kvh * kAttnDim);
    constexpr int kHalfRow = kAttnDim / 8;
    float4 kk[kHalfRow];
#pragma unroll
    for (int m = 0; m < kHalfRow; ++m) kk[m] = k4[m];
    __builtin_amdgcn_sched_barrier(0);
    {
        const float4 *q4 = reinterpret_cast<const float4 *>(q + (size_t)t * kQDim + h0 * kAttnDim);
        float4 qv[HPL];
#pragma unroll
        for (int j = 0; j < HPL; ++j) qv[j] = q4[lane + 64 * j];
#pragma unroll
        for (int j = 0; j < HPL; ++j) qs4[lane + 64 * j] = qv[j];
    }
    __syncthreads();
    float acc[HPL];
    for (int j = 0; j < HPL; ++j) acc[j] = 0.0f;
    /* the chain runs over d in order */
    for (int c = 0; c < 2; ++c) {
        if (c == 1) {
#pragma unroll
            for (int m = 0; m < kHalfRow; ++m) kk[m] = k4[kHalfRow + m];
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int m = 0; m < kHalfRow; ++m) {
            const float kv[4] = {kk[m].x, kk[m].y, kk[m].z, kk[m].w};
            for (int e = 0; e < 4; ++e) {
                const int d = (c * kHalfRow + m) * 4 + e;
                for (int j = 0; j < HPL; ++j)
                    acc[j] = __builtin_fmaf(reinterpret_cast<const float *>(qs4)[j * kAttnDim + d], kv[e], acc[j]);
            }
        }
    }
    if (p >= n) return;
    for (int j = 0; j < HPL; ++j)
        scores[((size_t)t * kAttnHeads + h0 + j) * context + p] = __fmul_rn(acc[j], 0.0625f);
}

/* Attention scores of a prompt batch: T rows x 64 positions x the six q
 * heads of one KV head per workgroup, the same fmaf chain over the 256 dims
 * in order per (row, head, position) as attn_scores_kernel.  Each lane
 * takes its key row 16 dims at a time and runs them against all T rows, so a
 * key chunk is read once per T rows instead of once per row; the q values
 * are wave-uniform and come in through scalar loads (no LDS operand per
 * multiply-add).  Same XCD placement as attn_scores_kernel; workgroups
 * whose chunk starts past the tile's last visible position exit at once. */
template <int T>
__global__ __launch_bounds__(64) void attn_scores_rows_kernel(float *__restrict__ scores, const float *__restrict__ q,
                                                              const float *__restrict__ key_cache, int context,
                                                              const uint32_t *__restrict__ position_ptr, int rows)
{
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, lane = threadIdx.x;
    const int half_chunks = ((context + kScoreChunk - 1) / kScoreChunk + 1) / 2;
    const int kvh = xcd >> 1;
    const int chunk = 2 * (slot % half_chunks) + (xcd & 1);
    const int t0 = (slot / half_chunks) * T;
    const int pos0 = (int)*position_ptr;
    const int tlast = (t0 + T < rows ? t0 + T : rows) - 1;
    const int nmax = pos0 + tlast + 1;   /* positions the tile's last row sees */
    if (t0 >= rows || chunk * kScoreChunk >= nmax) return;
    const int p = chunk * kScoreChunk + lane;
    const float4 *k4 =
        reinterpret_cast<const float4 *>(key_cache + (size_t)(p < nmax ? p : nmax - 1) * kKVDim + kvh * kAttnDim);
    float acc[T][6];
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
        for (int j = 0; j < 6; ++j) acc[tt][j] = 0.0f;
    /* rows past the batch run on the last row's q and store nothing */
    const float *qrow[T];
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
        qrow[tt] = q + (size_t)(t0 + tt < rows ? t0 + tt : rows - 1) * kQDim + kvh * 6 * kAttnDim;
    /* the chains run over d in order, 16 dims per step */
#pragma unroll 1
    for (int d0 = 0; d0 < kAttnDim; d0 += 16) {
        float4 kk[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) kk[m] = k4[d0 / 4 + m];
        const float kv[16] = {kk[0].x, kk[0].y, kk[0].z, kk[0].w, kk[1].x, kk[1].y, kk[1].z, kk[1].w,
                              kk[2].x, kk[2].y, kk[2].z, kk[2].w, kk[3].x, kk[3].y, kk[3].z, kk[3].w};
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                const float *qd = qrow[tt] + j * kAttnDim + d0;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[tt][j] = __builtin_fmaf(qd[e], kv[e], acc[tt][j]);
            }
    }
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
        const int t = t0 + tt;
        if (t >= rows || p >= pos0 + t + 1) continue;
#pragma unroll
        for (int j = 0; j < 6; ++j)
            scores[((size_t)t * kAttnHeads + kvh * 6 + j) * context + p] = __fmul_rn(acc[tt][j], 0.0625f);
    }
}

/* Softmax of q head blockIdx.x of row blockIdx.y (qwen38_model.c:863-876):
 * maximum over the scores (the reference's running max from -inf, which
 * NaN never wins); e_p = expf(score_p - max); the denominator summed in
 * position order; then the probability e_p / denominator of every position
 * written over its score, the input of attn_mix_kernel.  IN_LDS: the e_p
 * are staged in dynamic LDS for the sequential sum (context <= 32768),
 * otherwise they live in the scores row itself. */
template <bool IN_LDS>
__global__ __launch_bounds__(256) void attn_softmax_kernel(float *__restrict__ scores, int context,
                                                           const uint32_t *__restrict__ position_ptr)
{
    extern __shared__ __attribute__((aligned(16))) float lds_e[];
    __shared__ float red[4];
    __shared__ float den_s;
    __shared__ uint64_t exp_tab[32];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int n = (int)*position_ptr + t + 1;
    float *sc = scores + ((size_t)t * kAttnHeads + h) * context;
    float *e = IN_LDS ? lds_e : sc;
    /* maximum: eight score loads in flight per thread; with IN_LDS the
     * scores are kept in LDS for the exponentials */
    float local_max = -__builtin_inff();
    int p0 = tid;
    for (; p0 + 256 * 7 < n; p0 += 256 * 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = sc[p0 + 256 * k];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (IN_LDS) e[p0 + 256 * k] = v[k];
            local_max = fmaxf(local_max, v[k]);
        }
    }
    for (; p0 < n; p0 += 256) {
        const float v = sc[p0];
        if (IN_LDS) e[p0] = v;
        local_max = fmaxf(local_max, v);
    }
    for (int off = 32; off > 0; off >>= 1) local_max = fmaxf(local_max, __shfl_xor(local_max, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = local_max;
    if (tid < 32) exp_tab[tid] = q38_exp2_table_dev[tid];
    __syncthreads();
    const float maximum = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int p = tid; p < n; p += 256) e[p] = q38_expf_table(__fsub_rn(IN_LDS ? e[p] : sc[p], maximum), exp_tab);
    __syncthreads();
    if (tid == 0) {
        float d = 0.0f;
        int p = 0;
        if (IN_LDS) {
            /* position order, 32 weights per batch as 8 quads, three
             * batches in registers: batch c + 2 is read while batch c is
             * added, one LDS read between every four adds (the LDS row has
             * kSoftmaxPad floats past the context, so the read-ahead past
             * the last batch stays inside it) */
            const float4 *e4 = reinterpret_cast<const float4 *>(e);
            const int full = n / 32;
            float4 q0[8], q1[8], q2[8];
            auto step = [&d, e4](const float4 *cur, float4 *ahead, int batch) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    ahead[k] = e4[8 * batch + k];
                    d = __fadd_rn(d, cur[k].x);
                    d = __fadd_rn(d, cur[k].y);
                    d = __fadd_rn(d, cur[k].z);
                    d = __fadd_rn(d, cur[k].w);
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                }
            };
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                q0[k] = e4[k];
                q1[k] = e4[8 + k];
            }
            for (int c = 0; c < full; c += 3) {
                step(q0, q2, c + 2);
                if (c + 1 >= full) break;
                step(q1, q0, c + 3);
                if (c + 2 >= full) break;
                step(q2, q1, c + 4);
            }
            p = 32 * full;
        } else {
            /* position order; the weights of kAttnLoadBatch positions are
             * read ahead of their adds */
            for (; p + kAttnLoadBatch <= n; p += kAttnLoadBatch) {
                float a[kAttnLoadBatch];
#pragma unroll
                for (int k = 0; k < kAttnLoadBatch; ++k) a[k] = e[p + k];
#pragma unroll
                for (int k = 0; k < kAttnLoadBatch; ++k) d = __fadd_rn(d, a[k]);
            }
        }
        for (; p < n; ++p) d = __fadd_rn(d, e[p]);
        den_s = d;
    }
    __syncthreads();
    const float denominator = den_s;
    for (int p = tid; p < n; p += 256) sc[p] = div_rn(e[p], denominator);
}

/* Weighted sum of V (qwen38_model.c:877-884): out_i = fmaf-chain over the
 * positions in order of probability_p * v_p[i], then out_i *= sigmoid(gate_i).
 *
 * One workgroup per (row, q head, 64-dimension slice), so the chains of a
 * head are spread over four compute units.  Wavefront 0 runs the chains,
 * lane i that of dimension 64 * slice + i; wavefront 1 only streams: the
 * slice's channel rows of the channel-major value cache (128 contiguous
 * bytes per channel and chunk) and the probabilities go through an LDS ring
 * of kMixSlots chunks of kMixChunk positions, written by the load unit
 * itself (buffer loads with the LDS flag), up to kMixSlots - 1 chunks
 * ahead.  One barrier per chunk: at barrier c, chunk c + 1 has landed and
 * the chain wavefront has consumed chunk c - 1, whose slot the streaming
 * wavefront then refills; the chain wavefront reads chunk c + 1 into
 * registers (four positions of its channel per LDS read) while it runs the
 * links of chunk c.  The full chunks run through the pipeline; the n % 32
 * positions of a last, partial chunk are linked one by one, so no position
 * past n enters a chain.
 *
 * Workgroups go to the eight XCDs round-robin: XCD x = blockIdx.x % 8 takes
 * KV head x / 2 and the slice pair x % 2, so the value rows a KV head's
 * heads read stay in two L2s. */
constexpr int kMixChunk = 32;                              /* positions per ring slot */
constexpr int kMixSlots = 8;                               /* ring slots */
constexpr int kMixVOps = kMixChunk / 4;                    /* 1 KiB value loads per chunk */
constexpr int kMixSlotBytes = kMixChunk * 256 + 256;
constexpr int kMixLdsBytes = kMixSlots * kMixSlotBytes;
constexpr uint32_t kMixRawBuffer = 0x00020000u;   /* raw 32-bit buffer resource (gfx9) */

__device__ __forceinline__ uint32_t lds_address(const void *p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

template <int N>
__device__ __forceinline__ void mix_wait_vmcnt()
{
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ void mix_barrier() { asm volatile("s_barrier" ::: "memory"); }

/* chunk c into the ring slot at LDS address `slot`: eight value loads and
 * one probability load.  Value load j: lane i takes channel 8j + i / 8 of
 * the slice and its positions 32c + 4u .. 32c + 4u + 3 with
 * u = (i % 8) ^ (i / 8 % 8) ^ (j % 2), landing at slot + 1024 j + 16 i:
 * channel d's quad u sits at unit 64 (d / 8) + 8 (d % 8) + (u ^ s(d)),
 * s(d) = (d % 8) ^ (d / 8 % 2), so the chain's reads of one quad of 16
 * consecutive channels hit 16 different 16-byte bank groups.  v_lane[j] is the
 * lane's byte offset of its channel and quad in load j; the chunk goes into
 * the scalar offset, with c clamped to the last chunk holding positions
 * below n (`last`), so every address stays inside the layer's value block
 * whatever the range check does with the scalar offset (slots loaded past
 * the end are never read).  Probability load: lane i takes position
 * 32c + i, at slot + 8192 + 4 i; that resource ends at position n.  Inline
 * assembly, so the compiler's wait-count pass does not treat the loads as
 * LDS stores. */
__device__ __forceinline__ void mix_load_chunk(__amdgpu_buffer_rsrc_t vr, __amdgpu_buffer_rsrc_t pr,
                                               const uint32_t (&v_lane)[kMixVOps], uint32_t p_lane, int c, int last,
                                               uint32_t slot)
{
    const uint32_t chunk_off = (uint32_t)(c < last ? c : last) * (kMixChunk * 4);
#pragma unroll
    for (int j = 0; j < kMixVOps; ++j)
        asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds"
                     :: "v"(v_lane[j]), "s"(slot + 1024 * j), "s"(vr), "s"(chunk_off) : "memory", "m0");
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, 0 offen lds"
                 :: "v"(p_lane + (uint32_t)c * (kMixChunk * 4)), "s"(slot + kMixChunk * 256), "s"(pr)
                 : "memory", "m0");
}
constexpr int kMixOps = kMixVOps + 1;   /* loads per chunk */
static_assert(kMixOps * (kMixSlots - 1) <= 63, "loads in flight within the vmcnt range");

/* half a chunk of the ring (16 positions) in registers: v[k] = value of
 * position k in this lane's dimension, pr = the probabilities */
constexpr int kMixHalf = kMixChunk / 2;
struct MixHalf {
    float v[kMixHalf];
    float pr;   /* probability of position 16 half + lane % 16 of the chunk */
};

/* LDS address of channel d's quad u (positions 4u .. 4u + 3) in a slot */
__device__ __forceinline__ int mix_quad(int d, int u)
{
    return 1024 * (d >> 3) + 16 * (8 * (d & 7) + (u ^ (d & 7) ^ ((d >> 3) & 1)));
}

/* 5 LDS reads: four quads of the lane's channel and one probability per
 * lane (each 16-lane row holds the half's 16 probabilities) */
__device__ __forceinline__ void mix_read(MixHalf &r, const uint8_t *slot, int half, int lane, int pair = 0)
{
    const float *ps = reinterpret_cast<const float *>(slot + kMixChunk * 256) + pair * kMixChunk + half * kMixHalf;
    r.pr = ps[lane & 15];
#pragma unroll
    for (int k = 0; k < kMixHalf / 4; ++k) {
        const float4 q = *reinterpret_cast<const float4 *>(slot + mix_quad(lane, 4 * half + k));
        r.v[4 * k] = q.x;
        r.v[4 * k + 1] = q.y;
        r.v[4 * k + 2] = q.z;
        r.v[4 * k + 3] = q.w;
    }
}

/* the 16 links of a half in position order: o = fmaf(probability k, v[k],
 * o), probability k broadcast from lane k of each 16-lane row into the
 * fma's first operand (v_fmac_f32 with row_newbcast DPP: the same fused
 * multiply-add as fmaf).  One statement, so nothing is scheduled between
 * the links; it opens with the two wait states a DPP read of a VGPR written
 * by a VALU instruction just before needs. */
__device__ __forceinline__ float mix_links(const MixHalf &r, float o)
{
    asm volatile("s_nop 1\n\t"
                 "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf"
                 : "+v"(o)
                 : "v"(r.pr), "v"(r.v[0]), "v"(r.v[1]), "v"(r.v[2]), "v"(r.v[3]), "v"(r.v[4]), "v"(r.v[5]),
                   "v"(r.v[6]), "v"(r.v[7]), "v"(r.v[8]), "v"(r.v[9]), "v"(r.v[10]), "v"(r.v[11]), "v"(r.v[12]),
                   "v"(r.v[13]), "v"(r.v[14]), "v"(r.v[15]));
    return o;
}

/* the chain over chunk c (halves a0, a1, read earlier) while chunk c + 1
 * (landed at this chunk's barrier) is read into b0, b1: each half's links
 * wait only for that half's 12 reads, the other half's stay in flight.
 * After the last chunk the reads take a stale slot and are never used. */
__device__ __forceinline__ float mix_step(float o, const MixHalf &a0, const MixHalf &a1, MixHalf &b0, MixHalf &b1,
                                          const uint8_t *next_slot, int lane, int pair = 0)
{
    mix_barrier();
    __builtin_amdgcn_sched_barrier(0);
    o = mix_links(a0, o);
    __builtin_amdgcn_sched_barrier(0);
    mix_read(b0, next_slot, 0, lane, pair);
    __builtin_amdgcn_sched_barrier(0);
    o = mix_links(a1, o);
    __builtin_amdgcn_sched_barrier(0);
    mix_read(b1, next_slot, 1, lane, pair);
    __builtin_amdgcn_sched_barrier(0);
    return o;
}

/* The chain wavefront's part of the mix: the links of positions 0 .. n - 1
 * of its channel from the ring (chunk c in slot c % kMixSlots, probability
 * record `pair` of each slot), one barrier per chunk as the streaming
 * wavefront's (the chain of attn_mix_kernel). */
__device__ __forceinline__ float mix_chain(const uint8_t *ring, int slot_bytes, int n, int lane, int pair)
{
    const int full = n / kMixChunk, rest = n % kMixChunk;
    MixHalf a0, a1, b0, b1;
    mix_barrier();
    mix_read(a0, ring, 0, lane, pair);
    mix_read(a1, ring, 1, lane, pair);
    float o = 0.0f;
    int c = 0;
    static_assert(kMixSlots == 8, "the unrolled loop takes one ring turn per iteration");
#pragma unroll 1
    for (; c + kMixSlots <= full; c += kMixSlots) {
        o = mix_step(o, a0, a1, b0, b1, ring + 1 * slot_bytes, lane, pair);
        o = mix_step(o, b0, b1, a0, a1, ring + 2 * slot_bytes, lane, pair);
        o = mix_step(o, a0, a1, b0, b1, ring + 3 * slot_bytes, lane, pair);
        o = mix_step(o, b0, b1, a0, a1, ring + 4 * slot_bytes, lane, pair);
        o = mix_step(o, a0, a1, b0, b1, ring + 5 * slot_bytes, lane, pair);
        o = mix_step(o, b0, b1, a0, a1, ring + 6 * slot_bytes, lane, pair);
        o = mix_step(o, a0, a1, b0, b1, ring + 7 * slot_bytes, lane, pair);
        o = mix_step(o, b0, b1, a0, a1, ring, lane, pair);
    }
#pragma unroll 1
    for (; c + 2 <= full; c += 2) {
        o = mix_step(o, a0, a1, b0, b1, ring + ((c + 1) % kMixSlots) * slot_bytes, lane, pair);
        o = mix_step(o, b0, b1, a0, a1, ring + ((c + 2) % kMixSlots) * slot_bytes, lane, pair);
    }
    if (c < full) o = mix_step(o, a0, a1, b0, b1, ring + ((c + 1) % kMixSlots) * slot_bytes, lane, pair);
    if (rest) {
        /* the partial last chunk (landed at the previous barrier), link by
         * link up to position n - 1 */
        mix_barrier();
        const uint8_t *slot = ring + (full % kMixSlots) * slot_bytes;
        const float *ps = reinterpret_cast<const float *>(slot + kMixChunk * 256) + pair * kMixChunk;
        for (int k = 0; k < rest; ++k)
            o = __builtin_fmaf(ps[k], *reinterpret_cast<const float *>(slot + mix_quad(lane, k >> 2) + 4 * (k & 3)), o);
    }
    return o;
}

__global__ __launch_bounds__(128) void attn_mix_kernel(float *__restrict__ out, const float *__restrict__ prob,
                                                       const float *__restrict__ q_and_gate, long long qg_stride,
                                                       const float *__restrict__ value_cache, int context,
                                                       const uint32_t *__restrict__ position_ptr)
{
    __shared__ __attribute__((aligned(16))) uint8_t ring[kMixLdsBytes];
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3, lane = threadIdx.x & 63;
    const int kvh = xcd >> 1, slice = 2 * (xcd & 1) + ((j / 6) & 1);
    const int h = kvh * 6 + j % 6, t = j / 12;
    const int n = (int)*position_ptr + t + 1;
    const int chunks = (n + kMixChunk - 1) / kMixChunk;
    const uint32_t pitch4 = value_pitch((uint32_t)context) * 4u;
    if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) == 1) {
        /* streaming wavefront */
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(value_cache), 0, (int)(kKVDim * pitch4), kMixRawBuffer);
        const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(prob + ((size_t)t * kAttnHeads + h) * context), 0, n * 4, kMixRawBuffer);
        uint32_t v_lane[kMixVOps];
#pragma unroll
        for (int jj = 0; jj < kMixVOps; ++jj)
            v_lane[jj] = (uint32_t)(kvh * kAttnDim + 64 * slice + 8 * jj + (lane >> 3)) * pitch4 +
                         16u * (uint32_t)((lane & 7) ^ ((lane >> 3) & 7) ^ (jj & 1));
        const uint32_t p_lane = (uint32_t)lane * 4u;
        const uint32_t ring_base = __builtin_amdgcn_readfirstlane(lds_address(ring));
        const int last = chunks - 1;
#pragma unroll
        for (int c = 0; c < kMixSlots - 1; ++c)
            mix_load_chunk(vr, pr, v_lane, p_lane, c, last, ring_base + c * kMixSlotBytes);
        /* loads retire in order */
        mix_wait_vmcnt<kMixOps * (kMixSlots - 2)>();   /* chunk 0 */
        mix_barrier();
#pragma unroll 1
        for (int c = 0; c < chunks; ++c) {
            mix_wait_vmcnt<kMixOps * (kMixSlots - 3)>();   /* chunk c + 1 */
            mix_barrier();
            /* chunk c - 1 is consumed: its slot takes chunk c + kMixSlots - 1 */
            mix_load_chunk(vr, pr, v_lane, p_lane, c + kMixSlots - 1, last,
                           ring_base + ((c + kMixSlots - 1) % kMixSlots) * kMixSlotBytes);
        }
        mix_wait_vmcnt<0>();
        return;
    }
    /* chain wavefront: one barrier per chunk, as the streaming wavefront;
     * the gate is read before the chain so that its load is not waited
     * for after it */
    const float g = q_and_gate[(size_t)t * qg_stride + h * 2 * kAttnDim + kAttnDim + 64 * slice + lane];
    const float o = mix_chain(ring, kMixSlotBytes, n, lane, 0);
    const int dim = h * kAttnDim + 64 * slice + lane;
    out[(size_t)t * kQDim + dim] = __fmul_rn(o, sigmoidf_exact(g));
}

/* rows per workgroup of attn_mix_tile_kernel */
constexpr int kMixTileRows = 4;

/* attn_mix_kernel for prompt batches, register form: one 64-lane workgroup
 * per (KV head, 64-channel slice, R rows); lane = channel, and the lane runs
 * the 6 q heads x R rows of its channel as 6 R chains o = fmaf(prob, v, o)
 * over positions 0 .. n_row - 1 in order (the chain of attn_mix_kernel).
 * Each value is loaded once into a register and serves all 6 R chains; the
 * probabilities are wave-uniform and come in through scalar loads, 16
 * positions at a time while every row of the tile is still inside its
 * positions, then position by position to each row's end.  Tiles of later
 * rows (longer chains) are dispatched first. */
template <int R>
__global__ __launch_bounds__(64) void attn_mix_tile_kernel(float *__restrict__ out, const float *__restrict__ prob,
                                                           const float *__restrict__ q_and_gate, long long qg_stride,
                                                           const float *__restrict__ value_cache, int context,
                                                           const uint32_t *__restrict__ position_ptr, int rows)
{
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3, lane = threadIdx.x;
    const int kvh = xcd >> 1, slice = 2 * (xcd & 1) + (j & 1);
    const int tiles = (rows + R - 1) / R;
    const int t0 = (tiles - 1 - (j >> 1)) * R;
    if (t0 < 0) return;
    const int pos0 = (int)*position_ptr;
    const int nr = rows - t0 < R ? rows - t0 : R;
    const int nmin = pos0 + t0 + 1, nmax = pos0 + t0 + nr;
    const float *vrow = value_cache + (size_t)(kvh * kAttnDim + 64 * slice + lane) * value_pitch((uint32_t)context);
    /* probability rows of (row t0 + tt, head kvh * 6 + jh): prow[tt] + jh *
     * context; rows past the batch read row t0 and store nothing */
    const float *prow[R];
#pragma unroll
    for (int tt = 0; tt < R; ++tt)
        prow[tt] = prob + ((size_t)(t0 + (tt < nr ? tt : 0)) * kAttnHeads + kvh * 6) * context;
    float acc[R][6];
#pragma unroll
    for (int tt = 0; tt < R; ++tt)
#pragma unroll
        for (int jh = 0; jh < 6; ++jh) acc[tt][jh] = 0.0f;
    int p0 = 0;
#pragma unroll 1
    for (; p0 + 16 <= nmin; p0 += 16) {
        float4 v4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) v4[m] = reinterpret_cast<const float4 *>(vrow + p0)[m];
        const float v[16] = {v4[0].x, v4[0].y, v4[0].z, v4[0].w, v4[1].x, v4[1].y, v4[1].z, v4[1].w,
                             v4[2].x, v4[2].y, v4[2].z, v4[2].w, v4[3].x, v4[3].y, v4[3].z, v4[3].w};
#pragma unroll
        for (int tt = 0; tt < R; ++tt)
#pragma unroll
            for (int jh = 0; jh < 6; ++jh) {
                const float *pp = prow[tt] + (size_t)jh * context + p0;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[tt][jh] = __builtin_fmaf(pp[e], v[e], acc[tt][jh]);
            }
    }
    /* the last positions, each row up to its own end */
#pragma unroll 1
    for (; p0 < nmax; ++p0) {
        const float v = vrow[p0];
#pragma unroll
        for (int tt = 0; tt < R; ++tt) {
            if (tt >= nr || p0 >= nmin + tt) continue;
#pragma unroll
            for (int jh = 0; jh < 6; ++jh) acc[tt][jh] = __builtin_fmaf(prow[tt][(size_t)jh * context + p0], v,
                                                                        acc[tt][jh]);
        }
    }
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        if (tt >= nr) break;
        const int t = t0 + tt;
#pragma unroll
        for (int jh = 0; jh < 6; ++jh) {
            const int h = kvh * 6 + jh;
            const float g = q_and_gate[(size_t)t * qg_stride + h * 2 * kAttnDim + kAttnDim + 64 * slice + lane];
            out[(size_t)t * kQDim + h * kAttnDim + 64 * slice + lane] = __fmul_rn(acc[tt][jh], sigmoidf_exact(g));
        }
    }
}

/* ---- launchers ----------------------------------------------------------- */

void launch_norm_quant(float *norm_out, long long norm_stride, uint8_t *q_out, int q_stride_blocks, float *hidden,
                       long long in_stride, const float *branch, const float *weight, int rows, hipStream_t stream)
{
    if (branch)
        norm_quant_kernel<2, true><<<rows, kNormThreads, 0, stream>>>(norm_out, norm_stride, q_out, q_stride_blocks,
                                                                       hidden, in_stride, branch, weight);
    else
        norm_quant_kernel<2, false><<<rows, kNormThreads, 0, stream>>>(norm_out, norm_stride, q_out, q_stride_blocks,
                                                                        hidden, in_stride, nullptr, weight);
}

void launch_add(float *hidden, const float *branch, long long n, hipStream_t stream)
{
    add_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(hidden, branch, n);
}

void launch_swiglu_quant(uint8_t *q_out, const float *gate, const float *up, long long stride, int rows,
                         hipStream_t stream, float *f_out)
{
    const int nblocks = rows * (kFFNWidth / 256);
    swiglu_quant_kernel<<<(nblocks + 3) / 4, 256, 0, stream>>>(q_out, gate, up, stride, nblocks, f_out);
}

void launch_embed_q4k(float *out, const uint8_t *w, const uint32_t *tokens, int count, int width, uint32_t vocab,
                      hipStream_t stream)
{
    embed_q4k_kernel<<<dim3(width / 256, count), 256, 0, stream>>>(out, w, tokens, width / 256, vocab);
}

void launch_deltanet_prep(float *qkv, long long ld, int beta_off, int alpha_off, float *conv_state,
                          long long slot_stride, const uint32_t *slot, int rows, const float *conv_w,
                          const float *ssm_a, const float *ssm_dt, bool last_only, hipStream_t stream)
{
    deltanet_prep_kernel<<<kQKV / 128 + 1, 128, 0, stream>>>(qkv, ld, beta_off, alpha_off, conv_state, slot_stride,
                                                             slot, rows, conv_w, ssm_a, ssm_dt, last_only ? 1 : 0);
}

void launch_deltanet_prep_rows(float *out, const float *qkv, long long ld, int beta_off, int alpha_off,
                               float *conv_state, long long slot_stride, const uint32_t *slot, int rows,
                               const float *conv_w, const float *ssm_a, const float *ssm_dt, hipStream_t stream)
{
    deltanet_prep_rows_kernel<<<dim3(kQKV / 128 + 1, (rows + kPrepRows - 1) / kPrepRows), 128, 0, stream>>>(
        out, qkv, ld, beta_off, alpha_off, conv_state, slot_stride, slot, rows, conv_w, ssm_a, ssm_dt);
}

void launch_deltanet_state(float *attn, float *delta_state, long long slot_stride, const uint32_t *slot, int rows,
                           const float *qkv, long long ld, int beta_off, int alpha_off, float query_scale,
                           bool last_only, hipStream_t stream)
{
    deltanet_state_kernel<<<kVHeads * kHeadDim / kScan16Cols, 256, 0, stream>>>(
        attn, delta_state, slot_stride, slot, rows, qkv, ld, beta_off, alpha_off, query_scale, last_only ? 1 : 0);
}

bool launch_deltanet_fused(float *attn, float *delta_state, long long slot_stride, const uint32_t *slot, int rows,
                           const float *qkv, long long ld, int beta_off, int alpha_off, float query_scale,
                           float *conv_state, long long conv_stride, const float *conv_w, const float *ssm_a,
                           const float *ssm_dt, hipStream_t stream)
{
    if (rows < 1 || rows > kFusedRows) return false;
    deltanet_fused_kernel<<<kVHeads * kHeadDim / kFusedCols, 256, 0, stream>>>(attn, delta_state, slot_stride, slot, rows, qkv,
                                                                     ld, beta_off, alpha_off, query_scale, conv_state,
                                                                     conv_stride, conv_w, ssm_a, ssm_dt);
    return true;
}

void launch_deltanet_out_quant(float *attn, uint8_t *q_out, const float *z, long long z_stride, const float *ssm_norm,
                               int rows, hipStream_t stream)
{
    deltanet_out_quant_kernel<<<dim3(kVHeads / 2, rows), 256, 0, stream>>>(attn, q_out, z, z_stride, ssm_norm);
}

/* The dynamic-LDS limit of the in-LDS softmax kernel is a per-device
 * attribute of the function: it only ever grows, to the largest context
 * configured so far on the device, so a later model or call with a smaller
 * context never lowers it under an earlier one. */
bool configure_attention(int context)
{
    static std::mutex mutex;
    static std::vector<int> configured;
    if (context < 1 || (uint32_t)context > kMaxAttentionContext) return false;
    if (context > kMaxLdsPositions) return true;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return false;
    std::lock_guard<std::mutex> lock(mutex);
    if ((int)configured.size() <= device) configured.resize(device + 1, 0);
    if (context <= configured[device]) return true;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_softmax_kernel<true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (context + kSoftmaxPad) * 4) != hipSuccess)
        return false;
    configured[device] = context;
    return true;
}

/* RoPE table of positions [0, context): cos then sin of the 32 pair angles.
 * theta starts at the position and is multiplied by powf(1e7, -2/64) per
 * pair; cosf/sinf of the host C library, exactly the values q38_rope
 * computes (qwen38_model.c:697-713). */
void rope_table_host(float *table, uint32_t context)
{
    const float theta_scale = powf(10000000.0f, -2.0f / 64.0f);
    for (uint32_t pos = 0; pos < context; ++pos) {
        float theta = (float)pos;
        for (int pair = 0; pair < 32; ++pair) {
            table[(size_t)pos * 64 + pair] = cosf(theta);
            table[(size_t)pos * 64 + 32 + pair] = sinf(theta);
            theta *= theta_scale;
        }
    }
}

void launch_attention(float *attn, uint8_t *q_out, float *q_buf, const float *q_and_gate, const float *key,
                      const float *value, long long in_stride, const float *q_norm, const float *k_norm,
                      const float *rope, float *key_cache, float *value_cache, float *scores, int context,
                      const uint32_t *position, int rows, hipStream_t stream)
{
    attn_prep_kernel<<<dim3(kAttnHeads + kKVHeads + 1, rows), 256, 0, stream>>>(
        q_buf, q_and_gate, key, value, in_stride, q_norm, k_norm, rope, key_cache, value_cache,
        (int)value_pitch((uint32_t)context), position, 0);
    {
        const int half_chunks = ((context + kScoreChunk - 1) / kScoreChunk + 1) / 2;
        if (rows > (int)kRecurrentStateSlots - 1)
            attn_scores_rows_kernel<kScoreRows><<<dim3(8 * half_chunks * ((rows + kScoreRows - 1) / kScoreRows)), 64, 0,
                                                  stream>>>(scores, q_buf, key_cache, context, position, rows);
        else
            attn_scores_kernel<kScoreHeadsPerLane>
                <<<dim3(8 * (6 / kScoreHeadsPerLane) * half_chunks * rows), 64, 0, stream>>>(scores, q_buf, key_cache,
                                                                                            context, position);
    }
    if (context <= kMaxLdsPositions)
        attn_softmax_kernel<true><<<dim3(kAttnHeads, rows), 256, (size_t)(context + kSoftmaxPad) * 4, stream>>>(scores, context,
                                                                                              position);
    else
        attn_softmax_kernel<false><<<dim3(kAttnHeads, rows), 256, 0, stream>>>(scores, context, position);
    /* the row-group kernel only for prompt batches: at decode batches its
     * few workgroups lose to one workgroup per (row, head group, slice)
     * (3 rows: 40.3 against 23.1 us at a 4K cache, 8.8 against 6.2 us at
     * 512 positions) */
    if (rows > (int)kRecurrentStateSlots - 1)
        attn_mix_tile_kernel<kMixTileRows><<<dim3(16 * ((rows + kMixTileRows - 1) / kMixTileRows)), 64, 0, stream>>>(
            attn, scores, q_and_gate, in_stride, value_cache, context, position, rows);
    else
        attn_mix_kernel<<<dim3(8 * 12 * rows), 128, 0, stream>>>(attn, scores, q_and_gate, in_stride, value_cache,
                                                                context, position);
    launch_quantize(attn, q_out, (uint32_t)(rows * kAttnHeads), stream);
}

void launch_kv_write(const float *key, const float *value, long long in_stride, const float *k_norm,
                     const float *rope, float *key_cache, float *value_cache, int context, const uint32_t *position,
                     int rows, hipStream_t stream)
{
    attn_prep_kernel<<<dim3(kKVHeads + 1, rows), 256, 0, stream>>>(nullptr, nullptr, key, value, in_stride, nullptr,
                                                                  k_norm, rope, key_cache, value_cache,
                                                                  (int)value_pitch((uint32_t)context), position,
                                                                  kAttnHeads);
}

}  // namespace q38
