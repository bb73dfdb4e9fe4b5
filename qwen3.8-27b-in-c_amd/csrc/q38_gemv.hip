/* Lane-chain GEMV / small-M GEMM for Q4_K and Q6_K weights against Q8_K
 * activations on gfx950 (the decode kernel).
 *
 * The reference's AVX2 kernels keep eight fp32 accumulator lanes per row
 * (plus four min lanes for Q4_K) and, for every super-block in order, add
 * d_b * W[b][l] to lane l, where W[b][l] is an exact integer over a fixed
 * 32-element subset of the block (src/qwen38/qwen38_quant.c:1546-1634 for
 * Q4_K, :1727-1833 for Q6_K).  Here eight GPU lanes own the eight
 * accumulator lanes of a row: each computes its own W[b][l] with
 * v_dot4_i32_i8 from 16 bytes of packed quants and runs the fmaf chain in a
 * register right away, so the integer and fp32 phases need no exchange.
 * A wavefront holds 8 rows; the loads of the next P blocks of its rows are
 * in flight while the current block is computed.
 *
 * Activations (all M tokens, all blocks) are staged once per workgroup in
 * LDS, with the quants of each block permuted so that the 32 bytes a lane
 * needs are contiguous (two 16-byte LDS reads).
 */
#include "q38_device.h"

namespace q38 {

namespace {

constexpr int kActStride = 304;   /* bytes per staged Q8_K block: quants 256, sums 32, scale 4, pad */
constexpr int kSumsOff = 256;
constexpr int kScaleOff = 288;

/* destination dword of source quant dword d (elements 4d..4d+3) */
template <int TYPE>
__device__ __forceinline__ int perm_dword(int d)
{
    if (TYPE == kQ4K) {
        /* element 64c + 32h + 4l + u -> lane l, slot 2c + h */
        const int c = d >> 4, h = (d >> 3) & 1, l = d & 7;
        return 8 * l + 2 * c + h;
    }
    /* Q6_K: element 128h + 32j + 4l + u -> lane l, slot 4h + j */
    const int h = d >> 5, j = (d >> 3) & 3, l = d & 7;
    return 8 * l + 4 * h + j;
}

/* Copy the MT x nb Q8_K blocks into LDS (permuted quants, sums, scale),
 * eight dwords per thread in flight at a time. */
template <int TYPE>
__device__ __forceinline__ void stage(uint8_t *act, const uint8_t *x, int count)
{
    constexpr int kDepth = 8;
    const int nthreads = blockDim.x;
    const int total = count * 73;   /* 73 dwords per block: scale, 64 quants, 8 sums */
    const uint32_t *src = reinterpret_cast<const uint32_t *>(x);
    for (int i0 = threadIdx.x; i0 < total; i0 += kDepth * nthreads) {
        uint32_t v[kDepth];
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            const int i = i0 + u * nthreads;
            if (i < total) v[u] = src[i];
        }
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            const int i = i0 + u * nthreads;
            if (i < total) {
                const int blk = i / 73, d = i - blk * 73;
                int o;
                if (d == 0) o = kScaleOff / 4;
                else if (d <= 64) o = perm_dword<TYPE>(d - 1);
                else o = kSumsOff / 4 + (d - 65);
                reinterpret_cast<uint32_t *>(act + (size_t)blk * kActStride)[o] = v[u];
            }
        }
    }
}

/* one lane's share of a block: Q4_K quants dwords at 16 + 32c + 4l and the
 * 16-byte header; Q6_K ql dwords at 4l, 32+4l, 64+4l, 96+4l, qh dwords at
 * 128+4l, 160+4l, scales (16 bytes) and d */
template <int TYPE> struct Lane;

template <> struct Lane<kQ4K> {
    uint32_t q[4];
    uint4 hdr;
    __device__ __forceinline__ void load(const uint8_t *blk, int l)
    {
        hdr = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *reinterpret_cast<const uint32_t *>(blk + 16 + 32 * c + 4 * l);
    }
    __device__ __forceinline__ void zero()
    {
        hdr = make_uint4(0, 0, 0, 0);
        q[0] = q[1] = q[2] = q[3] = 0;
    }
};

__device__ __forceinline__ uint32_t ld32(const uint8_t *p)
{
    uint32_t v;
    __builtin_memcpy(&v, p, 4);   /* Q6_K blocks are 2-byte aligned */
    return v;
}

template <> struct Lane<kQ6K> {
    uint32_t ql[4], qh[2];
    uint32_t sc[4];
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *blk, int l)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i) ql[i] = ld32(blk + 32 * i + 4 * l);
        qh[0] = ld32(blk + 128 + 4 * l);
        qh[1] = ld32(blk + 160 + 4 * l);
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = ld32(blk + 192 + 4 * i);
        d = *reinterpret_cast<const uint16_t *>(blk + 208);
    }
    __device__ __forceinline__ void zero()
    {
        ql[0] = ql[1] = ql[2] = ql[3] = qh[0] = qh[1] = 0;
        sc[0] = sc[1] = sc[2] = sc[3] = 0;
        d = 0;
    }
};

__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ int sbyte_of(uint32_t w, int i) { return (int)(int8_t)((w >> (8 * i)) & 0xffu); }

/* Q4_K, lane l: W = sum_c sc[2c]*dot(lo nibbles, a) + sc[2c+1]*dot(hi nibbles, a);
 * lanes 0..3 also M = m[2l]*(s[4l]+s[4l+1]) + m[2l+1]*(s[4l+2]+s[4l+3])
 * (src/qwen38/qwen38_quant.c:1569-1620, scale/min unpacking :131-143). */
struct Q4KDecoded {
    int sc[8];
    int m0, m1;
    float d, dmin;
};

__device__ __forceinline__ Q4KDecoded q4k_decode(const Lane<kQ4K> &r, int l)
{
    Q4KDecoded o;
    const uint32_t Y = r.hdr.y, Z = r.hdr.z, Wd = r.hdr.w;
    const uint32_t sc_hi = (Wd & 0x0f0f0f0fu) | ((Y >> 2) & 0x30303030u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o.sc[i] = (int)((Y >> (8 * i)) & 63u);
        o.sc[4 + i] = byte_of(sc_hi, i);
    }
    const uint32_t m_lo = Z & 0x3f3f3f3fu;
    const uint32_t m_hi = ((Wd >> 4) & 0x0f0f0f0fu) | ((Z >> 2) & 0x30303030u);
    /* lane l < 4 uses sub-blocks 2l, 2l+1 */
    const uint32_t mw = (l & 2) ? m_hi : m_lo;
    const int sh = 16 * (l & 1);
    o.m0 = (int)((mw >> sh) & 0xffu);
    o.m1 = (int)((mw >> (sh + 8)) & 0xffu);
    o.d = f16_to_f32(r.hdr.x);
    o.dmin = f16_to_f32(r.hdr.x >> 16);
    return o;
}

__device__ __forceinline__ int q4k_w(const Lane<kQ4K> &r, const Q4KDecoded &dec, const uint8_t *a, int l)
{
    const int4 a0 = *reinterpret_cast<const int4 *>(a + 32 * l);
    const int4 a1 = *reinterpret_cast<const int4 *>(a + 32 * l + 16);
    const int av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    int w = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int lo = (int)(r.q[c] & 0x0f0f0f0fu);
        const int hi = (int)((r.q[c] >> 4) & 0x0f0f0f0fu);
        w = mad24(dot4z(lo, av[2 * c]), dec.sc[2 * c], w);
        w = mad24(dot4z(hi, av[2 * c + 1]), dec.sc[2 * c + 1], w);
    }
    return w;
}

__device__ __forceinline__ int q4k_m(const Q4KDecoded &dec, const uint8_t *a, int l)
{
    const uint2 s = *reinterpret_cast<const uint2 *>(a + kSumsOff + 8 * (l & 3));
    const int p0 = (int)(int16_t)(s.x & 0xffffu) + ((int)s.x >> 16);
    const int p1 = (int)(int16_t)(s.y & 0xffffu) + ((int)s.y >> 16);
    return mad24(dec.m0, p0, mul24(dec.m1, p1));
}

/* Q6_K, lane l: W = sum_{h,j} scale[8h+2j+(l>=4)] * dot(q6(h,j,4l..4l+3), a)
 * - 32*(s[2l]*scale[2l] + s[2l+1]*scale[2l+1])  (:1741-1814) */
__device__ __forceinline__ int q6k_w(const Lane<kQ6K> &r, const uint8_t *a, int l)
{
    const int4 a0 = *reinterpret_cast<const int4 *>(a + 32 * l);
    const int4 a1 = *reinterpret_cast<const int4 *>(a + 32 * l + 16);
    const int av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const int upper = l >= 4 ? 1 : 0;
    int w = 0;
    /* every r.sc[] index is a compile-time constant (a lane-dependent index
     * would keep the array in scratch memory): scale 8h + 2j + upper is
     * byte 2(j & 1) + upper of word 2h + j/2 */
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t low = r.ql[2 * h + (j & 1)];
            const uint32_t lo4 = (j < 2 ? low : (low >> 4)) & 0x0f0f0f0fu;
            const uint32_t hi2 = ((r.qh[h] >> (2 * j)) & 0x03030303u) << 4;
            const int q = (int)(lo4 | hi2);
            w = mad24(dot4z(q, av[4 * h + j]), sbyte_of(r.sc[2 * h + (j >> 1)], 2 * (j & 1) + upper), w);
        }
    }
    const uint32_t s = *reinterpret_cast<const uint32_t *>(a + kSumsOff + 4 * l);
    const int s0 = (int)(int16_t)(s & 0xffffu), s1 = (int)s >> 16;
    /* scales 2l and 2l + 1: bytes 2(l & 1), 2(l & 1) + 1 of word l / 2 */
    const uint32_t sw = (l & 4) ? ((l & 2) ? r.sc[3] : r.sc[2]) : ((l & 2) ? r.sc[1] : r.sc[0]);
    const int b0 = 2 * (l & 1);
    const int offset = 32 * mad24(s0, sbyte_of(sw, b0), mul24(s1, sbyte_of(sw, b0 + 1)));
    return w - offset;
}

}  // namespace

template <int TYPE, int MT, int P>
__global__ __launch_bounds__(256) void gemv_lanes(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                  float *__restrict__ y, uint32_t ldy, uint32_t rows, uint32_t nb)
{
    constexpr int BB = TYPE == kQ4K ? 144 : 210;
    extern __shared__ __align__(16) uint8_t act[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l = lane & 7, rw = lane >> 3;
    const uint32_t row = (blockIdx.x * 4u + (uint32_t)wave) * 8u + (uint32_t)rw;
    const bool row_ok = row < rows;
    const uint8_t *rowp = w + (size_t)(row_ok ? row : 0) * nb * BB;
    const int steps = (int)nb;

    Lane<TYPE> ring[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        if (row_ok && i < steps) ring[i].load(rowp + (size_t)i * BB, l);
        else ring[i].zero();
    }
    stage<TYPE>(act, x, MT * (int)nb);
    __syncthreads();

    float acc[MT], accm[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = accm[t] = 0.0f;

    for (int k0 = 0; k0 < steps; k0 += P) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int k = k0 + i;
            if (k >= steps) break;
            const Lane<TYPE> cur = ring[i];
            /* refill this slot with block k + P */
            if (row_ok && k + P < steps) ring[i].load(rowp + (size_t)(k + P) * BB, l);
            const int bs = k;
            float dw[MT], dm[MT];
            int iw[MT], im[MT];
            if constexpr (TYPE == kQ4K) {
                const Q4KDecoded dec = q4k_decode(cur, l);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const uint8_t *a = act + ((size_t)t * nb + bs) * kActStride;
                    const float xs = *reinterpret_cast<const float *>(a + kScaleOff);
                    iw[t] = q4k_w(cur, dec, a, l);
                    im[t] = q4k_m(dec, a, l);
                    dw[t] = fmul_rn(dec.d, xs);
                    dm[t] = -fmul_rn(dec.dmin, xs);
                }
            } else {
                const float d = f16_to_f32(cur.d);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const uint8_t *a = act + ((size_t)t * nb + bs) * kActStride;
                    const float xs = *reinterpret_cast<const float *>(a + kScaleOff);
                    iw[t] = q6k_w(cur, a, l);
                    im[t] = 0;
                    dw[t] = fmul_rn(d, xs);
                    dm[t] = 0.0f;
                }
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                acc[t] = __builtin_fmaf(dw[t], (float)iw[t], acc[t]);
                if (TYPE == kQ4K) accm[t] = __builtin_fmaf(dm[t], (float)im[t], accm[t]);
            }
        }
    }

    /* horizontal trees of the AVX2 build (qwen38_quant.c:303-310, 1626-1630)
     * over the 8 lanes of group 0: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)),
     * plus ((m0+m2)+(m1+m3)) for Q4_K */
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        float v = acc[t];
        v = fadd_rn(v, __shfl_down(v, 4, 8));
        v = fadd_rn(v, __shfl_down(v, 2, 8));
        v = fadd_rn(v, __shfl_down(v, 1, 8));
        if (TYPE == kQ4K) {
            float m = accm[t];
            m = fadd_rn(m, __shfl_down(m, 2, 8));
            m = fadd_rn(m, __shfl_down(m, 1, 8));
            v = fadd_rn(v, m);
        }
        if (row_ok && l == 0) y[(size_t)t * ldy + row] = v;
    }
}

/* Launch the lane-chain kernel if it applies: Q4_K / Q6_K with 2..4 tokens
 * whose activations fit in LDS (measured on MI355X: at one token the
 * two-phase kernels of q38_gemm.hip are as fast or faster; from two tokens
 * on this kernel's per-token cost is lower).  Returns false otherwise. */
template <int TYPE, int MT>
static bool launch_lanes_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                               uint32_t nb, hipStream_t stream)
{
    const size_t lds = (size_t)MT * nb * kActStride;
    if (MT < 2 || lds > 64 * 1024) return false;
    /* one row per 8 lanes, 32 rows per workgroup; P = 6 blocks in flight per
     * row (measured on the 3-row Q6_K LM head: 4 was 0.3 % slower in decode) */
    const dim3 grid((rows + 31) / 32);
    hipLaunchKernelGGL((gemv_lanes<TYPE, MT, 6>), grid, dim3(256), lds, stream, w, x, y, ldy, rows, nb);
    return true;
}

template <int TYPE>
static bool launch_lanes_m(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, hipStream_t stream)
{
    switch (m) {
    case 1: return launch_lanes_typed<TYPE, 1>(w, x, y, ldy, rows, nb, stream);
    case 2: return launch_lanes_typed<TYPE, 2>(w, x, y, ldy, rows, nb, stream);
    case 3: return launch_lanes_typed<TYPE, 3>(w, x, y, ldy, rows, nb, stream);
    case 4: return launch_lanes_typed<TYPE, 4>(w, x, y, ldy, rows, nb, stream);
    default: return false;
    }
}

bool launch_gemv_lanes(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                       uint32_t nb, hipStream_t stream)
{
    if (type == kQ4K) return launch_lanes_m<kQ4K>(m, w, x, y, ldy, rows, nb, stream);
    if (type == kQ6K) return launch_lanes_m<kQ6K>(m, w, x, y, ldy, rows, nb, stream);
    return false;
}

}  // namespace q38
