/* Quantised GEMV / small-M GEMM against Q8_K activations on gfx950.
 *
 * Computes what q38_tensor_gemv_q8_k / q38_tensor_gemm_q8_k compute
 * (src/qwen38/qwen38_quant.c:2833-3169 of the reference) for Q4_K, Q6_K and
 * IQ1_M weights, bit-identically to its x86 AVX2 build.
 *
 * Work split.  A workgroup owns `rw` consecutive weight rows and walks their
 * super-blocks in chunks of `ch` blocks:
 *   stage    the chunk's Q8_K activation blocks for every token into LDS;
 *   phase 1  every (row, block) pair of the chunk goes to a lane quad.  The
 *            quad streams the packed block from HBM with 16-byte loads,
 *            dequantises in registers and forms the block's exact int32 sums
 *            with v_dot4_i32_i8, reduced across the quad with DPP.  The sums
 *            land in LDS, one 16-dword slot per (pair, token);
 *   phase 2  "chain" lanes replay the reference's fp32 accumulation over the
 *            chunk's blocks in order: one lane per AVX2 accumulator lane
 *            (Q4_K: 8 weighted + 4 min lanes, Q6_K: 8, IQ1_M: 1 scalar), each
 *            a sequential fmaf chain, so the K dimension is split across
 *            lanes for the integer work but never for the fp32 work.
 * After the last chunk the chain lanes of a (row, token) combine with the
 * reference's fixed horizontal-add tree and write output[token * rows + row].
 */
#include "q38_device.h"

namespace q38 {

constexpr int kActStride = 304;  /* staged Q8_K block: 256 q, 16 sums, scale, pad */
constexpr int kActSumsOff = 256;
constexpr int kActScaleOff = 288;
constexpr int kSlot = 16;        /* dwords per (pair, token) result slot */

template <int TYPE> struct Format;
template <> struct Format<kQ4K> { static constexpr int bytes = 144, chains = 12, group = 16; };
template <> struct Format<kQ6K> { static constexpr int bytes = 210, chains = 8, group = 16; };
template <> struct Format<kIQ1M> { static constexpr int bytes = 56, chains = 1, group = 1; };

/* Copy the chunk's Q8_K blocks (AoS, 292-byte stride, 4-byte aligned) into
 * LDS with a 304-byte stride: quants at 0, sums at 256, scale at 288. */
__device__ __forceinline__ void stage_activations(uint8_t *act, const uint8_t *x, int tokens,
                                                  uint32_t nblk, uint32_t b0, int cb)
{
    const int total = tokens * cb * 73;
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int slot = i / 73, w = i - slot * 73;
        const int t = slot / cb, bl = slot - t * cb;
        const uint32_t *src = reinterpret_cast<const uint32_t *>(
            x + (static_cast<size_t>(t) * nblk + b0 + bl) * kQ8KBytes);
        const uint32_t v = src[w];
        int dst;
        if (w == 0) dst = kActScaleOff / 4;
        else if (w <= 64) dst = w - 1;
        else dst = kActSumsOff / 4 + (w - 65);
        reinterpret_cast<uint32_t *>(act + slot * kActStride)[dst] = v;
    }
}

/* ---- Q4_K --------------------------------------------------------------- */

/* Integer lanes of one Q4_K block (src/qwen38/qwen38_quant.c:1564-1620).
 * Quad lane j owns nibble chunk c = j: bytes 32j..32j+31 of qs, activation
 * elements 64j..64j+63, sub-blocks 2j (low nibbles) and 2j+1 (high). */
template <int MT>
__device__ __forceinline__ void q4k_pair(const uint8_t *blk, const uint8_t *act_chunk, int cb,
                                         int bl, int *res, int j)
{
    const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
    const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * j);
    const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * j);

    /* q38_scale_min_k4 for indices 2j and 2j+1 (qwen38_quant.c:131-143). */
    const uint32_t sh = 16u * (j & 1);
    uint32_t sc0, m0, sc1, m1;
    if (j < 2) {
        sc0 = (hdr.y >> sh) & 63u;
        m0 = (hdr.z >> sh) & 63u;
        sc1 = (hdr.y >> (sh + 8)) & 63u;
        m1 = (hdr.z >> (sh + 8)) & 63u;
    } else {
        sc0 = ((hdr.w >> sh) & 15u) | ((hdr.y >> (sh + 2)) & 0x30u);
        m0 = ((hdr.w >> (sh + 4)) & 15u) | ((hdr.z >> (sh + 2)) & 0x30u);
        sc1 = ((hdr.w >> (sh + 8)) & 15u) | ((hdr.y >> (sh + 10)) & 0x30u);
        m1 = ((hdr.w >> (sh + 12)) & 15u) | ((hdr.z >> (sh + 10)) & 0x30u);
    }
    const float dbase = f16_to_f32(hdr.x);
    const float mbase = f16_to_f32(hdr.x >> 16);
    const int q[8] = {(int)qa.x, (int)qa.y, (int)qa.z, (int)qa.w,
                      (int)qb.x, (int)qb.y, (int)qb.z, (int)qb.w};

#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint8_t *a = act_chunk + (t * cb + bl) * kActStride;
        const int4 a0 = *reinterpret_cast<const int4 *>(a + 64 * j);
        const int4 a1 = *reinterpret_cast<const int4 *>(a + 64 * j + 16);
        const int4 a2 = *reinterpret_cast<const int4 *>(a + 64 * j + 32);
        const int4 a3 = *reinterpret_cast<const int4 *>(a + 64 * j + 48);
        const int alo[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const int ahi[8] = {a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
        int W[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const int lo = dot4(q[l] & 0x0f0f0f0f, alo[l], 0);
            const int hi = dot4((q[l] >> 4) & 0x0f0f0f0f, ahi[l], 0);
            W[l] = quad_sum(lo * (int)sc0 + hi * (int)sc1);
        }
        const uint2 sums = *reinterpret_cast<const uint2 *>(a + kActSumsOff + 8 * j);
        /* _mm_hadd_epi16 pairs in 16-bit arithmetic, then _mm_madd_epi16. */
        const int p0 = (int16_t)((int16_t)(sums.x & 0xffff) + (int16_t)(sums.x >> 16));
        const int p1 = (int16_t)((int16_t)(sums.y & 0xffff) + (int16_t)(sums.y >> 16));
        const int M = (int)m0 * p0 + (int)m1 * p1;
        const float xs = *reinterpret_cast<const float *>(a + kActScaleOff);

        int *slot = res + t * kSlot;
        slot[8 + j] = M;
        if (j == 0) {
            *reinterpret_cast<int4 *>(slot) = make_int4(W[0], W[1], W[2], W[3]);
        } else if (j == 1) {
            *reinterpret_cast<int4 *>(slot + 4) = make_int4(W[4], W[5], W[6], W[7]);
        } else if (j == 2) {
            const float d = fmul_rn(dbase, xs);
            const float dm = fmul_rn(mbase, xs);
            *reinterpret_cast<float2 *>(slot + 12) = make_float2(d, -dm);
        }
    }
}

/* ---- IQ1_M -------------------------------------------------------------- */

/* Integer sums of one IQ1_M block (src/qwen38/qwen38_quant.c:1388-1544).
 * Quad lane j owns groups 2j and 2j+1 (sections 8j..8j+7, elements
 * 64j..64j+63).  The codebook is staged in LDS in nibble-pair form: byte i
 * of entry e holds (g_i + 1) | (g_{4+i} + 1) << 4, so a section's dot with
 * the activations is dot4(lo) + dot4(hi) - sum(a). */
template <int MT>
__device__ __forceinline__ void iq1m_pair(const uint8_t *blk, const uint8_t *act_chunk, int cb,
                                          int bl, int *res, int j, const uint32_t *grid)
{
    const uint2 qs = *reinterpret_cast<const uint2 *>(blk + 8 * j);
    const uint32_t qh = *reinterpret_cast<const uint32_t *>(blk + 32 + 4 * j);
    const uint2 sc = *reinterpret_cast<const uint2 *>(blk + 48);
    const uint32_t u0 = sc.x & 0xffffu, u1 = sc.x >> 16, u2 = sc.y & 0xffffu, u3 = sc.y >> 16;
    const uint32_t scale_bits = (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
    const float dbase = f16_to_f32(scale_bits);
    const uint32_t mine = (j & 2) ? ((j & 1) ? u3 : u2) : ((j & 1) ? u1 : u0);

    uint32_t entry[8];
    int negative[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const uint32_t low = ((s < 4 ? qs.x : qs.y) >> (8 * (s & 3))) & 0xffu;
        const uint32_t nib = qh >> (8 * (s >> 1) + 4 * (s & 1));
        entry[s] = grid[low | ((nib & 7u) << 8)];
        negative[s] = (nib >> 3) & 1;
    }
    int scale[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) scale[h] = 1 + 2 * (int)((mine >> (3 * h)) & 7u);

#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint8_t *a = act_chunk + (t * cb + bl) * kActStride + 64 * j;
        int av[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int4 x = *reinterpret_cast<const int4 *>(a + 16 * v);
            av[4 * v] = x.x; av[4 * v + 1] = x.y; av[4 * v + 2] = x.z; av[4 * v + 3] = x.w;
        }
        int weighted = 0, correction = 0;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            int dsum = 0, csum = 0;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int s = 2 * h + u;
                const int e = (int)entry[s];
                const int dn = dot4(e & 0x0f0f0f0f, av[2 * s], dot4((e >> 4) & 0x0f0f0f0f, av[2 * s + 1], 0));
                const int s8 = dot4(0x01010101, av[2 * s], dot4(0x01010101, av[2 * s + 1], 0));
                dsum += dn - s8;
                csum += negative[s] ? -s8 : s8;
            }
            weighted += scale[h] * dsum;
            correction += scale[h] * csum;
        }
        weighted = quad_sum(weighted);
        correction = quad_sum(correction);
        if (j == 0) {
            const float xs = *reinterpret_cast<const float *>(act_chunk + (t * cb + bl) * kActStride + kActScaleOff);
            int *slot = res + t * kSlot;
            *reinterpret_cast<int2 *>(slot) = make_int2(weighted, correction);
            reinterpret_cast<float *>(slot)[2] = fmul_rn(dbase, xs);
        }
    }
}

/* ---- Q6_K --------------------------------------------------------------- */

/* Integer lanes of one Q6_K block (src/qwen38/qwen38_quant.c:1727-1814).
 * Quad lane j = 2h + p owns half h and AVX2 lanes 4p..4p+3: bytes
 * 16p..16p+15 of ql[64h..], ql[64h+32..] and qh[32h..].  Lanes with h = 0
 * subtract the offset lanes 32*(s[2l]*sc[2l] + s[2l+1]*sc[2l+1]). */
__device__ __forceinline__ uint4 load16_unaligned(const uint8_t *p)
{
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

template <int MT>
__device__ __forceinline__ void q6k_pair(const uint8_t *blk, const uint8_t *act_chunk, int cb,
                                         int bl, int *res, int j)
{
    const int h = j >> 1, p = j & 1;
    const uint4 l0 = load16_unaligned(blk + 64 * h + 16 * p);
    const uint4 l1 = load16_unaligned(blk + 64 * h + 32 + 16 * p);
    const uint4 up = load16_unaligned(blk + 128 + 32 * h + 16 * p);
    const uint4 scv = load16_unaligned(blk + 192);
    uint16_t dbits;
    __builtin_memcpy(&dbits, blk + 208, 2);
    const float dbase = f16_to_f32(dbits);
    const int lo0[4] = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w};
    const int lo1[4] = {(int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
    const int upv[4] = {(int)up.x, (int)up.y, (int)up.z, (int)up.w};
    const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
    /* int8 scales[8h + 2q + p] for quarters q = 0..3 */
    int scale[4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        const int idx = 8 * h + 2 * qq + p;
        scale[qq] = (int)(int8_t)((scw[idx >> 2] >> (8 * (idx & 3))) & 0xffu);
    }
    int q6[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q6[0][i] = (lo0[i] & 0x0f0f0f0f) | ((upv[i] & 0x03030303) << 4);
        q6[1][i] = (lo1[i] & 0x0f0f0f0f) | (((upv[i] >> 2) & 0x03030303) << 4);
        q6[2][i] = ((lo0[i] >> 4) & 0x0f0f0f0f) | (((upv[i] >> 4) & 0x03030303) << 4);
        q6[3][i] = ((lo1[i] >> 4) & 0x0f0f0f0f) | (((upv[i] >> 6) & 0x03030303) << 4);
    }

#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint8_t *a = act_chunk + (t * cb + bl) * kActStride;
        int W[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) W[i] = 0;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int4 x = *reinterpret_cast<const int4 *>(a + 128 * h + 32 * qq + 16 * p);
            const int xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) W[i] += scale[qq] * dot4(q6[qq][i], xv[i], 0);
        }
        if (h == 0) {
            /* offset lanes l = 4p + i use sums/scales 2l, 2l+1 = 8p + 2i, 8p + 2i + 1 */
            const int4 s4 = *reinterpret_cast<const int4 *>(a + kActSumsOff + 16 * p);
            const uint32_t sv[4] = {(uint32_t)s4.x, (uint32_t)s4.y, (uint32_t)s4.z, (uint32_t)s4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int i0 = 8 * p + 2 * i, i1 = i0 + 1;
                const int c0 = (int)(int8_t)((scw[i0 >> 2] >> (8 * (i0 & 3))) & 0xffu);
                const int c1 = (int)(int8_t)((scw[i1 >> 2] >> (8 * (i1 & 3))) & 0xffu);
                const int s0 = (int)(int16_t)(sv[i] & 0xffffu);
                const int s1 = (int)(int16_t)(sv[i] >> 16);
                W[i] -= 32 * (s0 * c0 + s1 * c1);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) W[i] += quad_xor2(W[i]);
        int *slot = res + t * kSlot;
        if (h == 0) {
            *reinterpret_cast<int4 *>(slot + 4 * p) = make_int4(W[0], W[1], W[2], W[3]);
            if (p == 0) {
                const float xs = *reinterpret_cast<const float *>(a + kActScaleOff);
                reinterpret_cast<float *>(slot)[12] = fmul_rn(dbase, xs);
            }
        }
    }
}

/* ---- kernel ------------------------------------------------------------- */

template <int TYPE, int MT>
__global__ __launch_bounds__(256) void gemm_q8k_kernel(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ x, float *__restrict__ y,
    uint32_t rows, uint32_t nblk, uint32_t rw, uint32_t ch, const uint32_t *__restrict__ grid_src)
{
    using F = Format<TYPE>;
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *act = lds;
    int *res = reinterpret_cast<int *>(lds + MT * ch * kActStride);
    uint32_t *grid = reinterpret_cast<uint32_t *>(lds + MT * ch * kActStride + rw * ch * MT * kSlot * 4);

    const int tid = threadIdx.x;
    const int quad = tid >> 2, j = tid & 3, nquads = blockDim.x >> 2;
    const uint32_t row0 = blockIdx.x * rw;

    if (TYPE == kIQ1M) {
        for (int i = tid; i < 2048; i += blockDim.x) grid[i] = grid_src[i];
    }

    /* chain-lane role: (row r, token t, accumulator lane k) */
    const int g = tid / F::group, k = tid - g * F::group;
    const int rc = g / MT, tc = g - rc * MT;
    const bool chain = g < (int)rw * MT && row0 + rc < rows && k < F::chains;
    float acc = 0.0f;

    for (uint32_t b0 = 0; b0 < nblk; b0 += ch) {
        const int cb = (int)min(ch, nblk - b0);
        __syncthreads();
        stage_activations(act, x, MT, nblk, b0, cb);
        __syncthreads();

        const int npairs = (int)rw * cb;
        for (int p = quad; p < npairs; p += nquads) {
            const int r = p / cb, bl = p - r * cb;
            const uint32_t row = row0 + r;
            if (row >= rows) break;
            const uint8_t *blk = w + (static_cast<size_t>(row) * nblk + b0 + bl) * F::bytes;
            int *slot = res + p * MT * kSlot;
            if (TYPE == kQ4K) q4k_pair<MT>(blk, act, cb, bl, slot, j);
            else if (TYPE == kIQ1M) iq1m_pair<MT>(blk, act, cb, bl, slot, j, grid);
            else q6k_pair<MT>(blk, act, cb, bl, slot, j);
        }
        __syncthreads();

        if (chain) {
            const int *base = res + (rc * cb * MT + tc) * kSlot;
            const int stride = MT * kSlot;
            if (TYPE == kQ4K) {
                const int dsel = k < 8 ? 12 : 13;
                for (int bl = 0; bl < cb; ++bl) {
                    const int *s = base + bl * stride;
                    acc = __builtin_fmaf(reinterpret_cast<const float *>(s)[dsel], (float)s[k], acc);
                }
            } else if (TYPE == kQ6K) {
                for (int bl = 0; bl < cb; ++bl) {
                    const int *s = base + bl * stride;
                    acc = __builtin_fmaf(reinterpret_cast<const float *>(s)[12], (float)s[k], acc);
                }
            } else {
                for (int bl = 0; bl < cb; ++bl) {
                    const int *s = base + bl * stride;
                    const float corr = fmul_rn(0.125f, (float)s[1]);
                    const float inner = fadd_rn((float)s[0], corr);
                    acc = fadd_rn(acc, fmul_rn(reinterpret_cast<const float *>(s)[2], inner));
                }
            }
        }
    }

    /* Horizontal trees of the AVX2 build (qwen38_quant.c:303-310, 1626-1630). */
    if (TYPE == kIQ1M) {
        if (chain) y[static_cast<size_t>(tc) * rows + row0 + rc] = acc;
        return;
    }
    const int lane16 = tid & ~15;
    /* step A: lanes 0..3 -> a_k + a_{k+4}; lanes 8,9 -> m0 + m2, m1 + m3 */
    const int srcA = lane16 + (k < 8 ? k + 4 : k + 2);
    const float vA = acc + __shfl(acc, srcA & 63, 64);
    /* step B: lanes 0,1 -> (s0 + s2), (s1 + s3); lane 8 -> x8 + x9 */
    const int srcB = lane16 + (k < 8 ? k + 2 : k + 1);
    const float vB = vA + __shfl(vA, srcB & 63, 64);
    /* step C: lane 0 -> v0 + v1 */
    const float vC = vB + __shfl(vB, (lane16 + 1) & 63, 64);
    if (TYPE == kQ4K) {
        const float mins = __shfl(vB, (lane16 + 8) & 63, 64);
        if (chain && k == 0) y[static_cast<size_t>(tc) * rows + row0 + rc] = vC + mins;
    } else {
        if (chain && k == 0) y[static_cast<size_t>(tc) * rows + row0 + rc] = vC;
    }
}

/* ---- launcher ------------------------------------------------------------ */

struct GemmShape {
    uint32_t rw, ch;
    size_t lds;
};

template <int TYPE>
static GemmShape pick_shape(uint32_t rows, uint32_t nblk, int mt)
{
    using F = Format<TYPE>;
    GemmShape s;
    /* chain lanes: rw * mt groups of F::group lanes within 256 threads */
    uint32_t rw_max = 256u / (uint32_t)(F::group * mt);
    if (rw_max > 16) rw_max = 16;
    uint32_t rw = rw_max;
    /* keep at least ~8 workgroups per CU on 256 CUs when rows allow */
    while (rw > 1 && (rows + rw - 1) / rw < 2048u) rw >>= 1;
    uint32_t ch = nblk;
    auto lds_of = [&](uint32_t r, uint32_t c) {
        return (size_t)mt * c * kActStride + (size_t)r * c * mt * kSlot * 4 + (TYPE == kIQ1M ? 8192 : 0);
    };
    while (lds_of(rw, ch) > 48 * 1024 && ch > 8) ch = (ch + 1) / 2;
    s.rw = rw;
    s.ch = ch;
    s.lds = lds_of(rw, ch);
    return s;
}

template <int TYPE, int MT>
static void launch_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t rows, uint32_t nblk,
                         const uint32_t *grid, hipStream_t stream)
{
    const GemmShape s = pick_shape<TYPE>(rows, nblk, MT);
    const uint32_t groups = (rows + s.rw - 1) / s.rw;
    hipLaunchKernelGGL((gemm_q8k_kernel<TYPE, MT>), dim3(groups), dim3(256), s.lds, stream,
                       w, x, y, rows, nblk, s.rw, s.ch, grid);
}

template <int TYPE>
static void launch_m(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t rows, uint32_t nblk,
                     const uint32_t *grid, hipStream_t stream)
{
    switch (m) {
    case 1: launch_typed<TYPE, 1>(w, x, y, rows, nblk, grid, stream); break;
    case 2: launch_typed<TYPE, 2>(w, x, y, rows, nblk, grid, stream); break;
    case 3: launch_typed<TYPE, 3>(w, x, y, rows, nblk, grid, stream); break;
    case 4: launch_typed<TYPE, 4>(w, x, y, rows, nblk, grid, stream); break;
    case 5: launch_typed<TYPE, 5>(w, x, y, rows, nblk, grid, stream); break;
    case 6: launch_typed<TYPE, 6>(w, x, y, rows, nblk, grid, stream); break;
    case 7: launch_typed<TYPE, 7>(w, x, y, rows, nblk, grid, stream); break;
    default: launch_typed<TYPE, 8>(w, x, y, rows, nblk, grid, stream); break;
    }
}

/* Enqueue y[t * rows + row] = W_row . x_t for t < m (all device pointers).
 * x is m * nblk Q8_K blocks, token-major.  grid is the IQ1_M codebook in
 * nibble-pair form (unused for the other types). */
bool launch_gemm(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t rows,
                 uint32_t nblk, const uint32_t *grid, hipStream_t stream)
{
    if (m < 1 || m > 8) return false;
    switch (type) {
    case kQ4K: launch_m<kQ4K>(m, w, x, y, rows, nblk, grid, stream); return true;
    case kQ6K: launch_m<kQ6K>(m, w, x, y, rows, nblk, grid, stream); return true;
    case kIQ1M: launch_m<kIQ1M>(m, w, x, y, rows, nblk, grid, stream); return true;
    default: return false;
    }
}

}  // namespace q38
