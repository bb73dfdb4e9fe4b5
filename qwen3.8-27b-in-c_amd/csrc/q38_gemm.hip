/* Quantised GEMV / small-M GEMM against Q8_K activations on gfx950.
 *
 * Computes what q38_tensor_gemv_q8_k / q38_tensor_gemm_q8_k compute
 * (src/qwen38/qwen38_quant.c:2833-3169 of the reference) for Q4_K, Q6_K and
 * IQ1_M weights, bit-identically to its x86 AVX2 build.
 *
 * Two phases per tile of weight rows:
 *   phase 1  every (row, super-block) pair goes to a lane quad, which
 *            dequantises the packed block in registers and forms the
 *            block's exact int32 sums with v_dot4_i32_i8 against the Q8_K
 *            activations staged once in LDS.  The sums land in LDS in
 *            k-major order: one contiguous run of `nblk` values per
 *            (row, token, sum index);
 *   phase 2  "chain" lanes replay the reference's fp32 accumulation over the
 *            row's blocks in order: one lane per AVX2 accumulator lane
 *            (Q4_K: 8 weighted + 4 min lanes, Q6_K: 8, IQ1_M: 1 scalar), each
 *            a sequential fmaf chain reading its run with 16-byte LDS loads.
 *            The K dimension is split across lanes for the integer work and
 *            never for the fp32 work.  The lanes of a (row, token) combine
 *            with the reference's fixed horizontal-add tree (DPP row shifts)
 *            and write output[token * rows + row].
 *
 * Kernels: `ring` (the weights streamed into an LDS ring with direct
 * global->LDS copies, one workgroup per CU), `stream` (each wavefront
 * prefetches its next tile into registers; used where the ring's alignment
 * rules do not hold) and `chunked` (activations staged chunk by chunk, for
 * token counts whose activations exceed LDS).
 */
#include "q38_device.h"
#include "q38_kernels.h"

#include <map>
#include <mutex>
#include <utility>

namespace q38 {

/* staged Q8_K block in LDS: quants @0, sums @256, scale @288; IQ1_M adds the
 * 32 per-section (8-element) sums @304 */
constexpr int kActSumsOff = 256;
constexpr int kActScaleOff = 288;
constexpr int kActS8Off = 304;

/* slot = number of per-(row, token, block) values phase 1 leaves for phase 2:
 * Q4_K W[0..7], M[0..3], d, -dmin; Q6_K W[0..7], d; IQ1_M weighted,
 * correction, d */
template <int TYPE> struct Format;
template <> struct Format<kQ4K> {
    static constexpr int bytes = 144, chains = 12, group = 16, slot = 14, act = 304, prefetch = 5;
};
template <> struct Format<kQ6K> {
    static constexpr int bytes = 210, chains = 8, group = 16, slot = 9, act = 304, prefetch = 4;
};
template <> struct Format<kIQ1M> {
    static constexpr int bytes = 56, chains = 1, group = 1, slot = 3, act = 368, prefetch = 8;
};

/* Phase-1 output of one (row, block) pair: value (t, k) at p[(t*S + k)*nb]. */
struct PairOut {
    int *p;
    int nb;
    __device__ __forceinline__ int &at(int t, int k, int S) const { return p[(t * S + k) * nb]; }
};

/* ---- staging ------------------------------------------------------------ */

template <int TYPE>
__device__ __forceinline__ int act_dword_dst(int w)
{
    if (w == 0) return kActScaleOff / 4;
    if (w > 64) return kActSumsOff / 4 + (w - 65);
    const int d = w - 1;
    if (TYPE == kQ4K) {
        /* element e = 64c + 32h + 8j + u goes to byte 64j + 16c + 8h + u */
        const int c = d >> 4, h = (d >> 3) & 1, jj = (d >> 1) & 3;
        return 16 * jj + 4 * c + 2 * h + (d & 1);
    }
    return d;
}

/* Copy Q8_K blocks [b0, b0 + cb) of every token (AoS, 292-byte stride) into
 * LDS slots of F::act bytes; IQ1_M also gets the per-section sums.  Wavefront
 * w copies blocks w, w + nw, ...; lane l moves dwords l and 64 + l (l < 9),
 * eight blocks in flight at once.  Ends with a workgroup barrier. */
template <int TYPE>
__device__ __forceinline__ void stage_activations(uint8_t *act, const uint8_t *x, int tokens,
                                                  uint32_t nblk, uint32_t b0, int cb)
{
    using F = Format<TYPE>;
    constexpr int kDepth = 8;
    const int nslots = tokens * cb;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int dst0 = act_dword_dst<TYPE>(lane), dst1 = act_dword_dst<TYPE>(64 + lane);
    for (int sb = wave; sb < nslots; sb += kDepth * nw) {
        uint32_t v0[kDepth], v1[kDepth];
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            const int slot = sb + u * nw;
            if (slot < nslots) {
                const int t = slot / cb, bl = slot - t * cb;
                const uint32_t *src = reinterpret_cast<const uint32_t *>(
                    x + (static_cast<size_t>(t) * nblk + b0 + bl) * kQ8KBytes);
                v0[u] = src[lane];
                if (lane < 9) v1[u] = src[64 + lane];
            }
        }
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            const int slot = sb + u * nw;
            if (slot < nslots) {
                uint32_t *dst = reinterpret_cast<uint32_t *>(act + slot * F::act);
                dst[dst0] = v0[u];
                if (lane < 9) dst[dst1] = v1[u];
            }
        }
    }
    __syncthreads();
    if (TYPE == kIQ1M) {
        const int sections = tokens * cb * 32;
        for (int i = threadIdx.x; i < sections; i += blockDim.x) {
            const int slot = i >> 5, sct = i & 31;
            uint8_t *a = act + slot * F::act;
            const int2 v = *reinterpret_cast<const int2 *>(a + 8 * sct);
            const int s8 = dot4(0x01010101, v.x, dot4(0x01010101, v.y, 0));
            reinterpret_cast<int16_t *>(a + kActS8Off)[sct] = static_cast<int16_t>(s8);
        }
        __syncthreads();
    }
}

/* ---- per-type block loads (one quad lane's share; blk in HBM or LDS) ------ */

template <int TYPE> struct Raw;

template <> struct Raw<kQ4K> {
    uint4 hdr;
    uint2 q[4];
    __device__ __forceinline__ void load(const uint8_t *blk, int j)
    {
        hdr = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * c + 8 * j);
    }
};

template <> struct Raw<kIQ1M> {
    uint2 qs, sc;
    uint32_t qh;
    __device__ __forceinline__ void load(const uint8_t *blk, int j)
    {
        qs = *reinterpret_cast<const uint2 *>(blk + 8 * j);
        qh = *reinterpret_cast<const uint32_t *>(blk + 32 + 4 * j);
        sc = *reinterpret_cast<const uint2 *>(blk + 48);
    }
};

__device__ __forceinline__ uint4 load16_unaligned(const uint8_t *p)
{
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

template <> struct Raw<kQ6K> {
    uint4 l0, l1, up, scv;
    uint32_t dbits;
    __device__ __forceinline__ void load(const uint8_t *blk, int j)
    {
        const int h = j >> 1, p = j & 1;
        l0 = load16_unaligned(blk + 64 * h + 16 * p);
        l1 = load16_unaligned(blk + 64 * h + 32 + 16 * p);
        up = load16_unaligned(blk + 128 + 32 * h + 16 * p);
        scv = load16_unaligned(blk + 192);
        uint16_t d;
        __builtin_memcpy(&d, blk + 208, 2);
        dbits = d;
    }
};

/* ---- Q4_K integer lanes (src/qwen38/qwen38_quant.c:1564-1620) --------------
 * AVX2 lane l (l = 0..7) owns bytes 4l..4l+3 of each 32-byte nibble chunk c:
 * W[l] = sum_c sc[2c] * dot(lo nibbles, a[64c+4l..]) + sc[2c+1] * dot(hi
 * nibbles, a[64c+32+4l..]).  Quad lane j forms W[2j] and W[2j+1] over all four
 * chunks (no cross-lane reduction) and the min lane M[j] = m[2j](s[4j]+s[4j+1])
 * + m[2j+1](s[4j+2]+s[4j+3]).  The staged activations are permuted so lane j
 * reads its 64 bytes contiguously: [c][lo/hi][8 bytes]. */
template <int MT>
__device__ __forceinline__ void q4k_ints(const Raw<kQ4K> &raw, const uint8_t *act, int bl, int nb,
                                         PairOut out, int j)
{
    constexpr int S = Format<kQ4K>::slot;
    const uint32_t Y = raw.hdr.y, Z = raw.hdr.z, Wd = raw.hdr.w;
    /* q38_scale_min_k4 (qwen38_quant.c:131-143), all eight scales at once:
     * sub-blocks 0..3 take the low 6 bits of bytes 0..3; sub-blocks 4..7 take
     * the low nibble of bytes 8..11 plus the top 2 bits of bytes 0..3. */
    const uint32_t sc_hi = (Wd & 0x0f0f0f0fu) | ((Y >> 2) & 0x30303030u);
    int sc[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = (int)((Y >> (8 * i)) & 63u);
        sc[4 + i] = (int)((sc_hi >> (8 * i)) & 0xffu);
    }
    /* this lane's two mins, sub-blocks 2j and 2j+1 */
    const uint32_t m_lo = Z & 0x3f3f3f3fu;
    const uint32_t m_hi = ((Wd >> 4) & 0x0f0f0f0fu) | ((Z >> 2) & 0x30303030u);
    const uint32_t mw = (j & 2) ? m_hi : m_lo;
    const uint32_t msh = 16u * (j & 1);
    const int m0 = (int)((mw >> msh) & 0xffu), m1 = (int)((mw >> (msh + 8)) & 0xffu);

    int lo[4][2], hi[4][2];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        lo[c][0] = (int)(raw.q[c].x & 0x0f0f0f0fu);
        hi[c][0] = (int)((raw.q[c].x >> 4) & 0x0f0f0f0fu);
        lo[c][1] = (int)(raw.q[c].y & 0x0f0f0f0fu);
        hi[c][1] = (int)((raw.q[c].y >> 4) & 0x0f0f0f0fu);
    }
    const float dbase = f16_to_f32(raw.hdr.x), mbase = f16_to_f32(raw.hdr.x >> 16);

#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint8_t *a = act + (t * nb + bl) * Format<kQ4K>::act;
        int av[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int4 x = *reinterpret_cast<const int4 *>(a + 64 * j + 16 * v);
            av[4 * v] = x.x; av[4 * v + 1] = x.y; av[4 * v + 2] = x.z; av[4 * v + 3] = x.w;
        }
        int W0 = 0, W1 = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            /* av[4c + 2h + l']: chunk c, half h (lo/hi), lane 2j + l' */
            W0 = mad24(dot4z(lo[c][0], av[4 * c + 0]), sc[2 * c], W0);
            W0 = mad24(dot4z(hi[c][0], av[4 * c + 2]), sc[2 * c + 1], W0);
            W1 = mad24(dot4z(lo[c][1], av[4 * c + 1]), sc[2 * c], W1);
            W1 = mad24(dot4z(hi[c][1], av[4 * c + 3]), sc[2 * c + 1], W1);
        }
        const uint2 sums = *reinterpret_cast<const uint2 *>(a + kActSumsOff + 8 * j);
        /* the pair sums of _mm_hadd_epi16 cannot overflow 16 bits (|s| <= 2032) */
        const int p0 = (int)(int16_t)(sums.x & 0xffffu) + ((int)sums.x >> 16);
        const int p1 = (int)(int16_t)(sums.y & 0xffffu) + ((int)sums.y >> 16);
        out.at(t, 2 * j, S) = W0;
        out.at(t, 2 * j + 1, S) = W1;
        out.at(t, 8 + j, S) = mad24(m0, p0, mul24(m1, p1));
        if (j == 0) {
            const float xs = *reinterpret_cast<const float *>(a + kActScaleOff);
            out.at(t, 12, S) = __float_as_int(fmul_rn(dbase, xs));
            out.at(t, 13, S) = __float_as_int(-fmul_rn(mbase, xs));
        }
    }
}

/* ---- IQ1_M integer sums (src/qwen38/qwen38_quant.c:1388-1544) -------------
 * Quad lane j owns groups 2j and 2j+1 (sections 8j..8j+7, elements
 * 64j..64j+63).  The codebook sits in LDS as 8 int8 values per entry;
 * correction uses the staged per-section activation sums. */
template <int MT>
__device__ __forceinline__ void iq1m_ints(const Raw<kIQ1M> &raw, const uint8_t *act, int bl, int nb,
                                          PairOut out, int j, const uint2 *grid)
{
    constexpr int S = Format<kIQ1M>::slot;
    const uint32_t u0 = raw.sc.x & 0xffffu, u1 = raw.sc.x >> 16;
    const uint32_t u2 = raw.sc.y & 0xffffu, u3 = raw.sc.y >> 16;
    const uint32_t mine = (j & 2) ? ((j & 1) ? u3 : u2) : ((j & 1) ? u1 : u0);
    uint2 g[8];
    bool negative[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const uint32_t low = ((s < 4 ? raw.qs.x : raw.qs.y) >> (8 * (s & 3))) & 0xffu;
        const uint32_t nib = raw.qh >> (8 * (s >> 1) + 4 * (s & 1));
        g[s] = grid[low | ((nib & 7u) << 8)];
        negative[s] = (nib & 8u) != 0;
    }
    int scale[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) scale[h] = 1 + 2 * (int)((mine >> (3 * h)) & 7u);

#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint8_t *a = act + (t * nb + bl) * Format<kIQ1M>::act;
        int av[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int4 x = *reinterpret_cast<const int4 *>(a + 64 * j + 16 * v);
            av[4 * v] = x.x; av[4 * v + 1] = x.y; av[4 * v + 2] = x.z; av[4 * v + 3] = x.w;
        }
        const int4 s8v = *reinterpret_cast<const int4 *>(a + kActS8Off + 16 * j);
        const int s8w[4] = {s8v.x, s8v.y, s8v.z, s8v.w};
        int weighted = 0, correction = 0;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int e0 = 2 * h, e1 = 2 * h + 1;
            const int d0 = dot4((int)g[e0].x, av[2 * e0], dot4((int)g[e0].y, av[2 * e0 + 1], 0));
            const int d1 = dot4((int)g[e1].x, av[2 * e1], dot4((int)g[e1].y, av[2 * e1 + 1], 0));
            const int s0 = (int)(int16_t)(s8w[h] & 0xffff);
            const int s1 = s8w[h] >> 16;
            weighted = mad24(scale[h], d0 + d1, weighted);
            correction = mad24(scale[h], (negative[e0] ? -s0 : s0) + (negative[e1] ? -s1 : s1), correction);
        }
        weighted = quad_sum(weighted);
        correction = quad_sum(correction);
        if (j == 0) {
            const uint32_t bits = (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
            const float xs = *reinterpret_cast<const float *>(a + kActScaleOff);
            out.at(t, 0, S) = weighted;
            out.at(t, 1, S) = correction;
            out.at(t, 2, S) = __float_as_int(fmul_rn(f16_to_f32(bits), xs));
        }
    }
}

/* ---- Q6_K integer lanes (src/qwen38/qwen38_quant.c:1727-1814) -------------
 * Quad lane j = 2h + p owns half h and AVX2 lanes 4p..4p+3: bytes 16p..16p+15
 * of ql[64h..], ql[64h+32..] and qh[32h..].  Lanes with h = 0 subtract the
 * offset lanes 32*(s[2l]*sc[2l] + s[2l+1]*sc[2l+1]). */
template <int MT>
__device__ __forceinline__ void q6k_ints(const Raw<kQ6K> &raw, const uint8_t *act, int bl, int nb,
                                         PairOut out, int j)
{
    constexpr int S = Format<kQ6K>::slot;
    const int h = j >> 1, p = j & 1;
    const int lo0[4] = {(int)raw.l0.x, (int)raw.l0.y, (int)raw.l0.z, (int)raw.l0.w};
    const int lo1[4] = {(int)raw.l1.x, (int)raw.l1.y, (int)raw.l1.z, (int)raw.l1.w};
    const int upv[4] = {(int)raw.up.x, (int)raw.up.y, (int)raw.up.z, (int)raw.up.w};
    const uint32_t scw[4] = {raw.scv.x, raw.scv.y, raw.scv.z, raw.scv.w};
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
        const uint8_t *a = act + (t * nb + bl) * Format<kQ6K>::act;
        int W[4] = {0, 0, 0, 0};
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int4 x = *reinterpret_cast<const int4 *>(a + 128 * h + 32 * qq + 16 * p);
            const int xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) W[i] = mad24(scale[qq], dot4(q6[qq][i], xv[i], 0), W[i]);
        }
        if (h == 0) {
            const int4 s4 = *reinterpret_cast<const int4 *>(a + kActSumsOff + 16 * p);
            const uint32_t sv[4] = {(uint32_t)s4.x, (uint32_t)s4.y, (uint32_t)s4.z, (uint32_t)s4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int i0 = 8 * p + 2 * i, i1 = i0 + 1;
                const int c0 = (int)(int8_t)((scw[i0 >> 2] >> (8 * (i0 & 3))) & 0xffu);
                const int c1 = (int)(int8_t)((scw[i1 >> 2] >> (8 * (i1 & 3))) & 0xffu);
                W[i] -= 32 * mad24((int)(int16_t)(sv[i] & 0xffffu), c0, mul24((int)(int16_t)(sv[i] >> 16), c1));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) W[i] += quad_xor2(W[i]);
        if (h == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) out.at(t, 4 * p + i, S) = W[i];
            if (p == 0) {
                const float xs = *reinterpret_cast<const float *>(a + kActScaleOff);
                out.at(t, 8, S) = __float_as_int(fmul_rn(f16_to_f32(raw.dbits), xs));
            }
        }
    }
}

template <int TYPE, int MT>
__device__ __forceinline__ void block_ints(const Raw<TYPE> &raw, const uint8_t *act, int bl, int nb, PairOut out,
                                           int j, const uint2 *grid)
{
    if constexpr (TYPE == kQ4K) q4k_ints<MT>(raw, act, bl, nb, out, j);
    else if constexpr (TYPE == kIQ1M) iq1m_ints<MT>(raw, act, bl, nb, out, j, grid);
    else q6k_ints<MT>(raw, act, bl, nb, out, j);
}

/* Phase-1 output slot of pair (r, bl) of a tile. */
template <int TYPE, int MT>
__device__ __forceinline__ PairOut pair_out(int *res, int r, int bl, int nb)
{
    return PairOut{res + r * MT * Format<TYPE>::slot * nb + bl, nb};
}

/* ---- phase 2: the reference's sequential fp32 accumulation ---------------- */

/* Chain lane (row r, token t, lane k) over blocks [0, nb) of its run. */
template <int TYPE, int MT>
__device__ __forceinline__ float chain(const int *res, int r, int t, int k, int nb)
{
    constexpr int S = Format<TYPE>::slot;
    const int *row = res + (r * MT + t) * S * nb;
    float acc = 0.0f;
    if constexpr (TYPE == kIQ1M) {
        /* total += d * (weighted + 0.125f * correction), each op rounded */
        for (int bl = 0; bl < nb; ++bl) {
            const float corr = fmul_rn(0.125f, (float)row[nb + bl]);
            const float inner = fadd_rn((float)row[bl], corr);
            acc = fadd_rn(acc, fmul_rn(__int_as_float(row[2 * nb + bl]), inner));
        }
        return acc;
    } else {
        const int dsel = TYPE == kQ4K ? (k < 8 ? 12 : 13) : 8;
        const int *wk = row + k * nb;
        const int *dk = row + dsel * nb;
        int bl = 0;
        if ((nb & 3) == 0) {
            /* runs start on 16-byte boundaries when nb % 4 == 0 */
#pragma unroll 4
            for (; bl < nb; bl += 4) {
                const int4 iv = *reinterpret_cast<const int4 *>(wk + bl);
                const int4 dv = *reinterpret_cast<const int4 *>(dk + bl);
                acc = __builtin_fmaf(__int_as_float(dv.x), (float)iv.x, acc);
                acc = __builtin_fmaf(__int_as_float(dv.y), (float)iv.y, acc);
                acc = __builtin_fmaf(__int_as_float(dv.z), (float)iv.z, acc);
                acc = __builtin_fmaf(__int_as_float(dv.w), (float)iv.w, acc);
            }
        }
        for (; bl < nb; ++bl) acc = __builtin_fmaf(__int_as_float(dk[bl]), (float)wk[bl], acc);
        return acc;
    }
}

/* Value of lane (lane + n) of the same 16-lane DPP row (row_shl:n). */
template <int N>
__device__ __forceinline__ float row_shl(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, true));
}

/* Horizontal trees of the AVX2 build (qwen38_quant.c:303-310, 1626-1630) on a
 * 16-lane row holding the accumulator lanes (0..7 weighted, 8..11 min):
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)), plus ((m0+m2)+(m1+m3)) for Q4_K.
 * The result is valid in lane 0 of the row; every lane must call this. */
template <int TYPE>
__device__ __forceinline__ float chain_tree(float acc)
{
    if constexpr (TYPE == kIQ1M) {
        return acc;
    } else {
        const float vA = acc + row_shl<4>(acc);  /* lanes 0..3: a_i + a_{i+4} */
        const float vB = vA + row_shl<2>(vA);    /* lanes 0, 1 */
        const float vC = vB + row_shl<1>(vB);    /* lane 0 */
        if constexpr (TYPE == kQ4K) {
            const float mA = acc + row_shl<2>(acc);  /* lanes 8, 9: m0 + m2, m1 + m3 */
            const float mB = mA + row_shl<1>(mA);    /* lane 8 */
            return vC + row_shl<8>(mB);
        } else {
            return vC;
        }
    }
}

/* All (row, token) chains of a tile: groups of F::group lanes over nthreads
 * lanes (a multiple of 64; every lane must call this). */
template <int TYPE, int MT>
__device__ __forceinline__ void tile_chains(const int *res, float *y, uint32_t ldy, uint32_t row0, int tile_rows,
                                            int nb, int tid, int nthreads)
{
    using F = Format<TYPE>;
    const int groups = tile_rows * MT;
    const int per_pass = nthreads / F::group;
    for (int g0 = 0; g0 < groups; g0 += per_pass) {
        const int g = g0 + tid / F::group, k = tid % F::group;
        const int rc = g / MT, tc = g - rc * MT;
        const bool active = g < groups && k < F::chains;
        const float acc = active ? chain<TYPE, MT>(res, rc, tc, k, nb) : 0.0f;
        const float out = chain_tree<TYPE>(acc);
        if (active && k == 0) y[static_cast<size_t>(tc) * ldy + row0 + rc] = out;
    }
}

/* ---- direct global->LDS copies ---------------------------------------------- */

__device__ __forceinline__ uint32_t lds_address(const void *p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

/* 16 bytes per lane from gaddr to LDS at lds_base + 16 * lane (the wave's
 * 1 KiB is contiguous).  Issued from inline assembly so that the compiler's
 * wait-count pass does not treat it as an LDS store: it would otherwise drain
 * every outstanding copy before each later LDS read.  Callers place the
 * s_waitcnt themselves. */
__device__ __forceinline__ void lds_dma16(const void *gaddr, uint32_t lds_base)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(gaddr), "s"(lds_base) : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

/* ---- ring kernel ------------------------------------------------------------
 * One workgroup of WAVES wavefronts per CU owns an LDS ring of NR slots of
 * WAVES * LW KiB.  Tiles of `rw` whole rows (contiguous bytes in HBM) are
 * copied into the ring with global_load_lds_dwordx4, 1 KiB per wave
 * instruction, perfectly coalesced and without passing through VGPRs, NR - 1
 * tiles ahead of the tile being computed.  Vector-memory loads retire in
 * order, so after issuing tile k + NR - 1 the wait vmcnt((NR-1)*LW)
 * guarantees the wave's share of tile k has landed; a barrier then publishes
 * the whole tile. */
template <int TYPE, int MT, int NR, int WAVES, int LW>
__global__ __launch_bounds__(64 * WAVES) void gemm_q8k_ring(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ x, float *__restrict__ y, uint32_t ldy,
    uint32_t rows, uint32_t nblk, uint32_t rw, uint32_t ntiles, const uint2 *__restrict__ grid_src)
{
    using F = Format<TYPE>;
    constexpr uint32_t kSlotBytes = WAVES * LW * 1024u;
    constexpr int kQuads = 16 * WAVES;
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = (int)nblk;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gquad = threadIdx.x >> 2, j = threadIdx.x & 3;
    uint2 *grid = reinterpret_cast<uint2 *>(lds);
    uint8_t *act = lds + (TYPE == kIQ1M ? 16384 : 0);
    uint8_t *ring = act + MT * nb * F::act;
    int *res = reinterpret_cast<int *>(ring + NR * kSlotBytes);
    const uint32_t ring_lds = lds_address(ring);
    const size_t tile_bytes = static_cast<size_t>(rw) * nblk * F::bytes;
    const size_t total_bytes = static_cast<size_t>(rows) * nblk * F::bytes;

    /* copy this wave's LW KiB share of tile t into ring slot s.  The
     * launcher guarantees 16-byte aligned tiles and matrix end; lanes past
     * the end re-read byte 0 into slot bytes that are never used. */
    auto issue = [&](uint32_t t, int s) {
        const size_t base = static_cast<size_t>(t) * tile_bytes;
#pragma unroll
        for (int q = 0; q < LW; ++q) {
            const uint32_t chunk = (uint32_t)(wave * LW + q) * 1024u;
            size_t off = base + chunk + (size_t)lane * 16u;
            if (chunk >= tile_bytes || off + 16u > total_bytes) off = 0;
            lds_dma16(w + off, __builtin_amdgcn_readfirstlane(ring_lds + s * kSlotBytes + chunk));
        }
    };

    uint32_t tile = blockIdx.x;
#pragma unroll
    for (int s = 0; s < NR - 1; ++s)
        if (tile + s * gridDim.x < ntiles) issue(tile + s * gridDim.x, s);

    if (TYPE == kIQ1M) {
        for (int i = threadIdx.x; i < 2048; i += blockDim.x) grid[i] = grid_src[i];
    }
    stage_activations<TYPE>(act, x, MT, nblk, 0, nb);

    int slot = 0;
    for (; tile < ntiles; tile += gridDim.x) {
        const uint32_t ahead = tile + (NR - 1) * gridDim.x;
        if (ahead < ntiles) {
            issue(ahead, (slot + NR - 1) % NR);
            wait_vmcnt<(NR - 1) * LW>();
        } else {
            wait_vmcnt<0>();
        }
        /* every wave's share of this tile has landed, and the previous
         * tile's chains are done with `res` */
        __syncthreads();
        const uint32_t row0 = tile * rw;
        const int tile_rows = (int)min(rw, rows - row0);
        const int npairs = tile_rows * nb;
        const uint8_t *tb = ring + slot * kSlotBytes;
        for (int p = gquad; p < npairs; p += kQuads) {
            Raw<TYPE> raw;
            raw.load(tb + p * F::bytes, j);
            const int r = p / nb, bl = p - r * nb;
            block_ints<TYPE, MT>(raw, act, bl, nb, pair_out<TYPE, MT>(res, r, bl, nb), j, grid);
        }
        __syncthreads();
        tile_chains<TYPE, MT>(res, y, ldy, row0, tile_rows, nb, threadIdx.x, 64 * WAVES);
        slot = (slot + 1) % NR;
    }
    /* no copy may still be in flight into LDS when the workgroup retires */
    wait_vmcnt<0>();
}

/* ---- stream kernel: one independent pipeline per wavefront -----------------
 * After the workgroup stages the activations once, each wavefront walks its
 * own tiles of `rw` rows: the next tile's blocks are loaded into registers
 * while the current tile's integer sums and fp32 chains run.  Tile pairs
 * p = quad + 16 i (i < P) cover rw * nblk (row, block) pairs. */
template <int TYPE, int MT>
__global__ __launch_bounds__(256) void gemm_q8k_stream(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ x, float *__restrict__ y, uint32_t ldy,
    uint32_t rows, uint32_t nblk, uint32_t rw, uint32_t ntiles, const uint2 *__restrict__ grid_src)
{
    using F = Format<TYPE>;
    constexpr int P = F::prefetch;
    extern __shared__ __align__(16) uint8_t lds[];
    uint2 *grid = reinterpret_cast<uint2 *>(lds);
    uint8_t *act = lds + (TYPE == kIQ1M ? 16384 : 0);
    const int nb = (int)nblk;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int quad = lane >> 2, j = lane & 3;
    int *res = reinterpret_cast<int *>(act + MT * nb * F::act) + wave * (int)rw * nb * MT * F::slot;
    const uint32_t nwaves = gridDim.x * 4u;

    uint32_t tile = blockIdx.x * 4u + (uint32_t)wave;
    Raw<TYPE> raw[P];
    /* Rows are contiguous, so pair p of a tile is block (row0 * nblk + p) of
     * the matrix and its (row, column) within the tile is the same every tile. */
    int pair_r[P], pair_b[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        pair_r[i] = (quad + 16 * i) / nb;
        pair_b[i] = (quad + 16 * i) - pair_r[i] * nb;
    }
    auto prefetch = [&](uint32_t t) {
        const uint32_t row0 = t * rw;
        const int npairs = (int)min(rw, rows - row0) * nb;
        const uint8_t *tile_w = w + static_cast<size_t>(row0) * nblk * F::bytes;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int p = quad + 16 * i;
            if (p < npairs) raw[i].load(tile_w + (uint32_t)p * (uint32_t)F::bytes, j);
        }
    };
    if (tile < ntiles) prefetch(tile);

    if (TYPE == kIQ1M) {
        for (int i = threadIdx.x; i < 2048; i += blockDim.x) grid[i] = grid_src[i];
    }
    stage_activations<TYPE>(act, x, MT, nblk, 0, nb);

    for (; tile < ntiles; tile += nwaves) {
        const uint32_t row0 = tile * rw;
        const int tile_rows = (int)min(rw, rows - row0);
        const int npairs = tile_rows * nb;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int p = quad + 16 * i;
            if (p < npairs)
                block_ints<TYPE, MT>(raw[i], act, pair_b[i], nb, pair_out<TYPE, MT>(res, pair_r[i], pair_b[i], nb), j,
                                     grid);
        }
        if (tile + nwaves < ntiles) prefetch(tile + nwaves);
        /* LDS traffic of one wavefront completes in issue order; the fence
         * keeps the compiler from moving the chain reads above the writes. */
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        tile_chains<TYPE, MT>(res, y, ldy, row0, tile_rows, nb, lane, 64);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
}

/* ---- chunked kernel: activations staged chunk by chunk ---------------------- */

template <int TYPE, int MT>
__global__ __launch_bounds__(256) void gemm_q8k_chunked(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ x, float *__restrict__ y, uint32_t ldy,
    uint32_t rows, uint32_t nblk, uint32_t rw, uint32_t ch, const uint2 *__restrict__ grid_src)
{
    using F = Format<TYPE>;
    constexpr int S = F::slot;
    extern __shared__ __align__(16) uint8_t lds[];
    uint2 *grid = reinterpret_cast<uint2 *>(lds);
    uint8_t *act = lds + (TYPE == kIQ1M ? 16384 : 0);
    int *res = reinterpret_cast<int *>(act + MT * ch * F::act);

    const int tid = threadIdx.x, quad = tid >> 2, j = tid & 3, nquads = blockDim.x >> 2;
    const uint32_t row0 = blockIdx.x * rw;
    const int tile_rows = (int)min(rw, rows - row0);
    if (TYPE == kIQ1M) {
        for (int i = tid; i < 2048; i += blockDim.x) grid[i] = grid_src[i];
    }
    const int g = tid / F::group, k = tid % F::group;
    const int rc = g / MT, tc = g - rc * MT;
    const bool active = g < tile_rows * MT && k < F::chains;
    float acc = 0.0f;

    for (uint32_t b0 = 0; b0 < nblk; b0 += ch) {
        const int cb = (int)min(ch, nblk - b0);
        __syncthreads();
        stage_activations<TYPE>(act, x, MT, nblk, b0, cb);
        const int npairs = tile_rows * cb;
        for (int p = quad; p < npairs; p += nquads) {
            const int r = p / cb, bl = p - r * cb;
            Raw<TYPE> raw;
            raw.load(w + (static_cast<size_t>(row0 + r) * nblk + b0 + bl) * F::bytes, j);
            block_ints<TYPE, MT>(raw, act, bl, cb, pair_out<TYPE, MT>(res, r, bl, cb), j, grid);
        }
        __syncthreads();
        /* continue each chain over this chunk's blocks, in order */
        if (active) {
            const int *row = res + (rc * MT + tc) * S * cb;
            for (int bl = 0; bl < cb; ++bl) {
                if constexpr (TYPE == kIQ1M) {
                    const float corr = fmul_rn(0.125f, (float)row[cb + bl]);
                    const float inner = fadd_rn((float)row[bl], corr);
                    acc = fadd_rn(acc, fmul_rn(__int_as_float(row[2 * cb + bl]), inner));
                } else {
                    const int dsel = TYPE == kQ4K ? (k < 8 ? 12 : 13) : 8;
                    acc = __builtin_fmaf(__int_as_float(row[dsel * cb + bl]), (float)row[k * cb + bl], acc);
                }
            }
        }
    }
    const float out = chain_tree<TYPE>(acc);
    if (active && k == 0) y[static_cast<size_t>(tc) * ldy + row0 + rc] = out;
}

/* ---- launch policy ---------------------------------------------------------- */

constexpr size_t kLdsBudget = 64 * 1024;
constexpr size_t kRingLds = 160 * 1024;

static int device_cus()
{
    static std::mutex m;
    static std::map<int, int> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(m);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    cache[dev] = cus;
    return cus;
}

static int occupancy(const void *kernel, int threads, size_t lds)
{
    static std::mutex m;
    static std::map<std::pair<const void *, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(m);
    auto key = std::make_pair(kernel, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, lds) != hipSuccess || blocks <= 0)
        blocks = 1;
    cache[key] = blocks;
    return blocks;
}

template <int TYPE, int MT, int NR, int WAVES, int LW>
static bool try_ring(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t nblk,
                     const uint2 *grid, hipStream_t stream)
{
    using F = Format<TYPE>;
    constexpr size_t kSlotBytes = (size_t)WAVES * LW * 1024u;
    const size_t row_bytes = (size_t)nblk * F::bytes;
    uint32_t rw = (uint32_t)(kSlotBytes / row_bytes);
    if (rw > rows) rw = rows;
    /* the copies move whole 16-byte chunks: every tile and the matrix end
     * must sit on a 16-byte boundary (no chunk may straddle the end) */
    while (rw > 0 && (rw * row_bytes) % 16u) --rw;
    if (rw == 0 || ((size_t)rows * row_bytes) % 16u) return false;
    const size_t lds = (TYPE == kIQ1M ? 16384 : 0) + (size_t)MT * nblk * F::act + NR * kSlotBytes +
                       (size_t)rw * nblk * MT * F::slot * 4;
    if (lds > kRingLds) return false;
    static bool attr_set = false;
    const void *kernel = reinterpret_cast<const void *>(&gemm_q8k_ring<TYPE, MT, NR, WAVES, LW>);
    if (!attr_set) {
        if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRingLds) != hipSuccess)
            return false;
        attr_set = true;
    }
    const uint32_t tiles = (rows + rw - 1) / rw;
    uint32_t groups = (uint32_t)device_cus();
    if (groups > tiles) groups = tiles;
    hipLaunchKernelGGL((gemm_q8k_ring<TYPE, MT, NR, WAVES, LW>), dim3(groups), dim3(64 * WAVES), lds, stream,
                       w, x, y, ldy, rows, nblk, rw, tiles, grid);
    return true;
}

template <int TYPE, int MT>
static void launch_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t nblk,
                         const uint2 *grid, hipStream_t stream)
{
    using F = Format<TYPE>;
    /* Long rows (down projections) stream best through the LDS ring; short
     * rows through per-wave register prefetch.  Q6_K blocks (210 bytes) do
     * not sit on 16-byte boundaries in the ring and always stream. */
    if (TYPE != kQ6K && MT <= 2 && nblk >= 40 && try_ring<TYPE, MT, 3, 16, 2>(w, x, y, ldy, rows, nblk, grid, stream))
        return;

    const size_t grid_lds = TYPE == kIQ1M ? 16384 : 0;
    /* rows per wave tile: the tile's pairs fit the 16 quads' prefetch
     * registers and its (row, token) chain groups fit the 64 lanes */
    uint32_t rw = (16u * F::prefetch) / nblk;
    const uint32_t rw_chain = 64u / (uint32_t)(F::group * MT);
    if (rw > rw_chain) rw = rw_chain;
    if (rw > rows) rw = rows;
    if (rw >= 1) {
        const size_t lds = grid_lds + (size_t)MT * nblk * F::act + 4u * rw * nblk * MT * F::slot * 4;
        if (lds <= kLdsBudget) {
            const uint32_t tiles = (rows + rw - 1) / rw;
            const void *kernel = reinterpret_cast<const void *>(&gemm_q8k_stream<TYPE, MT>);
            const uint32_t capacity = 4u * (uint32_t)(device_cus() * occupancy(kernel, 256, lds));
            const uint32_t per_wave = (tiles + capacity - 1) / capacity;
            const uint32_t waves = (tiles + per_wave - 1) / per_wave;
            hipLaunchKernelGGL((gemm_q8k_stream<TYPE, MT>), dim3((waves + 3) / 4), dim3(256), lds, stream,
                               w, x, y, ldy, rows, nblk, rw, tiles, grid);
            return;
        }
    }
    uint32_t rwc = 256u / (uint32_t)(F::group * MT);
    if (rwc > 4) rwc = 4;
    if (rwc > rows) rwc = rows;
    uint32_t ch = nblk;
    auto lds_of = [&](uint32_t c) {
        return grid_lds + (size_t)MT * c * F::act + (size_t)rwc * c * MT * F::slot * 4;
    };
    while (lds_of(ch) > 48 * 1024 && ch > 4) ch = (ch + 1) / 2;
    hipLaunchKernelGGL((gemm_q8k_chunked<TYPE, MT>), dim3((rows + rwc - 1) / rwc), dim3(256), lds_of(ch), stream,
                       w, x, y, ldy, rows, nblk, rwc, ch, grid);
}

template <int TYPE>
static void launch_m(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t nblk,
                     const uint2 *grid, hipStream_t stream)
{
    switch (m) {
    case 1: launch_typed<TYPE, 1>(w, x, y, ldy, rows, nblk, grid, stream); break;
    case 2: launch_typed<TYPE, 2>(w, x, y, ldy, rows, nblk, grid, stream); break;
    case 3: launch_typed<TYPE, 3>(w, x, y, ldy, rows, nblk, grid, stream); break;
    case 4: launch_typed<TYPE, 4>(w, x, y, ldy, rows, nblk, grid, stream); break;
    case 5: launch_typed<TYPE, 5>(w, x, y, ldy, rows, nblk, grid, stream); break;
    case 6: launch_typed<TYPE, 6>(w, x, y, ldy, rows, nblk, grid, stream); break;
    case 7: launch_typed<TYPE, 7>(w, x, y, ldy, rows, nblk, grid, stream); break;
    default: launch_typed<TYPE, 8>(w, x, y, ldy, rows, nblk, grid, stream); break;
    }
}

/* Enqueue y[t * ldy + row] = W_row . x_t for t < m (all device pointers).
 * x is m * nblk Q8_K blocks, token-major.  grid is the IQ1_M codebook as
 * 2048 x 8 int8 (unused for the other types). */
bool launch_gemm_ld(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                    uint32_t nblk, const void *grid, hipStream_t stream)
{
    if (m < 1 || m > 8 || ldy < rows) return false;
    /* IQ1_M at the Qwen3.8 row widths: the matrix-core kernel (q38_iq1m.hip) */
    if (type == kIQ1M && launch_gemm_iq1m_mfma(m, w, x, y, ldy, rows, nblk, grid, stream)) return true;
    if (launch_gemv_lanes(type, m, w, x, y, ldy, rows, nblk, stream)) return true;
    const uint2 *g = static_cast<const uint2 *>(grid);
    switch (type) {
    case kQ4K: launch_m<kQ4K>(m, w, x, y, ldy, rows, nblk, g, stream); return true;
    case kQ6K: launch_m<kQ6K>(m, w, x, y, ldy, rows, nblk, g, stream); return true;
    case kIQ1M: launch_m<kIQ1M>(m, w, x, y, ldy, rows, nblk, g, stream); return true;
    default: return false;
    }
}

bool launch_gemm(int type, int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t rows,
                 uint32_t nblk, const void *grid, hipStream_t stream)
{
    return launch_gemm_ld(type, m, w, x, y, rows, rows, nblk, grid, stream);
}

}  // namespace q38
