/* Q4_K x Q8_K for 2..8 tokens on the gfx950 matrix cores, 32 weight rows per
 * wavefront (v_mfma_f32_32x32x16_f16), over the 16-row tiled copy built by
 * repack_q4k_tiles ([tile = row / 16][block][row % 16][144 bytes]).
 *
 * Arithmetic (as in q38_tiled.hip).  Per row, token and super-block b the
 * reference's AVX2 kernel (src/qwen38/qwen38_quant.c:1546-1634) forms eight
 * exact integers W[b][l] (l = AVX2 accumulator lane; lane l of chunk c is
 * quant dword l of the chunk: low nibbles = elements 64c + 4l + u, high
 * nibbles = elements 64c + 32 + 4l + u, scales sc[2c] and sc[2c + 1]) and
 * four min sums M[b][i], then runs fp32 chains acc[l] = fmaf(d_b, W, acc[l]),
 * accm[i] = fmaf(-dmin_b, M, accm[i]) over b in order.  Every product sc * q
 * (<= 945) and activation (int8) is exact in fp16 and every partial sum is
 * an integer below 2^22, so the matrix core returns W exactly.
 *
 * Mapping.  Lane i of a wavefront: r = i % 32 (tile row; the wavefront's 32
 * rows are two consecutive 16-row tiles), q = i / 32.  For chunk pair c2 and
 * AVX2 lane p (one MFMA):
 *   B (16 x 32): K-slots 8q..8q+7 of column r = the 8 quants of lane p in
 *     chunk c = 2 c2 + q of row r, as fp16 sc * q;
 *   A (32 x 16): row m = (g, t) = (m / 4, m % 4), K-slots 8q..8q+7 = token
 *     t's activations of lane g in chunk c (lane i supplies row m = r);
 *   D_p[(g, t)][r] accumulated over c2 = sum over all chunks of
 *     act(g) . w(p), which for g == p is W[b][p] of token t.
 * Lane (r, q) holds D rows 8 (j / 4) + 4 q + j % 4 in register j, i.e. the
 * diagonal of D_p for p = 2k + q at registers 4k .. 4k + 3: it owns AVX2
 * lanes q, q + 2, q + 4, q + 6 and min lanes (= chunks) q, q + 2 of row r.
 *
 * Work split.  S wavefronts share a 32-row tile; wavefront s computes the
 * integer sums of blocks b = s (mod S).  With S > 1 each round of S blocks
 * goes through a double-buffered LDS ring (per lane: W of every token, and
 * in a ring of its own the three header dwords the chains use), and after a barrier wavefront s advances the chains of
 * tokens t = s (mod S) over the round's blocks in block order, so the fp32
 * order is the reference's.  The owner of a token applies the reference's
 * final tree: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) + ((m0+m2)+(m1+m3))
 * (qwen38_quant.c:303-310, 1626-1630).
 *
 * Memory.  Buffer loads with the block offset in a scalar, P blocks ahead;
 * a ring slot is refilled right after its last use.
 */
#include "q38_device.h"
#include "q38_kernels.h"
#include "q38_q4k_mfma.h"

namespace q38 {

namespace {

/* loads of one block for one lane */
template <int TS>
struct Blk {
    uint4 h;                 /* header of row r: d|dmin, 12 scale/min bytes */
    uint4 w0[2], w1[2];      /* quant dwords 0..7 of chunk q (w0) and q + 2 (w1) */
    uint32_t lo[TS][2], hi[TS][2];   /* activations: token set, chunk pair */
};

}  // namespace

/* LDS bytes of one workgroup of gemm_q4k_t32 */
template <int MT, int NB, int S>
constexpr int t32_lds_bytes()
{
    return MT * NB * 8 * 2 + MT * NB * 4 + (S > 1 ? 2 * S * 64 * (MT * 16 + 3 * 4) : 0);
}

/* Wavefronts per SIMD the registers are held to: one block in flight with a
 * workgroup small enough for five per compute unit (64 KB of LDS per five,
 * less a 512-byte allocation granule each) runs five; otherwise no bound. */
template <int MT, int NB, int S, int P>
constexpr int t32_min_waves()
{
    return P == 1 && S == 4 && t32_lds_bytes<MT, NB, S>() <= 163840 / 5 - 512 ? 5 : 1;
}

template <int MT, int NB, int S, int P>
__global__ __launch_bounds__(64 * S, (t32_min_waves<MT, NB, S, P>())) void gemm_q4k_t32(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                       float *__restrict__ y, uint32_t ldy, uint32_t rows)
{
    constexpr int TS = (MT + 3) / 4;           /* MFMA token sets of four */
    constexpr int KB = (NB + S - 1) / S;       /* rounds */
    constexpr int NO = (MT + S - 1) / S;       /* chains' tokens per wavefront */
    constexpr int RP = S > 1 ? 2 : 1;
    constexpr int RING = S > 1 ? RP * S * MT * 64 : 1;
    constexpr int HRING = S > 1 ? RP * S * 3 * 64 : 1;
    /* 32-element sub-block sums of the activations, int16 (|sum| <= 4096),
     * sub-blocks 2c and 2c + 1 of chunk c in one dword */
    __shared__ __attribute__((aligned(16))) int16_t sub_s[MT * NB * 8];
    __shared__ float xs_s[MT * NB];
    __shared__ uint4 ring[RING];        /* [parity][wavefront][token][lane] */
    __shared__ uint32_t hring[HRING];   /* [parity][wavefront][header dword][lane] */

    const int lane = threadIdx.x & 63;
    const int sw = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = lane & 31, q = lane >> 5, g = r >> 2, tk = r & 3;
    const uint32_t ntiles = (rows + kRows16 - 1) / kRows16;
    const uint32_t t0 = 2 * blockIdx.x;
    const bool pair = t0 + 1 < ntiles;   /* second 16-row tile present */

    const uint8_t *tb = w + (size_t)t0 * NB * kTileBlock;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(tb), 0, (pair ? 2 : 1) * NB * kTileBlock, kRawBuffer);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(x), 0, MT * NB * kQ8KBytes, kRawBuffer);
    /* rows of a missing second tile re-read the first tile (never stored) */
    const uint32_t hoff = (uint32_t)((pair ? (r >> 4) : 0) * NB * kTileBlock + (r & 15) * kBlockBytes);
    const uint32_t q0off = hoff + 16 + 32 * q, q1off = q0off + 64;
    uint32_t xoff[TS];   /* token tk + 4s (clamped), lane g, chunk q, low half */
#pragma unroll
    for (int s = 0; s < TS; ++s) {
        const int t = tk + 4 * s < MT ? tk + 4 * s : MT - 1;
        xoff[s] = (uint32_t)(t * NB * kQ8KBytes + 4 + 64 * q + 4 * g);
    }
    auto block_of = [&](int k) {
        const int b = sw + S * k;
        return b < NB ? b : NB - 1;   /* past the end: re-read the last block, results unused */
    };
    auto load = [&](int k) {
        const int b = block_of(k);
        const int wo = b * kTileBlock, xo = b * kQ8KBytes;
        Blk<TS> c;
        int4v v = __builtin_amdgcn_raw_buffer_load_b128(wr, hoff, wo, 0);
        c.h = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q0off, wo, 0);
        c.w0[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q0off + 16, wo, 0);
        c.w0[1] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q1off, wo, 0);
        c.w1[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q1off + 16, wo, 0);
        c.w1[1] = make_uint4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int s = 0; s < TS; ++s)
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2) {
                c.lo[s][c2] = __builtin_amdgcn_raw_buffer_load_b32(xr, xoff[s] + 128 * c2, xo, 0);
                c.hi[s][c2] = __builtin_amdgcn_raw_buffer_load_b32(xr, xoff[s] + 128 * c2 + 32, xo, 0);
            }
        return c;
    };
    Blk<TS> slot[P];
#pragma unroll
    for (int i = 0; i < P; ++i) slot[i] = load(i);

    /* activation scales and min pair sums (Q8_K dword 0 and sum dwords
     * 65..72), eight loads in flight per thread */
    {
        constexpr int kTotal = MT * NB * 9, kThreads = 64 * S, kDepth = 8;
        for (int i0 = threadIdx.x; i0 < kTotal; i0 += kDepth * kThreads) {
            uint32_t v[kDepth];
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int i = i0 + u * kThreads < kTotal ? i0 + u * kThreads : kTotal - 1;
                const int blk = i / 9, k = i - blk * 9;
                v[u] = __builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)(blk * kQ8KBytes + (k == 0 ? 0 : 256 + 4 * k)), 0, 0);
            }
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int i = i0 + u * kThreads;
                if (i >= kTotal) break;
                const int blk = i / 9, k = i - blk * 9;
                if (k == 0) xs_s[blk] = __uint_as_float(v[u]);
                else sub_s[blk * 8 + (k - 1)] = (int16_t)((int)(int16_t)(v[u] & 0xffffu) + ((int)v[u] >> 16));
            }
        }
    }
    __syncthreads();

    constexpr int NC = S == 1 ? MT : NO;   /* chain token slots of this wavefront */
    float acc[NC][4], accm[NC][2];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[j][k] = 0.0f;
        accm[j][0] = accm[j][1] = 0.0f;
    }
    int own[NC];   /* token of chain slot j (clamped; slots past MT are dropped) */
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int t = S == 1 ? j : sw + S * j;
        own[j] = t < MT ? t : MT - 1;
    }

    uint32_t kMask = 0x000f000fu, kMaskHi = 0x00f000f0u, kMagic = 0x64006400u;
    asm volatile("" : "+v"(kMask), "+v"(kMaskHi), "+v"(kMagic));
    /* byte 2q of a scale word: sub-block 2q (low nibbles) of its chunk */
    const uint32_t sel_lo = 0x07000700u + (uint32_t)(2 * q) * 0x00010001u;

    /* integer sums of one block: wv[t][k] = W[b][2k + q] of token t */
    auto block_sums = [&](const Blk<TS> &c, float (&wv)[MT][4]) {
        const uint32_t Y = c.h.y, Wd = c.h.w;
        /* 6-bit scales (qwen38_quant.c:131-143): sub-blocks 2q, 2q+1 from
         * bytes 0..3, sub-blocks 4+2q, 5+2q from bytes 8..11 low nibbles and
         * the top bits of bytes 0..3 */
        const uint32_t scw[2] = {Y & 0x3f3f3f3fu, (Wd & 0x0f0f0f0fu) | ((Y >> 2) & 0x30303030u)};
        Scale sc[2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            const half2v SL = pair_byte(scw[c2], sel_lo), SH = pair_byte(scw[c2], sel_lo + 0x00010001u);
            sc[c2].sl = SL;
            sc[c2].nl = SL * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
            sc[c2].sh16 = SH * (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
            sc[c2].nh = SH * (half2v){(_Float16)-64.0f, (_Float16)-64.0f};
        }
        half8 av[TS][2];
#pragma unroll
        for (int s = 0; s < TS; ++s)
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2) av[s][c2] = act8(c.lo[s][c2], c.hi[s][c2]);
        const uint32_t q0[8] = {c.w0[0].x, c.w0[0].y, c.w0[0].z, c.w0[0].w, c.w0[1].x, c.w0[1].y, c.w0[1].z, c.w0[1].w};
        const uint32_t q1[8] = {c.w1[0].x, c.w1[0].y, c.w1[0].z, c.w1[0].w, c.w1[1].x, c.w1[1].y, c.w1[1].z, c.w1[1].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const half8 b00 = dequant(q0[2 * k], sc[0], kMask, kMaskHi, kMagic);
            const half8 b10 = dequant(q1[2 * k], sc[1], kMask, kMaskHi, kMagic);
            const half8 b01 = dequant(q0[2 * k + 1], sc[0], kMask, kMaskHi, kMagic);
            const half8 b11 = dequant(q1[2 * k + 1], sc[1], kMask, kMaskHi, kMagic);
#pragma unroll
            for (int s = 0; s < TS; ++s) {
                const float16v z = {};
                float16v d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[s][0], b00, z, 0, 0, 0);
                float16v d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[s][0], b01, z, 0, 0, 0);
                d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[s][1], b10, d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[s][1], b11, d1, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int t = 4 * s + j;
                    if (t < MT) wv[t][k] = q ? d1[4 * k + j] : d0[4 * k + j];
                }
            }
        }
    };

    /* the token-independent part of a block header for this lane's chains:
     * d and dmin (the block's fp16 pair), and the 6-bit mins
     * (qwen38_quant.c:131-143) of sub-blocks 2c, 2c + 1 of chunks c = q and
     * q + 2 as u16 pairs */
    const uint32_t min_sel = q ? 0x0c030c02u : 0x0c010c00u;
    auto chain_header = [&](const uint4 &h) {
        const uint32_t mw0 = h.z & 0x3f3f3f3fu, mw1 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        return make_uint3(h.x, __builtin_amdgcn_perm(0u, mw0, min_sel), __builtin_amdgcn_perm(0u, mw1, min_sel));
    };

    /* advance chain slot j (token t) over block b with W values wq and the
     * chain header h; the min sums m0 * s(2c) + m1 * s(2c + 1) are exact
     * int32 dot products */
    auto chain = [&](int j, int t, int b, const uint3 &h, const float (&wq)[4]) {
        const float xs = xs_s[t * NB + b];
        const float dx = fmul_rn(f16_to_f32(h.x), xs), mx = -fmul_rn(f16_to_f32(h.x >> 16), xs);
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[j][k] = __builtin_fmaf(dx, wq[k], acc[j][k]);
        const uint32_t *sub2 = reinterpret_cast<const uint32_t *>(sub_s) + (t * NB + b) * 4 + q;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            const int msum = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, c2 ? h.z : h.y),
                                                    __builtin_bit_cast(short2v, sub2[2 * c2]), 0, false);
            accm[j][c2] = __builtin_fmaf(mx, (float)msum, accm[j][c2]);
        }
    };

    auto round = [&](const Blk<TS> &c, int k) {
        float wv[MT][4];
        const uint3 hd = chain_header(c.h);
        block_sums(c, wv);
        if (S == 1) {
#pragma unroll
            for (int t = 0; t < MT; ++t) chain(t, t, k, hd, wv[t]);
            return;
        }
        const int base = ((k & 1) * S + sw) * MT * 64, hbase = ((k & 1) * S + sw) * 3 * 64;
#pragma unroll
        for (int t = 0; t < MT; ++t)
            ring[base + t * 64 + lane] =
                make_uint4(__float_as_uint(wv[t][0]), __float_as_uint(wv[t][1]), __float_as_uint(wv[t][2]),
                           __float_as_uint(wv[t][3]));
        hring[hbase + lane] = hd.x;
        hring[hbase + 64 + lane] = hd.y;
        hring[hbase + 128 + lane] = hd.z;
        __syncthreads();
#pragma unroll
        for (int f = 0; f < S; ++f) {
            const int b2 = f + S * k;
            if (b2 >= NB) break;
            const int fb = ((k & 1) * S + f) * MT * 64, fhb = ((k & 1) * S + f) * 3 * 64;
            const uint3 h = make_uint3(hring[fhb + lane], hring[fhb + 64 + lane], hring[fhb + 128 + lane]);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const uint4 v = ring[fb + own[j] * 64 + lane];
                const float wq[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                                     __uint_as_float(v.w)};
                chain(j, own[j], b2, h, wq);
            }
        }
    };

    constexpr int kFull = KB / P, kRem = KB % P;
#pragma unroll 1
    for (int it = 0; it < kFull; ++it) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int k = it * P + i;
            round(slot[i], k);
            /* refill the slot after its last use */
            slot[i] = load(k + P);
        }
    }
#pragma unroll
    for (int i = 0; i < kRem; ++i) round(slot[i], KB - kRem + i);

    /* final trees; lane q = 0 of each row stores */
    const uint32_t row = 32 * blockIdx.x + (uint32_t)r;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int t = S == 1 ? j : sw + S * j;
        if (t >= MT) break;
        float a = fadd_rn(fadd_rn(acc[j][0], acc[j][2]), fadd_rn(acc[j][1], acc[j][3]));
        a = fadd_rn(a, __shfl_xor(a, 32, 64));
        float m = fadd_rn(accm[j][0], accm[j][1]);
        m = fadd_rn(m, __shfl_xor(m, 32, 64));
        if (q == 0 && row < rows) y[(size_t)t * ldy + row] = fadd_rn(a, m);
    }
}

/* Role-split form of gemm_q4k_t32 for 2..4 tokens on matrices with fewer
 * 32-row tiles than the chip has compute units (the 5120-row projections),
 * where one wavefront per SIMD leaves every round's latency exposed.  S
 * producer wavefronts compute the integer sums of the tile's blocks (block
 * b by producer b mod S, the same MFMA products and lane mapping as
 * gemm_q4k_t32) into a double-buffered LDS ring, one round of S blocks per
 * iteration; MT chain wavefronts (one per token) run the fp32 chains of the
 * previous round's blocks in block order while the producers fill the next
 * round, so the chains never wait on the dequantisation.  One barrier per
 * iteration orders the ring: round k is written in iteration k and read in
 * iteration k + 1, when the other half is being written. */
template <int MT, int NB, int S, int P>
__global__ __launch_bounds__(64 * (S + MT)) void gemm_q4k_t32r(const uint8_t *__restrict__ w,
                                                              const uint8_t *__restrict__ x, float *__restrict__ y,
                                                              uint32_t ldy, uint32_t rows)
{
    static_assert(MT >= 2 && MT <= 4, "one MFMA token set");
    constexpr int KB = (NB + S - 1) / S;   /* rounds */
    __shared__ __attribute__((aligned(16))) int16_t sub_s[MT * NB * 8];
    __shared__ float xs_s[MT * NB];
    __shared__ uint4 ring[2 * S * MT * 64];       /* [parity][producer][token][lane] */
    __shared__ uint32_t hring[2 * S * 3 * 64];    /* [parity][producer][header dword][lane] */

    const int lane = threadIdx.x & 63;
    const int sw = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const bool producer = sw < S;
    const int r = lane & 31, q = lane >> 5, g = r >> 2, tk = r & 3;
    const uint32_t ntiles = (rows + kRows16 - 1) / kRows16;
    const uint32_t t0 = 2 * blockIdx.x;
    const bool pair = t0 + 1 < ntiles;

    const uint8_t *tb = w + (size_t)t0 * NB * kTileBlock;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(tb), 0, (pair ? 2 : 1) * NB * kTileBlock, kRawBuffer);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(x), 0, MT * NB * kQ8KBytes, kRawBuffer);
    const uint32_t hoff = (uint32_t)((pair ? (r >> 4) : 0) * NB * kTileBlock + (r & 15) * kBlockBytes);
    const uint32_t q0off = hoff + 16 + 32 * q, q1off = q0off + 64;
    const int tok = tk < MT ? tk : MT - 1;
    const uint32_t xoff = (uint32_t)(tok * NB * kQ8KBytes + 4 + 64 * q + 4 * g);
    auto load = [&](int k) {
        int b = sw + S * k;
        b = b < NB ? b : NB - 1;   /* past the end: re-read the last block, results unused */
        const int wo = b * kTileBlock, xo = b * kQ8KBytes;
        Blk<1> c;
        int4v v = __builtin_amdgcn_raw_buffer_load_b128(wr, hoff, wo, 0);
        c.h = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q0off, wo, 0);
        c.w0[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q0off + 16, wo, 0);
        c.w0[1] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q1off, wo, 0);
        c.w1[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, q1off + 16, wo, 0);
        c.w1[1] = make_uint4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            c.lo[0][c2] = __builtin_amdgcn_raw_buffer_load_b32(xr, xoff + 128 * c2, xo, 0);
            c.hi[0][c2] = __builtin_amdgcn_raw_buffer_load_b32(xr, xoff + 128 * c2 + 32, xo, 0);
        }
        return c;
    };
    Blk<1> slot[P];
    if (producer) {
#pragma unroll
        for (int i = 0; i < P; ++i) slot[i] = load(i);
    }

    /* activation scales and min pair sums, as gemm_q4k_t32 */
    {
        constexpr int kTotal = MT * NB * 9, kThreads = 64 * (S + MT), kDepth = 4;
        for (int i0 = threadIdx.x; i0 < kTotal; i0 += kDepth * kThreads) {
            uint32_t v[kDepth];
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int i = i0 + u * kThreads < kTotal ? i0 + u * kThreads : kTotal - 1;
                const int blk = i / 9, k = i - blk * 9;
                v[u] = __builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)(blk * kQ8KBytes + (k == 0 ? 0 : 256 + 4 * k)),
                                                            0, 0);
            }
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int i = i0 + u * kThreads;
                if (i >= kTotal) break;
                const int blk = i / 9, k = i - blk * 9;
                if (k == 0) xs_s[blk] = __uint_as_float(v[u]);
                else sub_s[blk * 8 + (k - 1)] = (int16_t)((int)(int16_t)(v[u] & 0xffffu) + ((int)v[u] >> 16));
            }
        }
    }
    __syncthreads();

    uint32_t kMask = 0x000f000fu, kMaskHi = 0x00f000f0u, kMagic = 0x64006400u;
    asm volatile("" : "+v"(kMask), "+v"(kMaskHi), "+v"(kMagic));
    const uint32_t sel_lo = 0x07000700u + (uint32_t)(2 * q) * 0x00010001u;
    const uint32_t min_sel = q ? 0x0c030c02u : 0x0c010c00u;

    /* producer: integer sums of one block into ring half `par` */
    auto produce = [&](const Blk<1> &c, int par) {
        const uint32_t Y = c.h.y, Wd = c.h.w;
        const uint32_t scw[2] = {Y & 0x3f3f3f3fu, (Wd & 0x0f0f0f0fu) | ((Y >> 2) & 0x30303030u)};
        Scale sc[2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            const half2v SL = pair_byte(scw[c2], sel_lo), SH = pair_byte(scw[c2], sel_lo + 0x00010001u);
            sc[c2].sl = SL;
            sc[c2].nl = SL * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
            sc[c2].sh16 = SH * (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
            sc[c2].nh = SH * (half2v){(_Float16)-64.0f, (_Float16)-64.0f};
        }
        half8 av[2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) av[c2] = act8(c.lo[0][c2], c.hi[0][c2]);
        const uint32_t q0[8] = {c.w0[0].x, c.w0[0].y, c.w0[0].z, c.w0[0].w, c.w0[1].x, c.w0[1].y, c.w0[1].z, c.w0[1].w};
        const uint32_t q1[8] = {c.w1[0].x, c.w1[0].y, c.w1[0].z, c.w1[0].w, c.w1[1].x, c.w1[1].y, c.w1[1].z, c.w1[1].w};
        float wv[MT][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const half8 b00 = dequant(q0[2 * k], sc[0], kMask, kMaskHi, kMagic);
            const half8 b10 = dequant(q1[2 * k], sc[1], kMask, kMaskHi, kMagic);
            const half8 b01 = dequant(q0[2 * k + 1], sc[0], kMask, kMaskHi, kMagic);
            const half8 b11 = dequant(q1[2 * k + 1], sc[1], kMask, kMaskHi, kMagic);
            const float16v z = {};
            float16v d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[0], b00, z, 0, 0, 0);
            float16v d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[0], b01, z, 0, 0, 0);
            d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[1], b10, d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[1], b11, d1, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < MT; ++j) wv[j][k] = q ? d1[4 * k + j] : d0[4 * k + j];
        }
        const int base = (par * S + sw) * MT * 64;
#pragma unroll
        for (int t = 0; t < MT; ++t)
            ring[base + t * 64 + lane] = make_uint4(__float_as_uint(wv[t][0]), __float_as_uint(wv[t][1]),
                                                    __float_as_uint(wv[t][2]), __float_as_uint(wv[t][3]));
        const uint32_t mw0 = c.h.z & 0x3f3f3f3fu, mw1 = ((c.h.w >> 4) & 0x0f0f0f0fu) | ((c.h.z >> 2) & 0x30303030u);
        const int hbase = (par * S + sw) * 3 * 64;
        hring[hbase + lane] = c.h.x;
        hring[hbase + 64 + lane] = __builtin_amdgcn_perm(0u, mw0, min_sel);
        hring[hbase + 128 + lane] = __builtin_amdgcn_perm(0u, mw1, min_sel);
    };

    /* chain wavefront of token t: acc over AVX2 lanes q, q+2, q+4, q+6, accm
     * over min lanes q, q+2 */
    const int t = producer ? 0 : sw - S;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accm[2] = {0.0f, 0.0f};
    auto consume = [&](int par, int k) {
#pragma unroll
        for (int f = 0; f < S; ++f) {
            const int b = f + S * k;
            if (b >= NB) break;
            const int fb = (par * S + f) * MT * 64, fhb = (par * S + f) * 3 * 64;
            const uint32_t hx = hring[fhb + lane], hy = hring[fhb + 64 + lane], hz = hring[fhb + 128 + lane];
            const uint4 v = ring[fb + t * 64 + lane];
            const float xs = xs_s[t * NB + b];
            const float dx = fmul_rn(f16_to_f32(hx), xs), mx = -fmul_rn(f16_to_f32(hx >> 16), xs);
            acc[0] = __builtin_fmaf(dx, __uint_as_float(v.x), acc[0]);
            acc[1] = __builtin_fmaf(dx, __uint_as_float(v.y), acc[1]);
            acc[2] = __builtin_fmaf(dx, __uint_as_float(v.z), acc[2]);
            acc[3] = __builtin_fmaf(dx, __uint_as_float(v.w), acc[3]);
            const uint32_t *sub2 = reinterpret_cast<const uint32_t *>(sub_s) + (t * NB + b) * 4 + q;
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2) {
                const int msum = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, c2 ? hz : hy),
                                                        __builtin_bit_cast(short2v, sub2[2 * c2]), 0, false);
                accm[c2] = __builtin_fmaf(mx, (float)msum, accm[c2]);
            }
        }
    };

#pragma unroll 1
    for (int k = 0; k <= KB; ++k) {
        if (producer) {
            if (k < KB) {
                const int i = k % P;
                /* the slot of round k (P rounds are in flight) */
#pragma unroll
                for (int u = 0; u < P; ++u)
                    if (u == i) {
                        if (sw + S * k < NB) produce(slot[u], k & 1);
                        slot[u] = load(k + P);
                    }
            }
        } else if (k > 0) {
            consume((k - 1) & 1, k - 1);
        }
        __syncthreads();
    }

    if (!producer) {
        /* the reference's final tree, as gemm_q4k_t32 */
        const uint32_t row = 32 * blockIdx.x + (uint32_t)r;
        float a = fadd_rn(fadd_rn(acc[0], acc[2]), fadd_rn(acc[1], acc[3]));
        a = fadd_rn(a, __shfl_xor(a, 32, 64));
        float m = fadd_rn(accm[0], accm[1]);
        m = fadd_rn(m, __shfl_xor(m, 32, 64));
        if (q == 0 && row < rows) y[(size_t)t * ldy + row] = fadd_rn(a, m);
    }
}

namespace {

/* Launch shape (measured on MI355X for 2..4 tokens and 5120..34816 rows):
 * four wavefronts per 32-row tile.  Wide matrices keep one block in flight
 * per wavefront (up to five wavefronts per SIMD where the LDS allows, see
 * t32_min_waves), which hides more latency than a deeper prefetch at three.  A
 * matrix with fewer tiles than the chip has compute units runs one
 * workgroup per unit (one wavefront per SIMD) and keeps two blocks in
 * flight. */
constexpr int kT32Waves = 4, kT32Prefetch = 1;
constexpr int kT32PrefetchNarrow = 2;
constexpr uint32_t kT32NarrowTiles = 256;
/* Narrow matrices at 2..4 tokens run the role-split kernel: 8 producer
 * wavefronts, one block in flight each.  Measured on MI355X (3 tokens, weights
 * rotated over 1 GiB): 5120 x 17408 25.8 -> 21.4 us, 5120 x 6144 11.3 -> 9.3 us
 * against gemm_q4k_t32 (6 or 12 producers, or two blocks in flight: 21.2 to
 * 22.7 and 9.3 to 12.6 us). */
constexpr int kT32rProducers = 8, kT32rPrefetch = 1;

template <int MT, int NB, int S, int P>
void launch_t32r(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, hipStream_t stream)
{
    hipLaunchKernelGGL((gemm_q4k_t32r<MT, NB, S, P>), dim3((rows + 31) / 32), dim3(64 * (S + MT)), 0, stream, w, x, y,
                       ldy, rows);
}

template <int MT, int NB>
bool launch_t32_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, hipStream_t stream)
{
    const uint32_t tiles32 = (rows + 31) / 32;
    if constexpr (MT <= 4) {
        if (tiles32 < kT32NarrowTiles) {
            launch_t32r<MT, NB, kT32rProducers, kT32rPrefetch>(w, x, y, ldy, rows, stream);
            return hipGetLastError() == hipSuccess;
        }
    }
    if (tiles32 < kT32NarrowTiles)
        hipLaunchKernelGGL((gemm_q4k_t32<MT, NB, kT32Waves, kT32PrefetchNarrow>), dim3(tiles32), dim3(64 * kT32Waves),
                           0, stream, w, x, y, ldy, rows);
    else
        hipLaunchKernelGGL((gemm_q4k_t32<MT, NB, kT32Waves, kT32Prefetch>), dim3(tiles32), dim3(64 * kT32Waves), 0,
                           stream, w, x, y, ldy, rows);
    return hipGetLastError() == hipSuccess;
}

template <int NB>
bool launch_t32_nb(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                   hipStream_t stream)
{
    switch (m) {
    case 2: return launch_t32_typed<2, NB>(w, x, y, ldy, rows, stream);
    case 3: return launch_t32_typed<3, NB>(w, x, y, ldy, rows, stream);
    case 4: return launch_t32_typed<4, NB>(w, x, y, ldy, rows, stream);
    case 5: return launch_t32_typed<5, NB>(w, x, y, ldy, rows, stream);
    case 6: return launch_t32_typed<6, NB>(w, x, y, ldy, rows, stream);
    case 7: return launch_t32_typed<7, NB>(w, x, y, ldy, rows, stream);
    case 8: return launch_t32_typed<8, NB>(w, x, y, ldy, rows, stream);
    default: return false;
    }
}

}  // namespace

/* y[t * ldy + row] = W_row . x_t (t < m) from the 16-row tiled copy, 32 rows
 * per wavefront; 2..8 tokens (5..8 take a second MFMA token set and about
 * twice the registers); false for unsupported shapes. */
bool launch_gemm_q4k_t32(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                         uint32_t nb, hipStream_t stream)
{
    if (!rows || ldy < rows) return false;
    switch (nb) {
    case 20: return launch_t32_nb<20>(m, w_tiled, x, y, ldy, rows, stream);
    case 24: return launch_t32_nb<24>(m, w_tiled, x, y, ldy, rows, stream);
    case 40: return launch_t32_nb<40>(m, w_tiled, x, y, ldy, rows, stream);
    case 68: return launch_t32_nb<68>(m, w_tiled, x, y, ldy, rows, stream);
    default: return false;
    }
}

}  // namespace q38
