/* Q4_K x Q8_K for 2..8 tokens on the gfx950 matrix cores, over a 16-row
 * tiled copy of the weights (the speculative verify batch and prefill).
 *
 * Layout.  The tiled copy of a Q4_K matrix of R rows x NB super-blocks is
 * [tile = row / 16][block][row % 16][144 bytes]: the 16 rows' blocks b sit
 * together (2304 contiguous bytes), so a wavefront walking a tile reads one
 * contiguous stretch per step.  The last tile is zero-padded.
 *
 * Arithmetic.  The reference's AVX2 kernel (src/qwen38/qwen38_quant.c:
 * 1546-1634) keeps, per row and token, eight fp32 accumulator lanes and four
 * min lanes; for every super-block b in order, lane l adds d_b * W[b][l] and
 * min lane i adds -dmin_b * M[b][i], with
 *   W[b][l] = sum_c sc[2c] * sum_u lo(q[32c+4l+u]) * a[64c+4l+u]
 *           + sc[2c+1] * sum_u hi(q[32c+4l+u]) * a[64c+32+4l+u]
 *   M[b][i] = m[2i] * (s[4i] + s[4i+1]) + m[2i+1] * (s[4i+2] + s[4i+3]).
 * W[b][l] is a 32-term integer dot product of sc * q (<= 945, exact in
 * fp16) with the int8 activations (exact in fp16); every product and every
 * partial sum is an integer below 2^22, so v_mfma_f32_16x16x32_f16 returns
 * it exactly whatever its internal order.  The fp32 chains then run in the
 * reference's order with its fmaf and product roundings.
 *
 * Mapping.  Two wavefronts share a tile: wavefront G owns AVX2 lanes
 * 4G..4G+3.  Lane i: row r = i % 16, chunk q = i / 16 (elements 64q..64q+63),
 * and as an A row m = (g, t) = (i / 4 % 4, i % 4).  For each p = 0..3:
 *   B_p (weights): K-slot q, column r = the 8 quants of AVX2 lane 4G + p in
 *     chunk q as fp16 sc * q (one dword: masks, then a packed fma per pair,
 *     (1024 + n) * sc - 1024 * sc);
 *   A (activations): row (g, t), K-slot q = token t's 8 activations of AVX2
 *     lane 4G + g in chunk q;
 *   D_p[(g, t)][r] = sum over chunks of act(4G + g) . w(4G + p), which for
 *     g == p is W[b][4G + p] for token t.
 * Lane (r, q) reads that diagonal from D_q: it runs the chains of AVX2 lane
 * 4G + q (tokens t = 0..MT-1, four per MFMA token set) and, in wavefront 0,
 * of min lane q.  Wavefront 1 hands its lanes to wavefront 0 through LDS for
 * the reference's final tree.
 *
 * Memory.  Weights and activations are read with buffer loads whose block
 * offset is a scalar, four blocks ahead of use; each ring slot is refilled
 * only after its last use so the loop-carried registers stay in place and
 * the waits count only the loads still needed.  Scales and min pair sums of
 * the activations are staged in LDS once per workgroup.
 */
#include "q38_device.h"
#include "q38_kernels.h"


namespace q38 {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int kTileRows = 16;
constexpr int kQ4KBytes = 144;
constexpr int kTileBlockBytes = kTileRows * kQ4KBytes;   /* 2304 */
constexpr uint32_t kBufferFlags = 0x00020000u;           /* raw 32-bit buffer resource (gfx9) */

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

/* fp16 pair (n, n) for an integer n < 1024: (1024 + n) - 1024 */
__device__ __forceinline__ half2v pair_of(uint32_t n)
{
    const half2v x = as_h2((n | (n << 16)) | 0x64006400u);
    return x - (half2v){(_Float16)1024.0f, (_Float16)1024.0f};
}

struct Slot {
    uint4 h;        /* block header: d, dmin, 12 scale/min bytes */
    uint4 qd;       /* quant dwords 4G .. 4G+3 of chunk q */
    uint32_t alo[2], ahi[2];   /* per token set: 4 activations of half 0 and of half 1 */
};

}  // namespace

/* TPW tiles per workgroup, 2 * S wavefronts per tile: wavefront (G, phase)
 * owns AVX2 lanes 4G..4G+3 and the blocks b = phase (mod S), P of them in
 * flight.
 * With S > 1 every round of S blocks passes through a double-buffered LDS
 * ring: each wavefront leaves its block's integer sums (and, in wavefront
 * G = 0, the min sums and the block's d/dmin), and after a barrier the
 * wavefronts (G, t mod S) advance token t's chains over the round's blocks
 * in block order. */
template <int MT, int NB, int S, int P, int TPW>
__global__ __launch_bounds__(128 * S * TPW) void gemm_q4k_tiled(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                           float *__restrict__ y, uint32_t ldy, uint32_t rows)
{
    static_assert(NB % S == 0, "the blocks must split evenly over the wavefronts of a tile");
    constexpr int TS = (MT + 3) / 4;            /* MFMA token sets of four */
    constexpr int KB = NB / S;                  /* rounds */
    constexpr int NT = (MT + S - 1) / S;        /* tokens whose chains a wavefront owns */
    constexpr int RP = S > 1 ? 2 : 1;           /* ring parities */
    __shared__ int2 pairs_s[MT * NB * 4];
    __shared__ float xs_s[MT * NB];
    /* ring record of wavefront (G, phase): W per token, M per token, d|dmin */
    __shared__ float ring_w[TPW][RP][S][2][MT][64];
    __shared__ int ring_m[TPW][RP][S][2][MT][64];
    __shared__ uint32_t ring_d[TPW][RP][S][2][64];
    __shared__ float xch[TPW][MT][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int G = wave & 1, phase = (wave >> 1) % S, tl = wave / (2 * S);
    const int r = lane & 15, q = lane >> 4, g = (lane >> 2) & 3, tk = lane & 3;
    const uint32_t ntiles = (rows + kTileRows - 1) / kTileRows;
    const uint32_t tile_raw = blockIdx.x * TPW + (uint32_t)tl;
    const uint32_t tile = tile_raw < ntiles ? tile_raw : ntiles - 1;   /* idle waves re-read the last tile */

    /* uniform bases plus 32-bit per-lane offsets */
    const uint8_t *tb = w + (size_t)tile * NB * kTileBlockBytes;
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(tb), 0, NB * kTileBlockBytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(x), 0, MT * NB * kQ8KBytes, kBufferFlags);
    const uint32_t hoff = (uint32_t)(r * kQ4KBytes), qoff = hoff + 16 + 32 * q + 16 * G;
    uint32_t xoff[TS];   /* token tk + 4s (clamped), AVX2 lane 4G + g, chunk q, half 0 */
#pragma unroll
    for (int s = 0; s < TS; ++s) {
        const int t = tk + 4 * s < MT ? tk + 4 * s : MT - 1;
        xoff[s] = (uint32_t)(t * NB * kQ8KBytes + 4 + 64 * q + 4 * (4 * G + g));
    }
    /* this wavefront's k-th block (clamped: loads past the end re-read the
     * last block and are never used) */
    auto block_of = [&](int k) {
        const int b = phase + S * k;
        return b < NB ? b : NB - 1;
    };
    /* tokens owned: t_j = phase + S * j (clamped; chains of t_j >= MT are
     * computed and dropped, which keeps the loop free of branches) */
    int own[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) own[j] = phase + S * j < MT ? phase + S * j : MT - 1;
    auto load = [&](int k) {
        const int b = block_of(k);
        Slot sl;
        const int4v h = __builtin_amdgcn_raw_buffer_load_b128(wr, hoff, b * kTileBlockBytes, 0);
        const int4v qv = __builtin_amdgcn_raw_buffer_load_b128(wr, qoff, b * kTileBlockBytes, 0);
        sl.h = make_uint4(h[0], h[1], h[2], h[3]);
        sl.qd = make_uint4(qv[0], qv[1], qv[2], qv[3]);
#pragma unroll
        for (int s = 0; s < TS; ++s) {
            sl.alo[s] = __builtin_amdgcn_raw_buffer_load_b32(xr, xoff[s], b * kQ8KBytes, 0);
            sl.ahi[s] = __builtin_amdgcn_raw_buffer_load_b32(xr, xoff[s] + 32, b * kQ8KBytes, 0);
        }
        return sl;
    };
    Slot ring[P];
#pragma unroll
    for (int i = 0; i < P; ++i) ring[i] = load(i);

    /* activation scales and min pair sums: Q8_K dword 0 and bsum dwords
     * 65..72, loaded in batches of eight per thread (indices past the end are
     * clamped and their values dropped) so the loads overlap */
    {
        constexpr int kTotal = MT * NB * 9, kThreads = 128 * S * TPW, kDepth = 8;
        const __amdgpu_buffer_rsrc_t sr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(x), 0, MT * NB * kQ8KBytes, kBufferFlags);
        for (int i0 = threadIdx.x; i0 < kTotal; i0 += kDepth * kThreads) {
            uint32_t v[kDepth];
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int i = i0 + u * kThreads < kTotal ? i0 + u * kThreads : kTotal - 1;
                const int blk = i / 9, k = i - blk * 9;
                v[u] = __builtin_amdgcn_raw_buffer_load_b32(sr, (uint32_t)(blk * kQ8KBytes + (k == 0 ? 0 : 256 + 4 * k)), 0, 0);
            }
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int i = i0 + u * kThreads;
                if (i >= kTotal) break;
                const int blk = i / 9, k = i - blk * 9;
                if (k == 0) xs_s[blk] = __uint_as_float(v[u]);
                else reinterpret_cast<int *>(pairs_s)[blk * 8 + (k - 1)] =
                    (int)(int16_t)(v[u] & 0xffffu) + ((int)v[u] >> 16);
            }
        }
    }
    __syncthreads();

    /* S == 1: chains of every token; S > 1: of the owned tokens */
    constexpr int NC = S == 1 ? MT : NT;
    float acc[NC], accm[NC];
#pragma unroll
    for (int t = 0; t < NC; ++t) acc[t] = accm[t] = 0.0f;

    /* loop-invariant per-lane values (the masks live in registers: VOP3
     * forms cannot take two literals) */
    uint32_t kMask = 0x000f000fu, kMaskHi = 0x00f000f0u, kMagic = 0x64006400u;
    asm volatile("" : "+v"(kMask), "+v"(kMaskHi), "+v"(kMagic));
    const int sh = (q & 1) * 16;
    const bool hi_chunk = q >= 2, q_odd = (q & 1) != 0;
    const uint32_t kLow = hi_chunk ? 0x0f0f0f0fu : 0x3f3f3f3fu, kHigh = hi_chunk ? 0x30303030u : 0u;

    /* integer sums of one block: W[b][4G + q] per token into wv[], and in
     * wavefront 0 the min sums M[b][q] into mv[] */
    auto block_sums = [&](const Slot &c, int b, float (&wv)[MT], int (&mv)[MT]) {
        const uint32_t Y = c.h.y, Z = c.h.z, Wd = c.h.w;
        /* 6-bit scales of sub-blocks 2q, 2q+1 (src/qwen38/qwen38_quant.c:131-143) */
        const uint32_t scw = ((hi_chunk ? Wd : Y) & kLow) | ((Y >> 2) & kHigh);
        /* low nibbles sit in bits 0..3 of each half: fp16 1024 + n, times sc,
         * minus 1024 sc.  High nibbles are taken in place from bits 4..7:
         * fp16 1024 + 16 n, times sc / 16, minus 64 sc.  Both products and
         * sums are exact (sc / 16 and 64 sc are exact in fp16). */
        const half2v SL = pair_of((scw >> sh) & 0xffu), SH = pair_of((scw >> (sh + 8)) & 0xffu);
        const half2v k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
        const half2v k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
        const half2v k64 = {(_Float16)-64.0f, (_Float16)-64.0f};
        const half2v NL = SL * k1024, SH16 = SH * k16th, NH = SH * k64;
        half8 bv[4];
        const uint32_t qw[4] = {c.qd.x, c.qd.y, c.qd.z, c.qd.w};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            /* element order per half: u = 0, 2, 1, 3 (the activations use the same) */
            const uint32_t wd = qw[p], w8 = wd >> 8;
            const half2v b0 = __builtin_elementwise_fma(as_h2((wd & kMask) | kMagic), SL, NL);
            const half2v b1 = __builtin_elementwise_fma(as_h2((w8 & kMask) | kMagic), SL, NL);
            const half2v b2 = __builtin_elementwise_fma(as_h2((wd & kMaskHi) | kMagic), SH16, NH);
            const half2v b3 = __builtin_elementwise_fma(as_h2((w8 & kMaskHi) | kMagic), SH16, NH);
            bv[p][0] = b0[0]; bv[p][1] = b0[1]; bv[p][2] = b1[0]; bv[p][3] = b1[1];
            bv[p][4] = b2[0]; bv[p][5] = b2[1]; bv[p][6] = b3[0]; bv[p][7] = b3[1];
        }
#pragma unroll
        for (int s = 0; s < TS; ++s) {
            /* int8 -> fp16: bytes biased by 128 under 0x64 are 1024 + 128 + a */
            const half2v k1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
            const uint32_t ua = c.alo[s] ^ 0x80808080u, ub = c.ahi[s] ^ 0x80808080u;
            const half2v a02 = as_h2(__builtin_amdgcn_perm(0x64646464u, ua, 0x04020400u)) + k1152;
            const half2v a13 = as_h2(__builtin_amdgcn_perm(0x64646464u, ua, 0x04030401u)) + k1152;
            const half2v b02 = as_h2(__builtin_amdgcn_perm(0x64646464u, ub, 0x04020400u)) + k1152;
            const half2v b13 = as_h2(__builtin_amdgcn_perm(0x64646464u, ub, 0x04030401u)) + k1152;
            half8 av;
            av[0] = a02[0]; av[1] = a02[1]; av[2] = a13[0]; av[3] = a13[1];
            av[4] = b02[0]; av[5] = b02[1]; av[6] = b13[0]; av[7] = b13[1];
            float4v D[4];
#pragma unroll
            for (int p = 0; p < 4; ++p)
                D[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[p], (float4v){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 4 * s + j;
                if (t >= MT) break;
                /* the diagonal: lane (r, q) takes D_q */
                const float w01 = q_odd ? D[1][j] : D[0][j], w23 = q_odd ? D[3][j] : D[2][j];
                wv[t] = hi_chunk ? w23 : w01;
            }
        }
        /* 6-bit mins of sub-blocks 2q, 2q+1 (both wavefronts compute them,
         * which keeps the loop free of branches; only wavefront 0's min
         * chains are used) */
        const uint32_t mw = ((hi_chunk ? (Wd >> 4) : Z) & kLow) | ((Z >> 2) & kHigh);
        const int m0 = (int)((mw >> sh) & 0xffu), m1 = (int)((mw >> (sh + 8)) & 0xffu);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int2 pr = pairs_s[(t * NB + b) * 4 + q];
            mv[t] = mad24(m0, pr.x, mul24(m1, pr.y));
        }
    };
    /* chain slot j (token t) for block b with d, dmin of the block */
    auto chain = [&](int j, int t, int b, float d, float dmin, float wq, int mq) {
        const float xs = xs_s[t * NB + b];
        acc[j] = __builtin_fmaf(fmul_rn(d, xs), wq, acc[j]);
        accm[j] = __builtin_fmaf(-fmul_rn(dmin, xs), (float)mq, accm[j]);
    };

    auto round = [&](const Slot &c, int k) {
        const int b = phase + S * k;
        float wv[MT];
        int mv[MT];
        block_sums(c, b, wv, mv);
        if (S == 1) {
            const float d = f16_to_f32(c.h.x), dmin = f16_to_f32(c.h.x >> 16);
#pragma unroll
            for (int t = 0; t < MT; ++t) chain(t, t, b, d, dmin, wv[t], mv[t]);
            return;
        }
        const int par = k & 1;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            ring_w[tl][par][phase][G][t][lane] = wv[t];
            ring_m[tl][par][phase][G][t][lane] = mv[t];
        }
        ring_d[tl][par][phase][G][lane] = c.h.x;
        __syncthreads();
#pragma unroll
        for (int f = 0; f < S; ++f) {
            const int b2 = f + S * k;
            const uint32_t dpair = ring_d[tl][par][f][G][lane];
            const float d = f16_to_f32(dpair), dmin = f16_to_f32(dpair >> 16);
#pragma unroll
            for (int j = 0; j < NC; ++j)
                chain(j, own[j], b2, d, dmin, ring_w[tl][par][f][G][own[j]][lane], ring_m[tl][par][f][0][own[j]][lane]);
        }
    };

    constexpr int kFull = KB / P, kRem = KB % P;   /* rounds in ring-sized groups, then the rest */
#pragma unroll 1
    for (int it = 0; it < kFull; ++it) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int k = it * P + i;
            round(ring[i], k);
            /* refill the slot after its last use */
            ring[i] = load(k + P);
        }
    }
#pragma unroll
    for (int i = 0; i < kRem; ++i) round(ring[i], KB - kRem + i);

    /* the G = 1 owner of token t hands AVX2 lanes 4..7 to the G = 0 owner,
     * which applies the reference's trees: ((a0+a4)+(a2+a6)) +
     * ((a1+a5)+(a3+a7)), then ((m0+m2)+(m1+m3)) (qwen38_quant.c:303-310,
     * 1626-1630) */
    if (G == 1) {
#pragma unroll
        for (int j = 0; j < NC; ++j)
            if (S == 1 || phase + S * j < MT) xch[tl][S == 1 ? j : own[j]][lane] = acc[j];
    }
    __syncthreads();
    if (G == 0) {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int t = S == 1 ? j : own[j];
            if (S > 1 && phase + S * j >= MT) continue;
            float v = fadd_rn(acc[j], xch[tl][t][lane]);
            v = fadd_rn(v, __shfl_xor(v, 32, 64));
            v = fadd_rn(v, __shfl_xor(v, 16, 64));
            float m = accm[j];
            m = fadd_rn(m, __shfl_xor(m, 32, 64));
            m = fadd_rn(m, __shfl_xor(m, 16, 64));
            const uint32_t row = tile_raw * kTileRows + (uint32_t)r;
            if (q == 0 && tile_raw < ntiles && row < rows) y[(size_t)t * ldy + row] = fadd_rn(v, m);
        }
    }
}

/* Row-major Q4_K (rows x nb blocks) -> tiled copy; one thread per 16-byte
 * piece of the destination, pad rows of the last tile are zero. */
__global__ __launch_bounds__(256) void repack_q4k_tiles(uint4 *__restrict__ dst, const uint8_t *__restrict__ src,
                                                        uint32_t rows, uint32_t nb, size_t pieces)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    const size_t block_index = i / 9, k = i - block_index * 9;   /* 9 pieces per 144-byte block */
    const size_t per_tile = (size_t)nb * kTileRows;
    const size_t tile = block_index / per_tile, rem = block_index - tile * per_tile;
    const size_t b = rem / kTileRows, rr = rem - b * kTileRows;
    const size_t row = tile * kTileRows + rr;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < rows) {
        const uint8_t *p = src + (row * nb + b) * kQ4KBytes + k * 16;
        __builtin_memcpy(&v, p, 16);
    }
    dst[i] = v;
}

size_t tiled_q4k_bytes(uint32_t rows, uint32_t nb)
{
    return (size_t)((rows + kTileRows - 1) / kTileRows) * nb * kTileBlockBytes;
}

bool launch_repack_q4k_tiles(uint8_t *dst, const uint8_t *src, uint32_t rows, uint32_t nb, hipStream_t stream)
{
    if (!rows || !nb || (reinterpret_cast<uintptr_t>(dst) & 15)) return false;
    const size_t pieces = tiled_q4k_bytes(rows, nb) / 16;
    hipLaunchKernelGGL(repack_q4k_tiles, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<uint4 *>(dst), src, rows, nb, pieces);
    return hipGetLastError() == hipSuccess;
}

namespace {

/* Launch shape (measured on MI355X): with 5..8 tokens, two tiles of 2
 * wavefronts per workgroup; with 2..4 tokens, each tile's blocks split over
 * 2 wavefront pairs for tall matrices and 4 for short ones. */
int tiled_shape(uint32_t tiles, int mt)
{
    if (mt >= 5) return 12;
    return tiles >= 768 ? 2 : 4;
}

template <int MT, int NB>
void launch_tiled_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, hipStream_t stream)
{
    const uint32_t tiles = (rows + kTileRows - 1) / kTileRows;
    switch (tiled_shape(tiles, MT)) {
    case 12:
        hipLaunchKernelGGL((gemm_q4k_tiled<MT, NB, 1, 4, 2>), dim3((tiles + 1) / 2), dim3(256), 0, stream, w, x, y,
                           ldy, rows);
        break;
    case 2:
        hipLaunchKernelGGL((gemm_q4k_tiled<MT, NB, 2, 4, 1>), dim3(tiles), dim3(256), 0, stream, w, x, y, ldy, rows);
        break;
    default:
        hipLaunchKernelGGL((gemm_q4k_tiled<MT, NB, 4, 4, 1>), dim3(tiles), dim3(512), 0, stream, w, x, y, ldy, rows);
        break;
    }
}

template <int NB>
bool launch_tiled_nb(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                     hipStream_t stream)
{
    switch (m) {
    case 2: launch_tiled_typed<2, NB>(w, x, y, ldy, rows, stream); return true;
    case 3: launch_tiled_typed<3, NB>(w, x, y, ldy, rows, stream); return true;
    case 4: launch_tiled_typed<4, NB>(w, x, y, ldy, rows, stream); return true;
    case 5: launch_tiled_typed<5, NB>(w, x, y, ldy, rows, stream); return true;
    case 6: launch_tiled_typed<6, NB>(w, x, y, ldy, rows, stream); return true;
    case 7: launch_tiled_typed<7, NB>(w, x, y, ldy, rows, stream); return true;
    case 8: launch_tiled_typed<8, NB>(w, x, y, ldy, rows, stream); return true;
    default: return false;
    }
}

}  // namespace

/* Enqueue y[t * ldy + row] = W_row . x_t (t < m) from the tiled copy; the
 * row widths of the Qwen3.8 matrices (5120, 6144, 10240, 17408) and 2..8
 * tokens are supported, false otherwise. */
bool launch_gemm_q4k_tiled(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, hipStream_t stream)
{
    if (!rows || ldy < rows || m < 1) return false;
    /* one token: v_dot4 / v_dot2 lanes, one per AVX2 accumulator lane
     * (q38_q4k_gemv.hip) */
    if (m == 1) return launch_gemv_q4k_tiled(w_tiled, x, y, rows, nb, stream);
    /* prefill batches: the 64 x 64 matrix-core tiles of q38_wide.hip */
    if (m >= kWideMinTokens) return launch_gemm_q4k_wide((uint32_t)m, w_tiled, x, y, ldy, rows, nb, stream);
    /* 2..4 tokens on the widest 20-block matrices (FFN gate|up): 16 rows
     * per wavefront, weights streamed through LDS (q38_mm16.hip) */
    if (m <= 4 && nb == 20 && rows >= kMm16MinRows && launch_gemm_q4k_mm16(m, w_tiled, x, y, ldy, rows, nb, stream))
        return true;
    /* 4096 rows or more: 32 rows per wavefront (measured faster there; the
     * 16-row kernel keeps the small matrices) */
    if (rows >= 4096) return launch_gemm_q4k_t32(m, w_tiled, x, y, ldy, rows, nb, stream);
    switch (nb) {
    case 20: return launch_tiled_nb<20>(m, w_tiled, x, y, ldy, rows, stream);
    case 24: return launch_tiled_nb<24>(m, w_tiled, x, y, ldy, rows, stream);
    case 40: return launch_tiled_nb<40>(m, w_tiled, x, y, ldy, rows, stream);
    case 68: return launch_tiled_nb<68>(m, w_tiled, x, y, ldy, rows, stream);
    default: return false;
    }
}

}  // namespace q38
