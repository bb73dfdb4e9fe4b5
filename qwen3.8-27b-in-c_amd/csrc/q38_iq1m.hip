/* IQ1_M x Q8_K for 1..8 tokens on the gfx950 matrix cores
 * (v_mfma_i32_16x16x64_i8), row-major GGUF blocks.
 *
 * Arithmetic.  Per row, token and 56-byte block the reference
 * (src/qwen38/qwen38_quant.c:1388-1544) forms two exact integers,
 *   weighted   = sum_e s(e) * grid(e) * a(e)
 *   correction = sum_e s(e) * sign(e) * a(e)
 * (grid values in {-1, 0, 1} from the 2048-entry codebook, s the odd 3-bit
 * sub-scale of the element's half group, sign the section's delta sign), and
 * runs one fp32 chain total += d * (weighted + 0.125f * correction).  With
 * |8 weighted + correction| < 2^23 the bracket is exactly E / 8 for the
 * integer E = 8 weighted + correction, so the chain here is
 * total += d * (float(E) * 0.125f), bit for bit the reference's.
 *
 * E comes from two int8 matrix products per 64-element chunk with the
 * activations as the A operand (16 token rows) and, as B operand per weight
 * row, s * grid and s * sign (bytes in -15..15):
 *   E = 8 * A.[s grid] + A.[s sign],
 * exact in int32.
 *
 * Mapping (lane i of a wavefront, 16 weight rows per tile): r = i % 16 is the
 * weight row (B column) and the token (A row).  E is a sum over the whole
 * block, so the 16-element sub-block a lane feeds to the K slots it owns may
 * be chosen freely, as long as A and B agree: in chunk c lane q = i / 16 takes
 * sub-block k = 4q + c (elements 16k..16k+15: index bytes qs[2k], qs[2k+1],
 * high nibbles qh[k], sub-scale bits 3(k % 4) of scale word k / 4).  Over its
 * four chunks a lane thus reads the row's qs[8q..8q+7], qh[4q..4q+3] and
 * scale word q, 14 of the block's 56 bytes, and the four lanes of a row
 * together read the block once.  D register j of lane (r, q) is token 4q + j
 * of row r.  S wavefronts split the blocks of a tile (block b to
 * wavefront b mod S); every block's E and scale land in LDS, and after one
 * barrier one lane per (row, token) runs the fp32 chain in block order.
 * Workgroups stride over the tiles (the codebook is staged in LDS once per
 * workgroup) and load ahead across tile boundaries.  For one token the
 * activation quants (at most 17 KB) are staged in LDS too, once per
 * workgroup, since every tile reads the same ones.
 */
#include "q38_device.h"
#include "q38_kernels.h"

namespace q38 {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int2v __attribute__((ext_vector_type(2)));

constexpr int kIQ1MBytes = 56;
constexpr uint32_t kRawBuf = 0x00020000u;   /* raw 32-bit buffer resource (gfx9) */

template <int TS>
struct IQBlk {
    uint32_t qs[2], qh, sc[2];      /* the lane's index bytes and high nibbles, the scale words */
    int4v a[TS][4];                 /* activations per token set and chunk */
};

}  // namespace

template <int MT, int NB, int S, int P, bool TILED>
__global__ __launch_bounds__(64 * S) void gemm_iq1m_mfma(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                         float *__restrict__ y, uint32_t ldy, uint32_t rows,
                                                         const uint2 *__restrict__ grid)
{
    constexpr int TS = (MT + 15) / 16;   /* token sets of 16 (MT <= 8: one) */
    constexpr int KB = (NB + S - 1) / S;
    constexpr bool STAGE = MT == 1;       /* activation quants in LDS */
    __shared__ uint2 grid_s[2048];        /* codebook entries as bytes grid + 1 */
    __shared__ int4v act_s[STAGE ? MT * NB * 16 : 1];   /* [token][block][16 bytes] */
    __shared__ float e_s[2 * NB * MT * 16];   /* [tile parity][block][token][row] */
    __shared__ float d_s[2 * NB * 16];        /* [tile parity][block][row] super-scale */
    __shared__ float xs_s[MT * NB];

    const int lane = threadIdx.x & 63;
    const int sw = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const uint32_t ntiles = (rows + 15) / 16;

    /* once per workgroup: the codebook and the activation scales */
    for (int i = threadIdx.x; i < 2048; i += 64 * S) {
        /* bytes {-1, 0, 1} -> {0, 1, 2}: add 1 to the low 7 bits of every
         * byte (no carry out of a byte), then flip bit 7 back */
        const uint2 v = grid[i];
        grid_s[i] = make_uint2(((v.x & 0x7f7f7f7fu) + 0x01010101u) ^ (v.x & 0x80808080u),
                               ((v.y & 0x7f7f7f7fu) + 0x01010101u) ^ (v.y & 0x80808080u));
    }
    for (int i = threadIdx.x; i < MT * NB; i += 64 * S)
        xs_s[i] = *reinterpret_cast<const float *>(x + (size_t)i * kQ8KBytes);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0,
                                          (TILED ? ntiles * 16 : rows) * NB * kIQ1MBytes, kRawBuf);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(x), 0, MT * NB * kQ8KBytes, kRawBuf);
    if (STAGE)
        for (int i = threadIdx.x; i < MT * NB * 16; i += 64 * S)
            act_s[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)((i >> 4) * kQ8KBytes + 4 + 16 * (i & 15)),
                                                             0, 0);
    __syncthreads();   /* every wavefront reads the whole codebook */

    uint32_t xoff[TS];   /* token r + 16s (clamped), quants of sub-block 4q */
    int aidx[TS];        /* the same in act_s */
#pragma unroll
    for (int s = 0; s < TS; ++s) {
        const int t = r + 16 * s < MT ? r + 16 * s : MT - 1;
        xoff[s] = (uint32_t)(t * NB * kQ8KBytes + 4 + 64 * q);
        aidx[s] = t * NB * 16 + 4 * q;
    }

    /* The workgroup's work is a stream of items n = (j-th tile of the
     * workgroup, k-th round of its blocks): tile blockIdx.x + j * gridDim.x,
     * block sw + S * k.  Loads run P items ahead, across tile boundaries.
     * After the last round of a tile a barrier publishes its E and scales
     * (double-buffered by tile parity) and one lane per (row, token) runs the
     * tile's fp32 chains. */
    const uint32_t my_tiles = ntiles > blockIdx.x ? (ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    const int items = (int)my_tiles * KB;
    auto tile_of = [&](int n) {
        const uint32_t j = (uint32_t)(n / KB);
        const uint32_t t = blockIdx.x + j * gridDim.x;
        return t < ntiles ? t : ntiles - 1;   /* past the end: re-read the last tile, unused */
    };
    auto load = [&](int n) {
        const uint32_t tile = tile_of(n);
        const uint32_t row = tile * 16 + (uint32_t)r < rows ? tile * 16 + (uint32_t)r : rows - 1;
        int b = sw + S * (n % KB);
        b = b < NB ? b : NB - 1;   /* past the end: re-read the last block, unused */
        /* row-major: row `row`, block b; tiled: the 16 rows of block b of
         * the tile are one contiguous 896 bytes */
        const uint32_t woff = TILED ? (uint32_t)r * kIQ1MBytes : row * NB * kIQ1MBytes;
        const int soff = TILED ? (int)((tile * NB + (uint32_t)b) * 16u * kIQ1MBytes) : b * kIQ1MBytes;
        IQBlk<TS> c;
        const int2v qs = __builtin_bit_cast(int2v, __builtin_amdgcn_raw_buffer_load_b64(wr, woff + 8 * q, soff, 0));
        c.qs[0] = (uint32_t)qs[0];
        c.qs[1] = (uint32_t)qs[1];
        c.qh = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, woff + 32 + 4 * q, soff, 0);
        const int2v sc = __builtin_bit_cast(int2v, __builtin_amdgcn_raw_buffer_load_b64(wr, woff + 48, soff, 0));
        c.sc[0] = (uint32_t)sc[0];
        c.sc[1] = (uint32_t)sc[1];
#pragma unroll
        for (int s = 0; s < TS; ++s)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                c.a[s][cc] = STAGE ? act_s[aidx[s] + 16 * b + cc]
                                   : __builtin_amdgcn_raw_buffer_load_b128(xr, xoff[s] + 16 * cc, b * kQ8KBytes, 0);
        return c;
    };

    auto block = [&](const IQBlk<TS> &c, int n) {
        const int b = sw + S * (n % KB);
        const int par = (n / KB) & 1;
        int4v d1[TS], d2[TS];
#pragma unroll
        for (int t = 0; t < TS; ++t) d1[t] = d2[t] = (int4v){0, 0, 0, 0};
        const uint32_t scw = (q & 2 ? c.sc[1] : c.sc[0]) >> (16 * (q & 1));   /* scale word q */
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            /* sub-block 4q + cc of this row: two 8-element sections */
            const uint32_t ib = (c.qs[cc >> 1] >> (16 * (cc & 1))) & 0xffffu;   /* two index bytes */
            const uint32_t hb = (c.qh >> (8 * cc)) & 0xffu;                     /* two high nibbles */
            const uint32_t i0 = (ib & 0xffu) | ((hb & 7u) << 8);
            const uint32_t i1 = (ib >> 8) | ((hb & 0x70u) << 4);
            const uint32_t s = 2u * ((scw >> (3 * cc)) & 7u) + 1u;
            const uint2 g0 = grid_s[i0], g1 = grid_s[i1];
            /* s * g per byte: the bytes g + 1 in {0, 1, 2} select from the
             * byte table {-s, 0, s} */
            const uint32_t ns = 256u - s;
            const uint32_t lut = ns | (s << 16);
            int4v bw, bs;
            bw[0] = (int)__builtin_amdgcn_perm(0u, lut, g0.x);
            bw[1] = (int)__builtin_amdgcn_perm(0u, lut, g0.y);
            bw[2] = (int)__builtin_amdgcn_perm(0u, lut, g1.x);
            bw[3] = (int)__builtin_amdgcn_perm(0u, lut, g1.y);
            /* s * sign in every byte of each section */
            const uint32_t c0 = __builtin_amdgcn_perm(0u, (hb & 0x08u) ? ns : s, 0u);
            const uint32_t c1 = __builtin_amdgcn_perm(0u, (hb & 0x80u) ? ns : s, 0u);
            bs[0] = (int)c0; bs[1] = (int)c0; bs[2] = (int)c1; bs[3] = (int)c1;
#pragma unroll
            for (int t = 0; t < TS; ++t) {
                d1[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c.a[t][cc], bw, d1[t], 0, 0, 0);
                d2[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c.a[t][cc], bs, d2[t], 0, 0, 0);
            }
        }
        if (b < NB) {
#pragma unroll
            for (int t = 0; t < TS; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int tok = 16 * t + 4 * q + j;
                    if (tok < MT) e_s[((par * NB + b) * MT + tok) * 16 + r] = (float)(8 * d1[t][j] + d2[t][j]);
                }
            if (q == 0) {
                const uint32_t u0 = c.sc[0] & 0xffffu, u1 = c.sc[0] >> 16, u2 = c.sc[1] & 0xffffu,
                               u3 = c.sc[1] >> 16;
                const uint32_t bits = (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
                d_s[(par * NB + b) * 16 + r] = f16_to_f32(bits);
            }
        }
        if (n % KB == KB - 1) {
            /* the tile's last round: publish, then its fp32 chains in block
             * order, total += d * (E * 0.125) with d = dscale * xs */
            __syncthreads();
            const uint32_t row0 = tile_of(n) * 16;
            for (int idx = threadIdx.x; idx < 16 * MT; idx += 64 * S) {
                const int rr = idx & 15, t = idx >> 4;
                float total = 0.0f;
                for (int bb = 0; bb < NB; ++bb) {
                    const float d = fmul_rn(d_s[(par * NB + bb) * 16 + rr], xs_s[t * NB + bb]);
                    total = fadd_rn(total, fmul_rn(d, fmul_rn(e_s[((par * NB + bb) * MT + t) * 16 + rr], 0.125f)));
                }
                if (row0 + (uint32_t)rr < rows) y[(size_t)t * ldy + row0 + rr] = total;
            }
        }
    };

    IQBlk<TS> slot[P];
#pragma unroll
    for (int i = 0; i < P; ++i) slot[i] = load(i);
    const int full = items / P, rem = items % P;
#pragma unroll 1
    for (int it = 0; it < full; ++it) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int n = it * P + i;
            block(slot[i], n);
            slot[i] = load(n + P);
        }
    }
#pragma unroll
    for (int i = 0; i < P; ++i)
        if (i < rem) block(slot[i], full * P + i);
}

namespace {

/* Launch shape (measured on MI355X): 4 wavefronts per 16-row tile (8 for
 * one token, whose activations come from LDS), 512 workgroups striding over
 * the tiles, 2 blocks in flight per wavefront. */
constexpr int kIQ1MWaves = 4, kIQ1MWavesOneToken = 8;
constexpr uint32_t kIQ1MGroups = 512;
constexpr int kIQ1MPrefetch = 2;

template <int MT, int NB, int S, bool TILED>
void launch_iq1m_s(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, const uint2 *grid,
                   hipStream_t stream)
{
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t groups = tiles < kIQ1MGroups ? tiles : kIQ1MGroups;
    hipLaunchKernelGGL((gemm_iq1m_mfma<MT, NB, S, kIQ1MPrefetch, TILED>), dim3(groups), dim3(64 * S), 0, stream, w, x, y,
                       ldy, rows, grid);
}

template <int MT, int NB, bool TILED>
bool launch_iq1m_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, const uint2 *grid,
                       hipStream_t stream)
{
    launch_iq1m_s<MT, NB, MT == 1 ? kIQ1MWavesOneToken : kIQ1MWaves, TILED>(w, x, y, ldy, rows, grid, stream);
    return hipGetLastError() == hipSuccess;
}

template <int NB, bool TILED>
bool launch_iq1m_nb(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                    const uint2 *grid, hipStream_t stream)
{
    switch (m) {
    case 1: return launch_iq1m_typed<1, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 2: return launch_iq1m_typed<2, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 3: return launch_iq1m_typed<3, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 4: return launch_iq1m_typed<4, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 5: return launch_iq1m_typed<5, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 6: return launch_iq1m_typed<6, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 7: return launch_iq1m_typed<7, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    case 8: return launch_iq1m_typed<8, NB, TILED>(w, x, y, ldy, rows, grid, stream);
    default: return false;
    }
}

}  // namespace

/* IQ1_M x Q8_K for prefill batches (any token count): the products of
 * gemm_iq1m_mfma (per 16-row x 16-token tile and 64-element chunk,
 * E = 8 * A.[s grid] + A.[s sign] on v_mfma_i32_16x16x64_i8, the lane
 * (r, q) taking sub-block 4q + c of the chunk c) with the fp32 chain
 * total += d * (float(E) * 0.125f), d = dscale * xs, in block order per
 * (row, token) in registers.  A workgroup of 8 wavefronts covers 256 rows x
 * 64 tokens: wavefront w takes rows 32w .. 32w + 31 (two 16-row tiles)
 * against all 64 tokens (four token tiles), so each decoded weight operand
 * serves four token tiles and each activation operand two row tiles.  Lane
 * (r, q) of tile pair (rt, tt) owns tokens 16 tt + 4 q + j of row 16 rt + r.
 * The workgroup stages each block's activation quants of its 64 tokens in
 * LDS once (one block ahead), and every wavefront reads its A operands from
 * there, so the address unit handles only the weight loads and one 32-byte
 * staging copy per thread and block. */
constexpr int kIQWideRows = 256, kIQWideTokens = 64, kIQWideWaves = 8;

template <int NB>
__global__ __launch_bounds__(64 * kIQWideWaves, 1) void gemm_iq1m_wide(const uint8_t *__restrict__ w,
                                                                      const uint8_t *__restrict__ x,
                                                                      float *__restrict__ y, uint32_t ldy,
                                                                      uint32_t rows, uint32_t tokens,
                                                                      const uint2 *__restrict__ grid)
{
    __shared__ uint2 grid_s[2048];
    __shared__ float xs_s[NB * kIQWideTokens];   /* [block][token] */
    /* the activation quants of one block for the 64 tokens, double-buffered:
     * [parity][token][kActStride bytes] (256 quants + 16 bytes of padding, so
     * the 16 tokens one A-operand read touches fall on distinct banks) */
    constexpr int kActStride = 272;
    __shared__ __attribute__((aligned(16))) uint8_t act_s[2][kIQWideTokens * kActStride];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const uint32_t row0 = blockIdx.x * kIQWideRows + 32 * wv, tok0 = blockIdx.y * kIQWideTokens;
    const uint32_t wtok = tokens - tok0 < (uint32_t)kIQWideTokens ? tokens - tok0 : kIQWideTokens;

    for (int i = threadIdx.x; i < 2048; i += 64 * kIQWideWaves) {
        const uint2 v = grid[i];
        grid_s[i] = make_uint2(((v.x & 0x7f7f7f7fu) + 0x01010101u) ^ (v.x & 0x80808080u),
                               ((v.y & 0x7f7f7f7fu) + 0x01010101u) ^ (v.y & 0x80808080u));
    }
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0, rows * NB * kIQ1MBytes, kRawBuf);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(x + (size_t)tok0 * NB * kQ8KBytes), 0, wtok * NB * kQ8KBytes, kRawBuf);
    for (int i = threadIdx.x; i < NB * kIQWideTokens; i += 64 * kIQWideWaves) {
        const int t = i % kIQWideTokens, b = i / kIQWideTokens;
        xs_s[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)((t * NB + b) * kQ8KBytes), 0, 0));
    }
    __syncthreads();

    /* weight rows of the lane (rows past the matrix read as zero) */
    uint32_t woff[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) woff[rt] = (row0 + 16 * rt + (uint32_t)r) * NB * kIQ1MBytes;
    /* staging of a block's activations: thread i copies bytes 32 (i % 8) ..
     * + 31 of token i / 8's quants (tokens past the batch read as zero) */
    static_assert(64 * kIQWideWaves == 8 * kIQWideTokens, "one staging thread per 32 bytes");
    const uint32_t st_tok = threadIdx.x >> 3, st_part = threadIdx.x & 7;
    auto fetch_act = [&](int b, int4v (&v)[2]) {
        const uint32_t off = (st_tok * NB + (uint32_t)b) * kQ8KBytes + 4 + 32 * st_part;
        v[0] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
        v[1] = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0);
    };
    auto store_act = [&](int par, const int4v (&v)[2]) {
        int4v *d = reinterpret_cast<int4v *>(&act_s[par][st_tok * kActStride + 32 * st_part]);
        d[0] = v[0];
        d[1] = v[1];
    };
    /* the lane's A operand of token tile tt, chunk cc: 16 quants of token
     * 16 tt + r at 64 q + 16 cc */
    auto act = [&](int par, int tt, int cc) {
        return *reinterpret_cast<const int4v *>(&act_s[par][(16 * tt + r) * kActStride + 64 * q + 16 * cc]);
    };
    int4v stage_v[2];
    fetch_act(0, stage_v);
    store_act(0, stage_v);
    __syncthreads();

    struct WLoad {
        uint32_t qs[2], qh, sc[2];
    };
    auto load_w = [&](int rt, int b) {
        WLoad c;
        const int2v qs = __builtin_bit_cast(
            int2v, __builtin_amdgcn_raw_buffer_load_b64(wr, woff[rt] + 8 * q, b * kIQ1MBytes, 0));
        c.qs[0] = (uint32_t)qs[0];
        c.qs[1] = (uint32_t)qs[1];
        c.qh = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, woff[rt] + 32 + 4 * q, b * kIQ1MBytes, 0);
        const int2v sc = __builtin_bit_cast(
            int2v, __builtin_amdgcn_raw_buffer_load_b64(wr, woff[rt] + 48, b * kIQ1MBytes, 0));
        c.sc[0] = (uint32_t)sc[0];
        c.sc[1] = (uint32_t)sc[1];
        return c;
    };

    float total[2][4][4];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j) total[rt][tt][j] = 0.0f;

    WLoad wc[2] = {load_w(0, 0), load_w(1, 0)};

#pragma unroll 1
    for (int b = 0; b < NB; ++b) {
        const int bn = b + 1 < NB ? b + 1 : b;   /* the next block's loads (the last re-reads, unused) */
        const int par = b & 1;
        const WLoad wn[2] = {load_w(0, bn), load_w(1, bn)};
        if (b + 1 < NB) fetch_act(b + 1, stage_v);
        int4v d1[2][4], d2[2][4];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) d1[rt][tt] = d2[rt][tt] = (int4v){0, 0, 0, 0};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            int4v bw[2], bs[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const WLoad &c = wc[rt];
                const uint32_t scw = (q & 2 ? c.sc[1] : c.sc[0]) >> (16 * (q & 1));   /* scale word q */
                const uint32_t ib = (c.qs[cc >> 1] >> (16 * (cc & 1))) & 0xffffu;
                const uint32_t hb = (c.qh >> (8 * cc)) & 0xffu;
                const uint32_t i0 = (ib & 0xffu) | ((hb & 7u) << 8);
                const uint32_t i1 = (ib >> 8) | ((hb & 0x70u) << 4);
                const uint32_t sv = 2u * ((scw >> (3 * cc)) & 7u) + 1u;
                const uint2 g0 = grid_s[i0], g1 = grid_s[i1];
                const uint32_t ns = 256u - sv;
                const uint32_t lut = ns | (sv << 16);
                bw[rt][0] = (int)__builtin_amdgcn_perm(0u, lut, g0.x);
                bw[rt][1] = (int)__builtin_amdgcn_perm(0u, lut, g0.y);
                bw[rt][2] = (int)__builtin_amdgcn_perm(0u, lut, g1.x);
                bw[rt][3] = (int)__builtin_amdgcn_perm(0u, lut, g1.y);
                const uint32_t c0 = __builtin_amdgcn_perm(0u, (hb & 0x08u) ? ns : sv, 0u);
                const uint32_t c1 = __builtin_amdgcn_perm(0u, (hb & 0x80u) ? ns : sv, 0u);
                bs[rt][0] = (int)c0;
                bs[rt][1] = (int)c0;
                bs[rt][2] = (int)c1;
                bs[rt][3] = (int)c1;
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const int4v a = act(par, tt, cc);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    d1[rt][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw[rt], d1[rt][tt], 0, 0, 0);
                    d2[rt][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bs[rt], d2[rt][tt], 0, 0, 0);
                }
            }
        }
        /* the chains of this block */
        float dsc[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const uint32_t u0 = wc[rt].sc[0] & 0xffffu, u1 = wc[rt].sc[0] >> 16, u2 = wc[rt].sc[1] & 0xffffu,
                           u3 = wc[rt].sc[1] >> 16;
            const uint32_t bits = (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
            dsc[rt] = f16_to_f32(bits);
        }
        const float *xsb = xs_s + b * kIQWideTokens + 4 * q;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float xsv = xsb[16 * tt + j];
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const float d = fmul_rn(dsc[rt], xsv);
                    const float e = (float)(8 * d1[rt][tt][j] + d2[rt][tt][j]);
                    total[rt][tt][j] = fadd_rn(total[rt][tt][j], fmul_rn(d, fmul_rn(e, 0.125f)));
                }
            }
        wc[0] = wn[0];
        wc[1] = wn[1];
        /* the next block's activations into the other buffer */
        if (b + 1 < NB) store_act(par ^ 1, stage_v);
        __syncthreads();
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const uint32_t row = row0 + 16 * rt + (uint32_t)r;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t tok = tok0 + 16 * tt + 4 * q + j;
                if (row < rows && tok < tokens) y[(size_t)tok * ldy + row] = total[rt][tt][j];
            }
    }
}

namespace {
template <int NB>
bool launch_iq1m_wide_nb(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t tokens,
                         const uint2 *grid, hipStream_t stream)
{
    hipLaunchKernelGGL(gemm_iq1m_wide<NB>,
                       dim3((rows + kIQWideRows - 1) / kIQWideRows, (tokens + kIQWideTokens - 1) / kIQWideTokens),
                       dim3(64 * kIQWideWaves), 0, stream, w, x, y, ldy, rows, tokens, grid);
    return hipGetLastError() == hipSuccess;
}
}  // namespace

bool launch_gemm_iq1m_wide(uint32_t tokens, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, const void *grid, hipStream_t stream)
{
    if (!rows || !tokens || ldy < rows || !grid || tokens > 65535u * kIQWideTokens) return false;
    const uint2 *g = static_cast<const uint2 *>(grid);
    switch (nb) {
    case 20: return launch_iq1m_wide_nb<20>(w, x, y, ldy, rows, tokens, g, stream);
    case 24: return launch_iq1m_wide_nb<24>(w, x, y, ldy, rows, tokens, g, stream);
    case 40: return launch_iq1m_wide_nb<40>(w, x, y, ldy, rows, tokens, g, stream);
    case 68: return launch_iq1m_wide_nb<68>(w, x, y, ldy, rows, tokens, g, stream);
    default: return false;
    }
}

/* y[t * ldy + row] = W_row . x_t (t < m <= 8) for IQ1_M weights of the
 * Qwen3.8 row widths (5120, 6144, 10240, 17408); false otherwise. */
bool launch_gemm_iq1m_mfma(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, const void *grid, hipStream_t stream)
{
    if (!rows || ldy < rows || !grid) return false;
    const uint2 *g = static_cast<const uint2 *>(grid);
    switch (nb) {
    case 20: return launch_iq1m_nb<20, false>(m, w, x, y, ldy, rows, g, stream);
    case 24: return launch_iq1m_nb<24, false>(m, w, x, y, ldy, rows, g, stream);
    case 40: return launch_iq1m_nb<40, false>(m, w, x, y, ldy, rows, g, stream);
    case 68: return launch_iq1m_nb<68, false>(m, w, x, y, ldy, rows, g, stream);
    default: return false;
    }
}

bool launch_gemm_iq1m_tiled(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                            uint32_t nb, const void *grid, hipStream_t stream)
{
    if (!rows || ldy < rows || !grid) return false;
    const uint2 *g = static_cast<const uint2 *>(grid);
    switch (nb) {
    case 20: return launch_iq1m_nb<20, true>(m, w_tiled, x, y, ldy, rows, g, stream);
    case 24: return launch_iq1m_nb<24, true>(m, w_tiled, x, y, ldy, rows, g, stream);
    case 40: return launch_iq1m_nb<40, true>(m, w_tiled, x, y, ldy, rows, g, stream);
    case 68: return launch_iq1m_nb<68, true>(m, w_tiled, x, y, ldy, rows, g, stream);
    default: return false;
    }
}

namespace {

/* dst [tile][block][row % 16][56 bytes] from the row-major blocks, in 8-byte
 * pieces (7 per block); rows past the last are zero */
__global__ __launch_bounds__(256) void repack_iq1m_tiles_kernel(uint2 *__restrict__ dst, const uint8_t *__restrict__ src,
                                                                uint32_t rows, uint32_t nb, size_t pieces)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    const uint32_t k = (uint32_t)(i % 7);
    const size_t blk = i / 7;                       /* (tile, block, row % 16) */
    const uint32_t r = (uint32_t)(blk % 16);
    const size_t tb = blk / 16;                     /* tile * nb + block */
    const uint32_t b = (uint32_t)(tb % nb);
    const uint32_t row = (uint32_t)(tb / nb) * 16 + r;
    uint2 v = make_uint2(0, 0);
    if (row < rows) __builtin_memcpy(&v, src + ((size_t)row * nb + b) * kIQ1MBytes + 8 * k, 8);
    dst[i] = v;
}

}  // namespace

size_t tiled_iq1m_bytes(uint32_t rows, uint32_t nb)
{
    return (size_t)((rows + 15) / 16) * nb * 16 * kIQ1MBytes;
}

bool launch_repack_iq1m_tiles(uint8_t *dst, const uint8_t *src, uint32_t rows, uint32_t nb, hipStream_t stream)
{
    if (!rows || !nb || (reinterpret_cast<uintptr_t>(dst) & 7)) return false;
    const size_t pieces = tiled_iq1m_bytes(rows, nb) / 8;
    hipLaunchKernelGGL(repack_iq1m_tiles_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<uint2 *>(dst), src, rows, nb, pieces);
    return hipGetLastError() == hipSuccess;
}

}  // namespace q38
