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
#include <type_traits>

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

/* IQ1_M x Q8_K for ONE token on the vector ALU (v_dot4_i32_i8), over the
 * 16-row tiled copy.  The sign of each 8-element section is folded into the
 * codebook: the table that follows the 2048 grid entries in device memory
 * holds 4096 entries, index = qs byte | (qh nibble << 8) with the nibble's
 * sign bit as index bit 11, whose bytes are 8 g + delta (g in {-1, 0, 1},
 * delta = -1 when the bit is set, else +1: bytes in {-9, -7, -1, 1, 7, 9}).
 * For a 16-element half group with odd sub-scale s the block integer of the
 * reference (E = 8 weighted + correction, see the header) gains
 * s * sum_e (8 g(e) + delta) a(e): four v_dot4_i32_i8 of codebook bytes and
 * activation quants and one multiply-add.  E is exact in int32 and the fp32
 * chain is the reference's, total += d * (float(E) * 0.125f),
 * d = dscale * xs, in block order.
 *
 * Work unit: a quad of 4 weight rows.  Workgroup w of G owns quads
 * [w Q / G, (w + 1) Q / G) (Q = rows / 4), so 256 workgroups split both the
 * 17408- and the 5120-row shapes evenly.  A wavefront item is one quad x 4
 * consecutive blocks (4 pieces of 224 contiguous bytes, copied into the
 * wavefront's LDS ring by one global_load_lds_dwordx4 of 56 lanes): lane
 * (j, r, q) = (lane / 16, lane / 4 % 4, lane % 4) takes row r of the quad,
 * block 4 g + j of the item's block group g and elements 64 q .. 64 q + 63
 * of it (qs[8q..8q+7], qh[4q..4q+3], scale word q: its 4 half groups); the
 * 4 lanes of a row sum their E with two DPP quad permutations.  Items go to
 * the S wavefronts round-robin; when S is a multiple of the number of block
 * groups every item of a wavefront has the same blocks and its activation
 * quants stay in registers.  Each item's per-(row, block) products
 * t = d * (E * 0.125f) land in LDS; after the last item and one barrier one
 * thread per row adds its terms in block order.
 *
 * Every global read is an LDS copy with explicit vmcnt waits: per
 * wavefront, first its share of the staging (the 32 KiB table, the
 * activation quants, the scales), then the first P items; copies retire in
 * issue order, so after the staging wait and one barrier an item's wait
 * only counts the items issued after it. */
constexpr uint32_t kDot4Groups = 256;   /* persistent workgroups: one per CU */
constexpr int kDot4TFloats = 6144;      /* LDS terms [quad][block][row % 4], one token */
/* LDS terms for MT tokens: 34816 x 20-block matrices put 34 quads on a
 * workgroup, 34 x 20 x 4 x 3 = 8160 terms */
template <int MT>
constexpr int dot4_t_floats()
{
    return MT == 1 ? kDot4TFloats : 8192;
}
constexpr int kDot4ActStride = 272;     /* activation quants per block in LDS (256 + 16: no bank aliasing) */
constexpr int kDot4Slot = 896;          /* LDS ring slot: one item */

namespace {

__device__ __forceinline__ uint32_t dot4_lds_address(const void *p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

/* 16 bytes per lane from gaddr to LDS at m0 + 16 * lane, or 4 bytes to
 * m0 + 4 * lane.  Inline assembly keeps the compiler's wait-count pass
 * from draining these copies before unrelated LDS accesses; callers wait. */
__device__ __forceinline__ void dot4_copy16(const void *gaddr, uint32_t m0)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gaddr), "s"(m0) : "memory", "m0");
}

__device__ __forceinline__ void dot4_copy4(const void *gaddr, uint32_t m0)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(gaddr), "s"(m0) : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void dot4_wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/* wait until at most c (0..7, wave-uniform) vector memory operations are
 * outstanding */
__device__ __forceinline__ void dot4_wait_vm_upto(int c)
{
    switch (c) {
    case 0: dot4_wait_vm<0>(); break;
    case 1: dot4_wait_vm<1>(); break;
    case 2: dot4_wait_vm<2>(); break;
    case 3: dot4_wait_vm<3>(); break;
    case 4: dot4_wait_vm<4>(); break;
    case 5: dot4_wait_vm<5>(); break;
    case 6: dot4_wait_vm<6>(); break;
    default: dot4_wait_vm<7>(); break;
    }
}

}  // namespace

template <int NB, int S, int P, int MT>
__global__ __launch_bounds__(64 * S) void gemm_iq1m_dot4(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                         float *__restrict__ y, uint32_t ldy, uint32_t rows,
                                                         const uint2 *__restrict__ grid)
{
    static_assert(MT >= 1 && MT <= 3, "1..3 tokens");
    constexpr int NG = NB / 4;              /* block groups */
    constexpr bool ACT_REG = S % NG == 0;   /* fixed block group per wavefront */
    static_assert(NB % 4 == 0, "blocks per row must be a multiple of 4");
    static_assert(P >= 1 && P <= 4, "1..4 items in flight");
    __shared__ __attribute__((aligned(16))) uint2 cb_s[4096];
    __shared__ __attribute__((aligned(16))) uint8_t act_s[MT * NB * kDot4ActStride];   /* [token][block] */
    __shared__ float xs_s[MT * NB > 64 ? (MT * NB > 128 ? 256 : 128) : 64];            /* [token][block] */
    __shared__ float t_s[dot4_t_floats<MT>()];                                         /* [quad][block][row % 4][token] */
    __shared__ __attribute__((aligned(16))) uint8_t ring_s[S * P * kDot4Slot];

    const uint32_t nquads = (rows + 3) / 4;
    const uint32_t q0 = (uint32_t)(((uint64_t)blockIdx.x * nquads) / gridDim.x);
    const uint32_t q1 = (uint32_t)(((uint64_t)(blockIdx.x + 1) * nquads) / gridDim.x);
    if (q0 == q1) return;
    const int items = (int)(q1 - q0) * NG;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane >> 4, r = (lane >> 2) & 3, q = lane & 3;
    const int mine = wv < items ? (items - wv + S - 1) / S : 0;   /* the wavefront's items: wv + S n */

    /* staging copies, round-robin over the wavefronts: 32 x 1 KiB of the
     * table, one 256-byte block of activation quants per copy (16 lanes;
     * the tokens' Q8_K blocks are consecutive), the scales (4 bytes per
     * lane) */
    const uint8_t *table = reinterpret_cast<const uint8_t *>(grid + 2048);
    for (int k = wv; k < 32; k += S) dot4_copy16(table + 1024 * k + 16 * lane, dot4_lds_address(cb_s) + 1024 * k);
    for (int b = (wv + S - 32 % S) % S; b < MT * NB; b += S)
        if (lane < 16)
            dot4_copy16(x + (size_t)b * kQ8KBytes + 4 + 16 * lane, dot4_lds_address(act_s) + b * kDot4ActStride);
    if (wv == S - 1) {
#pragma unroll
        for (int k0 = 0; k0 < MT * NB; k0 += 64)
            if (lane < MT * NB - k0) dot4_copy4(x + (size_t)(lane + k0) * kQ8KBytes, dot4_lds_address(xs_s) + 4 * k0);
    }

    /* item n of the wavefront into ring slot n % P: lane l < 56 copies
     * bytes 16 (l % 14) .. + 15 of piece l / 14 (block 4 g + l / 14, the
     * quad's 4 rows) to slot byte 16 l */
    const uint32_t ring = dot4_lds_address(ring_s) + (uint32_t)(wv * P * kDot4Slot);
    const int cj = lane / 14, cp = lane - 14 * (lane / 14);
    auto issue = [&](int n, int slot) {
        const int i = wv + S * n;
        const uint32_t quad = q0 + (uint32_t)(i / NG);
        const uint32_t b = (uint32_t)(4 * (i % NG) + cj);
        const uint8_t *src = w + (size_t)(((quad >> 2) * NB + b) * 16u + ((quad & 3u) << 2)) * kIQ1MBytes + 16 * cp;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   /* the slot's previous reads are done */
        if (lane < 56) dot4_copy16(src, ring + (uint32_t)(slot * kDot4Slot));
    };
#pragma unroll
    for (int i = 0; i < P; ++i)
        if (i < mine) issue(i, i);
    dot4_wait_vm_upto(mine < P ? mine : P);   /* this wavefront's staging copies have landed */
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    int4v ar[MT][4];   /* activation quants of the fixed block group */
    if (ACT_REG) {
        const int b = 4 * (wv % NG) + j;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                ar[t][k] =
                    *reinterpret_cast<const int4v *>(act_s + (t * NB + b) * kDot4ActStride + 64 * q + 16 * k);
    }
    const uint8_t *rowp = ring_s + wv * P * kDot4Slot + 224 * j + 56 * r;

    auto item = [&](int n, int slot) {
        const int left = mine - 1 - n;   /* copies issued after this item's */
        dot4_wait_vm_upto(left < P - 1 ? left : P - 1);
        const uint8_t *bp = rowp + slot * kDot4Slot;
        const int2v qs = *reinterpret_cast<const int2v *>(bp + 8 * q);
        const uint32_t qh = *reinterpret_cast<const uint32_t *>(bp + 32 + 4 * q);
        const int2v sc = *reinterpret_cast<const int2v *>(bp + 48);
        const uint32_t qs0 = (uint32_t)qs[0], qs1 = (uint32_t)qs[1], sc0 = (uint32_t)sc[0], sc1 = (uint32_t)sc[1];
        const int i = wv + S * n;
        const int ql = i / NG;
        const int b = 4 * (i % NG) + j;
        int4v a[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                a[t][k] = ACT_REG ? ar[t][k]
                                  : *reinterpret_cast<const int4v *>(act_s + (t * NB + b) * kDot4ActStride + 64 * q +
                                                                     16 * k);
        /* 12-bit table indices of the lane's 8 sections, two per dword,
         * pre-shifted to byte offsets (x 8) */
        const uint32_t nlo = qh & 0x0f0f0f0fu, nhi = (qh >> 4) & 0x0f0f0f0fu;
        const uint32_t n03 = __builtin_amdgcn_perm(nhi, nlo, 0x05010400u);   /* nibbles 0, 1, 2, 3 */
        const uint32_t n47 = __builtin_amdgcn_perm(nhi, nlo, 0x07030602u);   /* nibbles 4, 5, 6, 7 */
        const uint32_t p[4] = {__builtin_amdgcn_perm(n03, qs0, 0x05010400u) << 3,
                               __builtin_amdgcn_perm(n03, qs0, 0x07030602u) << 3,
                               __builtin_amdgcn_perm(n47, qs1, 0x05010400u) << 3,
                               __builtin_amdgcn_perm(n47, qs1, 0x07030602u) << 3};
        const char *cb = reinterpret_cast<const char *>(cb_s);
        const uint32_t scw = ((q & 2) ? sc1 : sc0) >> (16 * (q & 1));   /* scale word q */
        int e[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) e[t] = 0;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            /* half group h: sections 2h, 2h + 1 = elements 64 q + 16 h .. + 15 */
            const uint2 e0 = *reinterpret_cast<const uint2 *>(cb + (p[h] & 0x7ff8u));
            const uint2 e1 = *reinterpret_cast<const uint2 *>(cb + (p[h] >> 16));
            const int sv = (int)(2u * ((scw >> (3 * h)) & 7u) + 1u);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int4v av4 = a[t][h];
                int acc = dot4z((int)e0.x, av4[0]);
                acc = dot4((int)e0.y, av4[1], acc);
                acc = dot4((int)e1.x, av4[2], acc);
                acc = dot4((int)e1.y, av4[3], acc);
                e[t] = mad24(sv, acc, e[t]);
            }
        }
        const uint32_t bits =
            ((sc0 >> 12) & 0x000fu) | ((sc0 >> 24) & 0x00f0u) | ((sc1 >> 4) & 0x0f00u) | ((sc1 >> 16) & 0xf000u);
        const float ds = f16_to_f32(bits);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            /* sum over the 4 lanes of the row (quad_perm [1,0,3,2], [2,3,0,1]) */
            int et = e[t];
            et += __builtin_amdgcn_update_dpp(0, et, 0xb1, 0xf, 0xf, false);
            et += __builtin_amdgcn_update_dpp(0, et, 0x4e, 0xf, 0xf, false);
            const float d = fmul_rn(ds, xs_s[t * NB + b]);
            const float term = fmul_rn(d, fmul_rn((float)et, 0.125f));
            if (q == 0) t_s[((ql * NB + b) * 4 + r) * MT + t] = term;
        }
    };

    const int full = mine / P, rem = mine % P;
#pragma unroll 1
    for (int it = 0; it < full; ++it) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int n = it * P + i;
            item(n, i);
            if (n + P < mine) issue(n + P, i);
        }
    }
#pragma unroll
    for (int i = 0; i < P; ++i)
        if (i < rem) item(full * P + i, i);
    __syncthreads();

    /* one thread per (row, token): the fp32 chain in block order */
    for (int c = tid; c < (int)(q1 - q0) * 4 * MT; c += 64 * S) {
        const int t = c % MT, ql = c / (4 * MT), rr = (c / MT) & 3;
        float total = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) total = fadd_rn(total, t_s[((ql * NB + b) * 4 + rr) * MT + t]);
        const uint32_t row = (q0 + (uint32_t)ql) * 4 + (uint32_t)rr;
        if (row < rows) y[(size_t)t * ldy + row] = total;
    }
}

namespace {

/* wavefronts per workgroup: a multiple of the block groups (NB / 4) where
 * that fits in 16, so the activation quants stay in registers */
template <int NB>
constexpr int dot4_waves()
{
    return NB == 20 ? 15 : NB == 24 ? 12 : NB == 40 ? 10 : 16;
}
constexpr int kDot4Prefetch = 2;

template <int NB, int MT>
bool launch_iq1m_dot4(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, const uint2 *grid,
                      hipStream_t stream)
{
    const uint32_t nquads = (rows + 3) / 4;
    const uint32_t groups = nquads < kDot4Groups ? nquads : kDot4Groups;
    const uint32_t per = (nquads + groups - 1) / groups;
    if ((size_t)per * NB * 4 * MT > (size_t)dot4_t_floats<MT>()) return false;
    hipLaunchKernelGGL((gemm_iq1m_dot4<NB, dot4_waves<NB>(), kDot4Prefetch, MT>), dim3(groups),
                       dim3(64 * dot4_waves<NB>()), 0, stream, w, x, y, ldy, rows, grid);
    return hipGetLastError() == hipSuccess;
}

template <int NB>
bool launch_iq1m_dot4_m(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                        const uint2 *grid, hipStream_t stream)
{
    switch (m) {
    case 1: return launch_iq1m_dot4<NB, 1>(w, x, y, ldy, rows, grid, stream);
    case 2: return launch_iq1m_dot4<NB, 2>(w, x, y, ldy, rows, grid, stream);
    case 3: return launch_iq1m_dot4<NB, 3>(w, x, y, ldy, rows, grid, stream);
    default: return false;
    }
}

}  // namespace

/* IQ1_M x Q8_K for prefill batches of 9..127 tokens: the products of
 * gemm_iq1m_mfma (per 16-row x 16-token tile and 64-element chunk on
 * v_mfma_i32_16x16x64_i8, the lane (r, q) taking sub-block 4q + c of the
 * chunk c), both into one int32 per (row, token) -- the grid operand carries
 * 8 s grid (at most 120 in magnitude), the sign operand s sign, so the sum is
 * E itself -- with the fp32 chain total += d * (float(E) * 0.125f),
 * d = dscale * xs, in block order per (row, token) in registers.  The chain
 * step of block b runs while block b + 1's products do (two accumulator
 * sets).  A workgroup of 8 wavefronts covers 256 rows x
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

    /* E of block b for the lane's 32 (row, token) pairs: both products
     * accumulate into one int32 per pair, the grid operand carrying 8 s g
     * (at most 8 * 15 = 120 in magnitude) and the sign operand s (-1)^sign,
     * so acc = 8 A.[s grid] + A.[s sign] = E exactly */
    auto products = [&](int b, const WLoad (&c)[2], int4v (&acc)[2][4]) {
        const int par = b & 1;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) acc[rt][tt] = (int4v){0, 0, 0, 0};
        uint32_t scw[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) scw[rt] = (q & 2 ? c[rt].sc[1] : c[rt].sc[0]) >> (16 * (q & 1));
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            int4v bw[2], bs[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const uint32_t ib = (c[rt].qs[cc >> 1] >> (16 * (cc & 1))) & 0xffffu;
                const uint32_t hb = (c[rt].qh >> (8 * cc)) & 0xffu;
                const uint32_t i0 = (ib & 0xffu) | ((hb & 7u) << 8);
                const uint32_t i1 = (ib >> 8) | ((hb & 0x70u) << 4);
                const uint2 g0 = grid_s[i0], g1 = grid_s[i1];
                const uint32_t t3 = (scw[rt] >> (3 * cc)) & 7u;
                /* grid selectors 0 / 1 / 2 pick -8 s / 0 / 8 s, s = 2 t3 + 1 */
                const uint32_t s8 = (t3 << 4) | 8u;
                const uint32_t lut = (256u - s8) | (s8 << 16);
                bw[rt][0] = (int)__builtin_amdgcn_perm(0u, lut, g0.x);
                bw[rt][1] = (int)__builtin_amdgcn_perm(0u, lut, g0.y);
                bw[rt][2] = (int)__builtin_amdgcn_perm(0u, lut, g1.x);
                bw[rt][3] = (int)__builtin_amdgcn_perm(0u, lut, g1.y);
                /* s and -s in every byte; the group's sign bit picks one */
                const uint32_t pos = __builtin_amdgcn_perm(0u, (t3 << 1) | 1u, 0u);
                const uint32_t neg = 0x01010100u - pos;
                const uint32_t m0 = (uint32_t)((int32_t)(c[rt].qh << (28 - 8 * cc)) >> 31);
                const uint32_t m1 = (uint32_t)((int32_t)(c[rt].qh << (24 - 8 * cc)) >> 31);
                const int c0 = (int)((m0 & neg) | (~m0 & pos)), c1 = (int)((m1 & neg) | (~m1 & pos));
                bs[rt] = (int4v){c0, c0, c1, c1};
            }
            int4v a[4];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) a[tt] = act(par, tt, cc);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    acc[rt][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[tt], bw[rt], acc[rt][tt], 0, 0, 0);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    acc[rt][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[tt], bs[rt], acc[rt][tt], 0, 0, 0);
        }
    };
    /* the block's dscale per row tile */
    auto dscale = [&](const WLoad (&c)[2], float (&dsc)[2]) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const uint32_t u0 = c[rt].sc[0] & 0xffffu, u1 = c[rt].sc[0] >> 16, u2 = c[rt].sc[1] & 0xffffu,
                           u3 = c[rt].sc[1] >> 16;
            const uint32_t bits = (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
            dsc[rt] = f16_to_f32(bits);
        }
    };
    /* the fp32 chain step of block b */
    auto chain = [&](int b, const int4v (&e)[2][4], const float (&dsc)[2]) {
        const float *xsb = xs_s + b * kIQWideTokens + 4 * q;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float xsv = xsb[16 * tt + j];
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const float d = fmul_rn(dsc[rt], xsv);
                    total[rt][tt][j] = fadd_rn(total[rt][tt][j], fmul_rn(d, fmul_rn((float)e[rt][tt][j], 0.125f)));
                }
            }
    };
    /* one block: its loads one block ahead, its products, and the chain step
     * of the block before (independent of the products, so the two
     * interleave); with_prev false only for block 0 */
    auto block = [&](int b, int4v (&cur)[2][4], float (&dcur)[2], const int4v (&prev)[2][4],
                     const float (&dprev)[2], bool with_prev, const WLoad (&wc)[2], WLoad (&wn)[2]) {
        const int bn = b + 1 < NB ? b + 1 : b;   /* the next block's loads (the last re-reads, unused) */
        wn[0] = load_w(0, bn);
        wn[1] = load_w(1, bn);
        if (b + 1 < NB) fetch_act(b + 1, stage_v);
        products(b, wc, cur);
        dscale(wc, dcur);
        if (with_prev) {
            chain(b - 1, prev, dprev);
#pragma unroll
            for (int i = 0; i < 64; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
        }
        /* the next block's activations into the other buffer */
        if (b + 1 < NB) store_act((b & 1) ^ 1, stage_v);
        __syncthreads();
    };
    static_assert(NB % 2 == 0, "blocks taken in pairs");
    int4v acc0[2][4], acc1[2][4];
    float dsc0[2], dsc1[2];
    WLoad w0[2] = {load_w(0, 0), load_w(1, 0)}, w1[2];
    block(0, acc0, dsc0, acc1, dsc1, false, w0, w1);
#pragma unroll 1
    for (int b = 1; b + 1 < NB; b += 2) {
        block(b, acc1, dsc1, acc0, dsc0, true, w1, w0);
        block(b + 1, acc0, dsc0, acc1, dsc1, true, w0, w1);
    }
    block(NB - 1, acc1, dsc1, acc0, dsc0, true, w1, w0);
    chain(NB - 1, acc1, dsc1);
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

/* IQ1_M x Q8_K for prompt batches of 128 tokens and more: the same E and
 * fp32 chain as gemm_iq1m_wide, with two changes that take work off the
 * vector ALU, which bounds that kernel.
 *
 * 1. The sign products.  A.[s sign] is constant over each 8-element group,
 *    so it equals sum_g s_g sign_g A8_g with A8_g the group's activation sum
 *    (in -1024..1016).  Split A8 = 8 h + l (h = A8 >> 3 in -128..127,
 *    l = A8 & 7): then 8 A.[s grid] + A.[s sign] =
 *      A.[8 s grid] + sum_g (h_g * 8 s_g sign_g + l_g * s_g sign_g),
 *    all int8 operands (8 s <= 120), so E takes the four grid products of
 *    the block with the B operand 8 s grid, plus ONE more K = 64 product whose
 *    A operand holds (h_g, l_g) byte pairs for the 32 groups (staged per token
 *    and block) and whose B operand holds (8 s_g sign_g, s_g sign_g): five
 *    products per tile and block where gemm_iq1m_wide takes eight, and no
 *    per-chunk sign operand.  Lane q's 16 bytes are groups 8q..8q+7, the
 *    groups of the sub-blocks 4q..4q+3 whose scale word and high nibbles the
 *    lane already holds; its sign word per sub-block comes from a 32-entry
 *    LDS table indexed by (sub-scale, both group signs).
 * 2. The chain step.  float(E) * 0.125f is exact, and d * (E / 8) equals
 *    (d / 8) * E bit for bit whenever d / 8 = fmul(dscale / 8, xs) is exact,
 *    i.e. unless 0 < |dscale * xs| < 2^-123; dscale >= 2^-24 (smallest
 *    fp16), so every Q8_K scale xs of the workgroup's tokens being 0 or
 *    >= 2^-99 in magnitude rules that out.  A workgroup checks its scales
 *    once and runs total += fmul(dscale / 8 * xs, float(E)) (three steps
 *    per pair and block instead of four, plus the scale product), else the
 *    literal chain.
 * A workgroup covers 256 rows x 128 tokens (wavefront w: rows 32w..32w+31,
 * two row tiles, against all eight token tiles), so each decoded weight
 * operand serves eight token tiles. */
constexpr int kIQW2Tokens = 128, kIQW2Waves = 8;

/* RT row tiles of 16 per wavefront: 128 RT rows per workgroup */
template <int NB, int RT>
__global__ __launch_bounds__(64 * kIQW2Waves, 1) void gemm_iq1m_wide128(const uint8_t *__restrict__ w,
                                                                         const uint8_t *__restrict__ x,
                                                                         float *__restrict__ y, uint32_t ldy,
                                                                         uint32_t rows, uint32_t tokens,
                                                                         const uint2 *__restrict__ grid)
{
    /* per token row: 256 quants + 16 bytes of padding / 64 (h, l) bytes +
     * 16 bytes of padding, so the 16 tokens of one A-operand read fall on
     * distinct banks */
    constexpr int kActStride = 272, kA8Stride = 80;
    __shared__ uint2 grid_s[2048];
    __shared__ uint32_t sign_s[32];               /* entry sign_a + 16 sign_b + 2 t (t: sub-scale) */
    __shared__ float xs_s[NB * kIQW2Tokens];      /* [block][token] */
    __shared__ __attribute__((aligned(16))) uint8_t act_s[2][kIQW2Tokens * kActStride];
    __shared__ __attribute__((aligned(16))) uint8_t a8_s[2][kIQW2Tokens * kA8Stride];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const uint32_t row0 = blockIdx.x * (128 * RT) + 16 * RT * wv, tok0 = blockIdx.y * kIQW2Tokens;
    const uint32_t wtok = tokens - tok0 < (uint32_t)kIQW2Tokens ? tokens - tok0 : kIQW2Tokens;

    for (int i = threadIdx.x; i < 2048; i += 64 * kIQW2Waves) {
        const uint2 v = grid[i];
        grid_s[i] = make_uint2(((v.x & 0x7f7f7f7fu) + 0x01010101u) ^ (v.x & 0x80808080u),
                               ((v.y & 0x7f7f7f7fu) + 0x01010101u) ^ (v.y & 0x80808080u));
    }
    if (threadIdx.x < 32) {
        /* bytes (8 s sign_a, s sign_a, 8 s sign_b, s sign_b), s = 2 t + 1; the
         * 32 entries sit in 32 distinct banks */
        const uint32_t i = threadIdx.x, s = 2u * ((i >> 1) & 7u) + 1u;
        const uint32_t pa = (i & 1u) ? ((256u - 8u * s) | ((256u - s) << 8)) : ((8u * s) | (s << 8));
        const uint32_t pb = (i & 16u) ? ((256u - 8u * s) | ((256u - s) << 8)) : ((8u * s) | (s << 8));
        sign_s[i] = pa | (pb << 16);
    }
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0, rows * NB * kIQ1MBytes, kRawBuf);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(x + (size_t)tok0 * NB * kQ8KBytes), 0, wtok * NB * kQ8KBytes, kRawBuf);
    int tiny = 0;
    for (int i = threadIdx.x; i < NB * kIQW2Tokens; i += 64 * kIQW2Waves) {
        const int t = i % kIQW2Tokens, b = i / kIQW2Tokens;
        const float v =
            __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)((t * NB + b) * kQ8KBytes), 0, 0));
        xs_s[i] = v;
        tiny |= v != 0.0f && fabsf(v) < 0x1p-99f;
    }
    const bool fold = !__syncthreads_or(tiny);

    uint32_t woff[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) woff[rt] = (row0 + 16 * rt + (uint32_t)r) * NB * kIQ1MBytes;
    /* staging of a block: thread i takes quants 64 (i % 4) .. + 63 of token
     * i / 4 (tokens past the batch read as zero), i.e. groups 8 (i % 4) ..
     * + 7, and writes their (h, l) pairs too */
    static_assert(64 * kIQW2Waves == 4 * kIQW2Tokens, "one staging thread per 64 quants");
    const uint32_t st_tok = threadIdx.x >> 2, st_part = threadIdx.x & 3;
    auto fetch_act = [&](int b, int4v (&v)[4]) {
        const uint32_t off = (st_tok * NB + (uint32_t)b) * kQ8KBytes + 4 + 64 * st_part;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16 * k, 0, 0);
    };
    auto store_act = [&](int par, const int4v (&v)[4]) {
        int4v *d = reinterpret_cast<int4v *>(&act_s[par][st_tok * kActStride + 64 * st_part]);
#pragma unroll
        for (int k = 0; k < 4; ++k) d[k] = v[k];
        int4v hl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t half[2];
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const int j = 2 * k + g;   /* group j of the part: dwords 2j, 2j + 1 */
                const int s8 = __builtin_amdgcn_sdot4(v[j >> 1][(2 * j) & 3 | 1], 0x01010101,
                                                      dot4z(v[j >> 1][(2 * j) & 3], 0x01010101), false);
                half[g] = ((uint32_t)s8 >> 3 & 0xffu) | (((uint32_t)s8 & 7u) << 8);
            }
            hl[k] = (int)(half[0] | (half[1] << 16));
        }
        *reinterpret_cast<int4v *>(&a8_s[par][st_tok * kA8Stride + 16 * st_part]) = hl;
    };
    int4v stage_v[4];
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

    float total[RT][8][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = 0; tt < 8; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j) total[rt][tt][j] = 0.0f;

    auto run = [&](auto fold_tag) {
        constexpr bool kFold = decltype(fold_tag)::value;
        WLoad wc[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) wc[rt] = load_w(rt, 0);
#pragma unroll 1
        for (int b = 0; b < NB; ++b) {
            const int bn = b + 1 < NB ? b + 1 : b;   /* the next block's loads (the last re-reads, unused) */
            const int par = b & 1;
            WLoad wn[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) wn[rt] = load_w(rt, bn);
            if (b + 1 < NB) fetch_act(b + 1, stage_v);
            int4v acc[RT][8];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int tt = 0; tt < 8; ++tt) acc[rt][tt] = (int4v){0, 0, 0, 0};
            uint32_t scw[RT];
            int4v xb[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                scw[rt] = (q & 2 ? wc[rt].sc[1] : wc[rt].sc[0]) >> (16 * (q & 1));
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    /* sign bits 3 and 7 of high byte cc to bits 2 and 6: the byte offset of
                     * entry sign_a + 16 sign_b + 2 t */
                    const uint32_t sb = (wc[rt].qh >> (8 * cc + 1)) & 0x44u;
                    xb[rt][cc] = (int)sign_s[(sb | (((scw[rt] >> (3 * cc)) & 7u) << 3)) >> 2];
                }
            }
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                int4v bw[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const WLoad &c = wc[rt];
                    const uint32_t ib = (c.qs[cc >> 1] >> (16 * (cc & 1))) & 0xffffu;
                    const uint32_t hb = (c.qh >> (8 * cc)) & 0xffu;
                    const uint32_t i0 = (ib & 0xffu) | ((hb & 7u) << 8);
                    const uint32_t i1 = (ib >> 8) | ((hb & 0x70u) << 4);
                    const uint2 g0 = grid_s[i0], g1 = grid_s[i1];
                    /* grid selectors 0 / 1 / 2 pick -8 s / 0 / 8 s, s = 2 t + 1 */
                    const uint32_t s8 = (((scw[rt] >> (3 * cc)) & 7u) << 4) | 8u;
                    const uint32_t lut = (256u - s8) | (s8 << 16);
                    bw[rt][0] = (int)__builtin_amdgcn_perm(0u, lut, g0.x);
                    bw[rt][1] = (int)__builtin_amdgcn_perm(0u, lut, g0.y);
                    bw[rt][2] = (int)__builtin_amdgcn_perm(0u, lut, g1.x);
                    bw[rt][3] = (int)__builtin_amdgcn_perm(0u, lut, g1.y);
                }
#pragma unroll
                for (int tt = 0; tt < 8; ++tt) {
                    const int4v a = *reinterpret_cast<const int4v *>(
                        &act_s[par][(16 * tt + r) * kActStride + 64 * q + 16 * cc]);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        acc[rt][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw[rt], acc[rt][tt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                const int4v a = *reinterpret_cast<const int4v *>(&a8_s[par][(16 * tt + r) * kA8Stride + 16 * q]);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    acc[rt][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, xb[rt], acc[rt][tt], 0, 0, 0);
            }
            /* the chain step of this block */
            float dsc[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint32_t u0 = wc[rt].sc[0] & 0xffffu, u1 = wc[rt].sc[0] >> 16, u2 = wc[rt].sc[1] & 0xffffu,
                               u3 = wc[rt].sc[1] >> 16;
                const uint32_t bits =
                    (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
                dsc[rt] = kFold ? f16_to_f32(bits) * 0.125f : f16_to_f32(bits);   /* exact */
            }
            const float *xsb = xs_s + b * kIQW2Tokens + 4 * q;
#pragma unroll
            for (int tt = 0; tt < 8; ++tt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float xsv = xsb[16 * tt + j];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const float d = fmul_rn(dsc[rt], xsv);
                        const float e = (float)acc[rt][tt][j];
                        total[rt][tt][j] =
                            fadd_rn(total[rt][tt][j], kFold ? fmul_rn(d, e) : fmul_rn(d, fmul_rn(e, 0.125f)));
                    }
                }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) wc[rt] = wn[rt];
            /* the next block's activations into the other buffer */
            if (b + 1 < NB) store_act(par ^ 1, stage_v);
            __syncthreads();
        }
    };
    if (fold)
        run(std::true_type{});
    else
        run(std::false_type{});
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t row = row0 + 16 * rt + (uint32_t)r;
#pragma unroll
        for (int tt = 0; tt < 8; ++tt)
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

template <int NB>
bool launch_iq1m_wide128_nb(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                            uint32_t tokens, const uint2 *grid, hipStream_t stream)
{
    /* 256-row workgroups also where 128-row ones would fill the chip better
     * (the 5120-row down projection at 4096 tokens: 640 workgroups take
     * 916 us, 1280 of 128 rows 1119 us, each of those reading its activation
     * operands for half as many rows) */
    hipLaunchKernelGGL((gemm_iq1m_wide128<NB, 2>), dim3((rows + 255) / 256, (tokens + kIQW2Tokens - 1) / kIQW2Tokens),
                       dim3(64 * kIQW2Waves), 0, stream, w, x, y, ldy, rows, tokens, grid);
    return hipGetLastError() == hipSuccess;
}

/* batches from this size on take the 128-token tiles */
constexpr uint32_t kIQW2MinTokens = 128;
}  // namespace

/* the buffer-resource kernels address a matrix with 32-bit byte offsets */
static bool iq1m_extent_ok(uint32_t rows, uint32_t nb)
{
    return (uint64_t)((rows + 15) / 16 * 16) * nb * kIQ1MBytes <= 0xffffffffull;
}

bool launch_gemm_iq1m_wide(uint32_t tokens, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, const void *grid, hipStream_t stream)
{
    if (!rows || !tokens || ldy < rows || !grid || tokens > 65535u * kIQWideTokens || !iq1m_extent_ok(rows, nb))
        return false;
    const uint2 *g = static_cast<const uint2 *>(grid);
    if (tokens >= kIQW2MinTokens) switch (nb) {
        case 20: return launch_iq1m_wide128_nb<20>(w, x, y, ldy, rows, tokens, g, stream);
        case 24: return launch_iq1m_wide128_nb<24>(w, x, y, ldy, rows, tokens, g, stream);
        case 40: return launch_iq1m_wide128_nb<40>(w, x, y, ldy, rows, tokens, g, stream);
        case 68: return launch_iq1m_wide128_nb<68>(w, x, y, ldy, rows, tokens, g, stream);
        default: return false;
        }
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
    if (!rows || ldy < rows || !grid || !iq1m_extent_ok(rows, nb)) return false;
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
    if (!rows || ldy < rows || !grid || !iq1m_extent_ok(rows, nb)) return false;
    const uint2 *g = static_cast<const uint2 *>(grid);
    if (m <= 3) {
        bool ok = false;
        switch (nb) {
        case 20: ok = launch_iq1m_dot4_m<20>(m, w_tiled, x, y, ldy, rows, g, stream); break;
        case 24: ok = launch_iq1m_dot4_m<24>(m, w_tiled, x, y, ldy, rows, g, stream); break;
        case 40: ok = launch_iq1m_dot4_m<40>(m, w_tiled, x, y, ldy, rows, g, stream); break;
        case 68: ok = launch_iq1m_dot4_m<68>(m, w_tiled, x, y, ldy, rows, g, stream); break;
        default: break;
        }
        if (ok) return true;
    }
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
