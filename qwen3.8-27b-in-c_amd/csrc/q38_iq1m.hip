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
 * E comes from three int8 matrix products per 64-element chunk with the
 * activations as the A operand (16 token rows) and, as B operand per weight
 * row: s * (grid + 1) (bytes 0..30), s * sign (bytes +-15) and s (broadcast):
 *   E = 8 * (A.[s(g+1)] - A.[s]) + A.[s sign].
 * The products are exact int32.
 *
 * Mapping (lane i of a wavefront, 16 weight rows per tile): r = i % 16 is the
 * weight row (B column) and the token (A row), q = i / 16 picks bytes
 * 16q..16q+15 of each 64-element chunk c: group g = 2c + q/2, sections
 * 2(q&1) and 2(q&1)+1, one sub-scale.  D register j of lane (r, q) is token
 * 4q + j of row r.  S wavefronts split the blocks of a tile (block b to
 * wavefront b mod S); every block's E and scale land in LDS, and after one
 * barrier one lane per (row, token) runs the fp32 chain in block order.
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
    uint32_t qs[8], qh[4], sc[2];   /* the row's block: indices, high bits, scales */
    int4v a[TS][4];                 /* activations per token set and chunk */
};

}  // namespace

template <int MT, int NB, int S, int P>
__global__ __launch_bounds__(64 * S) void gemm_iq1m_mfma(const uint8_t *__restrict__ w, const uint8_t *__restrict__ x,
                                                         float *__restrict__ y, uint32_t ldy, uint32_t rows,
                                                         const uint2 *__restrict__ grid)
{
    constexpr int TS = (MT + 15) / 16;   /* token sets of 16 (MT <= 8: one) */
    constexpr int KB = (NB + S - 1) / S;
    __shared__ uint2 grid_s[2048];        /* codebook entries as bytes grid + 1 */
    __shared__ float e_s[NB * MT * 16];   /* [block][token][row] */
    __shared__ float d_s[NB * 16];        /* [block][row] super-scale */
    __shared__ float xs_s[MT * NB];

    const int lane = threadIdx.x & 63;
    const int sw = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const uint32_t row0 = blockIdx.x * 16;
    const uint32_t row = row0 + (uint32_t)r < rows ? row0 + (uint32_t)r : rows - 1;

    for (int i = threadIdx.x; i < 2048; i += 64 * S) {
        /* bytes {-1, 0, 1} -> {0, 1, 2}: add 1 to the low 7 bits of every
         * byte (no carry out of a byte), then flip bit 7 back */
        const uint2 v = grid[i];
        grid_s[i] = make_uint2(((v.x & 0x7f7f7f7fu) + 0x01010101u) ^ (v.x & 0x80808080u),
                               ((v.y & 0x7f7f7f7fu) + 0x01010101u) ^ (v.y & 0x80808080u));
    }
    for (int i = threadIdx.x; i < MT * NB; i += 64 * S)
        xs_s[i] = *reinterpret_cast<const float *>(x + (size_t)i * kQ8KBytes);
    __syncthreads();   /* every wavefront reads the whole codebook */

    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0, rows * NB * kIQ1MBytes, kRawBuf);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(x), 0, MT * NB * kQ8KBytes, kRawBuf);
    const uint32_t woff = row * NB * kIQ1MBytes;
    uint32_t xoff[TS];   /* token r + 16s (clamped), bytes 16q.. of chunk 0 */
#pragma unroll
    for (int s = 0; s < TS; ++s) {
        const int t = r + 16 * s < MT ? r + 16 * s : MT - 1;
        xoff[s] = (uint32_t)(t * NB * kQ8KBytes + 4 + 16 * q);
    }
    auto load = [&](int k) {
        int b = sw + S * k;
        b = b < NB ? b : NB - 1;   /* past the end: re-read the last block, unused */
        IQBlk<TS> c;
#pragma unroll
        for (int h = 0; h < 7; ++h) {
            const int2v v = __builtin_bit_cast(int2v, __builtin_amdgcn_raw_buffer_load_b64(wr, woff + 8 * h,
                                                                                           b * kIQ1MBytes, 0));
            const uint32_t lo = (uint32_t)v[0], hi = (uint32_t)v[1];
            if (h < 4) { c.qs[2 * h] = lo; c.qs[2 * h + 1] = hi; }
            else if (h < 6) { c.qh[2 * (h - 4)] = lo; c.qh[2 * (h - 4) + 1] = hi; }
            else { c.sc[0] = lo; c.sc[1] = hi; }
        }
#pragma unroll
        for (int s = 0; s < TS; ++s)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                c.a[s][cc] = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff[s] + 64 * cc, b * kQ8KBytes, 0);
        return c;
    };
    IQBlk<TS> slot[P];
#pragma unroll
    for (int i = 0; i < P; ++i) slot[i] = load(i);

    const int qhi = q >> 1, qlo = q & 1;
    const uint32_t soff = (uint32_t)(6 * qhi + 3 * qlo);   /* sub-scale bits inside the group's u16 */

    auto block = [&](const IQBlk<TS> &c, int k) {
        const int b = sw + S * k;
        int4v d1[TS], d2[TS], d3[TS];
#pragma unroll
        for (int s = 0; s < TS; ++s) d1[s] = d2[s] = d3[s] = (int4v){0, 0, 0, 0};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            /* group 2cc + q/2, sections 2(q&1) and 2(q&1)+1 of this row */
            const uint32_t qsd = qhi ? c.qs[2 * cc + 1] : c.qs[2 * cc];
            const uint32_t ib = (qsd >> (16 * qlo)) & 0xffffu;        /* two index bytes */
            const uint32_t hb = (c.qh[cc] >> (8 * q)) & 0xffu;         /* two high nibbles */
            const uint32_t i0 = (ib & 0xffu) | ((hb & 7u) << 8);
            const uint32_t i1 = (ib >> 8) | ((hb & 0x70u) << 4);
            const uint32_t s = 2u * ((c.sc[cc >> 1] >> (16 * (cc & 1) + soff)) & 7u) + 1u;
            const uint2 g0 = grid_s[i0], g1 = grid_s[i1];
            /* s * (g + 1) per byte: the bytes g + 1 in {0, 1, 2} select from
             * the byte table {0, s, 2s} */
            const uint32_t lut = s * 0x00020100u;
            int4v bw, bs, bb;
            bw[0] = (int)__builtin_amdgcn_perm(0u, lut, g0.x);
            bw[1] = (int)__builtin_amdgcn_perm(0u, lut, g0.y);
            bw[2] = (int)__builtin_amdgcn_perm(0u, lut, g1.x);
            bw[3] = (int)__builtin_amdgcn_perm(0u, lut, g1.y);
            /* s and -s in every byte */
            const uint32_t sp = __builtin_amdgcn_perm(0u, s, 0u), sn = __builtin_amdgcn_perm(0u, 256u - s, 0u);
            const uint32_t c0 = (hb & 0x08u) ? sn : sp, c1 = (hb & 0x80u) ? sn : sp;
            bs[0] = (int)c0; bs[1] = (int)c0; bs[2] = (int)c1; bs[3] = (int)c1;
            bb[0] = bb[1] = bb[2] = bb[3] = (int)sp;
#pragma unroll
            for (int t = 0; t < TS; ++t) {
                d1[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c.a[t][cc], bw, d1[t], 0, 0, 0);
                d2[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c.a[t][cc], bs, d2[t], 0, 0, 0);
                d3[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c.a[t][cc], bb, d3[t], 0, 0, 0);
            }
        }
        if (b >= NB) return;
#pragma unroll
        for (int t = 0; t < TS; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int tok = 16 * t + 4 * q + j;
                if (tok < MT) e_s[(b * MT + tok) * 16 + r] = (float)(8 * (d1[t][j] - d3[t][j]) + d2[t][j]);
            }
        if (q == 0) {
            const uint32_t u0 = c.sc[0] & 0xffffu, u1 = c.sc[0] >> 16, u2 = c.sc[1] & 0xffffu, u3 = c.sc[1] >> 16;
            const uint32_t bits = (u0 >> 12) | ((u1 >> 8) & 0x00f0u) | ((u2 >> 4) & 0x0f00u) | (u3 & 0xf000u);
            d_s[b * 16 + r] = f16_to_f32(bits);
        }
    };

    constexpr int kFull = KB / P, kRem = KB % P;
#pragma unroll 1
    for (int it = 0; it < kFull; ++it) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int k = it * P + i;
            block(slot[i], k);
            slot[i] = load(k + P);
        }
    }
#pragma unroll
    for (int i = 0; i < kRem; ++i) block(slot[i], KB - kRem + i);
    __syncthreads();

    /* fp32 chains in block order: total += d * (E * 0.125), d = dscale * xs */
    for (int idx = threadIdx.x; idx < 16 * MT; idx += 64 * S) {
        const int rr = idx & 15, t = idx >> 4;
        float total = 0.0f;
        for (int b = 0; b < NB; ++b) {
            const float d = fmul_rn(d_s[b * 16 + rr], xs_s[t * NB + b]);
            total = fadd_rn(total, fmul_rn(d, fmul_rn(e_s[(b * MT + t) * 16 + rr], 0.125f)));
        }
        if (row0 + (uint32_t)rr < rows) y[(size_t)t * ldy + row0 + rr] = total;
    }
}

namespace {

/* wavefronts per 16-row tile (measured on MI355X): 8 for rows of 20..40
 * blocks, 4 for the 68-block rows of the FFN down projection */
int iq1m_waves(int nb) { return nb >= 68 ? 4 : 8; }

template <int MT, int NB, int S>
void launch_iq1m_s(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, const uint2 *grid,
                   hipStream_t stream)
{
    hipLaunchKernelGGL((gemm_iq1m_mfma<MT, NB, S, 2>), dim3((rows + 15) / 16), dim3(64 * S), 0, stream, w, x, y, ldy,
                       rows, grid);
}

template <int MT, int NB>
bool launch_iq1m_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, const uint2 *grid,
                       hipStream_t stream)
{
    if (iq1m_waves(NB) == 4) launch_iq1m_s<MT, NB, 4>(w, x, y, ldy, rows, grid, stream);
    else launch_iq1m_s<MT, NB, 8>(w, x, y, ldy, rows, grid, stream);
    return hipGetLastError() == hipSuccess;
}

template <int NB>
bool launch_iq1m_nb(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                    const uint2 *grid, hipStream_t stream)
{
    switch (m) {
    case 1: return launch_iq1m_typed<1, NB>(w, x, y, ldy, rows, grid, stream);
    case 2: return launch_iq1m_typed<2, NB>(w, x, y, ldy, rows, grid, stream);
    case 3: return launch_iq1m_typed<3, NB>(w, x, y, ldy, rows, grid, stream);
    case 4: return launch_iq1m_typed<4, NB>(w, x, y, ldy, rows, grid, stream);
    case 5: return launch_iq1m_typed<5, NB>(w, x, y, ldy, rows, grid, stream);
    case 6: return launch_iq1m_typed<6, NB>(w, x, y, ldy, rows, grid, stream);
    case 7: return launch_iq1m_typed<7, NB>(w, x, y, ldy, rows, grid, stream);
    case 8: return launch_iq1m_typed<8, NB>(w, x, y, ldy, rows, grid, stream);
    default: return false;
    }
}

}  // namespace

/* y[t * ldy + row] = W_row . x_t (t < m <= 8) for IQ1_M weights of the
 * Qwen3.8 row widths (5120, 6144, 10240, 17408); false otherwise. */
bool launch_gemm_iq1m_mfma(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                           uint32_t nb, const void *grid, hipStream_t stream)
{
    if (!rows || ldy < rows || !grid) return false;
    const uint2 *g = static_cast<const uint2 *>(grid);
    switch (nb) {
    case 20: return launch_iq1m_nb<20>(m, w, x, y, ldy, rows, g, stream);
    case 24: return launch_iq1m_nb<24>(m, w, x, y, ldy, rows, g, stream);
    case 40: return launch_iq1m_nb<40>(m, w, x, y, ldy, rows, g, stream);
    case 68: return launch_iq1m_nb<68>(m, w, x, y, ldy, rows, g, stream);
    default: return false;
    }
}

}  // namespace q38
