/* Q4_K x Q8_K for ONE token on the vector ALU (v_dot4_i32_i8 and
 * v_dot2_i32_i16), over the 16-row tiled copy built by repack_q4k_tiles
 * ([tile = row / 16][block][row % 16][144 bytes]).
 *
 * Arithmetic: that of the reference's AVX2 kernel
 * (src/qwen38/qwen38_quant.c:1546-1634).  Per row and super-block b there
 * are eight exact integers W[b][l] (AVX2 lane l owns quant dword l of each
 * 32-byte chunk c: low nibbles = elements 64c + 4l + u with sub-block scale
 * sc[2c], high nibbles = elements 64c + 32 + 4l + u with sc[2c + 1]) and four
 * min sums M[b][i] = m[2i] p0 + m[2i+1] p1 with p0 = (int16)(s[4i] + s[4i+1])
 * and p1 = (int16)(s[4i+2] + s[4i+3]) over the Q8_K 16-element sums s.  The
 * fp32 chains acc[l] = fmaf(d_b, W, acc[l]), accm[i] = fmaf(-dmin_b, M,
 * accm[i]) run over b in order (d_b = f16(d) * xs_b, dmin_b likewise), and
 * the row's value is the tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) +
 * ((m0+m2)+(m1+m3)) (:303-310, 1626-1630).
 *
 * Mapping.  Lane (g, l) = (lane / 8, lane % 8) of a wavefront is row g of
 * the wavefront's 8-row group and AVX2 lane l: per block it loads the four
 * quant dwords it owns and the block's 16-byte header, and forms W[b][l]
 * with two v_dot4_i32_i8 per chunk (nibbles against the staged activation
 * quants) and one v_dot2_i32_i16 of the (low, high) dot pair against the
 * chunk's (sc[2c], sc[2c+1]) pair; lanes l < 4 also form M[b][l] with one
 * v_dot2_i32_i16.  Every product is below 2^22, so every integer is exact
 * and converts to fp32 exactly.  The lane keeps acc[l] (and accm[l], l < 4)
 * in registers, so the fp32 work is the reference's sequence with no
 * reduction across lanes until the final tree, done with DPP row shifts
 * inside each 8-lane group.
 *
 * Work split.  A workgroup covers R row groups x H block ranges: wavefront
 * (rg, h) runs blocks h NB / H .. (h + 1) NB / H - 1 (integer division: the
 * ranges differ by at most one block) of row group rg, and requests all of
 * them at once, right after the staging loads.  Range 0 chains its blocks
 * in registers; ranges h > 0 leave (W, M) per lane and (d_b, -dmin_b) per
 * row and block in LDS, and after one barrier range 0 continues its chains
 * over them in block order.  The activations of all NB blocks are staged in
 * LDS once per workgroup, reordered so that lane l reads its eight quant
 * dwords of a block as two 16-byte words, followed by the four (p0, p1)
 * pairs and the scale.  Many short ranges keep many blocks in flight per
 * compute unit (measured on MI355X: 17408 x 5120 in 11.6 us with 4 ranges of
 * 5 blocks against 12.6 us with 2 of 10; 5120 x 17408 in 14.8 us with 12
 * ranges of 5 or 6 blocks against 17.2 us with 4 of 17). */
#include "q38_device.h"
#include "q38_kernels.h"

namespace q38 {

namespace {

typedef short short2v __attribute__((ext_vector_type(2)));

constexpr int kQ4KBlockBytes = 144;
constexpr uint32_t kGemvRawBuffer = 0x00020000u;   /* raw 32-bit buffer resource (gfx9) */
/* staged activations of one block, in 16-byte words: [0, 16) quants (lane l:
 * words 2l = its low-nibble quants of chunks 0..3, 2l + 1 = high), word 16 =
 * the (p0, p1) pairs of chunks 0..3, word 17 = the scale */
constexpr int kStageWords = 18;

__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, a), __builtin_bit_cast(short2v, b), c, false);
}

__device__ __forceinline__ int sdot2z(uint32_t a, uint32_t b) { return sdot2(a, b, 0); }

/* value of lane i + N of the same 16-lane row (row_shl:N); only read where
 * i + N stays inside the lane's 8-lane group */
template <int N>
__device__ __forceinline__ float row_shl(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + N, 0xf, 0xf,
                                                                  false));
}

struct Q4Blk {
    uint4 hdr;        /* d | dmin << 16, then the 12 scale bytes */
    uint32_t q[4];    /* quant dword l of chunks 0..3 */
};

}  // namespace

/* first block of range h of NB blocks split into H ranges */
template <int NB, int H>
__host__ __device__ constexpr int range_first(int h)
{
    return h * NB / H;
}

template <int NB, int H, int R>
__global__ __launch_bounds__(64 * H * R) void gemv_q4k_lanes(const uint8_t *__restrict__ w,
                                                             const uint8_t *__restrict__ x, float *__restrict__ y,
                                                             uint32_t rows)
{
    constexpr int KMAX = (NB + H - 1) / H;   /* longest range */
    constexpr int NT = 64 * H * R;
    constexpr int NS = H > 1 ? (H - 1) * R : 1;
    __shared__ uint4 act_s[NB * kStageWords];
    __shared__ float2 wm_s[NS * KMAX * 64];   /* (W, M) per range > 0, row group, block and lane */
    __shared__ float2 dd_s[NS * KMAX * 8];    /* (d, -dmin) per range > 0, row group, block and row */

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = wv % H, rg = wv / H;
    const int g = lane >> 3, l = lane & 7;
    const int b0 = (h * NB) / H, len = ((h + 1) * NB) / H - b0;
    const uint32_t row = (blockIdx.x * R + (uint32_t)rg) * 8 + (uint32_t)g;
    const uint32_t ntiles = (rows + 15) / 16;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0,
                                                                        ntiles * 16 * NB * kQ4KBlockBytes,
                                                                        kGemvRawBuffer);
    /* rows past the last read the tile's zero rows or, past the copy, zeros */
    const uint32_t row_off = ((row >> 4) * NB * 16 + (row & 15)) * kQ4KBlockBytes;

    /* staging loads first: quant dwords, the sum dwords of the pairs, scales */
    constexpr int kQuantPer = (NB * 64 + NT - 1) / NT;
    constexpr int kPairPer = (NB * 4 + NT - 1) / NT;
    uint32_t qv[kQuantPer], pv[kPairPer][2];
    float xv = 0.0f;
#pragma unroll
    for (int k = 0; k < kQuantPer; ++k) {
        const int i = tid + k * NT;
        qv[k] = i < NB * 64 ? *reinterpret_cast<const uint32_t *>(x + (size_t)(i >> 6) * kQ8KBytes + 4 + 4 * (i & 63))
                            : 0u;
    }
#pragma unroll
    for (int k = 0; k < kPairPer; ++k) {
        const int i = tid + k * NT;
        if (i < NB * 4) {
            const uint32_t *s = reinterpret_cast<const uint32_t *>(x + (size_t)(i >> 2) * kQ8KBytes + 260);
            pv[k][0] = s[2 * (i & 3)];
            pv[k][1] = s[2 * (i & 3) + 1];
        }
    }
    if (tid < NB) xv = *reinterpret_cast<const float *>(x + (size_t)tid * kQ8KBytes);

    /* every block of the wavefront's range in flight at once */
    Q4Blk blk[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        const int b = b0 + (k < len ? k : len - 1);   /* past a shorter range: re-read, unused */
        const uint32_t off = row_off + (uint32_t)b * 16 * kQ4KBlockBytes;
        blk[k].hdr = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
            blk[k].q[cc] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, off + 16 + 32 * cc + 4 * l, 0, 0);
    }

    /* staging writes: quant dword d of a block (elements 4d .. 4d + 3: chunk
     * d / 16, high half (d / 8) % 2, AVX2 lane d % 8) to word 2 (d % 8) +
     * (d / 8) % 2, dword d / 16; the pairs with the int16 wrap of the AVX2
     * adds */
    uint32_t *act_w = reinterpret_cast<uint32_t *>(act_s);
#pragma unroll
    for (int k = 0; k < kQuantPer; ++k) {
        const int i = tid + k * NT;
        if (i < NB * 64) {
            const int b = i >> 6, d = i & 63;
            act_w[b * 4 * kStageWords + 4 * (2 * (d & 7) + ((d >> 3) & 1)) + (d >> 4)] = qv[k];
        }
    }
#pragma unroll
    for (int k = 0; k < kPairPer; ++k) {
        const int i = tid + k * NT;
        if (i < NB * 4) {
            const uint32_t a = pv[k][0], c = pv[k][1];
            const uint32_t p0 = (uint16_t)((int16_t)a + (int16_t)(a >> 16));
            const uint32_t p1 = (uint16_t)((int16_t)c + (int16_t)(c >> 16));
            act_w[(i >> 2) * 4 * kStageWords + 64 + (i & 3)] = p0 | (p1 << 16);
        }
    }
    if (tid < NB) act_w[tid * 4 * kStageWords + 68] = __builtin_bit_cast(uint32_t, xv);
    __syncthreads();

    /* (sc[2c], sc[2c+1]) and (m[2i], m[2i+1]) as int16 pairs from the
     * packed-byte forms: selector bytes 2c, 2c + 1 of {hi : lo}, zero bytes
     * (0x0c) between */
    const uint32_t msel = (uint32_t)(2 * (l & 3)) | 0x0c00u | ((uint32_t)(2 * (l & 3) + 1) << 16) | 0x0c000000u;
    float acc = 0.0f, accm = 0.0f;
    const int slot = (h - 1) * R + rg;   /* ranges > 0 */
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        if (k >= len) break;
        const Q4Blk &c = blk[k];
        const int b = b0 + k;
        const uint32_t s0 = c.hdr.y, s1 = c.hdr.z, s2 = c.hdr.w;
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
        const uint4 alo = act_s[b * kStageWords + 2 * l], ahi = act_s[b * kStageWords + 2 * l + 1];
        const uint32_t al[4] = {alo.x, alo.y, alo.z, alo.w}, ah[4] = {ahi.x, ahi.y, ahi.z, ahi.w};
        int wsum = 0;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const int dl = dot4z((int)(c.q[cc] & 0x0f0f0f0fu), (int)al[cc]);
            const int dh = dot4z((int)((c.q[cc] >> 4) & 0x0f0f0f0fu), (int)ah[cc]);
            const uint32_t dp = __builtin_amdgcn_perm((uint32_t)dh, (uint32_t)dl, 0x05040100u);
            const uint32_t sp = __builtin_amdgcn_perm(sc_hi, sc_lo, (uint32_t)(2 * cc) | 0x0c00u |
                                                                         ((uint32_t)(2 * cc + 1) << 16) | 0x0c000000u);
            wsum = sdot2(dp, sp, wsum);
        }
        const uint32_t m_lo = s1 & 0x3f3f3f3fu;
        const uint32_t m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
        const uint32_t pairs = reinterpret_cast<const uint32_t *>(act_s)[(b * kStageWords + 16) * 4 + (l & 3)];
        const int msum = sdot2z(__builtin_amdgcn_perm(m_hi, m_lo, msel), pairs);
        const float xs = reinterpret_cast<const float *>(act_s)[(b * kStageWords + 17) * 4];
        const float d = fmul_rn(f16_to_f32(c.hdr.x & 0xffffu), xs);
        const float ndmin = -fmul_rn(f16_to_f32(c.hdr.x >> 16), xs);
        if (h == 0) {
            acc = __builtin_fmaf(d, (float)wsum, acc);
            accm = __builtin_fmaf(ndmin, (float)msum, accm);
        } else {
            wm_s[(slot * KMAX + k) * 64 + lane] = make_float2((float)wsum, (float)msum);
            if (l == 0) dd_s[(slot * KMAX + k) * 8 + g] = make_float2(d, ndmin);
        }
    }

    if (H > 1) __syncthreads();
    if (h != 0) return;
#pragma unroll
    for (int hh = 1; hh < H; ++hh) {
        const int s = (hh - 1) * R + rg;
#pragma unroll
        for (int k = 0; k < range_first<NB, H>(hh + 1) - range_first<NB, H>(hh); ++k) {
            const float2 v = wm_s[(s * KMAX + k) * 64 + lane];
            const float2 dv = dd_s[(s * KMAX + k) * 8 + g];
            acc = __builtin_fmaf(dv.x, v.x, acc);
            accm = __builtin_fmaf(dv.y, v.y, accm);
        }
    }

    /* the reference's tree inside each 8-lane group: lane l < 4 takes
     * a[l] + a[l + 4], then (s0 + s2) + (s1 + s3); mins (m0 + m2) + (m1 + m3) */
    const float s4 = acc + row_shl<4>(acc);
    const float s2 = s4 + row_shl<2>(s4);
    const float total = s2 + row_shl<1>(s2);
    const float m2 = accm + row_shl<2>(accm);
    const float mt = m2 + row_shl<1>(m2);
    if (l == 0 && row < rows) y[row] = total + mt;
}

namespace {

template <int NB, int H, int R>
bool launch_gemv_q4k_shape(const uint8_t *w, const uint8_t *x, float *y, uint32_t rows, hipStream_t stream)
{
    const uint32_t groups = (rows + 8 * R - 1) / (8 * R);
    hipLaunchKernelGGL((gemv_q4k_lanes<NB, H, R>), dim3(groups), dim3(64 * H * R), 0, stream, w, x, y, rows);
    return hipGetLastError() == hipSuccess;
}

}  // namespace

bool launch_gemv_q4k_tiled(const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t rows, uint32_t nb,
                           hipStream_t stream)
{
    if (!rows) return false;
    switch (nb) {
    /* ranges per row group, measured on MI355X (5120 or 17408 rows) */
    case 20: return launch_gemv_q4k_shape<20, 4, 1>(w_tiled, x, y, rows, stream);
    case 24: return launch_gemv_q4k_shape<24, 4, 1>(w_tiled, x, y, rows, stream);
    case 40: return launch_gemv_q4k_shape<40, 8, 1>(w_tiled, x, y, rows, stream);
    case 68: return launch_gemv_q4k_shape<68, 12, 1>(w_tiled, x, y, rows, stream);
    default: return false;
    }
}

}  // namespace q38
