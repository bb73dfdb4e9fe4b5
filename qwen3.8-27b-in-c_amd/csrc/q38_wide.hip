/* Q4_K x Q8_K for prompt-length token counts (the prefill batch) on the
 * gfx950 matrix cores, over the 16-row tiled copy built by repack_q4k_tiles
 * ([tile = row / 16][block][row % 16][144 bytes]).
 *
 * Arithmetic: as the reference's AVX2 kernel (src/qwen38/qwen38_quant.c:
 * 1546-1634) for every (row, token): eight exact integers W[b][l] per
 * super-block b (l = AVX2 accumulator lane: quant dword l of each 32-byte
 * chunk c, low nibbles = elements 64c + 4l + u with scale sc[2c], high
 * nibbles = elements 64c + 32 + 4l + u with scale sc[2c + 1]), four min sums
 * M[b][i] = m[2i] (s[4i] + s[4i+1]) + m[2i+1] (s[4i+2] + s[4i+3]), the fp32
 * chains acc[l] = fmaf(d_b, W, acc[l]), accm[i] = fmaf(-dmin_b, M, accm[i])
 * over b in order (d_b = f16(d) * scale_b, dmin_b likewise), and the final
 * tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) + ((m0+m2)+(m1+m3))
 * (:303-310, 1626-1630).  The results are those of the one-token GEMV bit
 * for bit, whatever the token count.
 *
 * Matrix cores.  The K dimension of one AVX2 lane's product is exactly its
 * 32 elements of the block (4 low and 4 high of each chunk), so
 * W[b][l] = sum over K of (sc * q) * a with fp16 operands (sc * q <= 945
 * and int8 activations are exact in fp16, every partial sum is an integer
 * below 2^24): two v_mfma_f32_32x32x16_f16 per lane l, A = 32 tokens,
 * B = 32 weight rows, with no redundant products.  The min sums are
 * v_mfma_f32_32x32x2_f32 with K = the two sub-blocks of a chunk (products
 * below 2^19, exact).
 *
 * Layout.  A workgroup of 8 wavefronts covers 64 rows x 64 tokens.
 * Wavefront w: lane half lh = w & 1 (AVX2 lanes 4 lh .. 4 lh + 3, min lanes
 * 2 lh, 2 lh + 1), token tile tt = (w >> 1) & 1, row tile rt = w >> 2.
 * Lane i: r = i % 32, q = i / 32.  The MFMA inputs of lane (r, q) are the
 * chunks q and q + 2 (K-slots 8q .. 8q + 7 of the two products) of weight
 * row 32 rt + r and of token 32 tt + r; its outputs are row 32 rt + r and
 * the tokens 8 (j / 4) + 4 q + j % 4 of the tile (register j), whose chains
 * it owns.  The two lane halves of a (row, token) meet in LDS for the final
 * tree.  Activation scales and sub-block pair sums of the workgroup's 64
 * tokens are staged in LDS once.
 */
#include "q38_device.h"
#include "q38_kernels.h"
#include "q38_q4k_mfma.h"

namespace q38 {

namespace {

typedef float float16v_w __attribute__((ext_vector_type(16)));

constexpr int kWideRows = 64, kWideTokens = 64, kWideWaves = 8;

/* loads of one block for one lane */
struct WideBlk {
    uint4 h;          /* header of the lane's row: d|dmin, 12 scale/min bytes */
    uint4 wq[2];      /* quant dwords 4 lh .. 4 lh + 3 of chunks q and q + 2 */
    uint4 lo[2], hi[2];   /* activation dwords 4 lh .. of chunks q, q + 2: low and high halves */
};

/* LDS: the staged scales (fp32) and pair sums (8 x int16) of the tile's
 * tokens, later reused for the final exchange (four wavefronts x eight
 * tokens x six values x 64 lanes) */
template <int NB>
constexpr int wide_stage_bytes()
{
    return NB * kWideTokens * (4 + 16);
}
constexpr int kWideExchangeBytes = 4 * 8 * 6 * 64 * 4;
template <int NB>
constexpr int wide_lds_bytes()
{
    return wide_stage_bytes<NB>() > kWideExchangeBytes ? wide_stage_bytes<NB>() : kWideExchangeBytes;
}

template <int NB>
__global__ __launch_bounds__(64 * kWideWaves, 1) void gemm_q4k_wide(const uint8_t *__restrict__ w,
                                                                   const uint8_t *__restrict__ x,
                                                                   float *__restrict__ y, uint32_t ldy,
                                                                   uint32_t rows, uint32_t tokens)
{
    /* xs_s[b][t]: activation scale; ps_s[b][t][j]: pair sums s[2j] + s[2j+1] */
    __shared__ __attribute__((aligned(16))) uint8_t lds[wide_lds_bytes<NB>()];
    float *xs_s = reinterpret_cast<float *>(lds);
    int16_t *ps_s = reinterpret_cast<int16_t *>(lds + NB * kWideTokens * 4);

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lh = wv & 1, tt = (wv >> 1) & 1, rt = wv >> 2;
    const int r = lane & 31, q = lane >> 5;
    const uint32_t ntiles = (rows + kRows16 - 1) / kRows16;
    const uint32_t row0 = blockIdx.x * kWideRows, tok0 = blockIdx.y * kWideTokens;

    /* weights: the workgroup's (up to) four 16-row tiles; tiles past the
     * matrix read as zero through the buffer bound */
    const uint32_t tile0 = row0 / kRows16;
    const uint32_t wtiles = ntiles - tile0 < 4 ? ntiles - tile0 : 4;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w + (size_t)tile0 * NB * kTileBlock), 0, wtiles * NB * kTileBlock, kRawBuffer);
    const uint32_t lrow = 32 * rt + r;   /* row inside the workgroup */
    const uint32_t hoff = (lrow >> 4) * NB * kTileBlock + (lrow & 15) * kBlockBytes;
    const uint32_t woff0 = hoff + 16 + 32 * q + 16 * lh, woff1 = woff0 + 64;

    /* activations of the workgroup's tokens (tokens past the end read as 0) */
    const uint32_t wtok = tokens - tok0 < (uint32_t)kWideTokens ? tokens - tok0 : kWideTokens;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(x + (size_t)tok0 * NB * kQ8KBytes), 0, wtok * NB * kQ8KBytes, kRawBuffer);
    const uint32_t atok = 32 * tt + r;   /* token of this lane's A operand */
    const uint32_t xoff0 = atok * NB * kQ8KBytes + 4 + 64 * q + 16 * lh, xoff1 = xoff0 + 128;

    /* stage scales and pair sums of the tile's tokens */
    for (int i = threadIdx.x; i < NB * kWideTokens; i += 64 * kWideWaves) {
        const int t = i % kWideTokens, b = i / kWideTokens;
        const uint32_t base = (uint32_t)(t * NB + b) * kQ8KBytes;
        const uint32_t sc = __builtin_amdgcn_raw_buffer_load_b32(xr, base, 0, 0);
        const int4v s0 = __builtin_amdgcn_raw_buffer_load_b128(xr, base + 260, 0, 0);
        const int4v s1 = __builtin_amdgcn_raw_buffer_load_b128(xr, base + 276, 0, 0);
        xs_s[i] = __uint_as_float(sc);
        int16_t *ps = ps_s + (size_t)i * 8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ps[k] = (int16_t)((int)(int16_t)(s0[k] & 0xffff) + (s0[k] >> 16));
            ps[4 + k] = (int16_t)((int)(int16_t)(s1[k] & 0xffff) + (s1[k] >> 16));
        }
    }
    __syncthreads();

    auto load = [&](int b) {
        const int bb = b < NB ? b : NB - 1;   /* past the end: re-read the last block, unused */
        const int wo = bb * kTileBlock, xo = bb * kQ8KBytes;
        WideBlk c;
        int4v v = __builtin_amdgcn_raw_buffer_load_b128(wr, hoff, wo, 0);
        c.h = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, woff0, wo, 0);
        c.wq[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(wr, woff1, wo, 0);
        c.wq[1] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff0, xo, 0);
        c.lo[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff0 + 32, xo, 0);
        c.hi[0] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff1, xo, 0);
        c.lo[1] = make_uint4(v[0], v[1], v[2], v[3]);
        v = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff1 + 32, xo, 0);
        c.hi[1] = make_uint4(v[0], v[1], v[2], v[3]);
        return c;
    };

    float acc[16][4], accm[16][2];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[j][k] = 0.0f;
        accm[j][0] = accm[j][1] = 0.0f;
    }
    uint32_t kMask = 0x000f000fu, kMaskHi = 0x00f000f0u, kMagic = 0x64006400u;
    asm volatile("" : "+v"(kMask), "+v"(kMaskHi), "+v"(kMagic));
    const uint32_t sel_lo = 0x07000700u + (uint32_t)(2 * q) * 0x00010001u;
    /* LDS index of the lane's D tokens: 32 tt + 8 (j / 4) + 4 q + j % 4 */
    const int dtok = 32 * tt + 4 * q;

    WideBlk cur = load(0);
#pragma unroll 1
    for (int b = 0; b < NB; ++b) {
        const WideBlk nxt = load(b + 1);
        /* 6-bit scales of chunks q and q + 2 (qwen38_quant.c:131-143) */
        const uint32_t Y = cur.h.y, Z = cur.h.z, Wd = cur.h.w;
        const uint32_t scw[2] = {Y & 0x3f3f3f3fu, (Wd & 0x0f0f0f0fu) | ((Y >> 2) & 0x30303030u)};
        Scale sc[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const half2v SL = pair_byte(scw[kk], sel_lo), SH = pair_byte(scw[kk], sel_lo + 0x00010001u);
            sc[kk].sl = SL;
            sc[kk].nl = SL * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
            sc[kk].sh16 = SH * (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
            sc[kk].nh = SH * (half2v){(_Float16)-64.0f, (_Float16)-64.0f};
        }
        /* mins of sub-blocks 4 lh + q and 4 lh + 2 + q (bytes q, 2 + q) */
        const uint32_t mw = lh ? (((Wd >> 4) & 0x0f0f0f0fu) | ((Z >> 2) & 0x30303030u)) : (Z & 0x3f3f3f3fu);
        const float mn0 = (float)((mw >> (8 * q)) & 63u), mn1 = (float)((mw >> (8 * q + 16)) & 63u);
        /* pair sums of the A token for the two min products */
        const int16_t *ps = ps_s + ((size_t)b * kWideTokens + atok) * 8;
        const float pa0 = (float)ps[4 * lh + q], pa1 = (float)ps[4 * lh + 2 + q];
        const float16v_w z = {};
        const float dh = f16_to_f32(cur.h.x), dmh = f16_to_f32(cur.h.x >> 16);
        const float *xsb = xs_s + b * kWideTokens + dtok;
        float xsv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) xsv[j] = xsb[8 * (j >> 2) + (j & 3)];
        {
            const float16v_w m0 = __builtin_amdgcn_mfma_f32_32x32x2f32(pa0, mn0, z, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 16; ++j) accm[j][0] = __builtin_fmaf(-fmul_rn(dmh, xsv[j]), m0[j], accm[j][0]);
            const float16v_w m1 = __builtin_amdgcn_mfma_f32_32x32x2f32(pa1, mn1, z, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 16; ++j) accm[j][1] = __builtin_fmaf(-fmul_rn(dmh, xsv[j]), m1[j], accm[j][1]);
        }
        float dx[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) dx[j] = fmul_rn(dh, xsv[j]);
        const uint32_t wq0[4] = {cur.wq[0].x, cur.wq[0].y, cur.wq[0].z, cur.wq[0].w};
        const uint32_t wq1[4] = {cur.wq[1].x, cur.wq[1].y, cur.wq[1].z, cur.wq[1].w};
        const uint32_t lo0[4] = {cur.lo[0].x, cur.lo[0].y, cur.lo[0].z, cur.lo[0].w};
        const uint32_t hi0[4] = {cur.hi[0].x, cur.hi[0].y, cur.hi[0].z, cur.hi[0].w};
        const uint32_t lo1[4] = {cur.lo[1].x, cur.lo[1].y, cur.lo[1].z, cur.lo[1].w};
        const uint32_t hi1[4] = {cur.hi[1].x, cur.hi[1].y, cur.hi[1].z, cur.hi[1].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const half8 b0 = dequant(wq0[k], sc[0], kMask, kMaskHi, kMagic);
            const half8 b1 = dequant(wq1[k], sc[1], kMask, kMaskHi, kMagic);
            const half8 a0 = act8(lo0[k], hi0[k]);
            const half8 a1 = act8(lo1[k], hi1[k]);
            float16v_w d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, z, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, d, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[j][k] = __builtin_fmaf(dx[j], d[j], acc[j][k]);
        }
        cur = nxt;
    }

    /* final tree: the lane half lh = 1 hands its six values per (row, token)
     * to lh = 0 through LDS, eight tokens at a time (the staging area is
     * free now) */
    float *xch = reinterpret_cast<float *>(lds);
    const uint32_t row = row0 + lrow;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        __syncthreads();
        if (lh) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int j = 8 * half + jj;
                float *e = xch + (((size_t)(wv >> 1) * 8 + jj) * 6) * 64 + lane;
                e[0] = acc[j][0];
                e[64] = acc[j][1];
                e[128] = acc[j][2];
                e[192] = acc[j][3];
                e[256] = accm[j][0];
                e[320] = accm[j][1];
            }
        }
        __syncthreads();
        if (!lh) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int j = 8 * half + jj;
                const float *e = xch + (((size_t)(wv >> 1) * 8 + jj) * 6) * 64 + lane;
                const float a4 = e[0], a5 = e[64], a6 = e[128], a7 = e[192], m2 = e[256], m3 = e[320];
                const float s = fadd_rn(fadd_rn(fadd_rn(acc[j][0], a4), fadd_rn(acc[j][2], a6)),
                                        fadd_rn(fadd_rn(acc[j][1], a5), fadd_rn(acc[j][3], a7)));
                const float m = fadd_rn(fadd_rn(accm[j][0], m2), fadd_rn(accm[j][1], m3));
                const uint32_t tok = tok0 + dtok + 8 * (j >> 2) + (j & 3);
                if (row < rows && tok < tokens) y[(size_t)tok * ldy + row] = fadd_rn(s, m);
            }
        }
    }
}

template <int NB>
bool launch_wide_nb(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, uint32_t tokens,
                    hipStream_t stream)
{
    static_assert(wide_lds_bytes<NB>() <= 160 * 1024, "LDS");
    hipLaunchKernelGGL(gemm_q4k_wide<NB>, dim3((rows + kWideRows - 1) / kWideRows, (tokens + kWideTokens - 1) / kWideTokens),
                       dim3(64 * kWideWaves), 0, stream, w, x, y, ldy, rows, tokens);
    return hipGetLastError() == hipSuccess;
}

}  // namespace

bool launch_gemm_q4k_wide(uint32_t tokens, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy,
                          uint32_t rows, uint32_t nb, hipStream_t stream)
{
    if (!rows || !tokens || ldy < rows || tokens > 65535u * kWideTokens) return false;
    switch (nb) {
    case 20: return launch_wide_nb<20>(w_tiled, x, y, ldy, rows, tokens, stream);
    case 24: return launch_wide_nb<24>(w_tiled, x, y, ldy, rows, tokens, stream);
    case 40: return launch_wide_nb<40>(w_tiled, x, y, ldy, rows, tokens, stream);
    case 68: return launch_wide_nb<68>(w_tiled, x, y, ldy, rows, tokens, stream);
    default: return false;
    }
}

}  // namespace q38
