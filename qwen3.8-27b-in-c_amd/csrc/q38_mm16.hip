/* Q4_K x Q8_K for 1..4 tokens on the gfx950 matrix cores, 16 weight rows
 * per wavefront (v_mfma_f32_16x16x32_f16), over the 16-row tiled copy built
 * by repack_q4k_tiles ([tile = row / 16][block][row % 16][144 bytes]).
 *
 * Arithmetic: that of the reference's AVX2 kernel
 * (src/qwen38/qwen38_quant.c:1546-1634).  Per row, token and super-block b:
 * eight exact integers W[b][l] (l = AVX2 accumulator lane; lane l of chunk c
 * is quant dword l of the chunk: low nibbles = elements 64c + 4l + u with
 * scale sc[2c], high nibbles = elements 64c + 32 + 4l + u with sc[2c + 1]),
 * four min sums M[b][i] = m[2i] (s[4i] + s[4i+1]) + m[2i+1] (s[4i+2] +
 * s[4i+3]), the fp32 chains acc[l] = fmaf(d_b, W, acc[l]) and
 * accm[i] = fmaf(-dmin_b, M, accm[i]) over b in order (d_b = f16(d) *
 * scale_b, dmin_b likewise) and the final tree
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) + ((m0+m2)+(m1+m3)) (:303-310,
 * 1626-1630).  Every sc * q (<= 945) and activation is exact in fp16 and
 * every partial sum is an integer below 2^22, so the matrix core returns W
 * exactly, in any internal order.
 *
 * Mapping.  One MFMA per AVX2 lane l and block: K = 32 is the lane's 8
 * elements of each of the four chunks, and K-group g (lanes 16g .. 16g + 15
 * of the wavefront) holds chunk c = g.  So lane (j = i % 16, g = i / 16)
 * supplies, as the B operand, dword l of chunk g of weight row j (all eight
 * lanes of a chunk are one contiguous 32 bytes: two 16-byte loads), scaled
 * by that chunk's two sub-block scales only.  Token t sits in A-row 4t: the
 * lanes i % 16 = 4t supply its eight activations of lane l in chunk g as
 * fp16 (staged in LDS once per workgroup), every other lane supplies zeros.
 * The result D[4g + r][j] lands in register r of lane (j, g), so register 0
 * of lane (j, t) is W[b][l] of row j and token t: the lane owns that
 * (row, token)'s twelve chains and its final tree.
 *
 * Work split.  A wavefront runs every block of its own 16-row tile; a
 * workgroup holds T such wavefronts, which share the activations staged in
 * LDS once (fp16 in the A-operand order, a scale and the sub-block pair sums
 * per token and block).  T is picked from the tile count so that every
 * workgroup of the launch is resident at once (one per compute unit).
 *
 * Memory.  Each wavefront streams its tile through a ring of P tile-blocks
 * in LDS, written by the load unit itself (buffer loads with the LDS flag,
 * 2304 contiguous bytes per block), P - 1 blocks ahead of the one being
 * computed; no registers hold data in flight, and the compute of one block
 * overlaps the loads of the next three.  A block's thirteen LDS reads are
 * scheduled together ahead of its arithmetic.  Measured on MI355X (kernel
 * trace) for 3 tokens x 34816 x 5120: 25.6 us against 27.4 us for the
 * 32-row kernel (q38_tiled32.hip); the stream alone (no arithmetic) takes
 * 19 us and the arithmetic alone 23 us, so the kernel is issue-bound: about
 * 150 instructions per block and wavefront, 74 of them the fp16 dequant.
 */
#include "q38_device.h"
#include "q38_kernels.h"
#include "q38_q4k_mfma.h"

namespace q38 {

namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr uint32_t kComputeUnits = 256;   /* MI355X */

/* staged fp16 activations of one (token, block): [chunk][AVX2 lane][8] */
constexpr int kActHalf8 = 32;

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

/* Copy one 2304-byte tile-block (bytes `soff` .. of the tile behind `rsrc`)
 * to LDS at `dst`: two 1 KiB buffer loads of 16 bytes per lane and one of 4
 * bytes per lane, written by the load unit straight into LDS (lane i's bytes
 * land at dst + 16 i, dst + 1024 + 16 i and dst + 2048 + 4 i).  Inline
 * assembly, so the compiler's wait-count pass does not see LDS stores and
 * drain them before every LDS read; the caller waits with wait_vmcnt.  Out of
 * range bytes (past the resource) read as zero. */
__device__ __forceinline__ void dma_tile_block(__amdgpu_buffer_rsrc_t rsrc, int soff, uint32_t dst, int lane)
{
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds"
                 :: "v"(lane * 16), "s"(dst), "s"(rsrc), "s"(soff) : "memory", "m0");
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds"
                 :: "v"(1024 + lane * 16), "s"(dst + 1024), "s"(rsrc), "s"(soff) : "memory", "m0");
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, %3 offen lds"
                 :: "v"(2048 + lane * 4), "s"(dst + 2048), "s"(rsrc), "s"(soff) : "memory", "m0");
}
constexpr int kDmaOps = 3;   /* vector-memory operations per tile-block */

template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

/* LDS bytes of one workgroup: staged activations (+ 8 zero records), scales,
 * pair sums, and a ring of P tile-blocks per wavefront */
template <int MT, int NB, int T, int P>
constexpr int mm16_lds_bytes()
{
    return (MT * NB * kActHalf8 + MT + 8) * 16 + MT * NB * 4 + MT * NB * 16 + T * P * kTileBlock;
}

template <int MT, int NB, int T, int P, int BP>
__global__ __launch_bounds__(64 * T) void gemm_q4k_mm16(const uint8_t *__restrict__ w,
                                                      const uint8_t *__restrict__ x, float *__restrict__ y,
                                                      uint32_t ldy, uint32_t rows)
{
    static_assert(MT >= 1 && MT <= 4, "1..4 tokens");
    static_assert(NB > P, "prefetch deeper than the blocks");
    static_assert(P % BP == 0 && (NB - P) % BP == 0, "rounds of BP blocks");
    /* token t's records start t half8 further on (bank spread) */
    constexpr int kZero = MT * NB * kActHalf8 + MT;
    auto act_index = [](int t, int b) { return (t * NB + b) * kActHalf8 + t; };
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    half8 *act_s = reinterpret_cast<half8 *>(lds);
    float *xs_s = reinterpret_cast<float *>(lds + (kZero + 8) * 16);
    uint4 *sub_s = reinterpret_cast<uint4 *>(lds + (kZero + 8) * 16 + MT * NB * 4);
    uint8_t *ring = lds + (kZero + 8) * 16 + MT * NB * 20;

    const int lane = threadIdx.x & 63;
    const int tg = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const uint32_t ntiles = (rows + 15) / 16;
    uint32_t tile = blockIdx.x * T + tg;
    const bool live = tile < ntiles;
    if (!live) tile = ntiles - 1;

    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w + (size_t)tile * NB * kTileBlock), 0, NB * kTileBlock, kRawBuffer);
    uint8_t *my_ring = ring + tg * P * kTileBlock;
    const uint32_t ring_base = __builtin_amdgcn_readfirstlane(lds_addr(my_ring));
    /* the first P blocks are requested before the staging */
#pragma unroll
    for (int k = 0; k < P; ++k) dma_tile_block(wr, k * kTileBlock, ring_base + k * kTileBlock, lane);

    const int nthreads = 64 * T;
    {
        /* activations as fp16 in the MFMA order of act8 (low nibble
         * elements u = 0, 2, 1, 3 of the lane's dword, then the high ones);
         * eight units' loads in flight per thread */
        constexpr int kUnits = MT * NB * 32, kDepth = 8;
        for (int u0 = threadIdx.x; u0 < kUnits; u0 += kDepth * nthreads) {
            uint32_t lo[kDepth], hi[kDepth];
#pragma unroll
            for (int d = 0; d < kDepth; ++d) {
                const int u = u0 + d * nthreads < kUnits ? u0 + d * nthreads : kUnits - 1;
                const int tb = u >> 5, cl = u & 31, c = cl >> 3, l = cl & 7;
                const uint8_t *xb = x + (size_t)tb * kQ8KBytes + 4 + 64 * c + 4 * l;
                lo[d] = *reinterpret_cast<const uint32_t *>(xb);
                hi[d] = *reinterpret_cast<const uint32_t *>(xb + 32);
            }
            /* every load's value is stored (past the end: the last unit again,
             * the same bytes), so no load is still in flight after the
             * barrier where the compiler would not expect one */
#pragma unroll
            for (int d = 0; d < kDepth; ++d) {
                const int u = u0 + d * nthreads < kUnits ? u0 + d * nthreads : kUnits - 1;
                act_s[u + u / (NB * kActHalf8)] = act8(lo[d], hi[d]);
            }
        }
        if (threadIdx.x < 8) act_s[kZero + threadIdx.x] = (half8){};
    }
    for (int u = threadIdx.x; u < MT * NB; u += nthreads) {
        const uint8_t *xb = x + (size_t)u * kQ8KBytes;
        xs_s[u] = *reinterpret_cast<const float *>(xb);
        const uint32_t *sd = reinterpret_cast<const uint32_t *>(xb + 260);
        uint32_t p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = sd[2 * i], b = sd[2 * i + 1];
            const int sa = (int)(int16_t)(a & 0xffffu) + ((int)a >> 16);
            const int sb = (int)(int16_t)(b & 0xffffu) + ((int)b >> 16);
            p[i] = ((uint32_t)sa & 0xffffu) | ((uint32_t)sb << 16);
        }
        sub_s[u] = make_uint4(p[0], p[1], p[2], p[3]);
    }
    __syncthreads();

    /* A operand: token t = (j / 4) in A-row j when j % 4 == 0 */
    const int at = j >> 2;
    const bool aon = (j & 3) == 0 && at < MT;
    /* chains: lane (j, g) owns token g */
    const int ct = g < MT ? g : MT - 1;

    uint32_t kMask = 0x000f000fu, kMaskHi = 0x00f000f0u, kMagic = 0x64006400u;
    asm volatile("" : "+v"(kMask), "+v"(kMaskHi), "+v"(kMagic));
    /* scale bytes of chunk g: sub-blocks 2g, 2g + 1 are bytes 2 (g & 1),
     * 2 (g & 1) + 1 of the low (g < 2) or high scale word */
    const uint32_t sel_lo = 0x07000700u + (uint32_t)(2 * (g & 1)) * 0x00010001u;
    const uint32_t gmask = g >= 2 ? 0xffffffffu : 0u;
    const uint32_t hoff = (uint32_t)(j * kBlockBytes), qoff = hoff + 16 + 32 * g;

    float acc[8], accm[4];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) accm[i] = 0.0f;

    /* A operands: the lanes that hold no token read eight zero records */
    struct Ops {
        uint4 h, q0, q1, sp;
        half8 a[8];
        float xs;
    };
    auto fetch = [&](int b, int st, Ops &o) {
        const uint8_t *blk = my_ring + st * kTileBlock;
        o.h = *reinterpret_cast<const uint4 *>(blk + hoff);
        o.q0 = *reinterpret_cast<const uint4 *>(blk + qoff);
        o.q1 = *reinterpret_cast<const uint4 *>(blk + qoff + 16);
        const half8 *ap = act_s + (aon ? act_index(at, b) + 8 * g : kZero);
#pragma unroll
        for (int l = 0; l < 8; ++l) o.a[l] = ap[l];
        o.xs = xs_s[ct * NB + b];
        o.sp = sub_s[ct * NB + b];
    };
    /* wl[l] = W[b][l] of (row j, token g) */
    auto products = [&](const Ops &o, float (&wl)[8]) {
        const uint32_t Y = o.h.y, Wd = o.h.w;
        const uint32_t scw =
            ((Y & 0x3f3f3f3fu) & ~gmask) | (((Wd & 0x0f0f0f0fu) | ((Y >> 2) & 0x30303030u)) & gmask);
        Scale sc;
        const half2v SL = pair_byte(scw, sel_lo), SH = pair_byte(scw, sel_lo + 0x00010001u);
        sc.sl = SL;
        sc.nl = SL * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
        sc.sh16 = SH * (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
        sc.nh = SH * (half2v){(_Float16)-64.0f, (_Float16)-64.0f};
        const uint32_t qd[8] = {o.q0.x, o.q0.y, o.q0.z, o.q0.w, o.q1.x, o.q1.y, o.q1.z, o.q1.w};
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const half8 bw = dequant(qd[l], sc, kMask, kMaskHi, kMagic);
            const float4v z = {};
            const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.a[l], bw, z, 0, 0, 0);
            wl[l] = d[0];
        }
    };
    /* the chains of (row j, token ct) over block b */
    auto chains = [&](const Ops &o, const float (&wl)[8]) {
        const uint4 h = o.h;
        const float xs = o.xs;
        const float dx = fmul_rn(f16_to_f32(h.x), xs);
        const float mx = -fmul_rn(f16_to_f32(h.x >> 16), xs);
        const uint32_t mw0 = h.z & 0x3f3f3f3fu, mw1 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        const uint32_t mp[4] = {__builtin_amdgcn_perm(0u, mw0, 0x0c010c00u), __builtin_amdgcn_perm(0u, mw0, 0x0c030c02u),
                                __builtin_amdgcn_perm(0u, mw1, 0x0c010c00u), __builtin_amdgcn_perm(0u, mw1, 0x0c030c02u)};
        const uint32_t sv[4] = {o.sp.x, o.sp.y, o.sp.z, o.sp.w};
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(dx, wl[l], acc[l]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int msum = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, mp[i]),
                                                    __builtin_bit_cast(short2v, sv[i]), 0, false);
            accm[i] = __builtin_fmaf(mx, (float)msum, accm[i]);
        }
    };
    /* BP blocks k .. k + BP - 1 in stages st ..: their LDS reads go out
     * first (issued one by one just before their use, each would wait a
     * full LDS round trip), their products interleave, and the chains run
     * in block order */
    auto round = [&](int k, int st) {
        Ops o[BP];
        float wl[BP][8];
#pragma unroll
        for (int u = 0; u < BP; ++u) fetch(k + u, st + u, o[u]);
#pragma unroll
        for (int u = 0; u < BP; ++u) products(o[u], wl[u]);
#pragma unroll
        for (int u = 0; u < BP; ++u) chains(o[u], wl[u]);
        __builtin_amdgcn_sched_group_barrier(0x100, 13 * BP, 0);
        __builtin_amdgcn_sched_group_barrier(0x00f, 1000 * BP, 0);
    };

    /* steady state: block k is in stage k % P; after its round the stage
     * takes block k + P.  Loads retire in order, so with P - BP later
     * blocks in flight vmcnt(3 (P - BP)) means the round's blocks have
     * landed; the LDS reads of a stage are consumed before its refill is
     * issued. */
#pragma unroll 1
    for (int k = 0; k < NB - P; k += BP) {
        const int st = k % P;
        wait_vmcnt<kDmaOps * (P - BP)>();
        round(k, st);
#pragma unroll
        for (int u = 0; u < BP; ++u)
            dma_tile_block(wr, (k + P + u) * kTileBlock, ring_base + (st + u) * kTileBlock, lane);
    }
    /* the last P blocks, nothing more to load */
#pragma unroll 1
    for (int e = 0; e < P; e += BP) {
        const int k = NB - P + e;
        switch (P - BP - e) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<kDmaOps>(); break;
        case 2: wait_vmcnt<2 * kDmaOps>(); break;
        case 3: wait_vmcnt<3 * kDmaOps>(); break;
        case 4: wait_vmcnt<4 * kDmaOps>(); break;
        case 5: wait_vmcnt<5 * kDmaOps>(); break;
        case 6: wait_vmcnt<6 * kDmaOps>(); break;
        default: wait_vmcnt<0>(); break;
        }
        round(k, k % P);
    }

    const uint32_t row = 16 * tile + (uint32_t)j;
    if (!live || g >= MT || row >= rows) return;
    const float a = fadd_rn(fadd_rn(fadd_rn(acc[0], acc[4]), fadd_rn(acc[2], acc[6])),
                            fadd_rn(fadd_rn(acc[1], acc[5]), fadd_rn(acc[3], acc[7])));
    const float m = fadd_rn(fadd_rn(accm[0], accm[2]), fadd_rn(accm[1], accm[3]));
    y[(size_t)g * ldy + row] = fadd_rn(a, m);
}

template <int MT, int NB, int T, int P, int BP>
bool launch_mm16_cfg(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, hipStream_t stream)
{
    constexpr int lds = mm16_lds_bytes<MT, NB, T, P>();
    if constexpr (lds > 160 * 1024) {
        return false;
    } else {
        const void *kernel = reinterpret_cast<const void *>(&gemm_q4k_mm16<MT, NB, T, P, BP>);
        static bool configured = false;
        if (!configured) {
            if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) return false;
            configured = true;
        }
        const uint32_t ntiles = (rows + 15) / 16;
        hipLaunchKernelGGL((gemm_q4k_mm16<MT, NB, T, P, BP>), dim3((ntiles + T - 1) / T), dim3(64 * T), lds, stream, w, x,
                           y, ldy, rows);
        return hipGetLastError() == hipSuccess;
    }
}

/* T tiles per workgroup: the fewest that keep the launch within one
 * workgroup per compute unit (a second wave of workgroups would double the
 * time of the compute units that run it) */
template <int MT, int NB>
bool launch_mm16_typed(const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows, hipStream_t stream)
{
    const uint32_t ntiles = (rows + 15) / 16;
    if (ntiles <= 8 * kComputeUnits) return launch_mm16_cfg<MT, NB, 8, 4, 1>(w, x, y, ldy, rows, stream);
    if (ntiles <= 9 * kComputeUnits) return launch_mm16_cfg<MT, NB, 9, 4, 1>(w, x, y, ldy, rows, stream);
    return false;
}

template <int NB>
bool launch_mm16_nb(int m, const uint8_t *w, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                    hipStream_t stream)
{
    switch (m) {
    case 2: return launch_mm16_typed<2, NB>(w, x, y, ldy, rows, stream);
    case 3: return launch_mm16_typed<3, NB>(w, x, y, ldy, rows, stream);
    case 4: return launch_mm16_typed<4, NB>(w, x, y, ldy, rows, stream);
    default: return false;
    }
}

}  // namespace

/* y[t * ldy + row] = W_row . x_t (2 <= m <= 4) from the 16-row tiled copy
 * of a 20-block (5120-wide) matrix of up to 36864 rows, 16 rows per
 * wavefront; false for other shapes.  Measured faster than the 32-row
 * kernel only from about 32768 rows on (below that the launch cannot keep
 * one workgroup of eight or more wavefronts on every compute unit). */
bool launch_gemm_q4k_mm16(int m, const uint8_t *w_tiled, const uint8_t *x, float *y, uint32_t ldy, uint32_t rows,
                          uint32_t nb, hipStream_t stream)
{
    if (!rows || ldy < rows) return false;
    switch (nb) {
    case 20: return launch_mm16_nb<20>(m, w_tiled, x, y, ldy, rows, stream);
    default: return false;
    }
}

}  // namespace q38
