/* Single-precision exp and log for the decode path, host and device.
 *
 * The reference engine evaluates every transcendental with the host C
 * library (expf in sigmoid/SiLU/softplus/decay/softmax, logf in softplus;
 * src/qwen38/qwen38_model.c:439, 444, 554, 771, 867; its vectorised
 * approximation at :447 is compiled only under Q38_FAST_EXP, which no build
 * of the reference defines).  glibc's expf is the table-plus-polynomial
 * method published in ARM's optimized-routines (math/expf.c):
 * x*N/ln2 = k + r with N = 32, 2^(k/N) from a 32-entry table of 2^(i/32),
 * and a cubic in r, all in double precision.  q38_expf restates that method;
 * its table entries are 2^(i/32) rounded to double.  glibc's logf is the
 * companion method of the same collection (math/logf.c): x = 2^k z with z in
 * [0x3f330000, 2*0x3f330000), sixteen subintervals each with a (1/c, log c)
 * pair, and log1p(z/c - 1) from a cubic in double precision; q38_logf
 * restates it.  Both round once, at the end, and match the host expf / logf
 * on every input tests/test_libm_exhaustive.py checks (all 2^32 floats for
 * expf, every non-negative float and the special values for logf).
 *
 * Plain C: usable from HIP device code and from host C compilers.
 */
#ifndef Q38_LIBM_H
#define Q38_LIBM_H

#include <stdint.h>

#if defined(__HIPCC__)
#define Q38_LIBM_FN __host__ __device__ static inline
#else
#define Q38_LIBM_FN static inline
#endif

Q38_LIBM_FN double q38_bits_to_double(uint64_t u)
{
    union { uint64_t u; double d; } v;
    v.u = u;
    return v.d;
}

Q38_LIBM_FN uint64_t q38_double_to_bits(double d)
{
    union { uint64_t u; double d; } v;
    v.d = d;
    return v.u;
}

Q38_LIBM_FN uint32_t q38_float_to_bits(float f)
{
    union { uint32_t u; float f; } v;
    v.f = f;
    return v.u;
}

Q38_LIBM_FN float q38_bits_to_float(uint32_t u)
{
    union { uint32_t u; float f; } v;
    v.u = u;
    return v.f;
}

/* asuint64(2^(i/32)) - (i << 47): adding k << 47 for k = 32 q + i then
 * yields 2^q * 2^(i/32). */
#define Q38_EXP2_TABLE \
    { 0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull }

/* (1/c, log c) for the sixteen subintervals of [0x3f330000, 2*0x3f330000). */
#define Q38_LOGF_TABLE \
    { { 0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2 }, { 0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2 }, \
      { 0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2 },  { 0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3 }, \
      { 0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3 }, { 0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3 },   \
      { 0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4 }, { 0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4 }, \
      { 0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5 }, { 0x1p+0, 0x0p+0 },                              \
      { 0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5 },  { 0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4 },   \
      { 0x1.b2036576afce6p-1, 0x1.526e57720db08p-3 },  { 0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3 },   \
      { 0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2 },  { 0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2 } }

#if defined(__HIPCC__)
__device__ static const uint64_t q38_exp2_table_dev[32] = Q38_EXP2_TABLE;
__device__ static const double q38_logf_table_dev[16][2] = Q38_LOGF_TABLE;
#endif
static const uint64_t q38_exp2_table_host[32] = Q38_EXP2_TABLE;
static const double q38_logf_table_host[16][2] = Q38_LOGF_TABLE;

/* q38_expf with the 2^(i/32) table at `tab` (a copy of Q38_EXP2_TABLE, for
 * instance in LDS) */
Q38_LIBM_FN float q38_expf_table(float x, const uint64_t *tab)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    /* 2^(r/32) ~ 1 + c2 r + c1 r^2 + c0 r^3 (coefficients pre-scaled by 1/32) */
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;

    const uint32_t ux = q38_float_to_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                                   /* |x| >= 88 or nan */
        if (ux == 0xff800000u) return 0.0f;                  /* -inf */
        if (abstop >= 0x7f8) return x + x;                   /* inf or nan */
        if (x > 0x1.62e42ep6f) return q38_bits_to_float(0x7f800000u);   /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                /* underflow */
    }
    const double xd = (double)x;
    /* x * 32/ln2 is fused into both the rounding add and the remainder, as
     * the host library's build does; that fusion reproduces it on every input */
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = q38_double_to_bits(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = q38_bits_to_double(t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

Q38_LIBM_FN float q38_expf(float x)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return q38_expf_table(x, q38_exp2_table_dev);
#else
    return q38_expf_table(x, q38_exp2_table_host);
#endif
}

Q38_LIBM_FN float q38_logf(float x)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const double(*tab)[2] = q38_logf_table_dev;
#else
    const double(*tab)[2] = q38_logf_table_host;
#endif
    const double ln2 = 0x1.62e42fefa39efp-1;
    const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2, a2 = -0x1.ffffef20a4123p-2;
    uint32_t ix = q38_float_to_bits(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        if (ix * 2 == 0) return q38_bits_to_float(0xff800000u);            /* log(+-0) = -inf */
        if (ix == 0x7f800000u) return x;                                   /* log(inf) = inf */
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u)                   /* x < 0 or nan */
            return q38_bits_to_float(0x7fc00000u);
        ix = q38_float_to_bits(x * 0x1p23f);                              /* subnormal */
        ix -= 23u << 23;
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = (int)((tmp >> 19) % 16);
    const int k = (int32_t)tmp >> 23;
    const uint32_t iz = ix - (tmp & (0x1ffu << 23));
    const double invc = tab[i][0], logc = tab[i][1];
    const double z = (double)q38_bits_to_float(iz);
    const double r = __builtin_fma(z, invc, -1.0);
    const double y0 = __builtin_fma((double)k, ln2, logc);
    const double r2 = r * r;
    double y = __builtin_fma(a1, r, a2);
    y = __builtin_fma(a0, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
    return (float)y;
}

#endif
