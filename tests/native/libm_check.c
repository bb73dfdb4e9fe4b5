/* Exhaustive comparison of q38_expf and q38_logf with the host C library's
 * expf and logf over all 2^32 float bit patterns (NaN results compare equal
 * when both are NaN).
 * Prints "<name> checked <n> mismatches <m> first <hex>" per function.
 * With the argument "checksum" it instead prints, for the host C library's
 * expf and logf, the order-independent checksum that
 * tests/native/math_probe.hip forms on the device:
 * sum over x of mix64((x << 32) | bits(f(x))), NaN results as 0x7fc00000.
 * Built and run by tests/test_libm_exhaustive.py. */
#include <math.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>

#include "q38_libm.h"

#define CHECK_ALL(NAME, FN, HOST)                                                            \
    static void check_##NAME(void)                                                           \
    {                                                                                        \
        unsigned long long mismatches = 0, checked = 0;                                      \
        uint32_t first = 0;                                                                  \
        int have_first = 0;                                                                  \
        _Pragma("omp parallel for schedule(static) reduction(+ : mismatches, checked)")      \
        for (long long hi = 0; hi < 65536; ++hi) {                                           \
            for (uint32_t lo = 0; lo < 65536; ++lo) {                                        \
                const uint32_t bits = ((uint32_t)hi << 16) | lo;                             \
                const float x = q38_bits_to_float(bits);                                     \
                const float a = FN(x);                                                       \
                const float b = HOST(x);                                                     \
                ++checked;                                                                   \
                const int both_nan = (a != a) && (b != b);                                   \
                if (!both_nan && q38_float_to_bits(a) != q38_float_to_bits(b)) {             \
                    ++mismatches;                                                            \
                    _Pragma("omp critical")                                                  \
                    if (!have_first) { have_first = 1; first = bits; }                       \
                }                                                                            \
            }                                                                                \
        }                                                                                    \
        printf(#NAME " checked %llu mismatches %llu first %08x\n", checked, mismatches, first); \
    }

CHECK_ALL(expf, q38_expf, expf)
CHECK_ALL(logf, q38_logf, logf)

static uint64_t mix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static uint64_t checksum(float (*f)(float))
{
    uint64_t acc = 0;
#pragma omp parallel for schedule(static) reduction(+ : acc)
    for (long long hi = 0; hi < 65536; ++hi) {
        for (uint32_t lo = 0; lo < 65536; ++lo) {
            const uint64_t x = ((uint64_t)hi << 16) | lo;
            const float r = f(q38_bits_to_float((uint32_t)x));
            uint32_t bits = q38_float_to_bits(r);
            if (r != r) bits = 0x7fc00000u;
            acc += mix64((x << 32) | bits);
        }
    }
    return acc;
}

int main(int argc, char **argv)
{
    if (argc > 1 && strcmp(argv[1], "checksum") == 0) {
        printf("expf checksum %llu\n", (unsigned long long)checksum(expf));
        printf("logf checksum %llu\n", (unsigned long long)checksum(logf));
        return 0;
    }
    check_expf();
    check_logf();
    return 0;
}
