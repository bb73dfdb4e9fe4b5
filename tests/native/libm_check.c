/* Exhaustive comparison of q38_expf and q38_logf with the host C library's
 * expf and logf over all 2^32 float bit patterns (NaN results compare equal
 * when both are NaN).
 * Prints "<name> checked <n> mismatches <m> first <hex>" per function.
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

int main(void)
{
    check_expf();
    check_logf();
    return 0;
}
