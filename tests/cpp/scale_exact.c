/* Exhaustive CPU check of the rotate+quantise prologue's scale divisions
 * (phi-agent_amd/csrc/qt_scale.hpp) against IEEE division, which the
 * reference uses (core/host/quant.cpp:134-169: scale = amax / qmax,
 * inv = 1 / scale).  Test infrastructure.
 *
 *   qt_div_qmax: q0 = a * RN(1/qmax), q = fma(fma(-q0, qmax, a), RN(1/qmax), q0)
 *     must equal a / qmax for every integer qmax in [1, 127] and every
 *     significand of a, at the ends of its range [2^-90, 2^122) and at 1.
 *   qt_rcp_bits: y' = fma(fma(-b, y, 1), y, y) twice from any estimate y
 *     within 2 ulps of RN(1/b) must equal RN(1/b) for every significand of b
 *     but all ones, at the ends of b's range [2^-97, 2^122] and at 1; on the
 *     all-ones significand the bits ((253 - E) << 23) | 1 must equal 1 / b.
 *
 * Every value stays normal in these ranges, so exponent scaling is exact and
 * the result depends on the significand alone.  Prints the mismatch counts;
 * exit status 0 when all are zero. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* The same loops twice: with the FMA instruction where the CPU has it, and
 * with libm's fmaf (also exact, slower) where it does not. */
#define SCALE_LOOPS(NAME, FMA)                                                                  \
    static void NAME(long* div_bad, long* rcp_bad, long* ones_bad) {                            \
        static const int dexp[3] = {-90, 0, 121};                                               \
        for (int ei = 0; ei < 3; ei++) {                                                        \
            const uint32_t eb = (uint32_t)(127 + dexp[ei]) << 23;                               \
            for (int qm = 1; qm <= 127; qm++) {                                                 \
                const float b = (float)qm, y = 1.0f / b;                                        \
                for (uint32_t m = 0; m < (1u << 23); m++) {                                     \
                    const float a = from_bits(eb | m);                                          \
                    const float q0 = a * y;                                                     \
                    const float q = FMA(FMA(-q0, b, a), y, q0);                                 \
                    if (q != a / b) ++*div_bad;                                                 \
                }                                                                               \
            }                                                                                   \
        }                                                                                       \
        static const int rexp[3] = {-97, 0, 121};                                               \
        for (int ei = 0; ei < 3; ei++) {                                                        \
            const uint32_t eb = (uint32_t)(127 + rexp[ei]) << 23;                               \
            for (uint32_t m = 0; m < (1u << 23); m++) {                                         \
                const float b = from_bits(eb | m), rn = 1.0f / b;                               \
                if (m == 0x7fffffu) {                                                           \
                    if (to_bits(rn) != (((253u - ((eb | m) >> 23)) << 23) | 1u)) ++*ones_bad;   \
                    continue;                                                                   \
                }                                                                               \
                float est[5];                                                                   \
                est[0] = rn;                                                                    \
                est[1] = nextafterf(rn, 0.0f);                                                  \
                est[2] = nextafterf(rn, INFINITY);                                              \
                est[3] = nextafterf(est[1], 0.0f);                                              \
                est[4] = nextafterf(est[2], INFINITY);                                          \
                for (int k = 0; k < 5; k++) {                                                   \
                    const float y1 = FMA(FMA(-b, est[k], 1.0f), est[k], est[k]);                \
                    const float y2 = FMA(FMA(-b, y1, 1.0f), y1, y1);                            \
                    if (y2 != rn) ++*rcp_bad;                                                   \
                }                                                                               \
            }                                                                                   \
        }                                                                                       \
    }

#if defined(__x86_64__)
__attribute__((target("fma"))) static float fma_hw(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__attribute__((target("fma"))) SCALE_LOOPS(loops_hw, fma_hw)
#endif
SCALE_LOOPS(loops_libm, fmaf)

int main(void) {
    long div_bad = 0, rcp_bad = 0, ones_bad = 0;
#if defined(__x86_64__)
    if (__builtin_cpu_supports("fma"))
        loops_hw(&div_bad, &rcp_bad, &ones_bad);
    else
#endif
        loops_libm(&div_bad, &rcp_bad, &ones_bad);
    printf("div_qmax_mismatches %ld rcp_mismatches %ld all_ones_mismatches %ld\n", div_bad, rcp_bad, ones_bad);
    return div_bad || rcp_bad || ones_bad;
}
