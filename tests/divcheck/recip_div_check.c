/* Host check of the reciprocal division the int8 KV writes use on the GPU: with y = 1 / b (IEEE),
 * q0 = x * y, r = fma(-q0, b, x), q = fma(r, y, q0) is the IEEE quotient x / b (Markstein's
 * correction step) except where the quotient or the remainder underflows or overflows. The
 * kernels take the IEEE division instead for every row whose largest |x| is not below 2^100
 * (and for NaN), so the fast path serves |x| < 2^100 only. What the writes need there:
 *   cal   every bf16 |x| < 2^100 against every calibration the kernels write (1e-3 and every
 *         bf16 value of at least 1e-3): q == x / cal wherever either is at least 2^-64. Below
 *         that the value cannot reach an output: it quantizes to 0 against any row scale (at
 *         least 1e-6 / 127), and a row maximum below 1e-6 is raised to 1e-6.
 *   vrow  every bf16 x against the scale of every row whose largest |x| is a bf16 value a >= |x|
 *         (b = max(a, 1e-6) / 127: the V quantization, and K rows of calibration 1): the int8
 *         value clamp(rint(q), -127, 127) equals the one from x / b.
 *   krow  the same for random fp32 a < 2^110 and x with |x| <= a (the K quantization after the
 *         calibration division, whose quotients stay below 2^100 / 1e-3; N pairs, fixed seed).
 *   calr  as cal for random fp32 calibrations in [1e-3, 2^100) (calibrations a caller wrote
 *         itself) against random bf16 |x| < 2^100 (N pairs, fixed seed).
 * Build: gcc -O2 -ffp-contract=off -fopenmp recip_div_check.c -lm. Usage: prog cal|vrow|krow [N].
 * Prints the number of pairs checked and of mismatches; exits 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float rdiv(float x, float b, float y) {
    const float q0 = x * y;
    const float r = fmaf(-q0, b, x);
    return fmaf(r, y, q0);
}
static int same(float a, float b) { return u_of(a) == u_of(b); }
static int quant(float q) { return (int)fminf(fmaxf(rintf(q), -127.0f), 127.0f); }
static const float TINY = 0x1p-64f;
static const uint32_t XMAX_BF16 = 0x7180;  /* bf16 bits of 2^100: the fast path's bound on |x| */

int main(int argc, char** argv) {
    const char* mode = argc > 1 ? argv[1] : "cal";
    long long checked = 0, bad = 0;
    if (!strcmp(mode, "cal")) {
        /* b: 1e-3 then every finite positive bf16 >= 1e-3 */
        static uint32_t bs[40000];
        int nb = 0;
        bs[nb++] = u_of(1e-3f);
        for (uint32_t h = 0; h < 0x7f80; ++h) {
            const float b = f_of(h << 16);
            if (b >= 1e-3f) bs[nb++] = h << 16;
        }
#pragma omp parallel for reduction(+ : checked, bad) schedule(dynamic, 64)
        for (int i = 0; i < nb; ++i) {
            const float b = f_of(bs[i]), y = 1.0f / b;
            for (uint32_t h = 0; h < XMAX_BF16; ++h) {  /* x >= 0 (the identity is odd in x) */
                const float x = f_of(h << 16);
                ++checked;
                const float q = rdiv(x, b, y), want = x / b;
                if (!same(q, want) && (fabsf(q) >= TINY || fabsf(want) >= TINY)) {
                    if (bad < 5) printf("cal mismatch x=%a b=%a\n", x, b);
                    ++bad;
                }
            }
        }
    } else if (!strcmp(mode, "vrow")) {
#pragma omp parallel for reduction(+ : checked, bad) schedule(dynamic, 64)
        for (uint32_t ha = 1; ha < XMAX_BF16; ++ha) {
            const float a = f_of(ha << 16);
            const float b = fmaxf(a, 1e-6f) / 127.0f, y = 1.0f / b;
            for (uint32_t h = 0; h <= ha; ++h) {
                const float x = f_of(h << 16);
                ++checked;
                if (quant(rdiv(x, b, y)) != quant(x / b)) {
                    if (bad < 5) printf("vrow mismatch x=%a a=%a\n", x, a);
                    ++bad;
                }
            }
        }
    } else if (!strcmp(mode, "calr")) {
        const long long n = argc > 2 ? atoll(argv[2]) : 100000000LL;
#pragma omp parallel reduction(+ : checked, bad)
        {
            uint64_t s = 0xC2B2AE3D27D4EB4FULL;
#ifdef _OPENMP
            s ^= (uint64_t)(omp_get_thread_num() + 1) * 0x165667B19E3779F9ULL;
#endif
            const uint32_t lo = u_of(1e-3f), hi = 0x71800000u;  /* [1e-3, 2^100) */
#pragma omp for schedule(static)
            for (long long i = 0; i < n; ++i) {
                s ^= s << 13; s ^= s >> 7; s ^= s << 17;
                const float b = f_of(lo + (uint32_t)(s >> 32) % (hi - lo));
                const float x = f_of(((uint32_t)s % XMAX_BF16) << 16);
                const float y = 1.0f / b;
                const float q = rdiv(x, b, y), want = x / b;
                ++checked;
                if (!same(q, want) && (fabsf(q) >= TINY || fabsf(want) >= TINY)) {
                    if (bad < 5) printf("calr mismatch x=%a b=%a\n", x, b);
                    ++bad;
                }
            }
        }
    } else {
        const long long n = argc > 2 ? atoll(argv[2]) : 100000000LL;
#pragma omp parallel reduction(+ : checked, bad)
        {
            uint64_t s = 0x9E3779B97F4A7C15ULL;
#ifdef _OPENMP
            s ^= (uint64_t)(omp_get_thread_num() + 1) * 0xD1B54A32D192ED03ULL;
#endif
#pragma omp for schedule(static)
            for (long long i = 0; i < n; ++i) {
                s ^= s << 13; s ^= s >> 7; s ^= s << 17;
                /* a: any finite positive fp32; x: any fp32 of at most |a| */
                const float a = f_of((uint32_t)(s >> 32) % 0x76800000u);  /* < 2^110 */
                const float x = f_of((uint32_t)s % (u_of(a) + 1));
                const float b = fmaxf(a, 1e-6f) / 127.0f, y = 1.0f / b;
                ++checked;
                if (quant(rdiv(x, b, y)) != quant(x / b)) {
                    if (bad < 5) printf("krow mismatch x=%a a=%a\n", x, a);
                    ++bad;
                }
            }
        }
    }
    printf("%s: %lld pairs, %lld mismatches\n", mode, checked, bad);
    return bad != 0;
}
