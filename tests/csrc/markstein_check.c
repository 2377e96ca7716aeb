/*
 * markstein_check.c -- CPU check of the FP8 quantizer's division by the row
 * scale (kernel-craft_amd/csrc/fp8_quant.hip: row_div / div_scale<true>).
 *
 * The reference divides each element by the row scale s = absmax / 448 with
 * an IEEE division (fp8_quant.cu:121,126).  The kernel instead computes, with
 * r = RN(1/s),
 *     q0 = RN(x*r);  e = RN(x - s*q0) (one FMA);  q = copysign(RN(q0 + e*r), x)
 * for rows with 2^-60 <= absmax <= FLT_MAX.  Claim checked here, for such s:
 *   (a) |x| >= 2^-103 and RN(x/s) normal:  q == RN(x/s) bit for bit;
 *   (b) otherwise:  |q| < 2^-30 and |RN(x/s)| < 2^-30, both with the sign of
 *       x (both encode to E4M3 +-0, whose smallest nonzero step is 2^-9).
 *
 * usage: markstein_check <mode> <n> <seed>
 *   mode 0: n random rows' scales (absmax from a wide exponent range and
 *           mantissa patterns), 2^16 random x each plus edge cases
 *   mode 1: exhaustive over all 2^32 x for the n-th fixed scale
 * Prints "mismatches <count>" and exits 0 when there are none.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits_to_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t rng_state;
static uint64_t next_u64(void) {  /* splitmix64 */
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static float kernel_div(float x, float s, float r) {
    volatile float q0 = x * r;          /* volatile: no contraction into the FMA */
    float e = fmaf(-s, q0, x);
    return copysignf(fmaf(e, r, q0), x);
}

static long check(float x, float absmax) {
    if (isnan(x) || fabsf(x) > absmax) return 0;  /* a row never holds |x| > absmax */
    const float s = absmax / 448.0f, r = 1.0f / s;
    const float want = x / s, got = kernel_div(x, s, r);
    if (fabsf(x) >= 0x1p-103f && fabsf(want) >= 0x1p-126f) {
        if (f_to_bits(want) != f_to_bits(got)) {
            fprintf(stderr, "absmax=%a x=%a: x/s=%a kernel=%a\n", absmax, x, want, got);
            return 1;
        }
    } else {
        if (!(fabsf(got) < 0x1p-30f && fabsf(want) < 0x1p-30f && signbit(got) == signbit(x) &&
              signbit(want) == signbit(x))) {
            fprintf(stderr, "tiny absmax=%a x=%a: x/s=%a kernel=%a\n", absmax, x, want, got);
            return 1;
        }
    }
    return 0;
}

static const float kFixed[] = {448.0f, 3.0f, 1.0f, 235.0f, 5.5104f, 0x1p-60f, 3.40282347e38f,
                               1e-10f, 1e30f, 0.75f, 0x1.fffffep+0f, 0x1.000002p-30f};

int main(int argc, char** argv) {
    const int mode = argc > 1 ? atoi(argv[1]) : 0;
    const long n = argc > 2 ? atol(argv[2]) : 64;
    rng_state = argc > 3 ? strtoull(argv[3], NULL, 10) : 1;
    long bad = 0;
    if (mode == 0) {
        for (long k = 0; k < n; ++k) {
            /* absmax exponent in [-60, 127], random or extreme mantissa */
            const int ex = -60 + (int)(next_u64() % 188);
            uint32_t man = (uint32_t)(next_u64() & 0x7FFFFF);
            if (k % 4 == 1) man = 0x7FFFFF;
            if (k % 4 == 2) man = 0;
            float absmax = bits_to_f(((uint32_t)(ex + 127) << 23) | man);
            if (isinf(absmax)) absmax = 3.40282347e38f;
            for (long i = 0; i < 65536; ++i) {
                const uint64_t u = next_u64();
                float x;
                switch (i & 3) {
                    case 0: x = bits_to_f((uint32_t)u); break;                          /* any pattern */
                    case 1: x = absmax * (float)((int64_t)(u % 2000001) - 1000000) * 1e-6f; break;
                    case 2: x = ldexpf(1.0f + (float)(u & 0xFFFFF) / 1048576.0f,
                                       (int)((u >> 20) % 140) - 140) * ((u >> 40) & 1 ? -1.0f : 1.0f);
                            break;                                                         /* near 2^-103 */
                    default: x = bits_to_f(f_to_bits(absmax) - (uint32_t)(u % 64)) * ((u >> 8) & 1 ? -1.0f : 1.0f);
                }
                bad += check(x, absmax);
            }
            const float edge[] = {0.0f, -0.0f, absmax, -absmax, 0x1p-103f, -0x1p-103f,
                                  0x1.fffffep-104f, 0x1p-149f, -0x1p-149f, 0x1p-126f};
            for (unsigned i = 0; i < sizeof(edge) / sizeof(edge[0]); ++i) bad += check(edge[i], absmax);
        }
    } else {
        const float absmax = kFixed[n % (long)(sizeof(kFixed) / sizeof(kFixed[0]))];
        for (uint64_t u = 0; u < (1ull << 32); ++u) bad += check(bits_to_f((uint32_t)u), absmax);
    }
    printf("mismatches %ld\n", bad);
    return bad != 0;
}
