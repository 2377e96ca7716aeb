/*
 * markstein_check.c -- CPU check of the FP8 quantizer's divisions
 * (kernel-craft_amd/csrc/fp8_quant.hip: markstein(), row_div, and the
 * SmoothQuant route of quant_rows_smooth_kernel).
 *
 * The reference divides with IEEE divisions (fp8_quant.cu:121,126,183).  The
 * kernels instead compute, with r = RN(1/s),
 *     q0 = RN(x*r);  e = RN(s*q0 - x) (one FMA);  q = RN(q0 - e*r)
 * Claim checked by modes 0 and 1, for s in [2^-120, 2^120]:
 *   (a) |x| >= 2^-102 and RN(x/s) normal:  q == RN(x/s) bit for bit;
 *   (b) otherwise (finite x, |x/s| <= 2^126): q and RN(x/s) have the sign of
 *       x, zeros included, and magnitudes <= 2^-102/s + 2^-125.
 * Mode 2 checks the SmoothQuant route as a whole: rows are smoothed by the
 * Markstein step, kept when the largest quotient magnitude lies in
 * [max(2^-60, 2^-81/s_min), 2^126] with every factor in [2^-120, 2^120], and
 * then encoded with a Markstein division by the row scale; the E4M3 codes
 * and row scales of every kept row must equal those of the reference's
 * two-step pipeline (IEEE x/s, absmax, IEEE division by absmax/448).
 *
 * Mode 3 checks the row-scale route's codes completely: for every one of
 * the 2^23 significands of s (s in [1, 2)), every E4M3 rounding boundary m
 * (the midpoints of consecutive E4M3 magnitudes up to 448, and 2^-10 between
 * 0 and the smallest subnormal) and every x within 4 ulps of RN(m s), both
 * signs, the quotient bits of the two routes must agree (and so must the
 * codes).  Both quotients lie within 2 ulps of x/s, so a code can differ only
 * where x/s is that close to a boundary; and across the fast route's range
 * (absmax in [2^-60, FLT_MAX], so s = absmax/448 in [2^-68.8, 2^119.2], r =
 * 1/s normal, and every x whose code is not +-0 normal and above 2^-80) each
 * step scales exactly with a power of two of s or x, so s in [1, 2) stands
 * for every exponent.  Mode 4: every s significand against n random x each
 * (all exponents that keep x/s normal), quotient bits.
 *
 * usage: markstein_check <mode> <n> <seed>
 *   mode 0: n random scales (row scales absmax/448 with absmax in
 *           [2^-60, 2^127], and factors in [2^-120, 2^120]), 2^16 x each
 *           plus edge cases
 *   mode 1: exhaustive over all 2^32 x for the n-th fixed scale
 *   mode 2: n random rows of 512 elements through the SmoothQuant route
 *   mode 3: every s significand x every E4M3 boundary x 9 x neighbours x 2 signs
 *   mode 4: every s significand x n random x
 * Modes 1, 3 and 4 run on every OpenMP thread.
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
    volatile float e = fmaf(s, q0, -x);
    return fmaf(-e, r, q0);
}

static long check(float x, float s) {
    const float r = 1.0f / s;
    const float want = x / s;
    if (!isfinite(x) || !(fabsf(want) <= 0x1p126f)) return 0;  /* such rows divide exactly */
    const float got = kernel_div(x, s, r);
    if (fabsf(x) >= 0x1p-102f && fabsf(want) >= 0x1p-126f) {
        if (f_to_bits(want) != f_to_bits(got)) {
            fprintf(stderr, "s=%a x=%a: x/s=%a kernel=%a\n", s, x, want, got);
            return 1;
        }
    } else {
        const float bound = 0x1p-102f / s + 0x1p-125f;
        if (!(fabsf(got) <= bound && fabsf(want) <= bound && signbit(got) == signbit(x) &&
              signbit(want) == signbit(x))) {
            fprintf(stderr, "tiny s=%a x=%a: x/s=%a kernel=%a\n", s, x, want, got);
            return 1;
        }
    }
    return 0;
}

/* OCP E4M3 (no infinities, max 448), round to nearest even, of |v| <= 448. */
static uint8_t e4m3(float v) {
    static float mag[127];
    static int init = 0;
    if (!init) {
        for (int c = 0; c < 127; ++c) {
            const int e = c >> 3, m = c & 7;
            mag[c] = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + m / 8.0f, e - 7);
        }
        init = 1;
    }
    const uint8_t sign = signbit(v) ? 0x80 : 0;
    const float a = fabsf(v);
    int c = 0;
    while (c < 126 && mag[c + 1] <= a) ++c;      /* largest magnitude <= a */
    if (c < 126) {
        const double lo = a - mag[c], hi = mag[c + 1] - a;
        if (hi < lo || (hi == lo && (c & 1))) ++c;
    }
    return sign | (uint8_t)c;
}

static float clamp448(float v) {  /* fmaxf/fminf: NaN -> +448 */
    return fmaxf(-448.0f, fminf(448.0f, v));
}

#define ROW 512
static long fused_rows, fused_fast;

static long check_row(const float* x, const float* s) {
    /* reference: smooth, absmax, row scale, divide, clamp, encode */
    float q[ROW], amax = 0.0f;
    uint8_t want[ROW];
    for (int i = 0; i < ROW; ++i) { q[i] = x[i] / s[i]; amax = fmaxf(amax, fabsf(q[i])); }
    const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
    for (int i = 0; i < ROW; ++i) want[i] = e4m3(clamp448(q[i] / scale));
    /* kernel route */
    float smin = INFINITY;
    int factors_ok = 1;
    for (int i = 0; i < ROW; ++i) {
        if (!(s[i] >= 0x1p-120f && s[i] <= 0x1p120f)) factors_ok = 0;
        smin = fminf(smin, s[i]);
    }
    const uint32_t tlo = f_to_bits(fmaxf(0x1p-60f, 0x1p-81f / smin));
    float k[ROW];
    uint32_t um = 0;
    for (int i = 0; i < ROW; ++i) {
        k[i] = kernel_div(x[i], s[i], 1.0f / s[i]);
        const uint32_t b = f_to_bits(k[i]) & 0x7FFFFFFFu;
        if (b > um) um = b;
    }
    ++fused_rows;
    if (!(factors_ok && um >= tlo && um <= 0x7E800000u)) return 0;  /* exact route */
    ++fused_fast;
    const float sr = bits_to_f(um) / 448.0f, rr = 1.0f / sr;
    if (f_to_bits(sr) != f_to_bits(scale)) {
        fprintf(stderr, "row scale %a, reference %a\n", sr, scale);
        return 1;
    }
    for (int i = 0; i < ROW; ++i) {
        const float y = kernel_div(k[i], sr, rr);
        const uint8_t got = e4m3(fmaxf(-448.0f, fminf(448.0f, y)));  /* NaN-free: the median */
        if (got != want[i]) {
            fprintf(stderr, "x=%a s=%a: code %02x, reference %02x\n", x[i], s[i], got, want[i]);
            return 1;
        }
    }
    return 0;
}

static float random_exp(int lo, int hi) {
    const int ex = lo + (int)(next_u64() % (uint64_t)(hi - lo + 1));
    const float v = ldexpf(1.0f + (float)(next_u64() & 0x7FFFFF) / 8388608.0f, ex);
    return (next_u64() & 1) ? -v : v;
}

static const float kFixed[] = {448.0f / 448.0f,  3.0f / 448.0f, 0x1p-60f / 448.0f,
                               3.40282347e38f / 448.0f, 235.0f / 448.0f, 0x1p-120f,
                               0x1p120f, 1e-5f, 0x1.fffffep-1f, 0x1.000002p+0f,
                               0x1.5555p-3f, 0x1.234567p-100f};

int main(int argc, char** argv) {
    const int mode = argc > 1 ? atoi(argv[1]) : 0;
    const long n = argc > 2 ? atol(argv[2]) : 64;
    rng_state = argc > 3 ? strtoull(argv[3], NULL, 10) : 1;
    long bad = 0;
    if (mode == 0) {
        for (long k = 0; k < n; ++k) {
            uint32_t man = (uint32_t)(next_u64() & 0x7FFFFF);
            if (k % 4 == 1) man = 0x7FFFFF;
            if (k % 4 == 2) man = 0;
            float s;
            if (k % 2 == 0) {  /* row scale: absmax exponent in [-60, 127] */
                const int ex = -60 + (int)(next_u64() % 188);
                float absmax = bits_to_f(((uint32_t)(ex + 127) << 23) | man);
                if (isinf(absmax)) absmax = 3.40282347e38f;
                s = absmax / 448.0f;
            } else {           /* smoothing factor in [2^-120, 2^120] */
                const int ex = -120 + (int)(next_u64() % 240);
                s = bits_to_f(((uint32_t)(ex + 127) << 23) | man);
            }
            for (long i = 0; i < 65536; ++i) {
                const uint64_t u = next_u64();
                float x;
                switch (i & 3) {
                    case 0: x = bits_to_f((uint32_t)u); break;                          /* any pattern */
                    case 1: x = s * 448.0f * (float)((int64_t)(u % 2000001) - 1000000) * 1e-6f; break;
                    case 2: x = ldexpf(1.0f + (float)(u & 0xFFFFF) / 1048576.0f,
                                       (int)((u >> 20) % 140) - 140) * ((u >> 40) & 1 ? -1.0f : 1.0f);
                            break;                                                         /* near 2^-102 */
                    default: x = bits_to_f(f_to_bits(s) + (uint32_t)(u % 64)) * ((u >> 8) & 1 ? -1.0f : 1.0f);
                }
                bad += check(x, s);
            }
            const float edge[] = {0.0f, -0.0f, 0x1p-102f, -0x1p-102f, 0x1p-103f, -0x1p-103f,
                                  0x1.fffffep-103f, 0x1p-149f, -0x1p-149f, 0x1p-126f};
            for (unsigned i = 0; i < sizeof(edge) / sizeof(edge[0]); ++i) bad += check(edge[i], s);
        }
    } else if (mode == 1) {
        const float s = kFixed[n % (long)(sizeof(kFixed) / sizeof(kFixed[0]))];
#pragma omp parallel for reduction(+ : bad) schedule(static)
        for (int64_t hi = 0; hi < 65536; ++hi)
            for (uint32_t lo = 0; lo < 65536; ++lo)
                bad += check(bits_to_f(((uint32_t)hi << 16) | lo), s);
    } else if (mode == 3) {
        float bound[130];
        int nb = 0;
        e4m3(0.0f);  /* builds the magnitude table before the threads start */
        bound[nb++] = 0x1p-10f;
        {
            float prev = 0x1p-9f;
            for (int c = 2; c < 127; ++c) {
                const int e = c >> 3, m = c & 7;
                const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + m / 8.0f, e - 7);
                bound[nb++] = 0.5f * (prev + v);  /* exact: at most 5 significant bits */
                prev = v;
            }
        }
        long bits_bad = 0;
#pragma omp parallel for reduction(+ : bad, bits_bad) schedule(dynamic, 4096)
        for (int64_t man = 0; man < (1 << 23); ++man) {
            const float s = bits_to_f(0x3F800000u | (uint32_t)man);
            const float r = 1.0f / s;
            for (int b = 0; b < nb; ++b) {
                const uint32_t x0 = f_to_bits(bound[b] * s);
                for (int d = -4; d <= 4; ++d)
                    for (int sg = 0; sg < 2; ++sg) {
                        const float x = bits_to_f((x0 + (uint32_t)d) | (sg ? 0x80000000u : 0u));
                        const float want = x / s, got = kernel_div(x, s, r);
                        if (f_to_bits(want) != f_to_bits(got)) {
                            ++bits_bad;
                            if (e4m3(clamp448(want)) != e4m3(clamp448(got))) {
                                if (bad < 10) fprintf(stderr, "s=%a x=%a: codes differ\n", s, x);
                                ++bad;
                            }
                        }
                    }
            }
        }
        fprintf(stderr, "boundaries %d, checks %lld, quotient-bit differences %ld\n", nb,
                (long long)(1 << 23) * nb * 18, bits_bad);
        bad += bits_bad;
    } else if (mode == 4) {
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 4096)
        for (int64_t man = 0; man < (1 << 23); ++man) {
            const float s = bits_to_f(0x3F800000u | (uint32_t)man);
            uint64_t st = (uint64_t)man * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull;
            for (long i = 0; i < n; ++i) {
                st += 0x9E3779B97F4A7C15ull;
                uint64_t z = st;
                z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
                z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
                z ^= z >> 31;
                /* exponent of x in [-101, 126]: x/s stays normal, |x| >= 2^-102 */
                const uint32_t ex = 26u + (uint32_t)((z >> 32) % 228u);
                const float x = bits_to_f(((uint32_t)(z >> 63) << 31) | (ex << 23) | ((uint32_t)z & 0x7FFFFFu));
                bad += check(x, s);
            }
        }
    } else {
        float x[ROW], s[ROW];
        for (long k = 0; k < n; ++k) {
            const int kind = (int)(k % 8);
            /* factors: the SmoothQuant range, or wide but inside [2^-120, 2^120] */
            const int slo = kind < 4 ? -17 : -119, shi = kind < 4 ? 10 : 119;
            for (int i = 0; i < ROW; ++i) s[i] = fabsf(random_exp(slo, shi));
            if (k % 16 == 13) s[next_u64() % ROW] = 0x1p-121f;  /* outside: exact route */
            int xlo = -20, xhi = 10;
            switch (kind) {
                case 1: xlo = -149; xhi = -90; break;
                case 2: xlo = -140; xhi = 20; break;
                case 3: xlo = -70; xhi = -50; break;
                case 5: xlo = -149; xhi = 127; break;
                case 6: xlo = -110; xhi = -95; break;
                default: break;
            }
            for (int i = 0; i < ROW; ++i) {
                const uint64_t u = next_u64();
                if (u % 50 == 0) x[i] = (u >> 8) & 1 ? -0.0f : 0.0f;
                else if (u % 53 == 0) x[i] = bits_to_f((uint32_t)next_u64() & 0x807FFFFFu);  /* subnormal */
                else if (u % 97 == 0) x[i] = random_exp(-110, -100);
                else x[i] = random_exp(xlo, xhi);
                if (kind == 2 || kind == 5) x[i] = bits_to_f(f_to_bits(x[i]) & 0xFFFF0000u);  /* bf16 */
            }
            if (k % 16 == 9) x[next_u64() % ROW] = NAN;
            if (k % 16 == 11) x[next_u64() % ROW] = -INFINITY;
            bad += check_row(x, s);
        }
        /* the route must be exercised, not skipped */
        if (fused_fast * 4 < fused_rows) {
            fprintf(stderr, "only %ld of %ld rows took the Markstein route\n", fused_fast, fused_rows);
            ++bad;
        }
    }
    printf("mismatches %ld\n", bad);
    return bad != 0;
}
