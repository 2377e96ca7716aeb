/*
 * kc_oracle.c -- CPU restatement of kernel-craft's quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the thing
 * measured or shipped (bench.py's cpu_baseline leg times it as the CPU
 * baseline).  Built with gcc -O2 -ffp-contract=off and no fast-math, so every
 * fp32 operation below is one IEEE-754 operation with round-to-nearest-even,
 * as nvcc's defaults give the reference (no --use_fast_math anywhere in the
 * reference's CMakeLists.txt).
 *
 * Reference paths are relative to the kernel-craft repository root.
 *
 * How each function is pinned (see tests/test_oracle.py):
 *   kco_sext4, kco_dequantize_int4   reference KATs tests/test_quant_int4.cpp:35-88
 *                                    and :148-199, test_transformer_bindings.py:185-196
 *                                    (golden fixtures), closed-form invariants.
 *   kco_gemv_int4_*                  reference KATs test_quant_int4.cpp:90-146 and
 *                                    test_triton_kernels.py:76-119 (golden fixtures),
 *                                    numpy float64 matmul, linearity, brute force.
 *   kco_e4m3_encode / _decode        torch.float8_e4m3fn over every fp32 in the
 *                                    clamped domain and the full decode table, plus
 *                                    OCP special cases.
 *   kco_quantize_fp8_*               reference round-trip bounds
 *                                    (test_fp8_quant.cpp:34-71,137-174), zero rows,
 *                                    NaN/inf rows, numpy restatement of the scale.
 *   kco_smoothquant_scale            KAT test_fp8_quant.cpp:99-135, numpy divide.
 *   extensions                       composition identities with the pinned
 *                                    functions above (fused == two-step).
 *   kco_shuffle_int4_mfma            a numpy reshape/transpose restatement of the
 *                                    layout, a bijection check on unit indices, and
 *                                    the GEMMs on both layouts agreeing bit for bit.
 *   kco_rmsnorm_*                    reference KATs test_mamba_ops.cpp:219-300 (glibc
 *                                    srand/rand recipes) and test_mamba_bindings.py:
 *                                    251-290 (golden fixtures); constant rows, scale
 *                                    invariance, rms of the output.
 */
#include "kc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define E4M3_MAX 448.0f /* fp8_quant.cu:31 */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* CUDA's fmaxf/fminf (the reference's, fp8_quant.cu:105,127): a NaN operand,
 * quiet or signaling, is ignored and the other operand returned.  glibc's
 * fmaxf/fminf follow IEEE 754-2008 maxNum instead and return a quiet NaN for a
 * signaling operand, so they are not used.  Signed zeros never meet here (the
 * operands are |x| >= +0 or compared against +-448). */
static inline float cu_fmaxf(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a > b ? a : b;
}
static inline float cu_fminf(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a < b ? a : b;
}

/* quant_int4.cu:34-48: bits 3:0 (or 7:4) sign-extended from 4 bits. */
int kco_sext4(unsigned nibble) {
    nibble &= 0xFu;
    return (nibble & 0x8u) ? (int)nibble - 16 : (int)nibble;
}

/* OCP OFP8 v1.0 E4M3 ("FN"): bias 7, 3 mantissa bits, no infinities,
 * S.1111.111 is NaN, max finite 448 (S.1111.110), min subnormal 2^-9.
 * Round-to-nearest-even; magnitudes above 448 saturate to 448 (satfinite).
 * This is the conversion fp8_quant.cu:73,128 requests from __nv_fp8_e4m3;
 * it is written from the OCP specification, not from any CUDA header. */
uint8_t kco_e4m3_encode(float f) {
    uint32_t u = f2u(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);       /* NaN */
    if (a >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);      /* >= 448 */
    int e = (int)(a >> 23) - 127;
    if (e < -6) {
        /* E4M3 subnormal range: result = RNE(|x| * 2^9) units of 2^-9 */
        if ((a >> 23) == 0) return sign;                        /* fp32 denormal/0 */
        uint32_t m = (a & 0x7FFFFFu) | 0x800000u;               /* |x| = m*2^(e-23) */
        int shift = 14 - e;                                     /* >= 21 */
        if (shift > 24) return sign;                            /* < 0.5 unit */
        uint32_t half = 1u << (shift - 1);
        uint32_t q = (m + half - 1u + ((m >> shift) & 1u)) >> shift;
        return (uint8_t)(sign | q);            /* q == 8 encodes 2^-6 (E=1,M=0) */
    }
    uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);               /* RNE at bit 20 */
    int E = (int)(r >> 23) - 120;                               /* -127 + 7 */
    uint32_t m3 = (r >> 20) & 7u;
    if (E > 15 || (E == 15 && m3 == 7u)) return (uint8_t)(sign | 0x7Eu);
    return (uint8_t)(sign | ((uint32_t)E << 3) | m3);
}

float kco_e4m3_decode(uint8_t c) {
    int E = (c >> 3) & 0xF, M = c & 7;
    float v;
    if (E == 15 && M == 7) v = NAN;
    else if (E == 0) v = ldexpf((float)M, -9);
    else v = ldexpf(1.0f + (float)M / 8.0f, E - 7);
    return (c & 0x80) ? -v : v;
}

float kco_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t kco_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* fp8_quant.cu:126-129: clamp to +-448 (fmaxf/fminf drop NaN in favour of the
 * bound, so NaN becomes +448), then convert. */
static inline uint8_t clamp_encode(float q) {
    q = cu_fmaxf(-E4M3_MAX, cu_fminf(E4M3_MAX, q));
    return kco_e4m3_encode(q);
}

uint64_t kco_e4m3_sweep_mismatches(uint32_t start, uint64_t count,
                                   const uint8_t* codes, uint32_t* first_bad) {
    uint64_t bad = 0;
    uint32_t first = 0;
    for (uint64_t i = 0; i < count; ++i) {
        uint32_t bits = start + (uint32_t)i;
        if (clamp_encode(u2f(bits)) != codes[i]) {
            if (bad == 0) first = bits;
            ++bad;
        }
    }
    if (first_bad) *first_bad = first;
    return bad;
}

/* ---- INT4 ------------------------------------------------------------- */

/* Zero-point of group g of a row: byte zeros[row*(G/2) + g/2] (floor stride),
 * even g -> low nibble, odd g -> high nibble, read unsigned 0..15
 * (quant_int4.cu:93-96 and :152-156). */
static inline int zero_point(const uint8_t* zeros, int64_t row, int64_t G,
                             int64_t g) {
    uint8_t zb = zeros[row * (G / 2) + g / 2];
    return (g % 2 == 0) ? (zb & 0x0F) : (zb >> 4);
}

/* quant_int4.cu:68-105: W[n,k] = (float)(sext4(q) - z) * s, one fp32 rounding. */
void kco_dequantize_int4(const uint8_t* packed, const float* scales,
                         const uint8_t* zeros, float* out,
                         int64_t rows, int64_t cols, int64_t gs) {
    int64_t G = cols / gs;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; 2 * b < cols; ++b) {
            int64_t c0 = 2 * b, c1 = c0 + 1;
            uint8_t p = packed[r * (cols / 2) + b];
            int64_t g0 = c0 / gs, g1 = c1 / gs;
            float s0 = scales[r * G + g0], s1 = scales[r * G + g1];
            int z0 = zero_point(zeros, r, G, g0), z1 = zero_point(zeros, r, G, g1);
            out[r * cols + c0] = (float)(kco_sext4(p) - z0) * s0;
            if (c1 < cols) out[r * cols + c1] = (float)(kco_sext4(p >> 4) - z1) * s1;
        }
    }
}

/* The shuffled layout of the matrix-core kernels (no reference counterpart;
 * the reference has only the layout of quant_int4.cu:10-13): 16-byte unit l
 * (= 16 kb + i) of 1 KB block (tile t, k-block T) at byte (t * cols/128 + T)
 * * 1024 holds bytes 16 kb .. 16 kb + 15 of row 16 t + i's k-block T (64
 * bytes per k-block); rows past `rows` are zero.  cols % 128 == 0. */
void kco_shuffle_int4_mfma(const uint8_t* packed, uint8_t* out, int64_t rows, int64_t cols) {
    const int64_t nT = cols / 128, tiles = (rows + 15) / 16, rbytes = cols / 2;
    for (int64_t t = 0; t < tiles; ++t)
        for (int64_t T = 0; T < nT; ++T)
            for (int l = 0; l < 64; ++l) {
                uint8_t* dst = out + ((t * nT + T) * 64 + l) * 16;
                const int64_t row = 16 * t + (l % 16);
                if (row < rows) memcpy(dst, packed + row * rbytes + 64 * T + 16 * (l / 16), 16);
                else memset(dst, 0, 16);
            }
}

/* One dequantized weight exactly as quant_int4.cu:158-159 forms it. */
static inline float wq(const uint8_t* packed, const float* scales,
                       const uint8_t* zeros, int64_t r, int64_t k,
                       int64_t cols, int64_t gs) {
    int64_t G = cols / gs, g = k / gs;
    uint8_t p = packed[r * (cols / 2) + k / 2];
    int q = (k & 1) ? kco_sext4(p >> 4) : kco_sext4(p);
    return (float)(q - zero_point(zeros, r, G, g)) * scales[r * G + g];
}

void kco_gemv_int4_f64(const uint8_t* packed, const float* scales,
                       const uint8_t* zeros, const float* x, double* y,
                       int64_t rows, int64_t cols, int64_t gs) {
    for (int64_t r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int64_t k = 0; k < cols; ++k)
            acc += (double)wq(packed, scales, zeros, r, k, cols, gs) * (double)x[k];
        y[r] = acc;
    }
}

/* quant_int4.cu:140-174 with nvcc's default FMA contraction of
 * `partial += w * x` (fmaf), 256 strided partials, then the shared tree. */
void kco_gemv_int4_refkernel_f32(const uint8_t* packed, const float* scales,
                                 const uint8_t* zeros, const float* x, float* y,
                                 int64_t rows, int64_t cols, int64_t gs) {
    enum { BLOCK = 256 };
    float part[BLOCK];
    int64_t nbytes = cols / 2;
    for (int64_t r = 0; r < rows; ++r) {
        for (int t = 0; t < BLOCK; ++t) {
            float acc = 0.0f;
            for (int64_t b = t; b < nbytes; b += BLOCK) {
                int64_t c0 = 2 * b;
                float w0 = wq(packed, scales, zeros, r, c0, cols, gs);
                acc = fmaf(w0, x[c0], acc);
                if (c0 + 1 < cols) {
                    float w1 = wq(packed, scales, zeros, r, c0 + 1, cols, gs);
                    acc = fmaf(w1, x[c0 + 1], acc);
                }
            }
            part[t] = acc;
        }
        for (int stride = BLOCK / 2; stride >= 1; stride >>= 1)
            for (int t = 0; t < stride; ++t) part[t] += part[t + stride];
        y[r] = part[0];
    }
}

void kco_gemm_int4_bf16_f64(const uint8_t* packed, const float* scales,
                            const uint8_t* zeros, const uint16_t* x, double* y,
                            int64_t m, int64_t rows, int64_t cols, int64_t gs) {
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t i = 0; i < m; ++i) y[i * rows + r] = 0.0;
        for (int64_t k = 0; k < cols; ++k) {
            double w = (double)wq(packed, scales, zeros, r, k, cols, gs);
            for (int64_t i = 0; i < m; ++i)
                y[i * rows + r] += w * (double)kco_bf16_to_f32(x[i * cols + k]);
        }
    }
}

/* The same sums as kco_gemm_int4_bf16_f64, rows split over `threads` OpenMP
 * threads: each output y[i][r] starts at 0.0 and adds w(r, k) * x(i, k) for
 * k = 0, 1, ... in order, exactly as there (the loops are nested the other
 * way round so that a row's dequantized weights are formed once and x is
 * read contiguously). */
void kco_gemm_int4_bf16_f64_mt(const uint8_t* packed, const float* scales,
                               const uint8_t* zeros, const uint16_t* x, double* y,
                               int64_t m, int64_t rows, int64_t cols, int64_t gs,
                               int threads) {
    double* xd = (double*)malloc((size_t)(m * cols) * sizeof(double));
    if (!xd) return;
    for (int64_t j = 0; j < m * cols; ++j) xd[j] = (double)kco_bf16_to_f32(x[j]);
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        double* wr = (double*)malloc((size_t)cols * sizeof(double));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            if (!wr) continue;
            for (int64_t k = 0; k < cols; ++k) wr[k] = (double)wq(packed, scales, zeros, r, k, cols, gs);
            for (int64_t i = 0; i < m; ++i) {
                const double* xi = xd + i * cols;
                double acc = 0.0;
                for (int64_t k = 0; k < cols; ++k) acc += wr[k] * xi[k];
                y[i * rows + r] = acc;
            }
        }
        free(wr);
    }
    free(xd);
}

void kco_gemv_int4_bf16_f32(const uint8_t* packed, const float* scales,
                            const uint8_t* zeros, const uint16_t* x, float* y,
                            int64_t rows, int64_t cols, int64_t gs) {
    int64_t G = cols / gs;
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* pr = packed + r * (cols / 2);
        float acc = 0.0f;
        for (int64_t k = 0; k < cols; k += 2) {
            int64_t g = k / gs;
            float s = scales[r * G + g];
            int z = zero_point(zeros, r, G, g);
            uint8_t p = pr[k / 2];
            acc += (float)(kco_sext4(p) - z) * s * kco_bf16_to_f32(x[k]);
            acc += (float)(kco_sext4(p >> 4) - z) * s * kco_bf16_to_f32(x[k + 1]);
        }
        y[r] = acc;
    }
}

/* ---- FP8 -------------------------------------------------------------- */

/* fp8_quant.cu:103-107,120-121: absmax over the row with fmaxf from 0 (NaN is
 * dropped by fmaxf), scale = absmax/448 with an IEEE divide, 1 for an all-zero
 * (or all-NaN) row. */
static inline float row_scale(float amax) {
    return (amax > 0.0f) ? (amax / E4M3_MAX) : 1.0f;
}

/* fp8_quant.cu:89-131 */
void kco_quantize_fp8_per_token(const float* in, int8_t* out, float* scales,
                                int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* x = in + r * cols;
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; ++c) amax = cu_fmaxf(amax, fabsf(x[c]));
        float s = row_scale(amax);
        scales[r] = s;
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = (int8_t)clamp_encode(x[c] / s);
    }
}

/* fp8_quant.cu:62-75 (scale supplied by the caller, fp8_quant.cu:215-223) */
void kco_quantize_fp8_per_tensor(const float* in, int8_t* out, float scale,
                                 int64_t count) {
    for (int64_t i = 0; i < count; ++i)
        out[i] = (int8_t)clamp_encode(in[i] / scale);
}

/* fp8_quant.cu:145-160: exact decode times the scale (one fp32 rounding). */
void kco_dequantize_fp8(const int8_t* in, const float* scales, float* out,
                        int64_t rows, int64_t cols, int per_token) {
    for (int64_t r = 0; r < rows; ++r) {
        float s = per_token ? scales[r] : scales[0];
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = kco_e4m3_decode((uint8_t)in[r * cols + c]) * s;
    }
}

/* fp8_quant.cu:174-184 */
void kco_smoothquant_scale(const float* in, const float* smooth, float* out,
                           int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = in[r * cols + c] / smooth[c];
}

/* ---- extensions ------------------------------------------------------- */

/* Per-token quantization of bf16 activations: widen exactly, then
 * fp8_quant.cu:89-131 unchanged. */
void kco_quantize_fp8_per_token_bf16(const uint16_t* in, int8_t* out,
                                     float* scales, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * cols;
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; ++c)
            amax = cu_fmaxf(amax, fabsf(kco_bf16_to_f32(x[c])));
        float s = row_scale(amax);
        scales[r] = s;
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = (int8_t)clamp_encode(kco_bf16_to_f32(x[c]) / s);
    }
}

void kco_col_absmax_f32(const float* in, float* amax, int64_t rows, int64_t cols) {
    for (int64_t c = 0; c < cols; ++c) amax[c] = 0.0f;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            amax[c] = cu_fmaxf(amax[c], fabsf(in[r * cols + c]));
}

void kco_col_absmax_bf16(const uint16_t* in, float* amax, int64_t rows,
                         int64_t cols) {
    for (int64_t c = 0; c < cols; ++c) amax[c] = 0.0f;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            amax[c] = cu_fmaxf(amax[c], fabsf(kco_bf16_to_f32(in[r * cols + c])));
}

/* SmoothQuant factor with alpha = 0.5 (Xiao et al. 2023, eq. 4):
 * s_j = sqrt(max|X_j|) / sqrt(max(max|W_j|, 1e-5)), then s_j = max(s_j, 1e-5),
 * the clamps of the SmoothQuant authors' smooth_lm().  sqrtf and / are the
 * correctly rounded IEEE operations. */
void kco_smooth_factors(const float* amax_x, const float* amax_w, float* s,
                        int64_t cols) {
    for (int64_t c = 0; c < cols; ++c) {
        float v = sqrtf(amax_x[c]) / sqrtf(cu_fmaxf(amax_w[c], 1e-5f));
        s[c] = cu_fmaxf(v, 1e-5f);
    }
}

/* X/s (fp8_quant.cu:183) then per-token quantization (fp8_quant.cu:89-131):
 * the reference's two-launch pipeline, fused. */
void kco_quantize_fp8_smooth_div_f32(const float* in, const float* s,
                                     int8_t* out, float* scales,
                                     int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* x = in + r * cols;
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; ++c) amax = cu_fmaxf(amax, fabsf(x[c] / s[c]));
        float sc = row_scale(amax);
        scales[r] = sc;
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = (int8_t)clamp_encode((x[c] / s[c]) / sc);
    }
}

void kco_quantize_fp8_smooth_div_bf16(const uint16_t* in, const float* s,
                                      int8_t* out, float* scales,
                                      int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * cols;
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; ++c)
            amax = cu_fmaxf(amax, fabsf(kco_bf16_to_f32(x[c]) / s[c]));
        float sc = row_scale(amax);
        scales[r] = sc;
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] =
                (int8_t)clamp_encode((kco_bf16_to_f32(x[c]) / s[c]) / sc);
    }
}

/* W*s (fp32 multiply) then per-output-channel quantization, i.e. the
 * per-token quantizer applied to W's rows. */
void kco_quantize_fp8_smooth_mul_bf16(const uint16_t* in, const float* s,
                                      int8_t* out, float* scales,
                                      int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* w = in + r * cols;
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; ++c)
            amax = cu_fmaxf(amax, fabsf(kco_bf16_to_f32(w[c]) * s[c]));
        float sc = row_scale(amax);
        scales[r] = sc;
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] =
                (int8_t)clamp_encode((kco_bf16_to_f32(w[c]) * s[c]) / sc);
    }
}

/* RMSNorm, the reference's CPU check (tests/test_mamba_ops.cpp:89-101) of
 * rmsnorm.cu:40-70: per row, ss = sum x^2 in index order (one fp32 multiply
 * and one fp32 add per term), rms_inv = 1 / sqrt(ss / D + eps), and
 * y = (g * x) * rms_inv. */
void kco_rmsnorm_f32(const float* x, const float* g, float* y, int64_t rows,
                     int64_t D, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * D;
        float ss = 0.0f;
        for (int64_t i = 0; i < D; ++i) ss += xr[i] * xr[i];
        const float rms_inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (int64_t i = 0; i < D; ++i) y[r * D + i] = g[i] * xr[i] * rms_inv;
    }
}

/* The same with bf16 x, g and y (fp32 arithmetic, y rounded to nearest
 * even): the input the fused RMSNorm -> GEMV hands its GEMV. */
void kco_rmsnorm_bf16(const uint16_t* x, const uint16_t* g, uint16_t* y,
                      int64_t rows, int64_t D, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * D;
        float ss = 0.0f;
        for (int64_t i = 0; i < D; ++i) {
            const float v = kco_bf16_to_f32(xr[i]);
            ss += v * v;
        }
        const float rms_inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (int64_t i = 0; i < D; ++i)
            y[r * D + i] = kco_f32_to_bf16(kco_bf16_to_f32(g[i]) * kco_bf16_to_f32(xr[i]) * rms_inv);
    }
}

/* Sum of squares of one row in the library's fixed order (extension; the
 * reference's kernel sums in its own thread order, rmsnorm.cu:48-62, and its
 * CPU check in index order): lane l in [0, 64) accumulates, with one fused
 * multiply-add each, the elements i with floor(i / P) mod 64 == l in
 * increasing i, where P is the number of values in 16 bytes; the 64 lane sums
 * are then combined by the butterfly p[l] = p[l] + p[l ^ o], o = 32, ..., 1,
 * after which every lane holds the same value. */
static float sumsq_lanes(const float* v, int64_t D, int P) {
    float p[64];
    for (int l = 0; l < 64; ++l) {
        float s = 0.0f;
        for (int64_t slot = l; slot * P < D; slot += 64)
            for (int e = 0; e < P && slot * P + e < D; ++e) {
                const float x = v[slot * P + e];
                s = fmaf(x, x, s);
            }
        p[l] = s;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        float q[64];
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ o];
        memcpy(p, q, sizeof p);
    }
    return p[0];
}

/* kco_rmsnorm_f32 / kco_rmsnorm_bf16 with the sum of squares in the fixed
 * order above (the library's launch_rmsnorm / kc_rmsnorm_bf16); everything
 * else is the same expression: rms_inv = 1 / sqrt(ss / D + eps),
 * y = (g * x) * rms_inv. */
void kco_rmsnorm_f32_lanes(const float* x, const float* g, float* y, int64_t rows,
                           int64_t D, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * D;
        const float rms_inv = 1.0f / sqrtf(sumsq_lanes(xr, D, 4) / (float)D + eps);
        for (int64_t i = 0; i < D; ++i) y[r * D + i] = g[i] * xr[i] * rms_inv;
    }
}

void kco_rmsnorm_bf16_lanes(const uint16_t* x, const uint16_t* g, uint16_t* y,
                            int64_t rows, int64_t D, float eps, float* row_tmp) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * D;
        for (int64_t i = 0; i < D; ++i) row_tmp[i] = kco_bf16_to_f32(xr[i]);
        const float rms_inv = 1.0f / sqrtf(sumsq_lanes(row_tmp, D, 8) / (float)D + eps);
        for (int64_t i = 0; i < D; ++i)
            y[r * D + i] = kco_f32_to_bf16(kco_bf16_to_f32(g[i]) * row_tmp[i] * rms_inv);
    }
}

/* Extension: RMSNorm -> FP8 per-token quantization, defined as the
 * composition kco_rmsnorm_bf16_lanes, then kco_quantize_fp8_per_token_bf16 of
 * its bf16 output, row by row (the library's kc_rmsnorm_quantize_fp8_bf16).
 * row_tmp holds D floats, row_y D bf16 values. */
void kco_rmsnorm_quantize_fp8_bf16(const uint16_t* h, const uint16_t* g, float eps,
                                   int8_t* out, float* scales, int64_t rows, int64_t D,
                                   float* row_tmp, uint16_t* row_y) {
    for (int64_t r = 0; r < rows; ++r) {
        kco_rmsnorm_bf16_lanes(h + r * D, g, row_y, 1, D, eps, row_tmp);
        kco_quantize_fp8_per_token_bf16(row_y, out + r * D, scales + r, 1, D);
    }
}

/* ---- multi-threaded CPU baselines (bench.py's cpu_baseline leg) ---------
 * The same arithmetic as kco_gemv_int4_bf16_f32 and kco_quantize_fp8_per_token
 * (each row computed exactly as there), rows split over `threads` OpenMP
 * threads with a static schedule. */
void kco_gemv_int4_bf16_f32_mt(const uint8_t* packed, const float* scales,
                               const uint8_t* zeros, const uint16_t* x, float* y,
                               int64_t rows, int64_t cols, int64_t gs, int threads) {
    const int64_t G = cols / gs;
    const int64_t chunks = threads > 0 ? threads : 1;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t r0 = rows * c / chunks, r1 = rows * (c + 1) / chunks;
        kco_gemv_int4_bf16_f32(packed + r0 * (cols / 2), scales + r0 * G,
                               zeros + r0 * (G / 2), x, y + r0, r1 - r0, cols, gs);
    }
}

void kco_quantize_fp8_smooth_div_bf16_mt(const uint16_t* in, const float* s, int8_t* out,
                                         float* scales, int64_t rows, int64_t cols,
                                         int threads) {
    const int64_t chunks = threads > 0 ? threads : 1;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t r0 = rows * c / chunks, r1 = rows * (c + 1) / chunks;
        kco_quantize_fp8_smooth_div_bf16(in + r0 * cols, s, out + r0 * cols, scales + r0,
                                         r1 - r0, cols);
    }
}

void kco_quantize_fp8_smooth_mul_bf16_mt(const uint16_t* in, const float* s, int8_t* out,
                                         float* scales, int64_t rows, int64_t cols,
                                         int threads) {
    const int64_t chunks = threads > 0 ? threads : 1;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t r0 = rows * c / chunks, r1 = rows * (c + 1) / chunks;
        kco_quantize_fp8_smooth_mul_bf16(in + r0 * cols, s, out + r0 * cols, scales + r0,
                                         r1 - r0, cols);
    }
}

void kco_quantize_fp8_per_token_mt(const float* in, int8_t* out, float* scales,
                                   int64_t rows, int64_t cols, int threads) {
    const int64_t chunks = threads > 0 ? threads : 1;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t r0 = rows * c / chunks, r1 = rows * (c + 1) / chunks;
        kco_quantize_fp8_per_token(in + r0 * cols, out + r0 * cols, scales + r0, r1 - r0, cols);
    }
}
