/*
 * kc_oracle.h -- CPU restatement of kernel-craft's quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only as the checker (or, for bench.py, as the timed CPU baseline).
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the kernel-craft repository root).  Functions marked
 * "extension" have no reference code; their definition is this file.
 *
 * Conventions: rows = N (weight output features / tokens), cols = K.
 * All sizes are int64_t so the oracle itself never overflows.
 */
#ifndef KC_ORACLE_H
#define KC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
int      kco_sext4(unsigned nibble);            /* quant_int4.cu:34-48 */
uint8_t  kco_e4m3_encode(float f);              /* OCP OFP8 E4M3, RNE, satfinite */
float    kco_e4m3_decode(uint8_t code);         /* OCP OFP8 E4M3 -> fp32, exact */
float    kco_bf16_to_f32(uint16_t h);
uint16_t kco_f32_to_bf16(float f);              /* round-to-nearest-even */
/* Count mismatches between `codes[i]` and the product's clamp+encode of the
 * fp32 bit pattern (start + i), i.e. E4M3(fmaxf(-448, fminf(448, x))). */
uint64_t kco_e4m3_sweep_mismatches(uint32_t start, uint64_t count,
                                   const uint8_t* codes, uint32_t* first_bad);

/* ---- INT4 (quant_int4.cu) --------------------------------------------- */
void kco_dequantize_int4(const uint8_t* packed, const float* scales,
                         const uint8_t* zeros, float* out,
                         int64_t rows, int64_t cols, int64_t group_size);
/* the shuffled layout of the matrix-core GEMMs: [ceil(rows/16)*16, cols/2]
 * bytes, a permutation of 16-byte units plus zero pad rows (cols % 128 == 0) */
void kco_shuffle_int4_mfma(const uint8_t* packed, uint8_t* out, int64_t rows, int64_t cols);
/* fp64 dot of the reference's fp32-dequantized weights with x (truth) */
void kco_gemv_int4_f64(const uint8_t* packed, const float* scales,
                       const uint8_t* zeros, const float* x, double* y,
                       int64_t rows, int64_t cols, int64_t group_size);
/* the reference GPU kernel's own fp32 order: 256 strided FMA partials,
 * then the shared-memory tree (quant_int4.cu:140-174) */
void kco_gemv_int4_refkernel_f32(const uint8_t* packed, const float* scales,
                                 const uint8_t* zeros, const float* x, float* y,
                                 int64_t rows, int64_t cols, int64_t group_size);
/* extension: bf16 activations [M, K] -> fp64 truth [M, N] (per-row GEMV) */
void kco_gemm_int4_bf16_f64(const uint8_t* packed, const float* scales,
                            const uint8_t* zeros, const uint16_t* x, double* y,
                            int64_t m, int64_t rows, int64_t cols,
                            int64_t group_size);
/* single-threaded scalar GEMV used as the timed CPU baseline */
void kco_gemv_int4_bf16_f32(const uint8_t* packed, const float* scales,
                            const uint8_t* zeros, const uint16_t* x, float* y,
                            int64_t rows, int64_t cols, int64_t group_size);

/* ---- FP8 (fp8_quant.cu) ----------------------------------------------- */
void kco_quantize_fp8_per_token(const float* in, int8_t* out, float* scales,
                                int64_t rows, int64_t cols);
void kco_quantize_fp8_per_tensor(const float* in, int8_t* out, float scale,
                                 int64_t count);
void kco_dequantize_fp8(const int8_t* in, const float* scales, float* out,
                        int64_t rows, int64_t cols, int per_token);
void kco_smoothquant_scale(const float* in, const float* smooth, float* out,
                           int64_t rows, int64_t cols);

/* ---- extensions (no reference code; defined here) --------------------- */
void kco_quantize_fp8_per_token_bf16(const uint16_t* in, int8_t* out,
                                     float* scales, int64_t rows, int64_t cols);
void kco_col_absmax_f32(const float* in, float* amax, int64_t rows, int64_t cols);
void kco_col_absmax_bf16(const uint16_t* in, float* amax, int64_t rows,
                         int64_t cols);
void kco_smooth_factors(const float* amax_x, const float* amax_w, float* s,
                        int64_t cols);
void kco_quantize_fp8_smooth_div_f32(const float* in, const float* s,
                                     int8_t* out, float* scales,
                                     int64_t rows, int64_t cols);
void kco_quantize_fp8_smooth_div_bf16(const uint16_t* in, const float* s,
                                      int8_t* out, float* scales,
                                      int64_t rows, int64_t cols);
void kco_quantize_fp8_smooth_mul_bf16(const uint16_t* in, const float* s,
                                      int8_t* out, float* scales,
                                      int64_t rows, int64_t cols);

/* RMSNorm (tests/test_mamba_ops.cpp:89-101, rmsnorm.cu:40-70). */
void kco_rmsnorm_f32(const float* x, const float* g, float* y, int64_t rows,
                     int64_t D, float eps);
void kco_rmsnorm_bf16(const uint16_t* x, const uint16_t* g, uint16_t* y,
                      int64_t rows, int64_t D, float eps);

/* The same with the sum of squares in the library's fixed order (lane l of
 * 64 takes the 16-byte slots l, l + 64, ... with one FMA per element, then a
 * xor butterfly); row_tmp holds D floats.  Extension. */
void kco_rmsnorm_f32_lanes(const float* x, const float* g, float* y, int64_t rows,
                           int64_t D, float eps);
void kco_rmsnorm_bf16_lanes(const uint16_t* x, const uint16_t* g, uint16_t* y,
                            int64_t rows, int64_t D, float eps, float* row_tmp);
/* Extension: kco_rmsnorm_bf16_lanes then kco_quantize_fp8_per_token_bf16 on
 * its output, per row (row_tmp: D floats, row_y: D bf16 values). */
void kco_rmsnorm_quantize_fp8_bf16(const uint16_t* h, const uint16_t* g, float eps,
                                   int8_t* out, float* scales, int64_t rows, int64_t D,
                                   float* row_tmp, uint16_t* row_y);

/* Multi-threaded CPU baselines: the same rows as kco_gemv_int4_bf16_f32 and
 * kco_quantize_fp8_per_token, split over `threads` OpenMP threads. */
void kco_gemv_int4_bf16_f32_mt(const uint8_t* packed, const float* scales,
                               const uint8_t* zeros, const uint16_t* x, float* y,
                               int64_t rows, int64_t cols, int64_t group_size, int threads);
void kco_quantize_fp8_per_token_mt(const float* in, int8_t* out, float* scales,
                                   int64_t rows, int64_t cols, int threads);
/* Row splits used by the full-size GPU parity tests: the same rows as
 * kco_quantize_fp8_smooth_{div,mul}_bf16 and the same sums as
 * kco_gemm_int4_bf16_f64 (each output's terms added in k order from 0.0),
 * over `threads` OpenMP threads. */
void kco_quantize_fp8_smooth_div_bf16_mt(const uint16_t* in, const float* s, int8_t* out,
                                         float* scales, int64_t rows, int64_t cols,
                                         int threads);
void kco_quantize_fp8_smooth_mul_bf16_mt(const uint16_t* in, const float* s, int8_t* out,
                                         float* scales, int64_t rows, int64_t cols,
                                         int threads);
void kco_gemm_int4_bf16_f64_mt(const uint8_t* packed, const float* scales,
                               const uint8_t* zeros, const uint16_t* x, double* y,
                               int64_t m, int64_t rows, int64_t cols, int64_t group_size,
                               int threads);

#ifdef __cplusplus
}
#endif
#endif /* KC_ORACLE_H */
