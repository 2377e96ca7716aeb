/*
 * kernel_craft.h -- C ABI of libkernels.so, the MI355X (gfx950) build of
 * kernel-craft's quantized-inference path.
 *
 * Every pointer is a device pointer owned by the caller unless stated
 * otherwise; the library allocates nothing.  `rows` is N (weight output
 * features, or tokens), `cols` is K.  The stream argument is a hipStream_t
 * (an opaque pointer, ABI-identical to the reference's cudaStream_t); 0 is
 * the null stream.
 *
 * Part 1 keeps the reference launchers' names and signatures so that
 * ctypes.CDLL / pybind11 callers of the reference load this library
 * unchanged.  Like the reference they return void and synchronize their
 * stream before returning.  Unlike the reference they validate their
 * arguments: an invalid call launches nothing and records an error that
 * kc_get_last_error() reports (part 2).
 *
 * Part 3 adds entry points that have no reference counterpart (bf16
 * activations, the M>1 MFMA path, fused SmoothQuant, non-blocking variants).
 * They are stream-ordered (they do not synchronize) and return a kc_status.
 *
 * Part 4 exports the reference's out-of-scope launchers as stubs so that the
 * reference's loaders bind every symbol they expect; each stub prints
 * "[kernel-craft-hip stub] <name> not implemented" to stderr and records
 * KC_ERR_NOT_IMPLEMENTED.
 */
#ifndef KERNEL_CRAFT_H
#define KERNEL_CRAFT_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kc_stream_t; /* == hipStream_t */

/* ======================================================================
 * Part 1 -- reference launchers (blocking; void)
 * ==================================================================== */

/* W[n,k] = (float)(sext4(nibble) - zero) * scale.
 * packed [rows, cols/2] u8 (low nibble = even k), scales [rows, cols/gs]
 * fp32, zeros [rows, (cols/gs)/2] u8 (even group -> low nibble, unsigned).
 * Requires cols even and group_size dividing cols.
 * Replaces quant_int4.cu:193-206. */
void launch_dequantize_int4(const uint8_t* d_packed, const float* d_scales,
                            const uint8_t* d_zeros, float* d_output, int rows,
                            int cols, int group_size, kc_stream_t stream);

/* y[n] = sum_k W[n,k] * x[k], dequantizing on the fly; fp32 x and y.
 * Replaces quant_int4.cu:221-234. */
void launch_gemv_int4(const uint8_t* d_packed, const float* d_scales,
                      const uint8_t* d_zeros, const float* d_x, float* d_y,
                      int rows, int cols, int group_size, kc_stream_t stream);

/* FP8 E4M3 (OCP) quantization of fp32 [rows, cols]; codes are int8 bit
 * patterns.  per_token: scales[r] = absmax_r/448 (1 for an all-zero row),
 * written by the call.  Otherwise per-tensor: the call reads the scale from
 * d_scales[0].  q = E4M3_rne(clamp(x / scale, +-448)).
 * Replaces fp8_quant.cu:201-226. */
void launch_quantize_fp8(const float* d_input, int8_t* d_output,
                         float* d_scales, int rows, int cols, bool per_token,
                         kc_stream_t stream);

/* x = decode(code) * scale[row] (per_token) or * scale[0].
 * Replaces fp8_quant.cu:239-253. */
void launch_dequantize_fp8(const int8_t* d_input, const float* d_scales,
                           float* d_output, int rows, int cols, bool per_token,
                           kc_stream_t stream);

/* out[r,c] = in[r,c] / smooth[c].  Replaces fp8_quant.cu:265-278. */
void launch_smoothquant_scale(const float* d_input,
                              const float* d_smooth_scales, float* d_output,
                              int rows, int cols, kc_stream_t stream);

/* y[r,i] = (g[i] * x[r,i]) / sqrt(sum_j x[r,j]^2 / D + eps), fp32 [rows, D].
 * Replaces rmsnorm.cu:83-88; like that launcher (and unlike the others
 * here) it does not synchronize its stream. */
void launch_rmsnorm(const float* d_x, const float* d_g, float* d_y, int rows,
                    int D, float eps, kc_stream_t stream);

/* ======================================================================
 * Part 2 -- error channel (no reference counterpart: the reference's
 * launchers report nothing, quant_int4.cu:205,233, fp8_quant.cu:225)
 * ==================================================================== */

typedef enum kc_status {
    KC_SUCCESS = 0,
    KC_ERR_INVALID_ARGUMENT = 1,
    KC_ERR_NOT_IMPLEMENTED = 2,
    KC_ERR_HIP = 3,
    KC_ERR_UNSUPPORTED_DEVICE = 4
} kc_status;

/* Last error recorded on the calling thread; get_ clears it, peek_ keeps it. */
int kc_get_last_error(void);
int kc_peek_last_error(void);
/* Message of the last error on the calling thread ("" when none). */
const char* kc_last_error_string(void);
/* Library version string. */
const char* kc_version(void);

/* ======================================================================
 * Part 3 -- extensions (stream-ordered, return kc_status)
 * ==================================================================== */

/* Non-blocking launch_gemv_int4: identical arguments and results, no sync. */
int kc_gemv_int4_f32_async(const uint8_t* d_packed, const float* d_scales,
                           const uint8_t* d_zeros, const float* d_x, float* d_y,
                           int rows, int cols, int group_size,
                           kc_stream_t stream);

/* INT4 GEMV with bf16 activation and bf16 output, fp32 accumulation
 * (Llama-3-8B decode shapes).  x [cols] bf16, y [rows] bf16 (RNE). */
int kc_gemv_int4_bf16(const uint8_t* d_packed, const float* d_scales,
                      const uint8_t* d_zeros, const uint16_t* d_x,
                      uint16_t* d_y, int rows, int cols, int group_size,
                      kc_stream_t stream);

/* A decode step's INT4 GEMVs from one call (no counterpart in the
 * reference, whose decode loop calls launch_gemv_int4 once per projection,
 * quant_int4.cu:221-234).  Each op computes what kc_gemv_int4_bf16 computes,
 * in list order, so an op may read what earlier ops wrote (its x may be an
 * earlier op's y).  The list is cut into runs at dependencies (an op that
 * reads an earlier op's y, or writes what it reads or writes, starts a new
 * run); a run of two or more ops with K = 2048 KW (KW 2..8), a power-of-two
 * group of at least 32 and 16-byte aligned weights and x is one launch,
 * every other op its own kc_gemv_int4_bf16 launch.  Every op is validated
 * before the first launch; ops with rows == 0 are skipped. */
#define KC_GEMV_CHAIN_MAX_OPS 8
typedef struct kc_gemv_op {
    const uint8_t* packed;
    const float* scales;
    const uint8_t* zeros;
    const uint16_t* x;
    uint16_t* y;
    int rows, cols, group_size, reserved;
} kc_gemv_op;
int kc_gemv_int4_bf16_chain(const kc_gemv_op* ops, int n_ops, kc_stream_t stream);


/* RMSNorm with bf16 input, weight and output (fp32 arithmetic, output
 * rounded to nearest even): the bf16 counterpart of launch_rmsnorm,
 * rmsnorm.cu:40-70.  x, y [rows, D]; g [D].  Both RMSNorms sum the squares
 * in one fixed order: lane l of 64 accumulates, with one FMA each, the
 * elements i with floor(i / P) mod 64 == l (P = 4 fp32, 8 bf16 values per 16
 * bytes) in increasing i, then the 64 sums meet in a xor butterfly (offsets
 * 32, 16, ..., 1). */
int kc_rmsnorm_bf16(const uint16_t* d_x, const uint16_t* d_g, uint16_t* d_y,
                    int rows, int D, float eps, kc_stream_t stream);

/* The RMSNorm in front of a decoder GEMV, fused into it (no counterpart in
 * the reference, where rmsnorm.cu:83-88 and quant_int4.cu:221-234 are two
 * launches with the normalized vector in memory between them):
 *   y = rms_inv * (W x),  x[k] = bf16(gamma[k] * h[k]),
 *   rms_inv = 1 / sqrt(sum_k h[k]^2 / cols + eps)
 * h, gamma [cols] bf16; y [rows] bf16; W as in kc_gemv_int4_bf16.  The
 * same as kc_rmsnorm_bf16 followed by kc_gemv_int4_bf16 except that the
 * normalization is applied to the fp32 row sums instead of before x is
 * rounded to bf16 (one rounding less). */
int kc_rmsnorm_gemv_int4_bf16(const uint16_t* d_h, const uint16_t* d_gamma,
                              float eps, const uint8_t* d_packed,
                              const float* d_scales, const uint8_t* d_zeros,
                              uint16_t* d_y, int rows, int cols,
                              int group_size, kc_stream_t stream);

/* The RMSNorm in front of an FP8 linear, fused into its per-token
 * quantizer (no counterpart in the reference, where rmsnorm.cu:83-88 and
 * fp8_quant.cu:201-226 are two launches with the normalized rows in memory
 * between them):
 *   y[r, i]   = bf16((gamma[i] * h[r, i]) * rms_inv_r)     (kc_rmsnorm_bf16)
 *   scales[r] = absmax_r(y) / 448 (1 for an all-zero row)
 *   codes     = E4M3_rne(clamp(y / scales[r], +-448))     (kc_quantize_fp8_per_token_bf16)
 * h [rows, D] bf16, gamma [D] bf16, codes [rows, D] int8 bit patterns, scales
 * [rows] fp32.  Bit-identical to kc_rmsnorm_bf16 followed by
 * kc_quantize_fp8_per_token_bf16 on its output.  D == 0 writes nothing. */
int kc_rmsnorm_quantize_fp8_bf16(const uint16_t* d_h, const uint16_t* d_gamma,
                                 float eps, int8_t* d_codes, float* d_scales,
                                 int64_t rows, int64_t D, kc_stream_t stream);

/* GPTQ / AWQ INT4 checkpoints to the layout above (no counterpart in the
 * reference, which only describes its format as GPTQ/AWQ-style,
 * quant_int4.cu:5).  Sources, device pointers:
 *   GPTQ: qweight int32 [K/8, N] (nibble i of word (r, n) = input k 8r+i),
 *         qzeros int32 [K/gs, N/8] (nibble i = column 8c+i, stored minus
 *         zero_offset: 1 for the original AutoGPTQ format, 0 for v2),
 *         scales fp16 [K/gs, N]; perm int32 [K] or NULL: output column j
 *         takes input k = perm[j] (act-order checkpoints: perm sorts k by
 *         g_idx, and the caller applies the same permutation to x).
 *   AWQ:  qweight int32 [K, N/8], qzeros int32 [K/gs, N/8] (nibble i =
 *         column 8c + {0,2,4,6,1,3,5,7}[i]), scales fp16 [K/gs, N].
 * Outputs: packed [N, K/2] u8, scales [N, K/gs] fp32, zeros [N, K/gs/2] u8,
 * dequantizing to exactly (u - zu) * s (groups with zu <= 7 are stored with
 * a negated scale, so their zero weights dequantize to -0).  Requires K, N and group_size
 * multiples of 8, group_size dividing K, and an even K / group_size. */
int kc_convert_gptq_int4(const int32_t* d_qweight, const int32_t* d_qzeros,
                         const uint16_t* d_scales_f16, const int32_t* d_perm,
                         int K, int N, int group_size, int zero_offset,
                         uint8_t* d_packed, float* d_scales, uint8_t* d_zeros,
                         kc_stream_t stream);
int kc_convert_awq_int4(const int32_t* d_qweight, const int32_t* d_qzeros,
                        const uint16_t* d_scales_f16, int K, int N, int group_size,
                        uint8_t* d_packed, float* d_scales, uint8_t* d_zeros,
                        kc_stream_t stream);

/* Small-batch INT4 GEMM on MFMA: Y[m, n] = sum_k X[m,k] W[n,k].
 * X [m, cols] bf16 row-major, Y [m, rows] bf16 row-major, 1 <= m <= 64. */
int kc_gemm_int4_bf16(const uint8_t* d_packed, const float* d_scales,
                      const uint8_t* d_zeros, const uint16_t* d_x,
                      uint16_t* d_y, int m, int rows, int cols, int group_size,
                      kc_stream_t stream);

/* The pre-shuffled INT4 weight layout of the matrix-core kernels (the
 * optional "MFMA-friendly" layout of the weight-format bridge; no
 * counterpart in the reference, whose only layout is quant_int4.cu:10-13).
 * A permutation of the reference layout's 16-byte units: rows in tiles of
 * 16 (the last tile padded with zero rows), K in blocks of 128; block
 * (tile t, k-block T) is the 1 KB at byte (t * cols/128 + T) * 1024, and
 * its 16-byte unit l = 16 kb + i (i < 16, kb < 4) holds bytes
 * 16 kb .. 16 kb + 15 of row 16 t + i's k-block T.  Scales and zeros keep
 * the reference layout.
 *   kc_shuffled_int4_bytes: size of the shuffled buffer of a [rows, cols]
 *     matrix (rows rounded up to 16, times cols / 2), or -1 unless cols is a
 *     multiple of 128.
 *   kc_shuffle_int4_mfma: packed [rows, cols/2] -> that buffer (16-byte
 *     aligned, not overlapping).
 *   kc_gemm_int4_bf16_shuffled: kc_gemm_int4_bf16 on the shuffled weights,
 *     each wave-wide load reading 1 KB of the layout.  For m >= 9, and for
 *     m 2..8 with cols a multiple of 1024 up to 12288, the same kernel as
 *     kc_gemm_int4_bf16 on the same values: bit-identical results.  Other
 *     m 2..8 shapes run the K-split kernel here and the X-resident kernel
 *     on the reference layout (another summation order).  m == 1 runs a matrix-core GEMV when cols = 1024 * KW (KW <= 16), or
 *     cols = 512 * KW (KW <= 16) with rows <= 8192 (four k-blocks per wave);
 *     other cols take the m >= 2 kernel.  Within the bf16 tolerance of the
 *     reference GEMV.  Needs cols % 128 == 0, group_size a power of two
 *     >= 128, 16-byte aligned weights and x; cols == 0 writes Y = 0 and
 *     reads no weights. */
int64_t kc_shuffled_int4_bytes(int64_t rows, int64_t cols);
int kc_shuffle_int4_mfma(const uint8_t* d_packed, uint8_t* d_packed_shuffled,
                         int rows, int cols, kc_stream_t stream);
int kc_gemm_int4_bf16_shuffled(const uint8_t* d_packed_shuffled,
                               const float* d_scales, const uint8_t* d_zeros,
                               const uint16_t* d_x, uint16_t* d_y, int m,
                               int rows, int cols, int group_size,
                               kc_stream_t stream);

/* W8A8 FP8 GEMM (no counterpart in the reference, whose example dequantizes
 * the codes and multiplies in fp32, examples/python/transformer/
 * fp8_quant.py:55-60):  Y[m, n] = sx[m] * sw[n] * sum_k e4m3(qx[m,k]) *
 * e4m3(qw[n,k]).  qx [M, K] per-token codes with scales sx [M], qw [N, K]
 * per-output-channel codes with scales sw [N] (the quantizers below), Y
 * [M, N] row-major bf16 (RNE) or fp32.  K % 16 == 0 (K == 0 writes Y = 0),
 * qx and qw 16-byte aligned. */
int kc_gemm_fp8_w8a8_bf16(const int8_t* d_qx, const float* d_sx, const int8_t* d_qw,
                          const float* d_sw, uint16_t* d_y, int64_t M, int64_t N,
                          int64_t K, kc_stream_t stream);
int kc_gemm_fp8_w8a8_f32(const int8_t* d_qx, const float* d_sx, const int8_t* d_qw,
                         const float* d_sw, float* d_y, int64_t M, int64_t N, int64_t K,
                         kc_stream_t stream);

/* Non-blocking FP8 quantizers (same arithmetic as launch_quantize_fp8). */
int kc_quantize_fp8_per_token_f32(const float* d_input, int8_t* d_output,
                                  float* d_scales, int64_t rows, int64_t cols,
                                  kc_stream_t stream);
int kc_quantize_fp8_per_tensor_f32(const float* d_input, int8_t* d_output,
                                   const float* d_scale, int64_t rows,
                                   int64_t cols, kc_stream_t stream);
/* bf16 input, per row (per token for activations, per output channel for a
 * weight matrix [N, K]). */
int kc_quantize_fp8_per_token_bf16(const uint16_t* d_input, int8_t* d_output,
                                   float* d_scales, int64_t rows, int64_t cols,
                                   kc_stream_t stream);

/* SmoothQuant (alpha = 0.5).  Column absmax of a [rows, cols] tensor;
 * d_amax [cols] is overwritten (the call clears it first). */
int kc_col_absmax_bf16(const uint16_t* d_input, float* d_amax, int64_t rows,
                       int64_t cols, kc_stream_t stream);
int kc_col_absmax_f32(const float* d_input, float* d_amax, int64_t rows,
                      int64_t cols, kc_stream_t stream);
/* s[c] = max(sqrt(amax_x[c]) / sqrt(max(amax_w[c], 1e-5)), 1e-5) */
int kc_smooth_factors(const float* d_amax_x, const float* d_amax_w,
                      float* d_smooth, int64_t cols, kc_stream_t stream);
/* The SmoothQuant statistics of X [tokens, cols] and W [out_features,
 * cols] in one call: d_amax_x, d_amax_w and d_smooth [cols] get exactly what
 * kc_col_absmax_* on X, on W and kc_smooth_factors give, in three launches
 * instead of five (one fill for both maxima, one reduction grid over both
 * tensors).  No counterpart in the reference, which has no SmoothQuant
 * statistics (BASELINE cfg4 defines them). */
int kc_smoothquant_stats_bf16(const uint16_t* d_x, int64_t tokens,
                              const uint16_t* d_w, int64_t out_features,
                              int64_t cols, float* d_amax_x, float* d_amax_w,
                              float* d_smooth, kc_stream_t stream);
int kc_smoothquant_stats_f32(const float* d_x, int64_t tokens,
                             const float* d_w, int64_t out_features,
                             int64_t cols, float* d_amax_x, float* d_amax_w,
                             float* d_smooth, kc_stream_t stream);
/* One pass: X / s, per-row absmax, scale, E4M3.  Bit-identical to
 * launch_smoothquant_scale followed by launch_quantize_fp8(per_token). */
int kc_quantize_fp8_smooth_div_f32(const float* d_input, const float* d_smooth,
                                   int8_t* d_output, float* d_scales,
                                   int64_t rows, int64_t cols,
                                   kc_stream_t stream);
int kc_quantize_fp8_smooth_div_bf16(const uint16_t* d_input,
                                    const float* d_smooth, int8_t* d_output,
                                    float* d_scales, int64_t rows,
                                    int64_t cols, kc_stream_t stream);
/* One pass: W * s (fp32 multiply), per-output-channel absmax, E4M3. */
int kc_quantize_fp8_smooth_mul_bf16(const uint16_t* d_input,
                                    const float* d_smooth, int8_t* d_output,
                                    float* d_scales, int64_t rows,
                                    int64_t cols, kc_stream_t stream);

/* ======================================================================
 * Part 4 -- out-of-scope reference symbols (stubs).  Signatures from the
 * reference files cited; bound by kernel_craft_torch_ops.py:101-168 and
 * pybind_transformer.cpp:36-122.
 * ==================================================================== */

/* flash_attention.cu:177-180 */
void launch_flash_attention(const float* Q, const float* K, const float* V,
                            float* O, int B, int H, int H_kv, int N, int d,
                            bool causal, kc_stream_t stream);
/* paged_attention.cu:135-142 */
void launch_paged_attention(const float* Q, const int* block_table,
                            const float* K_pool, const float* V_pool, float* O,
                            const int* seq_lens, int B, int H, int H_kv, int d,
                            int block_size, int max_blocks, kc_stream_t stream);
/* speculative_decoding.cu:176-186 */
void launch_verify_draft_tokens(const float* d_draft_probs,
                                const float* d_target_probs,
                                const int* d_draft_tokens,
                                const float* d_rand_vals,
                                const float* d_rand_vals2, int* d_accepted,
                                int* d_corrected, int num_tokens,
                                int vocab_size, kc_stream_t stream);
/* speculative_decoding.cu:205-209 */
void launch_compute_prefix_length(const int* d_accepted, int* d_prefix_len,
                                  int num_tokens, kc_stream_t stream);
/* tensor_parallel.cu:93-97, :258-263, :209-211, :235-237 */
void launch_ring_allreduce(float** d_bufs, int count, int num_ranks,
                           kc_stream_t stream);
void launch_allgather(float** d_chunks, float* d_output, int chunk_size,
                      int num_ranks, kc_stream_t stream);
void launch_col_parallel_linear(const float* d_x, const float* d_W, float* d_y,
                                int M, int N_rank, int K, kc_stream_t stream);
void launch_row_parallel_linear(const float* d_x_rank, const float* d_W,
                                float* d_out, int M, int N, int K_rank,
                                kc_stream_t stream);
/* selective_scan.cu:104-109, depthwise_conv1d.cu:84-87 */
void launch_selective_scan(const float* d_u, const float* d_A_log,
                           const float* d_B, const float* d_C,
                           const float* d_delta, float* d_y, int B_, int L,
                           int D, int N_state, kc_stream_t stream);
void launch_depthwise_conv1d(const float* d_x, const float* d_w,
                             const float* d_bias, float* d_y, int B_, int D,
                             int L, int d_conv, kc_stream_t stream);
/* tensor_parallel_nccl.cu:171-198 (the reference's own no-NCCL stubs) */
void nccl_comm_init_all(void** comms, int num_comms, const int* devs);
void nccl_comm_destroy(void* comm);
void nccl_group_start(void);
void nccl_group_end(void);
void launch_ring_allreduce_nccl(void* comm, float* d_buf, int count,
                                kc_stream_t stream);
void launch_allgather_nccl(void* comm, const float* d_sendbuf,
                           float* d_recvbuf, int sendcount, kc_stream_t stream);
int nccl_comm_count(void* comm);     /* returns 0 */
int nccl_comm_user_rank(void* comm); /* returns -1 */

#ifdef __cplusplus
}
#endif
#endif /* KERNEL_CRAFT_H */
