// fp8_gemm.hip -- W8A8 FP8 GEMM on gfx950 matrix cores: the consumer of the
// FP8 quantizers (fp8_quant.hip).
//
//   Y[m, n] = sx[m] * sw[n] * sum_k e4m3(qx[m, k]) * e4m3(qw[n, k])
//
// qx [M, K] are per-token E4M3 codes of the activations with scales sx [M]
// (kc_quantize_fp8_per_token_* / _smooth_div_*), qw [N, K] per-output-channel
// codes of the weights with scales sw [N] (kc_quantize_fp8_per_token_* /
// _smooth_mul_bf16 on W).  The reference has no FP8 GEMM; its example
// dequantizes the codes and multiplies in fp32
// (examples/python/transformer/fp8_quant.py:55-60), which is what the tests'
// oracle does in fp64.
//
// Products of two E4M3 values are exact in fp32 (4-bit significands), and
// v_mfma_scale_f32_16x16x128_f8f6f4 accumulates them in fp32 (block scales
// fixed at 2^0).  The scales are applied once per output: (acc * sx) * sw.
//
// Tiling.  A 256-thread workgroup computes a 128 x 128 tile of Y; wave w
// owns the 64 x 64 quarter (w / 2, w % 2) as 4 x 4 MFMA tiles of 16 x 16.
// K advances 128 at a time: the workgroup's 128 rows of qx and of qw for the
// step (16 KB each) are staged in LDS, double-buffered, and each wave reads
// its operands from there: lane (i, kb) of an A or B operand holds bytes
// 32 kb .. 32 kb + 31 of row i of the 16-row block -- the same byte slots
// for both operands, so each product pairs equal k.  LDS rows are padded to
// 144 bytes, which spreads a 16-lane phase of 16-byte reads over all banks.
// Workgroups are ordered so that the eight XCDs each sweep a band of
// row tiles, sharing the qx rows in their L2.
#include <algorithm>

#include "kc_common.hpp"

namespace {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kRowPad = 144;                      // LDS bytes per staged row
constexpr int kStage = (kBM + kBN) * kRowPad;     // one buffer: A rows then B rows
constexpr int kE8M0One = 127;                     // block scale 2^0

// 128 rows x 128 bytes of a [rows, K] code matrix into registers: thread t
// loads 16 bytes of row t/8 + 32 q at byte 16 (t % 8), so that 8 lanes read
// one row's 128 contiguous bytes.  Rows or k past the end read as zeros.
__device__ __forceinline__ void load_tile(const int8_t* __restrict__ src, int64_t rows, int64_t K,
                                          int64_t r0, int64_t k0, u32x4 (&v)[4]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t r = r0 + t / 8 + 32 * q;
        const int64_t k = k0 + 16 * (t % 8);
        v[q] = u32x4{0u, 0u, 0u, 0u};
        if (r < rows && k < K)  // K % 16 == 0: a 16-byte piece is all in or all out
            v[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + r * K + k));
    }
}

__device__ __forceinline__ void store_tile(uint8_t* lds, const u32x4 (&v)[4]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x4*>(lds + (t / 8 + 32 * q) * kRowPad + 16 * (t % 8)) = v[q];
}

// Operand of a 16-row block starting at LDS row r0: lane (i, kb) reads
// bytes 32 kb .. 32 kb + 31 of row r0 + i.
__device__ __forceinline__ i32x8 read_operand(const uint8_t* lds, int r0, int lane) {
    const uint8_t* p = lds + (r0 + (lane & 15)) * kRowPad + 32 * (lane >> 4);
    const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16);
    return i32x8{static_cast<int32_t>(lo.x), static_cast<int32_t>(lo.y), static_cast<int32_t>(lo.z),
                 static_cast<int32_t>(lo.w), static_cast<int32_t>(hi.x), static_cast<int32_t>(hi.y),
                 static_cast<int32_t>(hi.z), static_cast<int32_t>(hi.w)};
}

template <bool YBF16>
__global__ __launch_bounds__(kThreads) void gemm_fp8_kernel(
    const int8_t* __restrict__ qx, const float* __restrict__ sx, const int8_t* __restrict__ qw,
    const float* __restrict__ sw, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int tiles_n, int tiles_m) {
    extern __shared__ __align__(16) uint8_t lds[];  // [2][kBM + kBN][kRowPad]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // XCD-aware order: workgroup b runs on XCD b % 8; XCD x takes the
    // (b / 8)-th tile of its contiguous share of the row-major tile list
    // (a bijection for any grid size: XCDs x < nb % 8 get one tile more).
    const int b = blockIdx.x, nb = gridDim.x;
    const int x = b % 8, q = nb / 8, r = nb % 8;
    const int lin = x * q + min(x, r) + b / 8;
    const int tm = lin / tiles_n, tn = lin % tiles_n;
    (void)tiles_m;
    const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int steps = static_cast<int>((K + kBK - 1) / kBK);
    u32x4 ra[4], rb[4];
    load_tile(qx, M, K, m0, 0, ra);
    load_tile(qw, N, K, n0, 0, rb);
    store_tile(lds, ra);
    store_tile(lds + kBM * kRowPad, rb);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        uint8_t* cur = lds + (s & 1) * kStage;
        uint8_t* nxt = lds + ((s + 1) & 1) * kStage;
        const bool more = s + 1 < steps;
        if (more) {
            load_tile(qx, M, K, m0, static_cast<int64_t>(s + 1) * kBK, ra);
            load_tile(qw, N, K, n0, static_cast<int64_t>(s + 1) * kBK, rb);
        }
        i32x8 a[4], bop[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = read_operand(cur, 64 * wm + 16 * i, lane);
#pragma unroll
        for (int j = 0; j < 4; ++j) bop[j] = read_operand(cur + kBM * kRowPad, 64 * wn + 16 * j, lane);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    a[i], bop[j], acc[i][j], 0, 0, 0, kE8M0One, 0, kE8M0One);
        if (more) {
            store_tile(nxt, ra);
            store_tile(nxt + kBM * kRowPad, rb);
        }
        __syncthreads();
    }

    // D layout of a 16 x 16 tile: lane (j, g) holds rows 4g + v, column j.
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        const int64_t n = n0 + 64 * wn + 16 * ni + j;
        if (n >= N) continue;
        const float swn = sw[n];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t m = m0 + 64 * wm + 16 * mi + 4 * g + v;
                if (m >= M) continue;
                const float r = (acc[mi][ni][v] * sx[m]) * swn;
                if constexpr (YBF16) static_cast<uint16_t*>(y)[m * N + n] = kc::f32_to_bf16(r);
                else static_cast<float*>(y)[m * N + n] = r;
            }
        }
    }
}

template <bool YBF16>
int gemm_fp8(const char* fn, const int8_t* qx, const float* sx, const int8_t* qw, const float* sw,
             void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative shape", fn);
    if (M == 0 || N == 0) return KC_SUCCESS;
    if (K % 16 != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: K=%lld must be a multiple of 16", fn,
                             (long long)K);
    if (!qx || !sx || !qw || !sw || !y)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    if (!kc::aligned(qx, 16) || !kc::aligned(qw, 16))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: qx and qw must be 16-byte aligned", fn);
    const int64_t tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
    if (tm * tn > INT32_MAX)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: too many tiles", fn);
    const size_t lds = 2 * static_cast<size_t>(kStage);
    static bool attr_set = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_fp8_kernel<YBF16>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(2 * kStage)) == hipSuccess;
    }();
    if (!attr_set) return kc::set_error(KC_ERR_HIP, "%s: cannot raise the LDS limit", fn);
    gemm_fp8_kernel<YBF16><<<static_cast<unsigned>(tm * tn), kThreads, lds, stream>>>(
        qx, sx, qw, sw, y, M, N, K, static_cast<int>(tn), static_cast<int>(tm));
    return kc::check_launch(fn);
}

}  // namespace

extern "C" int kc_gemm_fp8_w8a8_bf16(const int8_t* d_qx, const float* d_sx, const int8_t* d_qw,
                                     const float* d_sw, uint16_t* d_y, int64_t M, int64_t N,
                                     int64_t K, kc_stream_t stream) {
    return gemm_fp8<true>("kc_gemm_fp8_w8a8_bf16", d_qx, d_sx, d_qw, d_sw, d_y, M, N, K, stream);
}

extern "C" int kc_gemm_fp8_w8a8_f32(const int8_t* d_qx, const float* d_sx, const int8_t* d_qw,
                                    const float* d_sw, float* d_y, int64_t M, int64_t N, int64_t K,
                                    kc_stream_t stream) {
    return gemm_fp8<false>("kc_gemm_fp8_w8a8_f32", d_qx, d_sx, d_qw, d_sw, d_y, M, N, K, stream);
}
