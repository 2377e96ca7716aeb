// quant_int4.hip -- INT4 weight dequantization and dequant-on-the-fly GEMV
// for gfx950 (MI355X).
//
// Weight format (the reference's, quant_int4.cu:10-13, 34-48, 93-96):
//   packed [N, K/2] u8   two signed nibbles per byte, low nibble = even k,
//                        each sign-extended to [-8, 7]
//   scales [N, G] fp32   G = K / gs, one scale per group of gs k
//   zeros  [N, G/2] u8   row stride floor(G/2); group g -> byte g/2, even g in
//                        the low nibble; read unsigned 0..15
//   W[n,k] = (sext4(q) - z) * s
//
// Fast path (gs a power of two >= 32, 16-byte aligned rows): every lane owns
// 16-byte chunks (32 nibbles) of a row, which lie inside one group.  Using
// n' = q ^ 8 = sext4(q) + 8 in [0, 15]:
//     sum_k W x = s * (sum_k n' x - (8 + z) * sum_k x)        per chunk
// The per-chunk sum of x is computed once per workgroup while x is staged in
// LDS.  With bf16 x each nibble becomes the exact bf16 (128 + n') by one
// bitwise op, ((d ^ 0x00080008) & 0x000F000F) | 0x43004300 (v_bitop3_b32), and
// pairs of them meet pairs of x in v_dot2_f32_bf16 (exact products, fp32
// accumulation); the extra 128 * sum x is removed with the zero point.  With
// fp32 x (the reference ABI) each nibble goes through v_cvt_f32_ubyteN and an
// fp32 FMA, so every product is exact before its single rounding.
#include <algorithm>
#include <cstdlib>

#include "kc_common.hpp"

namespace {

using kc::kWave;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;                    // 4 waves per workgroup
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kMaxLdsBytes = 64 * 1024;

__device__ __forceinline__ int sext4(uint32_t v) { return static_cast<int>(v << 28) >> 28; }

// quant_int4.cu:93-96 / :152-156
__device__ __forceinline__ int zero_nibble(const uint8_t* zeros, int64_t row, int64_t G,
                                           int64_t g) {
    const uint32_t zb = zeros[row * (G >> 1) + (g >> 1)];
    return (g & 1) ? static_cast<int>(zb >> 4) : static_cast<int>(zb & 0xFu);
}

template <bool BF16>
__device__ __forceinline__ float load_x(const void* x, int64_t k) {
    if constexpr (BF16) return kc::bf16_to_f32(static_cast<const uint16_t*>(x)[k]);
    else return static_cast<const float*>(x)[k];
}

template <bool BF16>
__device__ __forceinline__ void store_y(void* y, int64_t n, float v) {
    if constexpr (BF16) static_cast<uint16_t*>(y)[n] = kc::f32_to_bf16(v);
    else static_cast<float*>(y)[n] = v;
}

// ---------------------------------------------------------------------------
// Generic GEMV: any even K and any group size dividing K.  One wave per row,
// lanes stride over bytes with the reference's own index arithmetic
// (quant_int4.cu:143-164), dequantizing each weight to fp32 as the reference
// does before the FMA.
// ---------------------------------------------------------------------------
template <bool XBF16, bool YBF16>
__global__ __launch_bounds__(kThreads) void gemv_int4_generic_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const void* __restrict__ x, void* __restrict__ y,
    int64_t rows, int64_t cols, int64_t gs) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t nbytes = cols >> 1;
    const int64_t G = cols / gs;
    const uint8_t* prow = packed + row * nbytes;
    float acc = 0.0f;
    for (int64_t b = lane; b < nbytes; b += kWave) {
        const int64_t c0 = 2 * b;
        const uint32_t p = prow[b];
        const int64_t g0 = c0 / gs, g1 = (c0 + 1) / gs;
        const float w0 =
            static_cast<float>(sext4(p) - zero_nibble(zeros, row, G, g0)) * scales[row * G + g0];
        const float w1 =
            static_cast<float>(sext4(p >> 4) - zero_nibble(zeros, row, G, g1)) * scales[row * G + g1];
        acc = fmaf(w0, load_x<XBF16>(x, c0), acc);
        acc = fmaf(w1, load_x<XBF16>(x, c0 + 1), acc);
    }
    acc = kc::wave_sum(acc);
    if (lane == 0) store_y<YBF16>(y, row, acc);
}

// ---------------------------------------------------------------------------
// Fast GEMV.
//
// LDS holds x for the whole K, split into chunks of 32 k.  A chunk is Q
// 16-byte quads (Q = 4 for bf16, 8 for fp32); quad q of chunk c lives at
// xq[q * cpr + c], so the 64 lanes of a wave, which work on 64 consecutive
// chunks, read 64 consecutive quads (conflict-free ds_read_b128).  For bf16
// the quad of k-block i (k = 8i..8i+7 of the chunk) stores the pairs
// (x0,x4) (x1,x5) (x2,x6) (x3,x7), the order in which the nibble unpack
// below produces weights.  xs[c] is the fp32 sum of the chunk's 32 x.
//
// Each wave owns R consecutive rows and walks their chunks c = lane,
// lane + 64, ... with one 16-byte load per row per step.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t nib_bf16_pair(uint32_t d) {
    // nibbles at bits 0-3 and 16-19 -> bf16 (128 + (q ^ 8)) in each half
    return ((d ^ 0x00080008u) & 0x000F000Fu) | 0x43004300u;
}

// Takes its operand by value: clang miscompiles __builtin_bit_cast applied to
// an element of an ext_vector reached through a reference (every element
// reads offset 0), so vector elements are always copied out first.
__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) {
    return __builtin_bit_cast(bf16x2_t, v);
}

__device__ __forceinline__ float dot8_bf16(uint32_t d, uint32_t x04, uint32_t x15, uint32_t x26,
                                           uint32_t x37, float a) {
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_bf16_pair(d)), as_bf16x2(x04), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_bf16_pair(d >> 4)), as_bf16x2(x15), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_bf16_pair(d >> 8)), as_bf16x2(x26), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_bf16_pair(d >> 12)), as_bf16x2(x37), a, false);
    return a;
}

__device__ __forceinline__ float dot8_f32(uint32_t d, f32x4 xa, f32x4 xb,
                                          float a) {
    const uint32_t o = d ^ 0x88888888u;  // n' = q ^ 8 in every nibble
    const uint32_t L = o & 0x0F0F0F0Fu;  // even k of each byte
    const uint32_t H = (o >> 4) & 0x0F0F0F0Fu;  // odd k
    a = fmaf(static_cast<float>(L & 0xFFu), xa.x, a);
    a = fmaf(static_cast<float>(H & 0xFFu), xa.y, a);
    a = fmaf(static_cast<float>((L >> 8) & 0xFFu), xa.z, a);
    a = fmaf(static_cast<float>((H >> 8) & 0xFFu), xa.w, a);
    a = fmaf(static_cast<float>((L >> 16) & 0xFFu), xb.x, a);
    a = fmaf(static_cast<float>((H >> 16) & 0xFFu), xb.y, a);
    a = fmaf(static_cast<float>(L >> 24), xb.z, a);
    a = fmaf(static_cast<float>(H >> 24), xb.w, a);
    return a;
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

template <bool XBF16>
__device__ __forceinline__ void stage_x(const void* __restrict__ x, u32x4* xq, float* xs,
                                        int cols) {
    const int cpr = cols >> 5;
    const int nblk = cols >> 3;  // multiple of 4, so a chunk's 4 blocks share a quad of lanes
    for (int b = threadIdx.x; b < nblk; b += kThreads) {
        const int c = b >> 2, i = b & 3;
        float part;
        if constexpr (XBF16) {
            const u32x4 d = static_cast<const u32x4*>(x)[b];
            u32x4 p;
            p.x = (d.x & 0xFFFFu) | (d.z << 16);
            p.y = (d.x >> 16) | (d.z & 0xFFFF0000u);
            p.z = (d.y & 0xFFFFu) | (d.w << 16);
            p.w = (d.y >> 16) | (d.w & 0xFFFF0000u);
            xq[i * cpr + c] = p;
            part = ((bf16_lo(d.x) + bf16_hi(d.x)) + (bf16_lo(d.y) + bf16_hi(d.y))) +
                   ((bf16_lo(d.z) + bf16_hi(d.z)) + (bf16_lo(d.w) + bf16_hi(d.w)));
        } else {
            const f32x4* src = static_cast<const f32x4*>(x) + 2 * b;
            const f32x4 a = src[0], e = src[1];
            xq[(2 * i) * cpr + c] = __builtin_bit_cast(u32x4, a);
            xq[(2 * i + 1) * cpr + c] = __builtin_bit_cast(u32x4, e);
            part = ((a.x + a.y) + (a.z + a.w)) + ((e.x + e.y) + (e.z + e.w));
        }
        part += __shfl_xor(part, 1, kWave);
        part += __shfl_xor(part, 2, kWave);
        if (i == 0) xs[c] = part;
    }
}

template <int R, bool XBF16, bool YBF16>
__global__ __launch_bounds__(kThreads) void gemv_int4_fast_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const void* __restrict__ x, void* __restrict__ y,
    int rows, int cols, int gshift) {
    extern __shared__ u32x4 lds[];
    constexpr int Q = XBF16 ? 4 : 8;
    const int cpr = cols >> 5;
    u32x4* xq = lds;
    float* xs = reinterpret_cast<float*>(lds + Q * cpr);
    stage_x<XBF16>(x, xq, xs, cols);
    __syncthreads();

    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * R;
    if (row0 >= rows) return;
    const int64_t rbytes = cols >> 1;
    const int G = cols >> (5 + gshift);
    const u32x4* prow[R];
    const float* srow[R];
    const uint8_t* zrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t rr = min(row0 + r, rows - 1);  // tail rows re-read the last row
        prow[r] = reinterpret_cast<const u32x4*>(packed + rr * rbytes);
        srow[r] = scales + rr * G;
        zrow[r] = zeros + rr * (G >> 1);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int c = lane; c < cpr; c += kWave) {
        const int g = c >> gshift;
        u32x4 w[R];
        float s[R];
        uint32_t zb[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            w[r] = __builtin_nontemporal_load(prow[r] + c);
            s[r] = srow[r][g];
            zb[r] = zrow[r][g >> 1];
        }
        const float xsum = xs[c];
        if constexpr (XBF16) {
            const u32x4 x0 = xq[c], x1 = xq[cpr + c], x2 = xq[2 * cpr + c], x3 = xq[3 * cpr + c];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t z = (g & 1) ? (zb[r] >> 4) : (zb[r] & 0xFu);
                const u32x4 wr = w[r];
                float a = dot8_bf16(wr.x, x0.x, x0.y, x0.z, x0.w, 0.0f);
                a = dot8_bf16(wr.y, x1.x, x1.y, x1.z, x1.w, a);
                a = dot8_bf16(wr.z, x2.x, x2.y, x2.z, x2.w, a);
                a = dot8_bf16(wr.w, x3.x, x3.y, x3.z, x3.w, a);
                acc[r] = fmaf(s[r], fmaf(-static_cast<float>(136u + z), xsum, a), acc[r]);
            }
        } else {
            f32x4 xf[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const u32x4 v = xq[q * cpr + c];
                xf[q] = __builtin_bit_cast(f32x4, v);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t z = (g & 1) ? (zb[r] >> 4) : (zb[r] & 0xFu);
                const u32x4 wr = w[r];
                float a = dot8_f32(wr.x, xf[0], xf[1], 0.0f);
                a = dot8_f32(wr.y, xf[2], xf[3], a);
                a = dot8_f32(wr.z, xf[4], xf[5], a);
                a = dot8_f32(wr.w, xf[6], xf[7], a);
                acc[r] = fmaf(s[r], fmaf(-static_cast<float>(8u + z), xsum, a), acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = kc::wave_sum(acc[r]);
        if (lane == 0 && row0 + r < rows) store_y<YBF16>(y, row0 + r, v);
    }
}

// ---------------------------------------------------------------------------
// Dequantization to fp32 (quant_int4.cu:68-105): exactly one fp32 rounding,
// (float)(sext4(q) - z) * s.
// ---------------------------------------------------------------------------

// Generic: one byte (two outputs) per thread, reference index arithmetic.
__global__ __launch_bounds__(kThreads) void dequant_int4_generic_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, float* __restrict__ out, int64_t rows, int64_t cols,
    int64_t gs) {
    const int64_t nbytes = cols >> 1;
    const int64_t G = cols / gs;
    const int64_t total = rows * nbytes;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t row = i / nbytes, b = i - row * nbytes;
        const int64_t c0 = 2 * b;
        const uint32_t p = packed[i];
        const int64_t g0 = c0 / gs, g1 = (c0 + 1) / gs;
        out[row * cols + c0] =
            static_cast<float>(sext4(p) - zero_nibble(zeros, row, G, g0)) * scales[row * G + g0];
        out[row * cols + c0 + 1] =
            static_cast<float>(sext4(p >> 4) - zero_nibble(zeros, row, G, g1)) *
            scales[row * G + g1];
    }
}

// Fast: 4 packed bytes -> 8 fp32 (two 16-byte stores) per thread; requires
// K % 8 == 0 and gs % 8 == 0 so the 8 outputs share one group.
__global__ __launch_bounds__(kThreads) void dequant_int4_fast_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, float* __restrict__ out, int64_t rows, int64_t cols,
    int64_t gs) {
    const int64_t bpr = cols >> 3;  // 8-element blocks per row
    const int64_t G = cols / gs;
    const int64_t total = rows * bpr;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t row = i / bpr, blk = i - row * bpr;
        const int64_t g = (blk << 3) / gs;
        const uint32_t d = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(packed) + i);
        const float s = scales[row * G + g];
        const int z = zero_nibble(zeros, row, G, g);
        f32x4 lo, hi;
        lo.x = static_cast<float>(sext4(d) - z) * s;
        lo.y = static_cast<float>(sext4(d >> 4) - z) * s;
        lo.z = static_cast<float>(sext4(d >> 8) - z) * s;
        lo.w = static_cast<float>(sext4(d >> 12) - z) * s;
        hi.x = static_cast<float>(sext4(d >> 16) - z) * s;
        hi.y = static_cast<float>(sext4(d >> 20) - z) * s;
        hi.z = static_cast<float>(sext4(d >> 24) - z) * s;
        hi.w = static_cast<float>(sext4(d >> 28) - z) * s;
        f32x4* o = reinterpret_cast<f32x4*>(out) + 2 * i;
        __builtin_nontemporal_store(lo, o);
        __builtin_nontemporal_store(hi, o + 1);
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

int check_int4_args(const char* fn, const void* packed, const void* scales, const void* zeros,
                    const void* x, const void* y, int64_t rows, int64_t cols, int64_t gs) {
    if (rows < 0 || cols < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative shape rows=%lld cols=%lld",
                             fn, (long long)rows, (long long)cols);
    if (gs <= 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: group_size=%lld must be > 0", fn,
                             (long long)gs);
    if (cols % 2 != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: cols=%lld must be even", fn,
                             (long long)cols);
    if (cols % gs != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                             "%s: group_size=%lld must divide cols=%lld", fn, (long long)gs,
                             (long long)cols);
    if (rows > 0 && (y == nullptr || (cols > 0 && (!packed || !scales || !zeros || !x))))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    return KC_SUCCESS;
}

int rows_per_wave_override() {
    static const int v = [] {
        const char* e = getenv("KC_GEMV_ROWS_PER_WAVE");
        return e ? atoi(e) : 0;
    }();
    return v;
}

template <int R, bool XB, bool YB>
void launch_fast(const uint8_t* packed, const float* scales, const uint8_t* zeros, const void* x,
                 void* y, int rows, int cols, int gshift, size_t lds, hipStream_t stream) {
    const int per_block = kWavesPerBlock * R;
    const unsigned grid = static_cast<unsigned>((rows + per_block - 1) / per_block);
    gemv_int4_fast_kernel<R, XB, YB><<<grid, kThreads, lds, stream>>>(packed, scales, zeros, x, y,
                                                                      rows, cols, gshift);
}

template <bool XB, bool YB>
int gemv_int4(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
              const void* x, void* y, int64_t rows, int64_t cols, int64_t gs,
              hipStream_t stream) {
    int st = check_int4_args(fn, packed, scales, zeros, x, y, rows, cols, gs);
    if (st != KC_SUCCESS) return st;
    if (rows == 0) return KC_SUCCESS;
    const size_t lds =
        static_cast<size_t>(cols >> 5) * ((XB ? 4 : 8) * 16 + 4);
    const bool fast = cols > 0 && gs >= 32 && kc::is_pow2(gs) && lds <= kMaxLdsBytes &&
                      rows <= INT32_MAX && kc::aligned(packed, 16) && kc::aligned(x, 16);
    if (fast) {
        const int gshift = kc::ilog2(gs) - 5;
        int R = rows_per_wave_override();
        if (R != 1 && R != 2 && R != 4 && R != 8) R = 4;
        const int r = static_cast<int>(rows), c = static_cast<int>(cols);
        switch (R) {
            case 1: launch_fast<1, XB, YB>(packed, scales, zeros, x, y, r, c, gshift, lds, stream); break;
            case 2: launch_fast<2, XB, YB>(packed, scales, zeros, x, y, r, c, gshift, lds, stream); break;
            case 8: launch_fast<8, XB, YB>(packed, scales, zeros, x, y, r, c, gshift, lds, stream); break;
            default: launch_fast<4, XB, YB>(packed, scales, zeros, x, y, r, c, gshift, lds, stream); break;
        }
    } else {
        const int64_t grid = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
        if (grid > INT32_MAX)
            return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: rows=%lld too large", fn,
                                 (long long)rows);
        gemv_int4_generic_kernel<XB, YB><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(
            packed, scales, zeros, x, y, rows, cols, gs);
    }
    return kc::check_launch(fn);
}

int dequant_int4(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                 float* out, int64_t rows, int64_t cols, int64_t gs, hipStream_t stream) {
    int st = check_int4_args(fn, packed, scales, zeros, packed, out, rows, cols, gs);
    if (st != KC_SUCCESS) return st;
    if (rows == 0 || cols == 0) return KC_SUCCESS;
    const bool fast = cols % 8 == 0 && gs % 8 == 0 && kc::aligned(packed, 4) &&
                      kc::aligned(out, 16);
    const int64_t work = fast ? rows * (cols >> 3) : rows * (cols >> 1);
    const int64_t blocks = std::min<int64_t>((work + kThreads - 1) / kThreads, 256 * 64);
    if (fast)
        dequant_int4_fast_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(
            packed, scales, zeros, out, rows, cols, gs);
    else
        dequant_int4_generic_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(
            packed, scales, zeros, out, rows, cols, gs);
    return kc::check_launch(fn);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" void launch_dequantize_int4(const uint8_t* d_packed, const float* d_scales,
                                       const uint8_t* d_zeros, float* d_output, int rows,
                                       int cols, int group_size, kc_stream_t stream) {
    if (dequant_int4("launch_dequantize_int4", d_packed, d_scales, d_zeros, d_output, rows, cols,
                     group_size, stream) == KC_SUCCESS)
        kc::sync_stream(stream, "launch_dequantize_int4");
}

extern "C" void launch_gemv_int4(const uint8_t* d_packed, const float* d_scales,
                                 const uint8_t* d_zeros, const float* d_x, float* d_y, int rows,
                                 int cols, int group_size, kc_stream_t stream) {
    if (gemv_int4<false, false>("launch_gemv_int4", d_packed, d_scales, d_zeros, d_x, d_y, rows,
                                cols, group_size, stream) == KC_SUCCESS)
        kc::sync_stream(stream, "launch_gemv_int4");
}

extern "C" int kc_gemv_int4_f32_async(const uint8_t* d_packed, const float* d_scales,
                                      const uint8_t* d_zeros, const float* d_x, float* d_y,
                                      int rows, int cols, int group_size, kc_stream_t stream) {
    return gemv_int4<false, false>("kc_gemv_int4_f32_async", d_packed, d_scales, d_zeros, d_x,
                                   d_y, rows, cols, group_size, stream);
}

extern "C" int kc_gemv_int4_bf16(const uint8_t* d_packed, const float* d_scales,
                                 const uint8_t* d_zeros, const uint16_t* d_x, uint16_t* d_y,
                                 int rows, int cols, int group_size, kc_stream_t stream) {
    return gemv_int4<true, true>("kc_gemv_int4_bf16", d_packed, d_scales, d_zeros, d_x, d_y,
                                 rows, cols, group_size, stream);
}
