// rmsnorm.hip -- RMSNorm on gfx950 (MI355X), the op in front of each
// quantized linear of a decoder layer, and its fusion into the FP8 per-token
// quantizer.
//
// The reference (rmsnorm.cu:40-70) computes, per row x of length D,
//     rms_inv = rsqrtf(sum_i x_i^2 / D + eps),   y_i = g_i * x_i * rms_inv
// with one thread block per row, strided fp32 partial sums and a shared-memory
// tree.  Here one wave owns a row: lane l holds the row's 16-byte slots l,
// l + 64, ... in registers (no second read of x), the sum of squares is a
// wave reduction (no LDS, no barrier), and y is written from the same
// registers.  rms_inv is computed as 1 / sqrtf(...) with IEEE division and
// square root, the expression of the reference's CPU check
// (tests/test_mamba_ops.cpp:89-101); the CUDA kernel's rsqrtf differs from
// it by a few ulp.  The product is evaluated as (g_i * x_i) * rms_inv, in
// the reference's order.
//
// Summation order (every kernel here, so results do not depend on the
// route a shape takes): with P values per 16-byte slot (4 fp32, 8 bf16),
// lane l accumulates, with one FMA each, the squares of the elements i with
// floor(i / P) mod 64 == l in increasing i; the 64 lane sums are then added
// by the butterfly v += v[lane ^ o] for o = 32, 16, 8, 4, 2, 1.  Rows whose
// pointers or D are not 16-byte granular take a scalar loop that visits the
// elements in the same order.
#include <type_traits>

#include "fp8_common.hpp"

namespace {

using kc::kWave;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / kWave;

template <bool BF16>
struct Elem;
template <>
struct Elem<false> {
    using T = float;
    static constexpr int kPerSlot = 4;  // values per 16-byte slot
    __device__ static float get(const float* p, int64_t i) { return p[i]; }
    __device__ static void put(float* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Elem<true> {
    using T = uint16_t;
    static constexpr int kPerSlot = 8;
    __device__ static float get(const uint16_t* p, int64_t i) { return kc::bf16_to_f32(p[i]); }
    __device__ static void put(uint16_t* p, int64_t i, float v) { p[i] = kc::f32_to_bf16(v); }
};

// One 16-byte slot as fp32 values.
template <bool BF16>
__device__ __forceinline__ void unpack(const u32x4 d, float (&v)[Elem<BF16>::kPerSlot]) {
    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
    if constexpr (BF16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = __uint_as_float(w[j]);
    }
}

template <bool BF16>
__device__ __forceinline__ u32x4 pack(const float (&v)[Elem<BF16>::kPerSlot]) {
    uint32_t w[4];
    if constexpr (BF16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = kc::pack_bf16x2(v[2 * j], v[2 * j + 1]);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = __float_as_uint(v[j]);
    }
    return u32x4{w[0], w[1], w[2], w[3]};
}

// Vector path: D a multiple of the slot width, 16-byte aligned rows, at most
// NS slots per lane (D <= NS * 64 * kPerSlot).  Lanes hold their slots across
// the reduction, so x is read once.
template <bool BF16, int NS>
__global__ __launch_bounds__(kThreads) void rmsnorm_wave_kernel(const typename Elem<BF16>::T* __restrict__ x,
                                                                const typename Elem<BF16>::T* __restrict__ g,
                                                                typename Elem<BF16>::T* __restrict__ y,
                                                                int rows, int D, float eps) {
    constexpr int P = Elem<BF16>::kPerSlot;
    // g, staged once per workgroup (its four rows share it) and read at its
    // use rather than re-read from the cache by every row: decode rows
    // (T = 1 / 64, D = 4096 bf16) 3.7 -> 3.4 / 4.6 -> 3.9 us, fp32 4096 x 4096
    // 22.4 -> 21.7 us, 16384 x 8192 bf16 1-2 % slower (91-92 -> 93-94 us).
    // Freeing the registers of the unpacked row across the reduction (5
    // instead of 3 waves per SIMD at NS = 16) measured no faster here.
    __shared__ u32x4 gl[NS * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const bool live = row < rows;
    const int nslots = D / P;
    const u32x4* xs = reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(live ? row : 0) * D);
    const u32x4* gs = reinterpret_cast<const u32x4*>(g);
    u32x4* ys = reinterpret_cast<u32x4*>(y + static_cast<int64_t>(row) * D);
    u32x4 xv[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int s = lane + j * kWave;
        xv[j] = s < nslots ? __builtin_nontemporal_load(xs + s) : u32x4{0u, 0u, 0u, 0u};
    }
    for (int s = threadIdx.x; s < nslots; s += kThreads) gl[s] = gs[s];
    __syncthreads();
    if (!live) return;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        float v[P];
        unpack<BF16>(xv[j], v);
#pragma unroll
        for (int e = 0; e < P; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = kc::wave_sum(ss);
    const float rms_inv = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int s = lane + j * kWave;
        if (s < nslots) {
            float v[P], gv[P];
            unpack<BF16>(xv[j], v);
            unpack<BF16>(gl[s], gv);
#pragma unroll
            for (int e = 0; e < P; ++e) v[e] = (gv[e] * v[e]) * rms_inv;
            __builtin_nontemporal_store(pack<BF16>(v), ys + s);
        }
    }
}

// Sum of squares of a row in the canonical order (see the header): lane
// `lane` of the wave takes the P-element slots lane, lane + 64, ...
template <bool BF16>
__device__ __forceinline__ float row_sumsq_scalar(const typename Elem<BF16>::T* x, int64_t base,
                                                  int D, int lane) {
    constexpr int P = Elem<BF16>::kPerSlot;
    float ss = 0.0f;
    for (int s = lane; s * P < D; s += kWave) {
#pragma unroll
        for (int e = 0; e < P; ++e) {
            const int i = s * P + e;
            if (i < D) {
                const float v = Elem<BF16>::get(x, base + i);
                ss = fmaf(v, v, ss);
            }
        }
    }
    return kc::wave_sum(ss);
}

// Any D and alignment: two passes over the row (the second from the cache).
template <bool BF16>
__global__ __launch_bounds__(kThreads) void rmsnorm_generic_kernel(const typename Elem<BF16>::T* __restrict__ x,
                                                                   const typename Elem<BF16>::T* __restrict__ g,
                                                                   typename Elem<BF16>::T* __restrict__ y,
                                                                   int rows, int D, float eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = static_cast<int64_t>(row) * D;
    const float ss = row_sumsq_scalar<BF16>(x, base, D, lane);
    const float rms_inv = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
    for (int i = lane; i < D; i += kWave)
        Elem<BF16>::put(y, base + i, (Elem<BF16>::get(g, i) * Elem<BF16>::get(x, base + i)) * rms_inv);
}

template <bool BF16>
int rmsnorm(const char* fn, const typename Elem<BF16>::T* x, const typename Elem<BF16>::T* g,
            typename Elem<BF16>::T* y, int rows, int D, float eps, hipStream_t stream) {
    if (rows < 0 || D < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative shape rows=%d D=%d", fn, rows, D);
    if (rows == 0 || D == 0) return KC_SUCCESS;
    if (!x || !g || !y) return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    constexpr int P = Elem<BF16>::kPerSlot;
    const unsigned grid = static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    const bool vec = D % P == 0 && kc::aligned(x, 16) && kc::aligned(g, 16) && kc::aligned(y, 16);
    const int ns = (D / P + kWave - 1) / kWave;
    if (vec && ns <= 4)
        rmsnorm_wave_kernel<BF16, 4><<<grid, kThreads, 0, stream>>>(x, g, y, rows, D, eps);
    else if (vec && ns <= 16)
        rmsnorm_wave_kernel<BF16, 16><<<grid, kThreads, 0, stream>>>(x, g, y, rows, D, eps);
    else
        rmsnorm_generic_kernel<BF16><<<grid, kThreads, 0, stream>>>(x, g, y, rows, D, eps);
    return kc::check_launch(fn);
}

// ---------------------------------------------------------------------------
// RMSNorm -> FP8 per-token quantization in one pass (bf16 h and gamma):
//   y_i          = bf16((gamma_i * h_i) * rms_inv)      as kc_rmsnorm_bf16
//   codes, scale = per-token E4M3 of the row y          as kc_quantize_fp8_per_token_bf16
// rms_inv uses the canonical summation order; y is rounded to bf16 and
// quantized from registers, so the normalized row never goes to memory.
// Every y is a rounded product, so a NaN among them is quiet and the absmax
// (fmaxf from 0) skips it, as the quantizer's does; it then encodes to +448.
// ---------------------------------------------------------------------------

// y of 8 values (one slot) as packed bf16, from h and gamma slots.
__device__ __forceinline__ u32x4 norm_slot(const u32x4 hv, const u32x4 gv, float rms_inv) {
    float v[8], g[8];
    unpack<true>(hv, v);
    unpack<true>(gv, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (g[e] * v[e]) * rms_inv;
    return pack<true>(v);
}

__device__ __forceinline__ float absmax_bf16x8(float m, const u32x4 y) {
    using kc::fp8::absmax4;
    using kc::fp8::bf16x4_to_f32;
    return absmax4(absmax4(m, bf16x4_to_f32(y.x, y.y)), bf16x4_to_f32(y.z, y.w));
}

// Vector path: D % 8 == 0, 16-byte aligned h and gamma, 8-byte aligned codes,
// D <= NS * 512.  One wave per row, lane l holding slots l, l + 64, ...
template <int NS>
__global__ __launch_bounds__(kThreads) void rmsnorm_fp8_wave_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ gamma, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t rows, int D, float eps) {
    using namespace kc::fp8;
    // gamma, staged once per workgroup (its four rows share it): read from
    // LDS at its use instead of held in registers across the reduction.
    __shared__ u32x4 gl[NS * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    const bool live = row < rows;
    const int nslots = D / 8;
    const u32x4* hs = reinterpret_cast<const u32x4*>(h + (live ? row : 0) * D);
    const u32x4* gs = reinterpret_cast<const u32x4*>(gamma);
    u32x4 xv[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int s = lane + j * kWave;
        xv[j] = s < nslots ? __builtin_nontemporal_load(hs + s) : u32x4{0u, 0u, 0u, 0u};
    }
    for (int s = threadIdx.x; s < nslots; s += kThreads) gl[s] = gs[s];
    __syncthreads();
    if (!live) return;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        float v[8];
        unpack<true>(xv[j], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = kc::wave_sum(ss);
    // Register fence: without it the compiler keeps the 8 * NS unpacked
    // values of the sum above alive across the reduction for the
    // normalization below (and the unpacked y across the next one), which
    // took this kernel to 251 VGPRs and 2 waves per SIMD; unpacking again
    // costs one instruction per value (154 VGPRs, 3 waves: 78.4 -> 75.4 us on
    // 16384 x 8192, with gamma from LDS).
#pragma unroll
    for (int j = 0; j < NS; ++j) asm volatile("" : "+v"(xv[j]) :: "memory");
    const float rms_inv = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        // Slots past the row hold h = 0 and give y = 0: no effect on the
        // absmax, and they are not stored.
        const int s = lane + j * kWave;
        const u32x4 g = s < nslots ? gl[s] : u32x4{0u, 0u, 0u, 0u};
        xv[j] = norm_slot(xv[j], g, rms_inv);
        m = absmax_bf16x8(m, xv[j]);
    }
    const RowDiv d = row_div(kc::wave_max(m));
#pragma unroll
    for (int j = 0; j < NS; ++j) asm volatile("" : "+v"(xv[j]));
    if (lane == 0) scales[row] = d.s;
    u32x2* dst = reinterpret_cast<u32x2*>(out + row * D);
    auto emit = [&](auto fast) {
        constexpr bool F = decltype(fast)::value;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int s = lane + j * kWave;
            if (s < nslots) {
                const u32x2 o{e4m3x4_div<F>(bf16x4_to_f32(xv[j].x, xv[j].y), d),
                              e4m3x4_div<F>(bf16x4_to_f32(xv[j].z, xv[j].w), d)};
                __builtin_nontemporal_store(o, dst + s);
            }
        }
    };
    if (d.fast) emit(std::true_type{});
    else emit(std::false_type{});
}

// Any D and alignment: the sum of squares in the canonical order, then two
// passes recomputing y (absmax, codes), all from the row in the cache.
__global__ __launch_bounds__(kThreads) void rmsnorm_fp8_generic_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ gamma, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t rows, int D, float eps) {
    using namespace kc::fp8;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = row * D;
    const float ss = row_sumsq_scalar<true>(h, base, D, lane);
    const float rms_inv = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
    auto y = [&](int i) {
        const float v = (kc::bf16_to_f32(gamma[i]) * kc::bf16_to_f32(h[base + i])) * rms_inv;
        return kc::bf16_to_f32(kc::f32_to_bf16(v));
    };
    float m = 0.0f;
    for (int i = lane; i < D; i += kWave) m = fmaxf(m, fabsf(y(i)));
    const RowDiv d = row_div(kc::wave_max(m));
    if (lane == 0) scales[row] = d.s;
    for (int i = lane; i < D; i += kWave)
        out[base + i] = static_cast<int8_t>(e4m3x1(d.fast ? div_scale<true>(y(i), d)
                                                          : div_scale<false>(y(i), d)));
}

}  // namespace

// rmsnorm.cu:83-88: asynchronous, like the reference's launcher (it does not
// synchronize its stream).
extern "C" void launch_rmsnorm(const float* d_x, const float* d_g, float* d_y, int rows, int D,
                               float eps, kc_stream_t stream) {
    rmsnorm<false>("launch_rmsnorm", d_x, d_g, d_y, rows, D, eps, stream);
}

extern "C" int kc_rmsnorm_bf16(const uint16_t* d_x, const uint16_t* d_g, uint16_t* d_y, int rows,
                               int D, float eps, kc_stream_t stream) {
    return rmsnorm<true>("kc_rmsnorm_bf16", d_x, d_g, d_y, rows, D, eps, stream);
}

extern "C" int kc_rmsnorm_quantize_fp8_bf16(const uint16_t* d_h, const uint16_t* d_gamma,
                                            float eps, int8_t* d_codes, float* d_scales,
                                            int64_t rows, int64_t D, kc_stream_t stream) {
    const char* fn = "kc_rmsnorm_quantize_fp8_bf16";
    if (rows < 0 || D < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative shape rows=%lld D=%lld", fn,
                             (long long)rows, (long long)D);
    if (D > INT32_MAX || rows > (int64_t{INT32_MAX} * kRowsPerBlock))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: rows=%lld D=%lld too large", fn,
                             (long long)rows, (long long)D);
    if (rows == 0 || D == 0) return KC_SUCCESS;
    if (!d_h || !d_gamma || !d_codes || !d_scales)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    const unsigned grid = static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    const int d = static_cast<int>(D);
    const bool vec = D % 8 == 0 && kc::aligned(d_h, 16) && kc::aligned(d_gamma, 16) &&
                     kc::aligned(d_codes, 8);
    const int64_t ns = (D / 8 + kWave - 1) / kWave;
    if (vec && ns <= 4)
        rmsnorm_fp8_wave_kernel<4><<<grid, kThreads, 0, stream>>>(d_h, d_gamma, d_codes, d_scales,
                                                                  rows, d, eps);
    else if (vec && ns <= 8)
        rmsnorm_fp8_wave_kernel<8><<<grid, kThreads, 0, stream>>>(d_h, d_gamma, d_codes, d_scales,
                                                                  rows, d, eps);
    else if (vec && ns <= 16)
        rmsnorm_fp8_wave_kernel<16><<<grid, kThreads, 0, stream>>>(d_h, d_gamma, d_codes,
                                                                   d_scales, rows, d, eps);
    else
        rmsnorm_fp8_generic_kernel<<<grid, kThreads, 0, stream>>>(d_h, d_gamma, d_codes, d_scales,
                                                                  rows, d, eps);
    return kc::check_launch(fn);
}
