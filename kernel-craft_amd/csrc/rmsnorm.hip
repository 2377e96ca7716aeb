// rmsnorm.hip -- RMSNorm on gfx950 (MI355X), the op in front of a decoder
// layer's first GEMV.
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
// the reference's order.  Rows whose pointers or D are not 16-byte
// granular take a scalar loop with the same arithmetic.
#include "kc_common.hpp"

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
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nslots = D / P;
    const u32x4* xs = reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(row) * D);
    const u32x4* gs = reinterpret_cast<const u32x4*>(g);
    u32x4* ys = reinterpret_cast<u32x4*>(y + static_cast<int64_t>(row) * D);
    u32x4 xv[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int s = lane + j * kWave;
        xv[j] = s < nslots ? __builtin_nontemporal_load(xs + s) : u32x4{0u, 0u, 0u, 0u};
    }
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
            unpack<BF16>(gs[s], gv);
#pragma unroll
            for (int e = 0; e < P; ++e) v[e] = (gv[e] * v[e]) * rms_inv;
            __builtin_nontemporal_store(pack<BF16>(v), ys + s);
        }
    }
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
    float ss = 0.0f;
    for (int i = lane; i < D; i += kWave) {
        const float v = Elem<BF16>::get(x, base + i);
        ss = fmaf(v, v, ss);
    }
    ss = kc::wave_sum(ss);
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
