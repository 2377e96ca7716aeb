// fp8_quant.hip -- FP8 E4M3 (OCP) quantization for gfx950 (MI355X).
//
// Arithmetic (fp8_quant.cu:62-75, 89-131, 145-160, 174-184), reproduced
// bit for bit:
//   absmax_r = max over the row of |x| (fmaxf from 0: NaN never wins)
//   scale_r  = absmax_r > 0 ? absmax_r / 448 : 1        (IEEE divide)
//   code     = E4M3_rne(fmaxf(-448, fminf(448, x / scale_r)))
// The divide is the compiler's correctly rounded fp32 division (HIP's default;
// this library is never built with fast-math or denormal flushing), and the
// clamp maps NaN to +448 exactly as CUDA's fmaxf/fminf do.  E4M3 encoding is
// gfx950's v_cvt_pk_fp8_f32, which produces OCP E4M3 with round-to-nearest-
// even; after the clamp every input is finite and within +-448.
//
// Per-token kernels read a row once: each thread keeps its slice of the row in
// registers across the absmax reduction, then converts and stores it.
#include <algorithm>
#include <type_traits>

#include "fp8_common.hpp"

namespace {

using kc::kWave;
using namespace kc::fp8;

typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;

// Block-wide max for 256 threads; every thread gets the result.
__device__ __forceinline__ float block_max(float m, float* red) {
    m = kc::wave_max(m);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = m;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Elementwise pre-transform applied before the absmax (SmoothQuant).
enum class Smooth { kNone, kDiv, kMul };

template <Smooth S>
__device__ __forceinline__ f32x4 apply_smooth(f32x4 v, const float* __restrict__ s, int64_t col) {
    if constexpr (S == Smooth::kNone) {
        return v;
    } else {
        const f32x4 f = quiet4(*reinterpret_cast<const f32x4*>(s + col));
        if constexpr (S == Smooth::kDiv)
            return f32x4{v.x / f.x, v.y / f.y, v.z / f.z, v.w / f.w};  // fp8_quant.cu:183
        else
            return f32x4{v.x * f.x, v.y * f.y, v.z * f.z, v.w * f.w};
    }
}

// ---------------------------------------------------------------------------
// Per-row quantizer, fast path.  One 256-thread workgroup per row; thread t
// holds float4 slots t, t+256, ... (NV of them) of the row in registers.
// Requires cols % 4 == 0 (fp32) / cols % 8 == 0 (bf16), 16-byte aligned rows
// and cols <= 1024*NV (fp32) / 2048*NV (bf16).
// ---------------------------------------------------------------------------
template <int NV, Smooth S>
__global__ __launch_bounds__(kThreads) void quant_rows_f32_kernel(
    const float* __restrict__ in, const float* __restrict__ smooth, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t cols) {
    __shared__ float red[kThreads / kWave];
    const int64_t row = blockIdx.x;
    const f32x4* src = reinterpret_cast<const f32x4*>(in + row * cols);
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + row * cols);
    const int n4 = static_cast<int>(cols >> 2);
    f32x4 v[NV];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < n4) {
            v[j] = apply_smooth<S>(quiet4(__builtin_nontemporal_load(src + i)), smooth,
                                   4 * int64_t{i});
            m = absmax4(m, v[j]);
        }
    }
    const RowDiv d = row_div(block_max(m, red));
    if (threadIdx.x == 0) scales[row] = d.s;
    auto emit = [&](auto fast) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int i = threadIdx.x + j * kThreads;
            if (i < n4) __builtin_nontemporal_store(e4m3x4_div<decltype(fast)::value>(v[j], d), dst + i);
        }
    };
    if (d.fast) emit(std::true_type{});
    else emit(std::false_type{});
}

template <int NV, Smooth S>
__global__ __launch_bounds__(kThreads) void quant_rows_bf16_kernel(
    const uint16_t* __restrict__ in, const float* __restrict__ smooth, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t cols) {
    __shared__ float red[kThreads / kWave];
    const int64_t row = blockIdx.x;
    const u32x4* src = reinterpret_cast<const u32x4*>(in + row * cols);  // 8 bf16 per u32x4
    u32x2* dst = reinterpret_cast<u32x2*>(out + row * cols);
    const int n8 = static_cast<int>(cols >> 3);
    f32x4 lo[NV], hi[NV];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < n8) {
            const u32x4 d = __builtin_nontemporal_load(src + i);
            lo[j] = apply_smooth<S>(quiet4(bf16x4_to_f32(d.x, d.y)), smooth, 8 * int64_t{i});
            hi[j] = apply_smooth<S>(quiet4(bf16x4_to_f32(d.z, d.w)), smooth, 8 * int64_t{i} + 4);
            m = absmax4(absmax4(m, lo[j]), hi[j]);
        }
    }
    const RowDiv d = row_div(block_max(m, red));
    if (threadIdx.x == 0) scales[row] = d.s;
    auto emit = [&](auto fast) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int i = threadIdx.x + j * kThreads;
            if (i < n8) {
                u32x2 o;
                o.x = e4m3x4_div<decltype(fast)::value>(lo[j], d);
                o.y = e4m3x4_div<decltype(fast)::value>(hi[j], d);
                __builtin_nontemporal_store(o, dst + i);
            }
        }
    };
    if (d.fast) emit(std::true_type{});
    else emit(std::false_type{});
}

// ---------------------------------------------------------------------------
// Per-row quantizer, one wave per row (rows of up to 4096 fp32 / 8192 bf16).
// Lane l holds 16-byte slots l, l+64, ... (NV of them) of the row in
// registers: the row is read once, its absmax is a wave reduction (no LDS,
// no barrier), and the codes are written from the same registers.  Each wave
// keeps its whole row (up to 16 KB) in flight.  With smoothing the smoothed
// fp32 values are kept instead of the raw input.
// ---------------------------------------------------------------------------
template <int NV, bool BF16, Smooth S>
__global__ __launch_bounds__(kWave) void quant_rows_wave_kernel(
    const void* __restrict__ in, const float* __restrict__ smooth, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t cols) {
    constexpr int kVals = BF16 ? 8 : 4;                 // values per 16-byte slot
    constexpr int kF4 = BF16 ? 2 : 1;                   // float4 per slot
    constexpr bool kKeep = S != Smooth::kNone;          // keep smoothed values
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int nslots = static_cast<int>(cols / kVals);
    const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const char*>(in) +
                                                      row * cols * (BF16 ? 2 : 4));
    u32x4 raw[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = j * kWave + lane;
        raw[j] = __builtin_nontemporal_load(src + (i < nslots ? i : 0));
    }
    auto values = [&](int j, int h) -> f32x4 {  // float4 h of slot j, before smoothing
        const u32x4 d = raw[j];
        if constexpr (BF16) return h == 0 ? bf16x4_to_f32(d.x, d.y) : bf16x4_to_f32(d.z, d.w);
        else return __builtin_bit_cast(f32x4, d);
    };
    f32x4 kept[kKeep ? NV * kF4 : 1];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = j * kWave + lane;
        if (i < nslots) {
#pragma unroll
            for (int h = 0; h < kF4; ++h) {
                const f32x4 v = apply_smooth<S>(quiet4(values(j, h)), smooth,
                                                int64_t{i} * kVals + 4 * h);
                if constexpr (kKeep) kept[j * kF4 + h] = v;
                m = absmax4(m, v);
            }
        }
    }
    const RowDiv d = row_div(kc::wave_max(m));
    if (lane == 0) scales[row] = d.s;
    auto emit = [&](auto fast) {
        constexpr bool F = decltype(fast)::value;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int i = j * kWave + lane;
            if (i >= nslots) continue;
            uint32_t o[kF4];
#pragma unroll
            for (int h = 0; h < kF4; ++h) {
                f32x4 v;
                if constexpr (kKeep) v = kept[j * kF4 + h];
                else v = F ? values(j, h) : quiet4(values(j, h));  // Markstein quiets sNaN itself
                o[h] = e4m3x4_div<F>(v, d);
            }
            if constexpr (BF16)
                __builtin_nontemporal_store(u32x2{o[0], o[1]}, reinterpret_cast<u32x2*>(out + row * cols) + i);
            else
                __builtin_nontemporal_store(o[0], reinterpret_cast<uint32_t*>(out + row * cols) + i);
        }
    };
    if (d.fast) emit(std::true_type{});
    else emit(std::false_type{});
}

// ---------------------------------------------------------------------------
// Row quantizer, persistent (SmoothQuant, and plain per-token rows of 1024
// 16-byte slots): one 256-thread workgroup per row, the
// grid sized to what the device holds at once; workgroup b takes rows b,
// b + G, b + 2G, ...  Thread t owns the 16-byte column slots t, t + 256, ...
// (NV of them).  Its smoothing factors (and, for the division, their
// reciprocals) are loaded once and stay in registers, so the factor vector
// is read once per workgroup instead of once per row; the slots of the next
// P-1 rows are in flight while a row is reduced and written.
//
// Division by the factors (fp8_quant.cu:183) uses the same Markstein step as
// the row scale (markstein() above).  It returns RN(x / s) for |x| >= 2^-102
// and a normal quotient when s lies in [2^-120, 2^120] (then r is normal),
// and a quotient with the sign of x otherwise.  Every inexact finite element
// has |q| and |x / s| below Q = max(2^-101 / s_min, 2^-125).  A row keeps
// these quotients when the maximum of their magnitude bits (an integer
// maximum, so a NaN or an infinity -- which only a non-finite x or an
// overflowing quotient produce -- exceeds every finite value) lies in
// [T, 2^126] with T = max(2^-60, 2^20 Q): the maximum is then an exact
// element, so the row scale is the reference's, and every inexact element is
// below 2^-20 absmax and encodes to +-0 with the sign of x on both routes.
// Such a row has no NaN, so the clamp to +-448 is one median.  Other rows are
// recomputed with IEEE divisions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, kWave)));
    return v;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fminf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

// The smoothing division's exact route for one row (rows that the check
// above rejects): IEEE divisions, as apply_smooth, re-reading the row and the
// factors slot by slot, so that this rare route adds no registers to the
// unrolled fast route.  Every thread of the workgroup calls it.
template <int NV, bool BF16>
__device__ void smooth_div_row_exact(const void* __restrict__ in, const float* __restrict__ smooth,
                                     int8_t* __restrict__ out, float* __restrict__ scales,
                                     int64_t r, int64_t cols, uint32_t* red) {
    constexpr int kVals = BF16 ? 8 : 4;
    constexpr int kF4 = kVals / 4;
    const int tid = threadIdx.x;
    const int nslots = static_cast<int>(cols / kVals);
    const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const char*>(in) +
                                                      r * cols * (BF16 ? 2 : 4));
    auto smoothed = [&](int i, int h) -> f32x4 {
        const u32x4 d = src[i];
        f32x4 x;
        if constexpr (BF16) x = h == 0 ? bf16x4_to_f32(d.x, d.y) : bf16x4_to_f32(d.z, d.w);
        else x = __builtin_bit_cast(f32x4, d);
        return apply_smooth<Smooth::kDiv>(quiet4(x), smooth, int64_t{i} * kVals + 4 * h);
    };
    float m = 0.0f;
#pragma unroll 1
    for (int j = 0; j < NV * kF4; ++j) {  // one float4 at a time
        const int i = tid + (j / kF4) * kThreads;
        if (i >= nslots) break;
        m = absmax4(m, smoothed(i, j % kF4));
    }
    m = kc::wave_max(m);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = __float_as_uint(m);
    __syncthreads();
    const RowDiv d = row_div(__uint_as_float(max(max(red[0], red[1]), max(red[2], red[3]))));
    if (tid == 0) scales[r] = d.s;
    auto emit = [&](auto fast) {
#pragma unroll 1
        for (int j = 0; j < NV * kF4; ++j) {  // one float4 at a time
            const int i = tid + (j / kF4) * kThreads, h = j % kF4;
            if (i >= nslots) break;
            reinterpret_cast<uint32_t*>(out + r * cols + int64_t{i} * kVals)[h] =
                e4m3x4_div<decltype(fast)::value>(smoothed(i, h), d);
        }
    };
    if (d.fast) emit(std::true_type{});
    else emit(std::false_type{});
}

template <int NV, bool BF16, Smooth S, int P, bool FULL>
__global__ __launch_bounds__(kThreads) void quant_rows_smooth_kernel(
    const void* __restrict__ in, const float* __restrict__ smooth, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t rows, int64_t cols) {
    constexpr int kVals = BF16 ? 8 : 4;  // values per 16-byte slot
    constexpr int kF4 = kVals / 4;       // float4 per slot
    constexpr int kWaves = kThreads / kWave;
    constexpr bool kDivide = S == Smooth::kDiv;
    constexpr bool kSmooth = S != Smooth::kNone;
    __shared__ uint32_t red[2][kWaves];  // row maxima, alternating rows
    __shared__ uint32_t red_exact[kWaves];
    __shared__ float red_min[kWaves];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const bool lead = (tid & (kWave - 1)) == 0;
    const int nslots = static_cast<int>(cols / kVals);
    const int64_t grid = gridDim.x;
    const int64_t row_bytes = cols * (BF16 ? 2 : 4);
    auto valid = [&](int j) { return FULL || tid + j * kThreads < nslots; };

    // Factors (quieted, as apply_smooth does) and their reciprocals.
    f32x4 f[kSmooth ? NV * kF4 : 1];
    f32x4 rf[kDivide ? NV * kF4 : 1];
    float smin = __builtin_inff();  // -1 once a factor is outside [2^-120, 2^120]
#pragma unroll
    for (int j = 0; j < (kSmooth ? NV : 0); ++j) {
#pragma unroll
        for (int h = 0; h < kF4; ++h) {
            f32x4 v = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
            if (valid(j))
                v = quiet4(*reinterpret_cast<const f32x4*>(
                    smooth + int64_t{tid + j * kThreads} * kVals + 4 * h));
            f[j * kF4 + h] = v;
            if constexpr (kDivide) {
                rf[j * kF4 + h] = f32x4{1.0f / v.x, 1.0f / v.y, 1.0f / v.z, 1.0f / v.w};
                if (valid(j)) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        smin = v[c] >= 0x1p-120f && v[c] <= 0x1p120f ? fminf(smin, v[c]) : -1.0f;
                }
            }
        }
    }
    uint32_t tlo_bits = 0;  // T above
    bool factors_ok = true;
    if constexpr (kDivide) {
        float m = wave_min(smin);
        if (lead) red_min[wave] = m;
        __syncthreads();
        m = fminf(fminf(red_min[0], red_min[1]), fminf(red_min[2], red_min[3]));
        factors_ok = m > 0.0f;
        tlo_bits = __float_as_uint(fmaxf(0x1p-60f, 0x1p-81f / m));
    }

    auto load_row = [&](u32x4 (&b)[NV], int64_t r) {
        const u32x4* src =
            reinterpret_cast<const u32x4*>(static_cast<const char*>(in) + r * row_bytes);
#pragma unroll
        for (int j = 0; j < NV; ++j)
            b[j] = __builtin_nontemporal_load(src + (valid(j) ? tid + j * kThreads : 0));
    };
    auto values = [](const u32x4& d, int h) -> f32x4 {  // float4 h of a slot
        if constexpr (BF16) return h == 0 ? bf16x4_to_f32(d.x, d.y) : bf16x4_to_f32(d.z, d.w);
        else return __builtin_bit_cast(f32x4, d);
    };
    auto store = [&](int64_t r, int j, const uint32_t (&o)[kF4]) {
        const int i = tid + j * kThreads;
        if constexpr (BF16)
            __builtin_nontemporal_store(u32x2{o[0], o[1]}, reinterpret_cast<u32x2*>(out + r * cols) + i);
        else
            __builtin_nontemporal_store(o[0], reinterpret_cast<uint32_t*>(out + r * cols) + i);
    };
    auto block_max = [&](uint32_t m, uint32_t* slot) {  // of non-negative floats' bits
        m = wave_max_u32(m);
        if (lead) slot[wave] = m;
        __syncthreads();
        return max(max(slot[0], slot[1]), max(slot[2], slot[3]));
    };

    int par = 0;
    auto process = [&](const u32x4 (&b)[NV], int64_t r) {
        f32x4 q[NV * kF4];
        uint32_t um = 0;
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
#pragma unroll
            for (int h = 0; h < kF4; ++h) {
                const f32x4 x = values(b[j], h);
                f32x4 v;
                if constexpr (kDivide) {
                    const f32x4 s = f[j * kF4 + h];
                    const f32x4 rr = rf[j * kF4 + h];
                    v = f32x4{markstein(x.x, s.x, rr.x), markstein(x.y, s.y, rr.y),
                              markstein(x.z, s.z, rr.z), markstein(x.w, s.w, rr.w)};
                    if (valid(j))
                        um = max(max(um, max(abs_bits(v.x), abs_bits(v.y))),
                                 max(abs_bits(v.z), abs_bits(v.w)));
                } else if constexpr (kSmooth) {
                    const f32x4 s = f[j * kF4 + h];
                    v = f32x4{x.x * s.x, x.y * s.y, x.z * s.z, x.w * s.w};  // fp8_quant.cu:183
                    if (valid(j)) m = absmax4(m, v);
                } else {
                    v = quiet4(x);
                    if (valid(j)) m = absmax4(m, v);
                }
                q[j * kF4 + h] = v;
            }
        }
        if constexpr (!kDivide) um = __float_as_uint(m);
        um = block_max(um, red[par]);
        par ^= 1;
        if constexpr (kDivide) {
            if (factors_ok && um >= tlo_bits && um <= 0x7E800000u) {  // 2^126
                const float sr = __uint_as_float(um) / kE4M3Max, rr = 1.0f / sr;
                if (tid == 0) scales[r] = sr;
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    if (!valid(j)) continue;
                    uint32_t o[kF4];
#pragma unroll
                    for (int h = 0; h < kF4; ++h) {
                        const f32x4 v = q[j * kF4 + h];
                        o[h] = e4m3x4_finite(markstein(v.x, sr, rr), markstein(v.y, sr, rr),
                                             markstein(v.z, sr, rr), markstein(v.w, sr, rr));
                    }
                    store(r, j, o);
                }
                return;
            }
            smooth_div_row_exact<NV, BF16>(in, smooth, out, scales, r, cols, red_exact);
        } else {
            const RowDiv d = row_div(__uint_as_float(um));
            if (tid == 0) scales[r] = d.s;
            auto emit = [&](auto fast) {
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    if (!valid(j)) continue;
                    uint32_t o[kF4];
#pragma unroll
                    for (int h = 0; h < kF4; ++h)
                        o[h] = e4m3x4_div<decltype(fast)::value>(q[j * kF4 + h], d);
                    store(r, j, o);
                }
            };
            if (d.fast) emit(std::true_type{});
            else emit(std::false_type{});
        }
    };

    u32x4 buf[P][NV];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int64_t r = blockIdx.x + k * grid;
        if (r < rows) load_row(buf[k], r);
    }
    for (int64_t base = blockIdx.x; base < rows; base += P * grid) {
#pragma unroll
        for (int k = 0; k < P; ++k) {
            const int64_t r = base + k * grid;
            if (r >= rows) break;
            process(buf[k], r);
            const int64_t nr = r + P * grid;
            if (nr < rows) load_row(buf[k], nr);
        }
    }
}

// ---------------------------------------------------------------------------
// Per-row quantizer, generic path: any cols >= 1, any alignment.  Two passes
// over the row (absmax, then quantize), scalar accesses.
// ---------------------------------------------------------------------------
template <bool BF16, Smooth S>
__device__ __forceinline__ float load_elem(const void* in, const float* smooth, int64_t row,
                                           int64_t cols, int64_t c) {
    float v;
    if constexpr (BF16) v = kc::bf16_to_f32(static_cast<const uint16_t*>(in)[row * cols + c]);
    else v = static_cast<const float*>(in)[row * cols + c];
    v = quiet(v);
    if constexpr (S == Smooth::kDiv) v = v / quiet(smooth[c]);
    if constexpr (S == Smooth::kMul) v = v * quiet(smooth[c]);
    return v;
}

template <bool BF16, Smooth S>
__global__ __launch_bounds__(kThreads) void quant_rows_generic_kernel(
    const void* __restrict__ in, const float* __restrict__ smooth, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t cols) {
    __shared__ float red[kThreads / kWave];
    const int64_t row = blockIdx.x;
    float m = 0.0f;
    for (int64_t c = threadIdx.x; c < cols; c += kThreads)
        m = fmaxf(m, fabsf(load_elem<BF16, S>(in, smooth, row, cols, c)));
    const RowDiv d = row_div(block_max(m, red));
    if (threadIdx.x == 0) scales[row] = d.s;
    for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
        const float v = load_elem<BF16, S>(in, smooth, row, cols, c);
        out[row * cols + c] = static_cast<int8_t>(e4m3x1(d.fast ? div_scale<true>(v, d) : div_scale<false>(v, d)));
    }
}

// ---------------------------------------------------------------------------
// Per-tensor quantizer (fp8_quant.cu:62-75).  The scale is read on the device
// from d_scale[0]; the reference copies the same word to the host first
// (fp8_quant.cu:215-219) and passes it by value.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void quant_tensor_f32_kernel(
    const float* __restrict__ in, const float* __restrict__ d_scale, int8_t* __restrict__ out,
    int64_t count, bool vec) {
    const float scale = quiet(*d_scale);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    int64_t done = 0;
    if (vec) {
        const int64_t n4 = count >> 2;
        const f32x4* src = reinterpret_cast<const f32x4*>(in);
        uint32_t* dst = reinterpret_cast<uint32_t*>(out);
        for (int64_t i = tid; i < n4; i += stride) {
            const f32x4 q = quiet4(__builtin_nontemporal_load(src + i));
            __builtin_nontemporal_store(e4m3x4(q.x / scale, q.y / scale, q.z / scale, q.w / scale),
                                        dst + i);
        }
        done = n4 << 2;
    }
    for (int64_t i = done + tid; i < count; i += stride)
        out[i] = static_cast<int8_t>(e4m3x1(quiet(in[i]) / scale));
}

// ---------------------------------------------------------------------------
// Dequantization (fp8_quant.cu:145-160): exact E4M3 decode
// (v_cvt_pk_f32_fp8), times the row's (or the tensor's) scale.
// Grid: one block per (row, 1024-column tile); the row index is uniform.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void dequant_fp8_kernel(
    const int8_t* __restrict__ in, const float* __restrict__ scales, float* __restrict__ out,
    int64_t cols, int64_t tiles_per_row, bool per_token, bool vec) {
    const int64_t row = blockIdx.x / tiles_per_row;
    const int64_t tile = blockIdx.x - row * tiles_per_row;
    const float s = per_token ? scales[row] : scales[0];
    const int64_t c = tile * 1024 + 4 * static_cast<int64_t>(threadIdx.x);
    const int8_t* src = in + row * cols;
    float* dst = out + row * cols;
    if (vec && c + 4 <= cols) {
        const uint32_t q = *reinterpret_cast<const uint32_t*>(src + c);
        const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(q), false);
        const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(q), true);
        __builtin_nontemporal_store(f32x4{a.x * s, a.y * s, b.x * s, b.y * s},
                                    reinterpret_cast<f32x4*>(dst + c));
    } else {
        for (int64_t k = c; k < std::min(c + 4, cols); ++k) {
            const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(static_cast<uint8_t>(src[k])), false);
            dst[k] = a.x * s;
        }
    }
}

// SmoothQuant divide (fp8_quant.cu:174-184): out = in / s[col].
__global__ __launch_bounds__(kThreads) void smooth_div_kernel(
    const float* __restrict__ in, const float* __restrict__ s, float* __restrict__ out,
    int64_t cols, int64_t tiles_per_row, bool vec) {
    const int64_t row = blockIdx.x / tiles_per_row;
    const int64_t tile = blockIdx.x - row * tiles_per_row;
    const int64_t c = tile * 1024 + 4 * static_cast<int64_t>(threadIdx.x);
    const float* src = in + row * cols;
    float* dst = out + row * cols;
    if (vec && c + 4 <= cols) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + c));
        const f32x4 f = *reinterpret_cast<const f32x4*>(s + c);
        __builtin_nontemporal_store(f32x4{v.x / f.x, v.y / f.y, v.z / f.z, v.w / f.w},
                                    reinterpret_cast<f32x4*>(dst + c));
    } else {
        for (int64_t k = c; k < std::min(c + 4, cols); ++k) dst[k] = src[k] / s[k];
    }
}

// ---------------------------------------------------------------------------
// SmoothQuant statistics: column absmax.  Each block reduces a band of
// kAbsmaxRowsPerBlock rows of 256 bf16 (128 fp32) columns in registers and
// folds it into d_amax with an integer atomic max (non-negative fp32 values
// order like their bit patterns; fmaxf from 0 keeps NaN out).  d_amax is
// cleared by a fill kernel first.
// ---------------------------------------------------------------------------
constexpr int kAbsmaxRowsPerBlock = 128;
constexpr int kAbsmaxUnroll = 4;  // row loads in flight per thread

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads)
        p[i] = 0.0f;
}

// A block covers a band of kAbsmaxRowsPerBlock rows and 32 16-byte column
// slots (256 bf16 or 128 fp32 columns).  Thread t reads slot t % 32 of rows
// t / 32, t / 32 + 8, ... (kAbsmaxUnroll loads in flight); the 8 row groups
// are max-reduced in LDS and each column gets one atomicMax per band.
// Measured at cfg4 (X 16384 x 8192, W 28672 x 8192 bf16): 128-row bands
// 42.8 / 74.8 us, 256-row 43.8 / 75.2, 512-row 45.2 / 76.8 (8 loads in
// flight), 64-row 42.8 / 74.6; wider column tiles (64 slots, 1 KB of a row
// per wave) 45-62 us.  A grid-stride form that keeps one column slot per
// thread (each wave reading 1 KB of a row, the grid in address order) ran
// 50-65 us: with few row phases too little is in flight, with many the
// atomics at the end of the kernel cost more than they save.
template <bool BF16>
__device__ __forceinline__ void col_absmax_block(const void* __restrict__ in,
                                                 float* __restrict__ amax, int64_t rows,
                                                 int64_t cols, int64_t tiles_per_band, bool vec,
                                                 int64_t block) {
    constexpr int kVals = BF16 ? 8 : 4;              // columns per 16-byte slot
    constexpr int kTileCols = 32 * kVals;
    __shared__ float red[8][kTileCols];
    const int64_t band = block / tiles_per_band;
    const int64_t tile = block - band * tiles_per_band;
    const int cg = threadIdx.x & 31, rg = threadIdx.x >> 5;
    const int64_t c = tile * kTileCols + cg * kVals;
    const int64_t r0 = band * kAbsmaxRowsPerBlock;
    const int64_t r1 = std::min(r0 + kAbsmaxRowsPerBlock, rows);
    float m[kVals];
#pragma unroll
    for (int k = 0; k < kVals; ++k) m[k] = 0.0f;
    if (vec && c + kVals <= cols) {
        for (int64_t r = r0 + rg; r < r1; r += 8 * kAbsmaxUnroll) {
            u32x4 d[kAbsmaxUnroll];
#pragma unroll
            for (int u = 0; u < kAbsmaxUnroll; ++u) {  // rows past the band re-read its last row
                const int64_t rr = std::min(r + 8 * u, r1 - 1);
                const char* base = static_cast<const char*>(in) + (rr * cols + c) * (BF16 ? 2 : 4);
                d[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base));
            }
#pragma unroll
            for (int u = 0; u < kAbsmaxUnroll; ++u) {
                // quieted: a signaling NaN must not win the max
                if constexpr (BF16) {
                    const f32x4 v0 = quiet4(bf16x4_to_f32(d[u].x, d[u].y));
                    const f32x4 v1 = quiet4(bf16x4_to_f32(d[u].z, d[u].w));
                    m[0] = fmaxf(m[0], fabsf(v0.x));
                    m[1] = fmaxf(m[1], fabsf(v0.y));
                    m[2] = fmaxf(m[2], fabsf(v0.z));
                    m[3] = fmaxf(m[3], fabsf(v0.w));
                    m[4] = fmaxf(m[4], fabsf(v1.x));
                    m[5] = fmaxf(m[5], fabsf(v1.y));
                    m[6] = fmaxf(m[6], fabsf(v1.z));
                    m[7] = fmaxf(m[7], fabsf(v1.w));
                } else {
                    const f32x4 v0 = quiet4(__builtin_bit_cast(f32x4, d[u]));
                    m[0] = fmaxf(m[0], fabsf(v0.x));
                    m[1] = fmaxf(m[1], fabsf(v0.y));
                    m[2] = fmaxf(m[2], fabsf(v0.z));
                    m[3] = fmaxf(m[3], fabsf(v0.w));
                }
            }
        }
    } else {
        // unaligned input, or the partial last slot of a row
        for (int64_t r = r0 + rg; r < r1; r += 8) {
#pragma unroll
            for (int k = 0; k < kVals; ++k) {
                if (c + k >= cols) break;
                float v;
                if constexpr (BF16) v = kc::bf16_to_f32(static_cast<const uint16_t*>(in)[r * cols + c + k]);
                else v = static_cast<const float*>(in)[r * cols + c + k];
                m[k] = fmaxf(m[k], fabsf(quiet(v)));
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kVals; ++k) red[rg][cg * kVals + k] = m[k];
    __syncthreads();
    for (int col = threadIdx.x; col < kTileCols; col += kThreads) {
        const int64_t gc = tile * kTileCols + col;
        if (gc >= cols) break;
        float v = red[0][col];
#pragma unroll
        for (int g = 1; g < 8; ++g) v = fmaxf(v, red[g][col]);
        atomicMax(reinterpret_cast<unsigned int*>(amax) + gc, __float_as_uint(v));
    }
}

template <bool BF16>
__global__ __launch_bounds__(kThreads) void col_absmax_kernel(const void* __restrict__ in,
                                                              float* __restrict__ amax,
                                                              int64_t rows, int64_t cols,
                                                              int64_t tiles_per_band, bool vec) {
    col_absmax_block<BF16>(in, amax, rows, cols, tiles_per_band, vec, blockIdx.x);
}

// Both column maxima of the SmoothQuant statistics in one grid: the first
// blocks_a blocks reduce A (rows_a x cols) into amax_a, the rest B into
// amax_b.  The two tensors' bands share one launch, so B's blocks fill the
// CUs that A's last blocks leave idle.
template <bool BF16>
__global__ __launch_bounds__(kThreads) void col_absmax2_kernel(
    const void* __restrict__ a, float* __restrict__ amax_a, int64_t rows_a, bool vec_a,
    int64_t blocks_a, const void* __restrict__ b, float* __restrict__ amax_b, int64_t rows_b,
    bool vec_b, int64_t cols, int64_t tiles_per_band) {
    const int64_t blk = blockIdx.x;
    if (blk < blocks_a) col_absmax_block<BF16>(a, amax_a, rows_a, cols, tiles_per_band, vec_a, blk);
    else col_absmax_block<BF16>(b, amax_b, rows_b, cols, tiles_per_band, vec_b, blk - blocks_a);
}

// Zeroes p[0, n) and q[0, n).
__global__ __launch_bounds__(kThreads) void fill_zero2_kernel(float* __restrict__ p,
                                                              float* __restrict__ q, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        p[i] = 0.0f;
        q[i] = 0.0f;
    }
}

// s = max(sqrt(ax) / sqrt(max(aw, 1e-5)), 1e-5); sqrtf and / correctly rounded.
__global__ __launch_bounds__(kThreads) void smooth_factor_kernel(const float* __restrict__ ax,
                                                                 const float* __restrict__ aw,
                                                                 float* __restrict__ s,
                                                                 int64_t cols) {
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c < cols;
         c += static_cast<int64_t>(gridDim.x) * kThreads)
        s[c] = fmaxf(sqrtf(ax[c]) / sqrtf(fmaxf(aw[c], 1e-5f)), 1e-5f);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

int check_rows(const char* fn, const void* in, const void* out, const void* scales, int64_t rows,
               int64_t cols) {
    if (rows < 0 || cols < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative shape rows=%lld cols=%lld",
                             fn, (long long)rows, (long long)cols);
    if (rows > INT32_MAX)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: rows=%lld exceeds 2^31-1", fn,
                             (long long)rows);
    if (rows > 0 && cols > 0 && (!scales || !in || !out))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    return KC_SUCCESS;
}

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Rows held by each workgroup of the persistent smoothing quantizer: the one
// being reduced and kSmoothDepth - 1 in flight.  Its grid is a multiple of
// what the device holds at once.  Workgroups that share a CU progress at
// different rates (on cfg4 X the first finished after 22 us, the last after
// 45 us, with the same row counts), so more, shorter workgroups shorten the
// tail, at the cost of one setup per workgroup: loading the factors and,
// for the division, their reciprocals (an IEEE division each).  For the
// multiplication (cfg4 W, 28672 x 8192: 121.9 -> 113.6 us) eight rounds
// pay; for the division (cfg4 X 70.5 against 72.2 us at four rounds) and the
// plain rows (cfg1) two.  More row slots in flight (depth 3-4) measured the
// same or up to 3 % slower.
constexpr int kSmoothDepth = 2;
constexpr int smooth_rounds(Smooth s) { return s == Smooth::kMul ? 8 : 2; }

template <int NV, bool BF16, Smooth S, bool FULL>
int launch_smooth(const char* fn, const void* in, const float* smooth, int8_t* out, float* scales,
                  int64_t rows, int64_t cols, hipStream_t stream) {
    auto kernel = quant_rows_smooth_kernel<NV, BF16, S, kSmoothDepth, FULL>;
    static const int per_cu = [&] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kThreads, 0) != hipSuccess || n < 1)
            n = 1;
        return n;
    }();
    const int64_t grid = std::min<int64_t>(rows, int64_t{smooth_rounds(S)} * per_cu * device_cus());
    kernel<<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(in, smooth, out, scales, rows, cols);
    return kc::check_launch(fn);
}

// Persistent route: rows of 256..1024 16-byte slots with smoothing, and
// rows of exactly 1024 slots (4096 fp32 / 8192 bf16 values) without.  Plain
// per-token rows of 1024 slots measured 7-9 % faster on this route than one
// wave per row (cold inputs, 4096 rows); shorter plain rows were slower.
// Returns false when the shape takes another route.
template <bool BF16, Smooth S>
bool try_smooth_persistent(const char* fn, const void* in, const float* smooth, int8_t* out,
                           float* scales, int64_t rows, int64_t cols, hipStream_t stream, int* st) {
    {
        const int64_t nslots = cols / (BF16 ? 8 : 4);
        if (nslots < kThreads || nslots > 4 * kThreads) return false;
        if (S == Smooth::kNone && nslots != 4 * kThreads) return false;
        const bool full = nslots % kThreads == 0;
        const int64_t nv = (nslots + kThreads - 1) / kThreads;
        if (nv == 1) *st = launch_smooth<1, BF16, S, true>(fn, in, smooth, out, scales, rows, cols, stream);
        else if (nv == 2 && full) *st = launch_smooth<2, BF16, S, true>(fn, in, smooth, out, scales, rows, cols, stream);
        else if (nv == 2) *st = launch_smooth<2, BF16, S, false>(fn, in, smooth, out, scales, rows, cols, stream);
        else if (full) *st = launch_smooth<4, BF16, S, true>(fn, in, smooth, out, scales, rows, cols, stream);
        else *st = launch_smooth<4, BF16, S, false>(fn, in, smooth, out, scales, rows, cols, stream);
        return true;
    }
}

template <Smooth S>
int quant_rows_f32(const char* fn, const float* in, const float* smooth, int8_t* out,
                   float* scales, int64_t rows, int64_t cols, hipStream_t stream) {
    int st = check_rows(fn, in, out, scales, rows, cols);
    if (st != KC_SUCCESS) return st;
    if (S != Smooth::kNone && rows > 0 && cols > 0 && !smooth)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null smoothing vector", fn);
    if (rows == 0 || cols == 0) return KC_SUCCESS;
    const unsigned grid = static_cast<unsigned>(rows);
    const bool vec = cols > 0 && cols % 4 == 0 && kc::aligned(in, 16) && kc::aligned(out, 4) &&
                     (S == Smooth::kNone || kc::aligned(smooth, 16));
    if (vec && try_smooth_persistent<false, S>(fn, in, smooth, out, scales, rows, cols, stream, &st))
        return st;
    const int64_t slots = (cols / 4 + kWave - 1) / kWave;  // 16-byte slots per lane, one wave per row
    if (vec && slots <= 16) {
        if (slots <= 1) quant_rows_wave_kernel<1, false, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else if (slots <= 2) quant_rows_wave_kernel<2, false, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else if (slots <= 4) quant_rows_wave_kernel<4, false, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else if (slots <= 8) quant_rows_wave_kernel<8, false, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else quant_rows_wave_kernel<16, false, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        return kc::check_launch(fn);
    }
    const int64_t nv = (cols + 1023) / 1024;
    if (vec && nv <= 1)
        quant_rows_f32_kernel<1, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else if (vec && nv <= 2)
        quant_rows_f32_kernel<2, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else if (vec && nv <= 4)
        quant_rows_f32_kernel<4, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else if (vec && nv <= 8)
        quant_rows_f32_kernel<8, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else
        quant_rows_generic_kernel<false, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales,
                                                                           cols);
    return kc::check_launch(fn);
}

template <Smooth S>
int quant_rows_bf16(const char* fn, const uint16_t* in, const float* smooth, int8_t* out,
                    float* scales, int64_t rows, int64_t cols, hipStream_t stream) {
    int st = check_rows(fn, in, out, scales, rows, cols);
    if (st != KC_SUCCESS) return st;
    if (S != Smooth::kNone && rows > 0 && cols > 0 && !smooth)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null smoothing vector", fn);
    if (rows == 0 || cols == 0) return KC_SUCCESS;
    const unsigned grid = static_cast<unsigned>(rows);
    const bool vec = cols > 0 && cols % 8 == 0 && kc::aligned(in, 16) && kc::aligned(out, 8) &&
                     (S == Smooth::kNone || kc::aligned(smooth, 16));
    if (vec && try_smooth_persistent<true, S>(fn, in, smooth, out, scales, rows, cols, stream, &st))
        return st;
    const int64_t slots = (cols / 8 + kWave - 1) / kWave;  // 16-byte slots per lane, one wave per row
    if (vec && slots <= 16) {
        if (slots <= 1) quant_rows_wave_kernel<1, true, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else if (slots <= 2) quant_rows_wave_kernel<2, true, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else if (slots <= 4) quant_rows_wave_kernel<4, true, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else if (slots <= 8) quant_rows_wave_kernel<8, true, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        else quant_rows_wave_kernel<16, true, S><<<grid, kWave, 0, stream>>>(in, smooth, out, scales, cols);
        return kc::check_launch(fn);
    }
    const int64_t nv = (cols + 2047) / 2048;
    if (vec && nv <= 1)
        quant_rows_bf16_kernel<1, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else if (vec && nv <= 2)
        quant_rows_bf16_kernel<2, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else if (vec && nv <= 4)
        quant_rows_bf16_kernel<4, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else if (vec && nv <= 8)
        quant_rows_bf16_kernel<8, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales, cols);
    else
        quant_rows_generic_kernel<true, S><<<grid, kThreads, 0, stream>>>(in, smooth, out, scales,
                                                                          cols);
    return kc::check_launch(fn);
}

int quant_tensor_f32(const char* fn, const float* in, int8_t* out, const float* d_scale,
                     int64_t rows, int64_t cols, hipStream_t stream) {
    int st = check_rows(fn, in, out, d_scale, rows, cols);
    if (st != KC_SUCCESS) return st;
    const int64_t count = rows * cols;
    if (count == 0) return KC_SUCCESS;
    const bool vec = kc::aligned(in, 16) && kc::aligned(out, 4);
    const int64_t work = vec ? (count + 3) / 4 : count;
    const int64_t blocks = std::min<int64_t>((work + kThreads - 1) / kThreads, 256 * 32);
    quant_tensor_f32_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(
        in, d_scale, out, count, vec);
    return kc::check_launch(fn);
}

int row_tiles(const char* fn, int64_t rows, int64_t cols, int64_t* tiles, unsigned* grid) {
    *tiles = (cols + 1023) / 1024;
    const int64_t g = rows * *tiles;
    if (g > INT32_MAX)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: tensor too large (rows=%lld cols=%lld)",
                             fn, (long long)rows, (long long)cols);
    *grid = static_cast<unsigned>(g);
    return KC_SUCCESS;
}

int dequant_fp8(const char* fn, const int8_t* in, const float* scales, float* out, int64_t rows,
                int64_t cols, bool per_token, hipStream_t stream) {
    int st = check_rows(fn, in, out, scales, rows, cols);
    if (st != KC_SUCCESS) return st;
    if (rows == 0 || cols == 0) return KC_SUCCESS;
    int64_t tiles;
    unsigned grid;
    if ((st = row_tiles(fn, rows, cols, &tiles, &grid)) != KC_SUCCESS) return st;
    const bool vec = cols % 4 == 0 && kc::aligned(in, 4) && kc::aligned(out, 16);
    dequant_fp8_kernel<<<grid, kThreads, 0, stream>>>(in, scales, out, cols, tiles, per_token, vec);
    return kc::check_launch(fn);
}

int smooth_div(const char* fn, const float* in, const float* s, float* out, int64_t rows,
               int64_t cols, hipStream_t stream) {
    int st = check_rows(fn, in, out, s, rows, cols);
    if (st != KC_SUCCESS) return st;
    if (rows == 0 || cols == 0) return KC_SUCCESS;
    int64_t tiles;
    unsigned grid;
    if ((st = row_tiles(fn, rows, cols, &tiles, &grid)) != KC_SUCCESS) return st;
    const bool vec = cols % 4 == 0 && kc::aligned(in, 16) && kc::aligned(out, 16) &&
                     kc::aligned(s, 16);
    smooth_div_kernel<<<grid, kThreads, 0, stream>>>(in, s, out, cols, tiles, vec);
    return kc::check_launch(fn);
}

template <bool BF16>
int col_absmax(const char* fn, const void* in, float* amax, int64_t rows, int64_t cols,
               hipStream_t stream) {
    int st = check_rows(fn, in, amax, amax, rows, cols);
    if (st != KC_SUCCESS) return st;
    if (cols == 0) return KC_SUCCESS;
    if (!amax) return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    const int64_t fill_blocks = std::min<int64_t>((cols + kThreads - 1) / kThreads, 1024);
    fill_zero_kernel<<<static_cast<unsigned>(fill_blocks), kThreads, 0, stream>>>(amax, cols);
    if ((st = kc::check_launch(fn)) != KC_SUCCESS) return st;
    if (rows == 0) return KC_SUCCESS;
    constexpr int64_t kCols = 32 * (BF16 ? 8 : 4);  // columns per block
    const int64_t tiles = (cols + kCols - 1) / kCols;
    const int64_t bands = (rows + kAbsmaxRowsPerBlock - 1) / kAbsmaxRowsPerBlock;
    if (bands * tiles > INT32_MAX)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: tensor too large", fn);
    const bool vec = cols % (BF16 ? 8 : 4) == 0 && kc::aligned(in, 16);
    col_absmax_kernel<BF16><<<static_cast<unsigned>(bands * tiles), kThreads, 0, stream>>>(
        in, amax, rows, cols, tiles, vec);
    return kc::check_launch(fn);
}

// X [tokens, cols] and W [out, cols]: amax_x, amax_w and the smoothing
// factors in three launches (one fill for both maxima, one reduction grid
// over both tensors, the factors), with the values of col_absmax on each
// tensor followed by smooth_factors.
template <bool BF16>
int smoothquant_stats(const char* fn, const void* x, int64_t tokens, const void* w, int64_t outs,
                      int64_t cols, float* amax_x, float* amax_w, float* smooth,
                      hipStream_t stream) {
    int st = check_rows(fn, x, amax_x, amax_x, tokens, cols);
    if (st != KC_SUCCESS) return st;
    if ((st = check_rows(fn, w, amax_w, amax_w, outs, cols)) != KC_SUCCESS) return st;
    if (cols == 0) return KC_SUCCESS;
    if (!amax_x || !amax_w || !smooth)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    const int64_t fill_blocks = std::min<int64_t>((cols + kThreads - 1) / kThreads, 1024);
    fill_zero2_kernel<<<static_cast<unsigned>(fill_blocks), kThreads, 0, stream>>>(amax_x, amax_w,
                                                                                  cols);
    if ((st = kc::check_launch(fn)) != KC_SUCCESS) return st;
    constexpr int64_t kCols = 32 * (BF16 ? 8 : 4);  // columns per block
    const int64_t tiles = (cols + kCols - 1) / kCols;
    const int64_t blocks_x = (tokens + kAbsmaxRowsPerBlock - 1) / kAbsmaxRowsPerBlock * tiles;
    const int64_t blocks_w = (outs + kAbsmaxRowsPerBlock - 1) / kAbsmaxRowsPerBlock * tiles;
    if (blocks_x + blocks_w > INT32_MAX)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: tensors too large", fn);
    if (blocks_x + blocks_w > 0) {
        const bool vec_x = cols % (BF16 ? 8 : 4) == 0 && kc::aligned(x, 16);
        const bool vec_w = cols % (BF16 ? 8 : 4) == 0 && kc::aligned(w, 16);
        col_absmax2_kernel<BF16><<<static_cast<unsigned>(blocks_x + blocks_w), kThreads, 0, stream>>>(
            x, amax_x, tokens, vec_x, blocks_x, w, amax_w, outs, vec_w, cols, tiles);
        if ((st = kc::check_launch(fn)) != KC_SUCCESS) return st;
    }
    const int64_t blocks = std::min<int64_t>((cols + kThreads - 1) / kThreads, 1024);
    smooth_factor_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(amax_x, amax_w,
                                                                                smooth, cols);
    return kc::check_launch(fn);
}

}  // namespace

// ===========================================================================
// C ABI -- reference launchers (blocking)
// ===========================================================================

extern "C" void launch_quantize_fp8(const float* d_input, int8_t* d_output, float* d_scales,
                                    int rows, int cols, bool per_token, kc_stream_t stream) {
    const char* fn = "launch_quantize_fp8";
    const int st = per_token ? quant_rows_f32<Smooth::kNone>(fn, d_input, nullptr, d_output,
                                                             d_scales, rows, cols, stream)
                             : quant_tensor_f32(fn, d_input, d_output, d_scales, rows, cols, stream);
    if (st == KC_SUCCESS) kc::sync_stream(stream, fn);
}

extern "C" void launch_dequantize_fp8(const int8_t* d_input, const float* d_scales,
                                      float* d_output, int rows, int cols, bool per_token,
                                      kc_stream_t stream) {
    const char* fn = "launch_dequantize_fp8";
    if (dequant_fp8(fn, d_input, d_scales, d_output, rows, cols, per_token, stream) == KC_SUCCESS)
        kc::sync_stream(stream, fn);
}

extern "C" void launch_smoothquant_scale(const float* d_input, const float* d_smooth_scales,
                                         float* d_output, int rows, int cols,
                                         kc_stream_t stream) {
    const char* fn = "launch_smoothquant_scale";
    if (smooth_div(fn, d_input, d_smooth_scales, d_output, rows, cols, stream) == KC_SUCCESS)
        kc::sync_stream(stream, fn);
}

// ===========================================================================
// C ABI -- extensions (stream-ordered)
// ===========================================================================

extern "C" int kc_quantize_fp8_per_token_f32(const float* d_input, int8_t* d_output,
                                             float* d_scales, int64_t rows, int64_t cols,
                                             kc_stream_t stream) {
    return quant_rows_f32<Smooth::kNone>("kc_quantize_fp8_per_token_f32", d_input, nullptr,
                                         d_output, d_scales, rows, cols, stream);
}

extern "C" int kc_quantize_fp8_per_tensor_f32(const float* d_input, int8_t* d_output,
                                              const float* d_scale, int64_t rows, int64_t cols,
                                              kc_stream_t stream) {
    return quant_tensor_f32("kc_quantize_fp8_per_tensor_f32", d_input, d_output, d_scale, rows,
                            cols, stream);
}

extern "C" int kc_quantize_fp8_per_token_bf16(const uint16_t* d_input, int8_t* d_output,
                                              float* d_scales, int64_t rows, int64_t cols,
                                              kc_stream_t stream) {
    return quant_rows_bf16<Smooth::kNone>("kc_quantize_fp8_per_token_bf16", d_input, nullptr,
                                          d_output, d_scales, rows, cols, stream);
}

extern "C" int kc_col_absmax_bf16(const uint16_t* d_input, float* d_amax, int64_t rows,
                                  int64_t cols, kc_stream_t stream) {
    return col_absmax<true>("kc_col_absmax_bf16", d_input, d_amax, rows, cols, stream);
}

extern "C" int kc_col_absmax_f32(const float* d_input, float* d_amax, int64_t rows, int64_t cols,
                                 kc_stream_t stream) {
    return col_absmax<false>("kc_col_absmax_f32", d_input, d_amax, rows, cols, stream);
}

extern "C" int kc_smoothquant_stats_bf16(const uint16_t* d_x, int64_t tokens, const uint16_t* d_w,
                                         int64_t out_features, int64_t cols, float* d_amax_x,
                                         float* d_amax_w, float* d_smooth, kc_stream_t stream) {
    return smoothquant_stats<true>("kc_smoothquant_stats_bf16", d_x, tokens, d_w, out_features, cols,
                                   d_amax_x, d_amax_w, d_smooth, stream);
}

extern "C" int kc_smoothquant_stats_f32(const float* d_x, int64_t tokens, const float* d_w,
                                        int64_t out_features, int64_t cols, float* d_amax_x,
                                        float* d_amax_w, float* d_smooth, kc_stream_t stream) {
    return smoothquant_stats<false>("kc_smoothquant_stats_f32", d_x, tokens, d_w, out_features, cols,
                                    d_amax_x, d_amax_w, d_smooth, stream);
}

extern "C" int kc_smooth_factors(const float* d_amax_x, const float* d_amax_w, float* d_smooth,
                                 int64_t cols, kc_stream_t stream) {
    const char* fn = "kc_smooth_factors";
    if (cols < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative cols", fn);
    if (cols == 0) return KC_SUCCESS;
    if (!d_amax_x || !d_amax_w || !d_smooth)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    const int64_t blocks = std::min<int64_t>((cols + kThreads - 1) / kThreads, 1024);
    smooth_factor_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(d_amax_x, d_amax_w,
                                                                                d_smooth, cols);
    return kc::check_launch(fn);
}

extern "C" int kc_quantize_fp8_smooth_div_f32(const float* d_input, const float* d_smooth,
                                              int8_t* d_output, float* d_scales, int64_t rows,
                                              int64_t cols, kc_stream_t stream) {
    return quant_rows_f32<Smooth::kDiv>("kc_quantize_fp8_smooth_div_f32", d_input, d_smooth,
                                        d_output, d_scales, rows, cols, stream);
}

extern "C" int kc_quantize_fp8_smooth_div_bf16(const uint16_t* d_input, const float* d_smooth,
                                               int8_t* d_output, float* d_scales, int64_t rows,
                                               int64_t cols, kc_stream_t stream) {
    return quant_rows_bf16<Smooth::kDiv>("kc_quantize_fp8_smooth_div_bf16", d_input, d_smooth,
                                         d_output, d_scales, rows, cols, stream);
}

extern "C" int kc_quantize_fp8_smooth_mul_bf16(const uint16_t* d_input, const float* d_smooth,
                                               int8_t* d_output, float* d_scales, int64_t rows,
                                               int64_t cols, kc_stream_t stream) {
    return quant_rows_bf16<Smooth::kMul>("kc_quantize_fp8_smooth_mul_bf16", d_input, d_smooth,
                                         d_output, d_scales, rows, cols, stream);
}
