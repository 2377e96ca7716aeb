// kc_common.hpp -- host/device utilities shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernel_craft.h"

namespace kc {

// ---- error channel (kc_status.cpp) --------------------------------------
// Records `code` and a printf-style message for the calling thread and
// returns `code`, so launchers can `return set_error(...)`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks hipGetLastError() after a launch; records KC_ERR_HIP on failure.
int check_launch(const char* what);
// hipStreamSynchronize with error recording (the reference launchers'
// blocking behaviour, quant_int4.cu:205,233, fp8_quant.cu:225,252,277).
int sync_stream(hipStream_t stream, const char* what);

// ---- device helpers -----------------------------------------------------
constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Two fp32 -> packed bf16 (lo in bits 0-15), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950.  Finite values and infinities convert as
// f32_to_bf16 does; a NaN stays a NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__host__ __device__ constexpr bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

inline int ilog2(int64_t v) {
    int r = 0;
    while ((int64_t{1} << (r + 1)) <= v) ++r;
    return r;
}

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

}  // namespace kc
