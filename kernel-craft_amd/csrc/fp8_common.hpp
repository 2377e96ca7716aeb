// fp8_common.hpp -- FP8 E4M3 (OCP) encoding and the division by a row
// scale, shared by the FP8 quantizers (fp8_quant.hip) and the RMSNorm ->
// FP8 fusion (rmsnorm.hip).
//
// Arithmetic (fp8_quant.cu:62-75, 89-131 in the reference):
//   absmax_r = max over the row of |x| (fmaxf from 0: NaN never wins)
//   scale_r  = absmax_r > 0 ? absmax_r / 448 : 1        (IEEE divide)
//   code     = E4M3_rne(fmaxf(-448, fminf(448, x / scale_r)))
#pragma once

#include "kc_common.hpp"

namespace kc {
namespace fp8 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kE4M3Max = 448.0f;  // fp8_quant.cu:31

__device__ __forceinline__ float clamp448(float v) { return fmaxf(-kE4M3Max, fminf(kE4M3Max, v)); }

// Every input element is quieted once as it is loaded (v_max_f32 x, x in IEEE
// mode; any other value, -0 and denormals included, is unchanged).  gfx950's
// division sequence passes a signaling NaN through unquieted, and the
// IEEE-mode v_min/v_max of the clamp then return NaN instead of the bound;
// CUDA's fminf/fmaxf (fp8_quant.cu:127) return the bound, +448, for every NaN.
// LLVM cannot drop the canonicalize of a loaded value, and treats its result
// as quiet from there on.
__device__ __forceinline__ float quiet(float x) { return __builtin_canonicalizef(x); }

__device__ __forceinline__ f32x4 quiet4(f32x4 v) {
    return f32x4{quiet(v.x), quiet(v.y), quiet(v.z), quiet(v.w)};
}

// 4 fp32 -> 4 E4M3 codes, byte i of the result holds input i.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    int v = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(a), clamp448(b), 0, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(c), clamp448(d), v, true);
    return static_cast<uint32_t>(v);
}

// The same for NaN-free input: the clamp is one median (v_med3_f32, which
// would not map NaN to +448).
__device__ __forceinline__ uint32_t e4m3x4_finite(float a, float b, float c, float d) {
    auto clamp = [](float v) { return __builtin_amdgcn_fmed3f(v, -kE4M3Max, kE4M3Max); };
    int v = __builtin_amdgcn_cvt_pk_fp8_f32(clamp(a), clamp(b), 0, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(clamp(c), clamp(d), v, true);
    return static_cast<uint32_t>(v);
}

__device__ __forceinline__ uint8_t e4m3x1(float a) {
    return static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(a), 0.0f, 0, false) & 0xFF);
}

__device__ __forceinline__ float row_scale(float amax) {
    return amax > 0.0f ? amax / kE4M3Max : 1.0f;  // fp8_quant.cu:121
}

// Division by the row scale.  The reference divides every element by its
// row's scale with an IEEE division (fp8_quant.cu:126).  With r = RN(1/s),
// computed once per row by a correctly rounded division, Markstein's
// correction step
//     q0 = RN(x * r),   e = RN(s * q0 - x) (one FMA),   q = RN(q0 - e * r)
// returns RN(x / s) whenever the residual is exactly representable and the
// quotient is a normal number, which holds for |x| >= 2^-102 and
// |x/s| >= 2^-126 when r is normal.  Every other finite x gets a q with the
// sign of x (zeros included: -0 gives -0) and |q| <= 2^-102/s + 2^-125.
// The row route uses it for rows with 2^-60 <= absmax <= FLT_MAX: there r is
// normal, and an element with |x| < 2^-102 has |x/s| < 2^-33, far below the
// smallest E4M3 step (2^-9), so its code is +0 or -0 with the sign of x on
// both routes.  Other rows (all-tiny or non-finite absmax) divide exactly.
// Three VALU operations instead of the ~10 of a correctly rounded division.
struct RowDiv {
    float s;      // row scale
    float r;      // RN(1 / s)
    bool fast;    // Markstein is exact for this row
};

__device__ __forceinline__ RowDiv row_div(float amax) {
    RowDiv d;
    d.s = row_scale(amax);
    d.r = 1.0f / d.s;
    d.fast = amax >= 0x1p-60f && amax <= 3.40282347e38f;
    return d;
}

// RN(x / s) for the element ranges stated above; r = RN(1/s).
__device__ __forceinline__ float markstein(float x, float s, float r) {
    const float q0 = __fmul_rn(x, r);
    const float e = fmaf(s, q0, -x);
    return fmaf(-e, r, q0);
}

template <bool FAST>
__device__ __forceinline__ float div_scale(float x, const RowDiv& d) {
    if constexpr (FAST) return markstein(x, d.s, d.r);
    else return x / d.s;
}

template <bool FAST>
__device__ __forceinline__ uint32_t e4m3x4_div(f32x4 v, const RowDiv& d) {
    return e4m3x4(div_scale<FAST>(v.x, d), div_scale<FAST>(v.y, d), div_scale<FAST>(v.z, d),
                  div_scale<FAST>(v.w, d));
}

__device__ __forceinline__ float absmax4(float m, f32x4 v) {
    return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}

__device__ __forceinline__ f32x4 bf16x4_to_f32(uint32_t a, uint32_t b) {
    return f32x4{__uint_as_float(a << 16), __uint_as_float(a & 0xFFFF0000u),
                 __uint_as_float(b << 16), __uint_as_float(b & 0xFFFF0000u)};
}

}  // namespace fp8
}  // namespace kc
