// int4_decode.hpp -- device helpers of the INT4 GEMV kernels
// (quant_int4.hip): nibble decode, the dot product of one
// 16-byte weight chunk with x staged in LDS, cross-lane row reductions, and
// the scale/zero slot map.  See quant_int4.hip for the encoding.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace kc {
namespace int4 {

// The GEMV kernels issue their loads at a raised wave priority and compute
// at the normal one (s_setprio).  When a workgroup's data land, its waves'
// decode bursts would otherwise hold the SIMD while waves of newly started
// workgroups wait to issue their loads, and the weight stream thins out
// (the decode layer's four GEMVs in one launch: 22.2 -> 20.1 us).
constexpr int kIssuePrio = 1;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The decode constants live in VGPRs: on gfx950 a VALU operation that reads
// an SGPR operand issues at half the rate of one with VGPR operands, and the
// compiler would otherwise put one of the two masks in an SGPR.  The asm
// makes the values opaque so they stay in VGPRs.
struct NibConsts {
    uint32_t mask;   // 0x000F000F
    uint32_t magic;  // 0x43084308 = 0x43004300 | (8 << 16) | 8
};

__device__ __forceinline__ NibConsts nib_consts() {
    NibConsts k;
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(k.mask));
    asm volatile("v_mov_b32 %0, 0x43084308" : "=v"(k.magic));
    return k;
}

// ((d ^ 0x00080008) & 0x000F000F) | 0x43004300 == (d & 0x000F000F) ^ 0x43084308
__device__ __forceinline__ uint32_t nib_pair(uint32_t d, NibConsts k) { return (d & k.mask) ^ k.magic; }

// Takes its operand by value: clang miscompiles __builtin_bit_cast applied to
// an element of an ext_vector reached through a reference (every element
// reads offset 0), so vector elements are always copied out first.
__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) {
    return __builtin_bit_cast(bf16x2_t, v);
}

__device__ __forceinline__ float dot8_bf16(uint32_t d, u32x4 xq, float a, NibConsts k) {
    const uint32_t x04 = xq.x, x15 = xq.y, x26 = xq.z, x37 = xq.w;
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_pair(d, k)), as_bf16x2(x04), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_pair(d >> 4, k)), as_bf16x2(x15), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_pair(d >> 8, k)), as_bf16x2(x26), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(nib_pair(d >> 12, k)), as_bf16x2(x37), a, false);
    return a;
}

// The masked words are made opaque to the optimizer: otherwise it merges the
// two masks of each byte into a bit-field extract per weight (v_bfe_u32 plus
// v_cvt_f32_ubyte0) instead of letting v_cvt_f32_ubyte1..3 pick the byte,
// 26 instead of 19 VALU operations per word (cfg0 5.14 -> 4.95 us).
__device__ __forceinline__ float dot8_f32(uint32_t d, f32x4 xa, f32x4 xb, float a) {
    uint32_t L = (d ^ 0x88888888u) & 0x0F0F0F0Fu;         // even k of each byte, n' = q ^ 8
    uint32_t H = ((d >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu;  // odd k
    asm volatile("" : "+v"(L), "+v"(H));
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

// Dot product of one 16-byte weight chunk with the chunk's x, read from LDS
// (bf16: 4 permuted quads; fp32: 8 quads of 4 values).
template <bool XBF16>
__device__ __forceinline__ float chunk_dot(const u32x4 w, const u32x4* xl, NibConsts k) {
    const uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
    if constexpr (XBF16) {
        float a = dot8_bf16(w0, xl[0], 0.0f, k);
        a = dot8_bf16(w1, xl[1], a, k);
        a = dot8_bf16(w2, xl[2], a, k);
        return dot8_bf16(w3, xl[3], a, k);
    } else {
        (void)k;
        const f32x4* xf = reinterpret_cast<const f32x4*>(xl);
        float a = dot8_f32(w0, xf[0], xf[1], 0.0f);
        a = dot8_f32(w1, xf[2], xf[3], a);
        a = dot8_f32(w2, xf[4], xf[5], a);
        return dot8_f32(w3, xf[6], xf[7], a);
    }
}

// Cross-lane steps, all VALU (no LDS round trip):
//   permlane32_swap(a, b) -> ([a 0-31, b 0-31], [a 32-63, b 32-63])
//   permlane16_swap(a, b) -> per 32-lane half, ([a 0-15, b 0-15], [a 16-31, b 16-31])
//   row_ror:n             -> lane i of each 16-lane row reads lane (i - n) mod 16
__device__ __forceinline__ float ror16(float v, int n) {
    const int iv = __builtin_bit_cast(int, v);
    switch (n) {
        case 8: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, false));
        case 4: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x124, 0xF, 0xF, false));
        case 2: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x122, 0xF, 0xF, false));
        default: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x121, 0xF, 0xF, false));
    }
}

// The swap builtins return a two-element vector; its elements are copied to
// scalars before __builtin_bit_cast, which reads element 0 for any element of
// a vector it is applied to directly (the same clang defect as above).
__device__ __forceinline__ float sum_swap32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a),
                                                    __builtin_bit_cast(unsigned, b), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float sum_swap16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a),
                                                    __builtin_bit_cast(unsigned, b), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float sum_row16(float t) {
    t += ror16(t, 8);
    t += ror16(t, 4);
    t += ror16(t, 2);
    return t + ror16(t, 1);
}

// Sums v[r] over the wave for R rows.  Afterwards lane (64/R)*r holds the
// total of row r (so do the other lanes of its group of 64/R).
template <int R>
__device__ __forceinline__ float wave_reduce_rows(const float (&v)[R]) {
    static_assert(R == 1 || R == 2 || R == 4, "rows per wave");
    if constexpr (R == 4) {
        const float a = sum_swap32(v[0], v[2]);  // lanes 0-31: row 0, 32-63: row 2
        const float b = sum_swap32(v[1], v[3]);  // lanes 0-31: row 1, 32-63: row 3
        return sum_row16(sum_swap16(a, b));     // rows 0, 1, 2, 3 in 16-lane rows
    } else if constexpr (R == 2) {
        const float t = sum_row16(sum_swap32(v[0], v[1]));  // halves: row 0, row 1
        return sum_swap16(t, t);
    } else {
        const float t = sum_row16(v[0]);
        const float u = sum_swap32(t, t);
        return sum_swap16(u, u);
    }
}

// Scale/zero items.  Slot (r, j) -- row r, chunk slot j -- covers the groups
// of chunks j*64 .. j*64+63 of its row: NG = max(1, 64 / (gs/32)) of them,
// at most SLOT items.  Slots are packed 64/SLOT to a register: slot s lives
// in register s / (64/SLOT), lanes (s % (64/SLOT)) * SLOT + gi.  One scale
// load and one zero-byte load per register bring in every (s, z) a wave
// needs; a lane then fetches the pair for its own chunk with ds_bpermute
// from a register index known at compile time.
//   SLOT = 16 serves gs >= 128, SLOT = 64 serves gs = 32 and 64.
template <int SLOT>
struct SlotMap {
    static constexpr int kPerReg = 64 / SLOT;
    static constexpr int reg(int s) { return s / kPerReg; }
    static constexpr int base_lane(int s) { return (s % kPerReg) * SLOT; }
};

}  // namespace int4
}  // namespace kc
