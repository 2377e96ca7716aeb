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
// A row is split into chunks of 32 k (16 bytes of packed weights).  One
// workgroup computes R consecutive rows; its W waves split K, wave w owning
// chunks [w*64*CPL, (w+1)*64*CPL) of every row and lane l the chunks
// w*64*CPL + 64*j + l (j < CPL), so each wave-wide load reads 1 KB of one
// row.  Every weight load of the workgroup is issued up front.  The lane's x
// for its chunks is loaded once into registers: for bf16 the quad of k-block
// i (k = 8i..8i+7 of a chunk) is rearranged into the pairs (x0,x4) (x1,x5)
// (x2,x6) (x3,x7), the order in which the nibble unpack produces weights;
// xs is the chunk's fp32 sum of x.  Partial sums are reduced across the wave
// with a transposed butterfly (R values in log2(64) + R - 1 shuffles) and
// across the W waves through LDS in a fixed order, so results do not depend
// on scheduling.
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

__device__ __forceinline__ float dot8_f32(uint32_t d, f32x4 xa, f32x4 xb, float a) {
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

// The lane's x for one chunk: bf16 as 4 quads of pairs, fp32 as 8 quads.
template <bool XBF16>
struct XChunk {
    u32x4 q[XBF16 ? 4 : 8];
    float sum;
};

template <bool XBF16>
__device__ __forceinline__ XChunk<XBF16> load_x_chunk(const void* __restrict__ x, int c) {
    XChunk<XBF16> xc;
    if constexpr (XBF16) {
        const u32x4* src = static_cast<const u32x4*>(x) + 4 * c;
        const bf16x2_t ones = as_bf16x2(0x3F803F80u);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 d = src[i];
            const uint32_t d0 = d.x, d1 = d.y, d2 = d.z, d3 = d.w;
            u32x4 p;
            p.x = (d0 & 0xFFFFu) | (d2 << 16);
            p.y = (d0 >> 16) | (d2 & 0xFFFF0000u);
            p.z = (d1 & 0xFFFFu) | (d3 << 16);
            p.w = (d1 >> 16) | (d3 & 0xFFFF0000u);
            xc.q[i] = p;
            sum = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d0), ones, sum, false);
            sum = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d1), ones, sum, false);
            sum = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d2), ones, sum, false);
            sum = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d3), ones, sum, false);
        }
        xc.sum = sum;
    } else {
        const f32x4* src = static_cast<const f32x4*>(x) + 8 * c;
        float part[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4 v = src[i];
            xc.q[i] = __builtin_bit_cast(u32x4, v);
            part[i] = (v.x + v.y) + (v.z + v.w);
        }
        xc.sum = ((part[0] + part[1]) + (part[2] + part[3])) +
                 ((part[4] + part[5]) + (part[6] + part[7]));
    }
    return xc;
}

template <bool XBF16>
__device__ __forceinline__ float chunk_dot(const u32x4 w, const XChunk<XBF16>& xc) {
    const uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
    if constexpr (XBF16) {
        const u32x4 a0 = xc.q[0], a1 = xc.q[1], a2 = xc.q[2], a3 = xc.q[3];
        float a = dot8_bf16(w0, a0.x, a0.y, a0.z, a0.w, 0.0f);
        a = dot8_bf16(w1, a1.x, a1.y, a1.z, a1.w, a);
        a = dot8_bf16(w2, a2.x, a2.y, a2.z, a2.w, a);
        return dot8_bf16(w3, a3.x, a3.y, a3.z, a3.w, a);
    } else {
        float a = dot8_f32(w0, __builtin_bit_cast(f32x4, xc.q[0]), __builtin_bit_cast(f32x4, xc.q[1]), 0.0f);
        a = dot8_f32(w1, __builtin_bit_cast(f32x4, xc.q[2]), __builtin_bit_cast(f32x4, xc.q[3]), a);
        a = dot8_f32(w2, __builtin_bit_cast(f32x4, xc.q[4]), __builtin_bit_cast(f32x4, xc.q[5]), a);
        return dot8_f32(w3, __builtin_bit_cast(f32x4, xc.q[6]), __builtin_bit_cast(f32x4, xc.q[7]), a);
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
__device__ __forceinline__ float wave_reduce_rows(float (&v)[R], int /*lane*/) {
    static_assert(R == 1 || R == 2 || R == 4, "rows per block");
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

constexpr int kMaxWaves = 16;

// Per row block, a lane needs for each of its CPL chunks and R rows the
// group's scale s and zero point z, folded as
//     acc += c1 * dot + c2 * sum(x),   c1 = s,  c2 = -s * (off + z)
// (off = 136 for the bf16 encoding 128 + (q ^ 8), 8 for fp32).  A wave's
// chunk slot j spans NG = max(1, 64 * 32 / gs) groups of a row, so the
// CPL * R * NG (<= 64) distinct (s, z) of a row block arrive with one
// coalesced scale load and one zero-byte load, lane i holding item
// i = (j * R + r) * NG + gi; every lane then picks up its own c1, c2 with
// ds_bpermute.
template <int R, int CPL>
struct RowBlock {
    u32x4 w[R][CPL];
    float s;       // item scale
    uint32_t zb;   // item zero byte
};

struct SzLayout {
    int ng;        // groups per chunk slot
    int gshift;    // log2(gs / 32)
    int G;         // groups per row
    int items;     // CPL * R * ng
};

template <int R, int CPL>
__device__ __forceinline__ void load_row_block(RowBlock<R, CPL>& b, const uint8_t* __restrict__ packed,
                                               const float* __restrict__ scales,
                                               const uint8_t* __restrict__ zeros, int row0, int rows,
                                               int64_t rbytes, const int (&cidx)[CPL],
                                               const SzLayout& L, int wave, int lane) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t rr = min(row0 + r, rows - 1);  // tail rows re-read the last row
        const u32x4* prow = reinterpret_cast<const u32x4*>(packed + rr * rbytes);
#pragma unroll
        for (int j = 0; j < CPL; ++j) b.w[r][j] = __builtin_nontemporal_load(prow + cidx[j]);
    }
    // item owned by this lane (lanes past `items` repeat item 0)
    const int item = lane < L.items ? lane : 0;
    const int gi = item % L.ng;
    const int jr = item / L.ng;
    const int r = jr % R, j = jr / R;
    const int gbase = ((wave * CPL + j) * kWave) >> L.gshift;
    const int g = min(gbase + gi, L.G - 1);
    const int64_t rr = min(row0 + r, rows - 1);
    b.s = scales[rr * L.G + g];
    b.zb = zeros[rr * (L.G >> 1) + (g >> 1)];
}

// Dot products of one row block, reduced over the wave and the workgroup,
// stored to y.  `red` is this iteration's half of the LDS exchange buffer.
template <int R, int CPL, bool XBF16, bool YBF16>
__device__ __forceinline__ void finish_row_block(const RowBlock<R, CPL>& b,
                                                 const XChunk<XBF16> (&xc)[CPL],
                                                 const bool (&act)[CPL], const SzLayout& L,
                                                 float (*red)[R], int row0, int rows, void* y,
                                                 int lane, int wave, int nwaves) {
    // this lane's item -> c1, c2
    const int item = lane < L.items ? lane : 0;
    const int g = min(((((item / L.ng) / R) * kWave + wave * CPL * kWave) >> L.gshift) + item % L.ng,
                      L.G - 1);
    const uint32_t z = (g & 1) ? (b.zb >> 4) : (b.zb & 0xFu);
    const float c1 = b.s;
    const float c2 = -b.s * static_cast<float>((XBF16 ? 136u : 8u) + z);
    const int gsub = L.ng > 1 ? (lane >> L.gshift) : 0;  // group of my chunk within its slot
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int src = ((j * R + r) * L.ng + gsub) << 2;
            float m1 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, c1)));
            float m2 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, c2)));
            m1 = act[j] ? m1 : 0.0f;
            m2 = act[j] ? m2 : 0.0f;
            acc[r] = fmaf(m1, chunk_dot<XBF16>(b.w[r][j], xc[j]), fmaf(m2, xc[j].sum, acc[r]));
        }
    }
    const float t = wave_reduce_rows<R>(acc, lane);
    constexpr int kGroup = kWave / R;
    if (nwaves == 1) {
        const int r = lane / kGroup;
        if ((lane & (kGroup - 1)) == 0 && row0 + r < rows) store_y<YBF16>(y, row0 + r, t);
        return;
    }
    if ((lane & (kGroup - 1)) == 0) red[wave][lane / kGroup] = t;
    __syncthreads();
    if (threadIdx.x < R) {
        float tot = red[0][threadIdx.x];
        for (int wv = 1; wv < nwaves; ++wv) tot += red[wv][threadIdx.x];
        if (row0 + static_cast<int>(threadIdx.x) < rows)
            store_y<YBF16>(y, row0 + threadIdx.x, tot);
    }
}

// Persistent: workgroup b computes row blocks b, b + gridDim.x, ...; the next
// block's weights are in flight while the current block is reduced.
template <int R, int CPL, bool XBF16, bool YBF16>
__global__ __launch_bounds__(CPL == 1 ? kMaxWaves * kWave : kWave) void gemv_int4_fast_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const void* __restrict__ x, void* __restrict__ y,
    int rows, int cols, int gshift) {
    __shared__ float red[2][kMaxWaves][R];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    const int cpr = cols >> 5;
    const int64_t rbytes = cols >> 1;
    const int nblocks = (rows + R - 1) / R;
    const int stride = gridDim.x;
    SzLayout L;
    L.gshift = gshift;
    L.ng = gshift >= 6 ? 1 : (64 >> gshift);
    L.G = cols >> (5 + gshift);
    L.items = CPL * R * L.ng;

    int cidx[CPL];
    bool act[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = (wave * CPL + j) * kWave + lane;
        act[j] = c < cpr;
        cidx[j] = act[j] ? c : 0;
    }
    int rb = blockIdx.x;
    RowBlock<R, CPL> bufA, bufB;
    load_row_block<R, CPL>(bufA, packed, scales, zeros, rb * R, rows, rbytes, cidx, L, wave, lane);
    XChunk<XBF16> xc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        xc[j] = load_x_chunk<XBF16>(x, cidx[j]);
        if (!act[j]) {  // lanes past the end of a row contribute nothing
#pragma unroll
            for (int q = 0; q < (XBF16 ? 4 : 8); ++q) xc[j].q[q] = u32x4{0u, 0u, 0u, 0u};
            xc[j].sum = 0.0f;
        }
    }

    // The prefetch is unconditional (the block past the end re-reads the last
    // one): a conditional load would make the compiler wait for every
    // outstanding load, prefetch included, before the current block's math.
    for (;;) {
        load_row_block<R, CPL>(bufB, packed, scales, zeros, min(rb + stride, nblocks - 1) * R,
                               rows, rbytes, cidx, L, wave, lane);
        finish_row_block<R, CPL, XBF16, YBF16>(bufA, xc, act, L, red[0], rb * R, rows, y, lane,
                                               wave, nwaves);
        rb += stride;
        if (rb >= nblocks) break;
        load_row_block<R, CPL>(bufA, packed, scales, zeros, min(rb + stride, nblocks - 1) * R,
                               rows, rbytes, cidx, L, wave, lane);
        finish_row_block<R, CPL, XBF16, YBF16>(bufB, xc, act, L, red[1], rb * R, rows, y, lane,
                                               wave, nwaves);
        rb += stride;
        if (rb >= nblocks) break;
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

int rows_per_block_override() {
    static const int v = [] {
        const char* e = getenv("KC_GEMV_ROWS_PER_BLOCK");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// Rows per workgroup iteration.
int pick_rows_per_block(int64_t rows, int waves_per_block) {
    const int o = rows_per_block_override();
    if (o == 1 || o == 2 || o == 4) return o;
    (void)rows;
    (void)waves_per_block;
    return 4;
}

int chunks_per_lane_override() {
    static const int v = [] {
        const char* e = getenv("KC_GEMV_CHUNKS_PER_LANE");
        return e ? atoi(e) : 0;
    }();
    return v;
}

int waves_per_cu_override() {
    static const int v = [] {
        const char* e = getenv("KC_GEMV_WAVES_PER_CU");
        return e ? atoi(e) : 0;
    }();
    return v;
}

int device_cu_count() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        return cus;
    }();
    return n;
}

// Persistent grid: as many workgroups as the CUs hold at once (from the
// occupancy of this kernel instance), with the same number of row blocks (to
// within one) for every workgroup.
template <int R, int CPL, bool XB, bool YB>
void launch_fast(const uint8_t* packed, const float* scales, const uint8_t* zeros, const void* x,
                 void* y, int rows, int cols, int gshift, int waves, hipStream_t stream) {
    const int threads = waves * kWave;
    static thread_local int cached_threads = -1, cached_occ = 1;
    if (cached_threads != threads) {
        int occ = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &occ, gemv_int4_fast_kernel<R, CPL, XB, YB>, threads, 0) != hipSuccess || occ < 1)
            occ = 1;
        cached_threads = threads;
        cached_occ = occ;
    }
    int per_cu = cached_occ;
    if (waves_per_cu_override() > 0) per_cu = std::max(1, std::min(per_cu, waves_per_cu_override() / waves));
    const int nblocks = (rows + R - 1) / R;
    const int max_grid = device_cu_count() * per_cu;
    const int iters = (nblocks + max_grid - 1) / max_grid;
    const unsigned grid = static_cast<unsigned>((nblocks + iters - 1) / iters);
    gemv_int4_fast_kernel<R, CPL, XB, YB><<<grid, threads, 0, stream>>>(
        packed, scales, zeros, x, y, rows, cols, gshift);
}

template <int CPL, bool XB, bool YB>
void launch_fast_r(int R, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                   const void* x, void* y, int rows, int cols, int gshift, int waves,
                   hipStream_t stream) {
    if (R >= 4) {
        if constexpr (CPL == 1)
            return launch_fast<4, 1, XB, YB>(packed, scales, zeros, x, y, rows, cols, gshift, waves, stream);
    }
    if (R >= 2) return launch_fast<2, CPL, XB, YB>(packed, scales, zeros, x, y, rows, cols, gshift, waves, stream);
    launch_fast<1, CPL, XB, YB>(packed, scales, zeros, x, y, rows, cols, gshift, waves, stream);
}

template <bool XB, bool YB>
int gemv_int4(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
              const void* x, void* y, int64_t rows, int64_t cols, int64_t gs,
              hipStream_t stream) {
    int st = check_int4_args(fn, packed, scales, zeros, x, y, rows, cols, gs);
    if (st != KC_SUCCESS) return st;
    if (rows == 0) return KC_SUCCESS;
    const int64_t cpr = cols >> 5;
    // one 16-byte chunk per lane per row: K <= 32 * 64 * 16 = 32768
    const bool fast = cols > 0 && gs >= 32 && kc::is_pow2(gs) && cpr <= 64 * kMaxWaves &&
                      rows <= INT32_MAX && kc::aligned(packed, 16) && kc::aligned(x, 16);
    if (fast) {
        const int gshift = kc::ilog2(gs) - 5;
        const int ng = gshift >= 6 ? 1 : (64 >> gshift);
        // K <= 4096: one wave covers a row with two chunks per lane (no
        // cross-wave reduction; the kernel is built for one-wave workgroups);
        // otherwise one chunk per lane and ceil(K/2048) waves.
        int cpl = (cpr <= 128 && 2 * ng <= 64) ? 2 : 1;
        if (chunks_per_lane_override() == 1) cpl = 1;
        const int waves = static_cast<int>((cpr + 64 * cpl - 1) / (64 * cpl));
        int R = pick_rows_per_block(rows, waves);
        while (R > 1 && cpl * R * ng > 64) R >>= 1;
        if (cpl == 2 && R > 2) R = 2;
        const int r = static_cast<int>(rows), c = static_cast<int>(cols);
        if (cpl == 2)
            launch_fast_r<2, XB, YB>(R, packed, scales, zeros, x, y, r, c, gshift, waves, stream);
        else
            launch_fast_r<1, XB, YB>(R, packed, scales, zeros, x, y, r, c, gshift, waves, stream);
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
