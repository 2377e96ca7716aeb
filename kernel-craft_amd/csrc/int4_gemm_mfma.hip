// int4_gemm_mfma.hip -- small-batch INT4 GEMM on gfx950 matrix cores.
//
// Y[m, n] = sum_k X[m, k] * W[n, k] for 1 <= M <= 64 activation rows (bf16),
// with W in the reference's INT4 format (quant_int4.cu:10-13): the
// reference's GEMV applied to every row of X, in one pass over the weights.
//
// v_mfma_f32_16x16x32_bf16 computes D[16 x 16] += A[16 x 32] * B[32 x 16].
// A is a 16-row tile of W, B a 16-row tile of X (transposed), D = Y^T.
// Operand layout (per lane l, i = l % 16, kb = l / 16):
//   A: 8 bf16 of W row i, k-slots 8*kb .. 8*kb+7
//   B: 8 bf16 of X row i, same k-slots
//   D: Y^T rows 4*kb + v (v = 0..3), column i
// Any bijection between k-slots and real k that A and B share gives the same
// contraction.  Each 128-k block is one lane-load of 16 bytes per W row (lane
// (i, kb) reads bytes 16*kb .. 16*kb+15 of the block, 32 nibbles); MFMA step t
// (t = 0..3) takes dword t, whose 8 nibbles become the bf16 pairs
// (k0,k4) (k1,k5) (k2,k6) (k3,k7) -- exact values 128 + (q ^ 8), one bitwise
// op each -- so the B operand holds X in the same pair order.
//
// The block lies inside one quantization group (gs a multiple of 128), so
// the block's MFMA sum C is folded into the fp32 accumulator as
//     acc += s * (C - (136 + z) * sum_k X[m, k])
// which removes the +128 encoding offset, the +8 of q ^ 8 and the zero point
// exactly as the GEMV does.  Groups smaller than 128 fall back to the GEMV
// per activation row.
#include <algorithm>

#include "kc_common.hpp"

namespace {

using kc::kWave;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kKBlock = 128;  // k per block: 64 bytes of each W row

__device__ __forceinline__ uint32_t nib_bf16_pair(uint32_t d) {
    return ((d ^ 0x00080008u) & 0x000F000Fu) | 0x43004300u;
}

__device__ __forceinline__ bf16x8_t a_operand(uint32_t d) {
    const u32x4 p{nib_bf16_pair(d), nib_bf16_pair(d >> 4), nib_bf16_pair(d >> 8),
                  nib_bf16_pair(d >> 12)};
    return __builtin_bit_cast(bf16x8_t, p);
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// LDS image of one 128-k block of X: B operands bop[mt][t][lane] (16 bytes)
// and the per-row block sums xsum[m].
template <int MT>
struct XBlock {
    u32x4 bop[MT][4][kWave];
    float xsum[MT * 16];
};

// All 256 threads stage X[0 .. 16*MT) x [k0, k0 + 128) into `xb`.  Item
// (m, u) is the 8-element slice k0 + 8u .. 8u + 7 of row m; it becomes the B
// operand of step t = u % 4 for lane (m % 16) + 16 * (u / 4).  Rows >= M are
// zero.  The 16 items of a row sit in 16 consecutive lanes for the row sum.
template <int MT>
__device__ __forceinline__ void stage_x_block(const uint16_t* __restrict__ X, int M, int K,
                                              int k0, XBlock<MT>& xb) {
#pragma unroll
    for (int it = 0; it < MT; ++it) {
        const int idx = it * kThreads + threadIdx.x;
        const int m = idx >> 4, u = idx & 15;
        u32x4 d{0u, 0u, 0u, 0u};
        if (m < M) d = *reinterpret_cast<const u32x4*>(X + static_cast<int64_t>(m) * K + k0 + 8 * u);
        u32x4 p;
        p.x = (d.x & 0xFFFFu) | (d.z << 16);
        p.y = (d.x >> 16) | (d.z & 0xFFFF0000u);
        p.z = (d.y & 0xFFFFu) | (d.w << 16);
        p.w = (d.y >> 16) | (d.w & 0xFFFF0000u);
        xb.bop[m >> 4][u & 3][(m & 15) + 16 * (u >> 2)] = p;
        float part = ((bf16_lo(d.x) + bf16_hi(d.x)) + (bf16_lo(d.y) + bf16_hi(d.y))) +
                     ((bf16_lo(d.z) + bf16_hi(d.z)) + (bf16_lo(d.w) + bf16_hi(d.w)));
        part += __shfl_xor(part, 1, kWave);
        part += __shfl_xor(part, 2, kWave);
        part += __shfl_xor(part, 4, kWave);
        part += __shfl_xor(part, 8, kWave);
        if (u == 0) xb.xsum[m] = part;
    }
}

template <int MT>
__global__ __launch_bounds__(kThreads) void gemm_int4_mfma_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int M, int N, int K, int gshift) {
    __shared__ XBlock<MT> xbuf[2];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int li = lane & 15, kb = lane >> 4;
    const int n0 = (blockIdx.x * kWaves + wave) * 16;
    const int G = K >> (7 + gshift);  // gs = 128 << gshift
    const int64_t rbytes = K >> 1;
    // this lane's A row and the 4 D rows (4*kb + v) whose scale/zero it needs
    const int64_t arow = std::min(n0 + li, N - 1);
    const u32x4* wptr = reinterpret_cast<const u32x4*>(packed + arow * rbytes) + kb;
    int64_t drow[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) drow[v] = std::min(n0 + 4 * kb + v, N - 1);

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nblk = K / kKBlock;
    stage_x_block<MT>(X, M, K, 0, xbuf[0]);
    u32x4 wv = __builtin_nontemporal_load(wptr);
    __syncthreads();
    for (int b = 0; b < nblk; ++b) {
        XBlock<MT>& cur = xbuf[b & 1];
        u32x4 wnext = wv;
        if (b + 1 < nblk) {
            stage_x_block<MT>(X, M, K, (b + 1) * kKBlock, xbuf[(b + 1) & 1]);
            wnext = __builtin_nontemporal_load(wptr + 4 * (b + 1));
        }
        const int g = (b * kKBlock) >> (7 + gshift);
        float s[4], zc[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            s[v] = scales[drow[v] * G + g];
            const uint32_t zb = zeros[drow[v] * (G >> 1) + (g >> 1)];
            zc[v] = -static_cast<float>(136u + ((g & 1) ? (zb >> 4) : (zb & 0xFu)));
        }
        f32x4 c[MT];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t d = t == 0 ? wv.x : t == 1 ? wv.y : t == 2 ? wv.z : wv.w;
            const bf16x8_t a = a_operand(d);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const u32x4 bv = cur.bop[mt][t][lane];
                const bf16x8_t bo = __builtin_bit_cast(bf16x8_t, bv);
                c[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    a, bo, t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : c[mt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const float xs = cur.xsum[mt * 16 + li];
            const f32x4 cm = c[mt];
            f32x4 a4 = acc[mt];
            a4.x = fmaf(s[0], fmaf(zc[0], xs, cm.x), a4.x);
            a4.y = fmaf(s[1], fmaf(zc[1], xs, cm.y), a4.y);
            a4.z = fmaf(s[2], fmaf(zc[2], xs, cm.z), a4.z);
            a4.w = fmaf(s[3], fmaf(zc[3], xs, cm.w), a4.w);
            acc[mt] = a4;
        }
        wv = wnext;
        __syncthreads();
    }
    // lane holds Y[m = 16*mt + li][n0 + 4*kb + v]
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + li;
        if (m >= M) continue;
        const f32x4 a4 = acc[mt];
        const float vals[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = n0 + 4 * kb + v;
            if (n < N) Y[static_cast<int64_t>(m) * N + n] = kc::f32_to_bf16(vals[v]);
        }
    }
}

template <int MT>
void launch_mfma(const uint8_t* packed, const float* scales, const uint8_t* zeros,
                 const uint16_t* X, uint16_t* Y, int M, int N, int K, int gshift,
                 hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>((N + 16 * kWaves - 1) / (16 * kWaves));
    gemm_int4_mfma_kernel<MT><<<grid, kThreads, 0, stream>>>(packed, scales, zeros, X, Y, M, N, K,
                                                             gshift);
}

}  // namespace

extern "C" int kc_gemm_int4_bf16(const uint8_t* d_packed, const float* d_scales,
                                 const uint8_t* d_zeros, const uint16_t* d_x, uint16_t* d_y,
                                 int m, int rows, int cols, int group_size, kc_stream_t stream) {
    const char* fn = "kc_gemm_int4_bf16";
    if (m < 0 || m > 64)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: m=%d must be in [0, 64]", fn, m);
    if (rows < 0 || cols < 0 || group_size <= 0 || cols % 2 != 0 || cols % group_size != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                             "%s: invalid shape rows=%d cols=%d group_size=%d", fn, rows, cols,
                             group_size);
    if (m == 0 || rows == 0) return KC_SUCCESS;
    if (!d_y || (cols > 0 && (!d_packed || !d_scales || !d_zeros || !d_x)))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    const bool fast = cols > 0 && cols % kKBlock == 0 && group_size % kKBlock == 0 &&
                      kc::is_pow2(group_size) && kc::aligned(d_packed, 16) &&
                      kc::aligned(d_x, 16);
    if (!fast) {
        // One GEMV per activation row: same results, no matrix cores.
        for (int i = 0; i < m; ++i) {
            const int st = kc_gemv_int4_bf16(d_packed, d_scales, d_zeros,
                                             d_x + static_cast<int64_t>(i) * cols,
                                             d_y + static_cast<int64_t>(i) * rows, rows, cols,
                                             group_size, stream);
            if (st != KC_SUCCESS) return st;
        }
        return KC_SUCCESS;
    }
    const int gshift = kc::ilog2(group_size) - 7;
    switch ((m + 15) / 16) {
        case 1: launch_mfma<1>(d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
        case 2: launch_mfma<2>(d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
        case 3: launch_mfma<3>(d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
        default: launch_mfma<4>(d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
    }
    return kc::check_launch(fn);
}
