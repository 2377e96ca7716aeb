// int4_convert.hip -- GPTQ / AWQ INT4 checkpoints to the reference layout
// (quant_int4.cu:10-13, 34-48, 93-96) on gfx950.
//
// Source formats (third-party; restated from their published packing, as
// the reference only describes its own format as "GPTQ/AWQ-style",
// quant_int4.cu:5):
//   GPTQ (AutoGPTQ 0.7):  qweight int32 [K/8, N], nibble i of word (r, n) is
//                         the unsigned weight of input k = 8r + i, column n;
//                         qzeros int32 [G, N/8], nibble i of word (g, c) is
//                         the zero point of column 8c + i, stored minus
//                         zero_offset (1 in the original format, 0 in v2);
//                         scales fp16 [G, N]; g_idx int32 [K] maps input k to
//                         its group (act-order checkpoints permute it).
//   AWQ (AutoAWQ 0.2, GEMM kernels): qweight int32 [K, N/8] and qzeros int32
//                         [G, N/8], nibble i of word (r, c) belongs to column
//                         8c + order[i], order = {0, 2, 4, 6, 1, 3, 5, 7};
//                         scales fp16 [G, N]; zero points stored as is.
//   Both dequantize as W[k, n] = (u - zu) * s (u, zu unsigned 0..15).
//
// Target: packed [N, K/2] u8 (signed nibbles, low nibble = even k), scales
// [N, G] fp32, zeros [N, G/2] u8 (unsigned), W[n, k] = (sext4(q) - z) * s'.
// The weight nibble is signed and the zero unsigned, so a group is mapped
// one of two ways, both exact (the integer difference is the same and the
// scale is negated exactly):
//   zu >= 8:  q = u - 8   (nibble u ^ 8), z = zu - 8, s' =  s
//   zu <= 7:  q = 7 - u   (nibble u ^ 7), z = 7 - zu, s' = -s
// so (sext4(q) - z) * s' == (u - zu) * s for every u, zu, s: the same value,
// and the same bits except that a zero weight (u == zu) of a group stored
// with -s dequantizes to -0.
// The reference's little-endian 32-bit word of four packed bytes holds
// nibble p = weight k = base + p, the same order as a GPTQ word: a GPTQ
// word becomes an output word by one XOR, and the conversion is a transpose
// of [K/8, N] words into [N, K/8] words through LDS tiles.
#include <algorithm>

#include "kc_common.hpp"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTile = 64;  // words per tile side: 64 columns x 64 words of 8 k

__device__ __forceinline__ int gptq_zero(const int32_t* qzeros, int N, int g, int n, int offset) {
    const uint32_t w = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N >> 3) + (n >> 3)]);
    return static_cast<int>((w >> (4 * (n & 7))) & 0xFu) + offset;
}

// AWQ: column 8c + order[i] sits in nibble i; inv[j] is the nibble of column 8c + j.
__device__ __forceinline__ int awq_nibble_of(int j) {
    constexpr int inv[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    return inv[j];
}

__device__ __forceinline__ int awq_zero(const int32_t* qzeros, int N, int g, int n) {
    const uint32_t w = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N >> 3) + (n >> 3)]);
    return static_cast<int>((w >> (4 * awq_nibble_of(n & 7))) & 0xFu);
}

__device__ __forceinline__ uint32_t flip_mask(int zu) { return zu >= 8 ? 0x88888888u : 0x77777777u; }

// 8 x 8 nibble transpose: on entry nibble i of a[p] is M[p][i], on return
// nibble p of a[i] is M[p][i] (three butterfly stages: 16-, 8-, 4-bit blocks).
__device__ __forceinline__ void transpose8x8_nibbles(uint32_t (&a)[8]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t t = ((a[p] >> 16) ^ a[p + 4]) & 0x0000FFFFu;
        a[p] ^= t << 16;
        a[p + 4] ^= t;
    }
#pragma unroll
    for (int p : {0, 1, 4, 5}) {
        const uint32_t t = ((a[p] >> 8) ^ a[p + 2]) & 0x00FF00FFu;
        a[p] ^= t << 8;
        a[p + 2] ^= t;
    }
#pragma unroll
    for (int p : {0, 2, 4, 6}) {
        const uint32_t t = ((a[p] >> 4) ^ a[p + 1]) & 0x0F0F0F0Fu;
        a[p] ^= t << 4;
        a[p + 1] ^= t;
    }
}

// Packed weights.  A workgroup converts a tile of TN columns x kTile output
// words (8 k each) in two phases.  Phase 1 builds each output word
// (column n, word kb) and XORs it with its group's mask:
//   GPTQ: the source word itself (16-byte loads, four columns per thread),
//         or with perm eight nibbles gathered from the words of the
//         permuted k;
//   AWQ:  thread t takes 8 x 8 nibble blocks (rows 8kb .. 8kb+7, source
//         word c): eight loads, one transpose, and the eight output words of
//         columns 8c + order[i]; the group's zero points are one qzeros word
//         in the same nibble order.
// Phase 2 writes the tile transposed, 256 contiguous bytes per column.
// The plain GPTQ tile is TN = 128 columns wide (512 contiguous source bytes
// per row; every load of a thread issued before the first is used): for the
// gate/up layer 26.1 -> 23.3 us per launch back to back, but only 32.7 -> 32.4
// us for a whole conversion call (this kernel, then the scales and zero points).
template <bool AWQ, bool PERM, int TN>
__device__ __forceinline__ void convert_packed_tile(
    const int32_t* __restrict__ qweight, const int32_t* __restrict__ qzeros,
    const int32_t* __restrict__ perm, int K, int N, int gs, int zero_offset,
    uint32_t* __restrict__ out, bool vec, int b, int nb, uint32_t (*tile)[TN + 1]) {
    static_assert(TN == kTile || (!AWQ && !PERM), "wider tiles for the plain GPTQ source only");
    // tile: [word kb][column n], kTile x (TN + 1) words of LDS
    const int KW = K >> 3;                       // output words per column
    const int NW = N >> 3;                       // source words per row (AWQ, qzeros)
    // Tiles in column-tile-major order.  AWQ reads 32 bytes of a source row
    // per tile, so there each XCD (workgroup b runs on XCD b % 8) takes a
    // contiguous share of the tiles: the column tiles that share a row's
    // 128-byte lines run on one XCD at about the same time and meet in its
    // L2 (56 -> 36 us on the gate/up layer).  GPTQ reads 256 or (plain
    // source) 512 contiguous bytes per row and keeps the plain order (64-column
    // tiles: 35.1 us remapped, 33.5 plain).
    const int xcd = b % 8, q = nb / 8, r = nb % 8;
    const int tile_id = AWQ ? xcd * q + min(xcd, r) + b / 8 : b;  // a bijection of [0, nb)
    const int ntn = (N + TN - 1) / TN;
    const int n0 = (tile_id % ntn) * TN, kb0 = (tile_id / ntn) * kTile;
    const int t = threadIdx.x;
    if constexpr (AWQ) {
        constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
#pragma unroll
        for (int i = 0; i < kTile * (kTile / 8) / kThreads; ++i) {
            const int kbl = t / 8 + (kThreads / 8) * i, kb = kb0 + kbl;
            const int cl = t % 8, c = (n0 >> 3) + cl;
            uint32_t a[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
            if (kb < KW && c < NW) {
#pragma unroll
                for (int p = 0; p < 8; ++p)
                    a[p] = static_cast<uint32_t>(qweight[static_cast<int64_t>(8 * kb + p) * NW + c]);
                transpose8x8_nibbles(a);
                const uint32_t zw = static_cast<uint32_t>(qzeros[static_cast<int64_t>((8 * kb) / gs) * NW + c]);
#pragma unroll
                for (int q = 0; q < 8; ++q) a[q] ^= flip_mask(static_cast<int>((zw >> (4 * q)) & 0xFu));
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) tile[kbl][8 * cl + order[q]] = a[q];
        }
    } else if constexpr (!PERM) {
        // thread t builds words (kb0 + t/kTPR + kRPI i, n0 + 4(t%kTPR) + c), c < 4:
        // every source load first, then the flips
        constexpr int kTPR = TN / 4, kRPI = kThreads / kTPR, kPasses = kTile / kRPI;
        u32x4 v[kPasses];
        uint32_t zw[kPasses];
#pragma unroll
        for (int i = 0; i < kPasses; ++i) {
            const int kb = kb0 + t / kTPR + kRPI * i, nb = n0 + 4 * (t % kTPR);
            v[i] = u32x4{0u, 0u, 0u, 0u};
            zw[i] = 0u;
            if (kb < KW && nb < N) {  // N % 8 == 0: all four columns or none
                v[i] = __builtin_bit_cast(
                    u32x4, *reinterpret_cast<const int32_t __attribute__((ext_vector_type(4)))*>(
                               qweight + static_cast<int64_t>(kb) * N + nb));
                zw[i] = static_cast<uint32_t>(qzeros[static_cast<int64_t>((8 * kb) / gs) * NW + (nb >> 3)]);
            }
        }
#pragma unroll
        for (int i = 0; i < kPasses; ++i) {
            const int kbl = t / kTPR + kRPI * i, nl0 = 4 * (t % kTPR), kb = kb0 + kbl, nb = n0 + nl0;
            const bool ok = kb < KW && nb < N;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                tile[kbl][nl0 + c] =
                    ok ? v[i][c] ^ flip_mask(static_cast<int>((zw[i] >> (4 * ((nb + c) & 7))) & 0xFu) + zero_offset)
                       : 0u;
        }
    } else {
        // act order: thread t builds words (kb0 + t/16 + 16i, n0 + 4(t%16) + c), c < 4,
        // each from the eight nibbles of the permuted k
        for (int i = 0; i < kTile / 16; ++i) {
            const int kbl = t / 16 + 16 * i, kb = kb0 + kbl;
            const int nl0 = 4 * (t % 16), nb = n0 + nl0;  // N % 8 == 0: all four columns or none
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            if (kb < KW && nb < N) {
                for (int c = 0; c < 4; ++c) {
                    for (int p = 0; p < 8; ++p) {
                        // clamped: a malformed permutation gives wrong
                        // values, never an access outside qweight
                        const int k = min(max(perm[8 * kb + p], 0), K - 1);
                        const uint32_t src = static_cast<uint32_t>(
                            qweight[static_cast<int64_t>(k >> 3) * N + nb + c]);
                        w[c] |= ((src >> (4 * (k & 7))) & 0xFu) << (4 * p);
                    }
                }
                const int g = (8 * kb) / gs;  // gs % 8 == 0: one group per word
                const uint32_t zw = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * NW + (nb >> 3)]);
                for (int c = 0; c < 4; ++c)
                    w[c] ^= flip_mask(static_cast<int>((zw >> (4 * ((nb + c) & 7))) & 0xFu) + zero_offset);
            }
            for (int c = 0; c < 4; ++c) tile[kbl][nl0 + c] = w[c];
        }
    }
    __syncthreads();
    // phase 2: thread t writes words (kb0 + 4(t%16) .. +3) of column n0 + t/16 + 16i
    for (int i = 0; i < TN / 16; ++i) {
        const int nl = t / 16 + 16 * i, n = n0 + nl;
        const int kbl = 4 * (t % 16), kb = kb0 + kbl;
        if (n >= N) continue;
        uint32_t* dst = out + static_cast<int64_t>(n) * KW + kb;
        if (vec && kb + 4 <= KW) {
            *reinterpret_cast<u32x4*>(dst) = u32x4{tile[kbl][nl], tile[kbl + 1][nl], tile[kbl + 2][nl], tile[kbl + 3][nl]};
        } else {
            for (int c = 0; c < 4 && kb + c < KW; ++c) dst[c] = tile[kbl + c][nl];
        }
    }
}

// Scales and zero points of 64 columns x 32 groups per workgroup, through
// LDS so that both the [G, N] sources and the [N, G] outputs are read and
// written along their rows.
constexpr int kMetaCols = 64, kMetaGroups = 32;

template <bool AWQ>
__device__ __forceinline__ void convert_meta_tile(
    const int32_t* __restrict__ qzeros, const uint16_t* __restrict__ scales16, int N, int G,
    int zero_offset, float* __restrict__ scales, uint8_t* __restrict__ zeros, int bx, int by,
    float (*sv)[kMetaCols + 1], uint8_t (*zv)[kMetaCols + 4]) {
    const int n0 = bx * kMetaCols, g0 = by * kMetaGroups;
    const int t = threadIdx.x;
    // read: thread t handles column n0 + t % 64 of groups g0 + t / 64 + 4i
    for (int i = 0; i < kMetaGroups / 4; ++i) {
        const int gl = t / kMetaCols + 4 * i, g = g0 + gl, nl = t % kMetaCols, n = n0 + nl;
        if (g < G && n < N) {
            const uint32_t zw = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N >> 3) + (n >> 3)]);
            const int zu = AWQ ? static_cast<int>((zw >> (4 * awq_nibble_of(n & 7))) & 0xFu)
                               : static_cast<int>((zw >> (4 * (n & 7))) & 0xFu) + zero_offset;
            // fp16 -> fp32 is exact
            const float s = static_cast<float>(__builtin_bit_cast(_Float16, scales16[static_cast<int64_t>(g) * N + n]));
            const bool up = zu >= 8;
            sv[gl][nl] = up ? s : -s;
            zv[gl][nl] = static_cast<uint8_t>(up ? zu - 8 : 7 - zu);
        }
    }
    __syncthreads();
    // write: scales row n, groups g0 .. g0 + 31 (thread t: column t / 4, 8 groups)
    {
        const int nl = t / 4, n = n0 + nl, gb = 8 * (t % 4);
        if (n < N) {
            float* dst = scales + static_cast<int64_t>(n) * G + g0 + gb;
            if ((G & 3) == 0 && g0 + gb + 8 <= G) {  // 16-byte aligned: G % 4 == 0
                reinterpret_cast<f32x4*>(dst)[0] = f32x4{sv[gb][nl], sv[gb + 1][nl], sv[gb + 2][nl], sv[gb + 3][nl]};
                reinterpret_cast<f32x4*>(dst)[1] = f32x4{sv[gb + 4][nl], sv[gb + 5][nl], sv[gb + 6][nl], sv[gb + 7][nl]};
            } else {
                for (int e = 0; e < 8 && g0 + gb + e < G; ++e) dst[e] = sv[gb + e][nl];
            }
        }
    }
    // zeros row n: bytes g0/2 .. g0/2 + 15 (thread t < 64: column t)
    if (t < kMetaCols) {
        const int n = n0 + t;
        if (n < N) {
            uint8_t* dst = zeros + static_cast<int64_t>(n) * (G >> 1) + (g0 >> 1);
            for (int e = 0; e < kMetaGroups / 2 && g0 + 2 * e + 1 < G; ++e)
                dst[e] = static_cast<uint8_t>(zv[2 * e][t] | (zv[2 * e + 1][t] << 4));
        }
    }
}

// One launch for both parts: blocks [0, meta_blocks) convert scales and zero
// points (tile (b % mx, b / mx) of 64 columns x 32 groups; blocks past the
// last tile pad meta_blocks to a multiple of 8 and return), the rest the
// packed weights, which then start on XCD 0 as in a launch of their own.  The
// two parts share one LDS buffer.  Against two launches, the short
// scales/zero-points tiles run beside the weight stream instead of after it.
template <bool AWQ, bool PERM, int TN>
__global__ __launch_bounds__(kThreads) void convert_kernel(
    const int32_t* __restrict__ qweight, const int32_t* __restrict__ qzeros,
    const int32_t* __restrict__ perm, const uint16_t* __restrict__ scales16, int K, int N, int gs,
    int zero_offset, uint32_t* __restrict__ out, bool vec, float* __restrict__ scales,
    uint8_t* __restrict__ zeros, int meta_blocks) {
    constexpr int kPackedWords = kTile * (TN + 1);
    constexpr int kMetaWords = kMetaGroups * (kMetaCols + 1) + kMetaGroups * (kMetaCols + 4) / 4;
    __shared__ uint32_t smem[kPackedWords > kMetaWords ? kPackedWords : kMetaWords];
    const int b = blockIdx.x;
    if (b < meta_blocks) {
        const int G = K / gs, mx = (N + kMetaCols - 1) / kMetaCols, my = (G + kMetaGroups - 1) / kMetaGroups;
        if (b >= mx * my) return;
        convert_meta_tile<AWQ>(qzeros, scales16, N, G, zero_offset, scales, zeros, b % mx, b / mx,
                               reinterpret_cast<float (*)[kMetaCols + 1]>(smem),
                               reinterpret_cast<uint8_t (*)[kMetaCols + 4]>(smem + kMetaGroups * (kMetaCols + 1)));
        return;
    }
    convert_packed_tile<AWQ, PERM, TN>(qweight, qzeros, perm, K, N, gs, zero_offset, out, vec,
                                       b - meta_blocks, static_cast<int>(gridDim.x) - meta_blocks,
                                       reinterpret_cast<uint32_t (*)[TN + 1]>(smem));
}

int check_convert(const char* fn, const void* qweight, const void* qzeros, const void* scales16,
                  int K, int N, int gs, const void* packed, const void* scales, const void* zeros) {
    if (K <= 0 || N <= 0 || gs <= 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: K=%d N=%d group_size=%d must be positive",
                             fn, K, N, gs);
    if (K % 8 || N % 8 || gs % 8 || K % gs)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                             "%s: K=%d and N=%d must be multiples of 8, group_size=%d a multiple "
                             "of 8 dividing K", fn, K, N, gs);
    if ((K / gs) % 2)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                             "%s: K / group_size = %d groups per row is odd; the zero-point layout "
                             "(row stride floor(G/2) bytes, quant_int4.cu:93) needs an even count",
                             fn, K / gs);
    if (!qweight || !qzeros || !scales16 || !packed || !scales || !zeros)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    return KC_SUCCESS;
}

template <bool AWQ>
int convert(const char* fn, const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales16,
            const int32_t* perm, int K, int N, int gs, int zero_offset, uint8_t* packed,
            float* scales, uint8_t* zeros, hipStream_t stream) {
    int st = check_convert(fn, qweight, qzeros, scales16, K, N, gs, packed, scales, zeros);
    if (st != KC_SUCCESS) return st;
    constexpr int kWide = 2 * kTile;  // the plain GPTQ tile's columns
    const bool wide = !AWQ && !perm;
    const int tn = wide ? kWide : kTile;
    const unsigned grid = static_cast<unsigned>(((N + tn - 1) / tn) * ((K / 8 + kTile - 1) / kTile));
    uint32_t* out = reinterpret_cast<uint32_t*>(packed);
    if (!kc::aligned(packed, 4) || !kc::aligned(qweight, 16) || !kc::aligned(qzeros, 4) ||
        !kc::aligned(scales16, 2) || !kc::aligned(scales, 16) || (perm && !kc::aligned(perm, 4)))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: misaligned pointer", fn);
    const bool vec = (K / 8) % 4 == 0 && kc::aligned(packed, 16);
    const int G = K / gs;
    const int meta = ((N + kMetaCols - 1) / kMetaCols) * ((G + kMetaGroups - 1) / kMetaGroups);
    const int meta_blocks = (meta + 7) / 8 * 8;
    const unsigned all = grid + static_cast<unsigned>(meta_blocks);
    if (AWQ)
        convert_kernel<true, false, kTile><<<all, kThreads, 0, stream>>>(qweight, qzeros, nullptr, scales16, K, N, gs, 0, out, vec, scales, zeros, meta_blocks);
    else if (perm)
        convert_kernel<false, true, kTile><<<all, kThreads, 0, stream>>>(qweight, qzeros, perm, scales16, K, N, gs, zero_offset, out, vec, scales, zeros, meta_blocks);
    else
        convert_kernel<false, false, kWide><<<all, kThreads, 0, stream>>>(qweight, qzeros, nullptr, scales16, K, N, gs, zero_offset, out, vec, scales, zeros, meta_blocks);
    return kc::check_launch(fn);
}

// ---------------------------------------------------------------------------
// The reference layout to the shuffled layout that the matrix-core GEMMs can
// also read (int4_gemm_mfma.hip, tile_lane_ptr).  Rows go in tiles of 16 (the
// last tile padded with zero rows), K in T-blocks of 128 (64 bytes of a
// row); block (tile t, T-block T) is the 1 KB at byte (t * K/128 + T) * 1024
// and its 16-byte unit l = 16 kb + i (i < 16, kb < 4) holds bytes
// 16 kb .. 16 kb + 15 of T-block T of row 16 t + i: the 16 bytes that lane l
// of a wave feeds to the matrix core for that tile and T-block.  A
// permutation of the 16-byte units, plus the pad.  One thread per output
// unit: the writes are in address order, each read is 16 bytes of a row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void shuffle_mfma_kernel(const u32x4* __restrict__ in,
                                                                u32x4* __restrict__ out, int64_t rows,
                                                                int64_t cols, int64_t units) {
    const int64_t nT = cols / 128;
    const int64_t row_units = cols / 32;  // 16-byte units of a row
    for (int64_t u = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; u < units;
         u += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t blk = u >> 6;
        const int l = static_cast<int>(u & 63);
        const int64_t tile = blk / nT, T = blk - tile * nT;
        const int64_t row = tile * 16 + (l & 15);
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (row < rows) v = in[row * row_units + T * 4 + (l >> 4)];
        out[u] = v;
    }
}

}  // namespace

extern "C" int64_t kc_shuffled_int4_bytes(int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0 || cols % 128 != 0) return -1;
    return (rows + 15) / 16 * 16 * (cols / 2);
}

extern "C" int kc_shuffle_int4_mfma(const uint8_t* d_packed, uint8_t* d_packed_shuffled, int rows,
                                    int cols, kc_stream_t stream) {
    const char* fn = "kc_shuffle_int4_mfma";
    if (rows < 0 || cols < 0 || cols % 128 != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                             "%s: rows=%d cols=%d (cols must be a multiple of 128)", fn, rows, cols);
    if (rows == 0 || cols == 0) return KC_SUCCESS;
    if (!d_packed || !d_packed_shuffled)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    if (!kc::aligned(d_packed, 16) || !kc::aligned(d_packed_shuffled, 16))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: both buffers must be 16-byte aligned", fn);
    const int64_t units = kc_shuffled_int4_bytes(rows, cols) / 16;
    const int64_t blocks = std::min<int64_t>((units + kThreads - 1) / kThreads, 8192);
    shuffle_mfma_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(
        reinterpret_cast<const u32x4*>(d_packed), reinterpret_cast<u32x4*>(d_packed_shuffled), rows,
        cols, units);
    return kc::check_launch(fn);
}

extern "C" int kc_convert_gptq_int4(const int32_t* d_qweight, const int32_t* d_qzeros,
                                    const uint16_t* d_scales_f16, const int32_t* d_perm, int K,
                                    int N, int group_size, int zero_offset, uint8_t* d_packed,
                                    float* d_scales, uint8_t* d_zeros, kc_stream_t stream) {
    const char* fn = "kc_convert_gptq_int4";
    if (zero_offset < 0 || zero_offset > 1)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: zero_offset=%d (0 or 1)", fn, zero_offset);
    return convert<false>(fn, d_qweight, d_qzeros, d_scales_f16, d_perm, K, N, group_size,
                          zero_offset, d_packed, d_scales, d_zeros, stream);
}

extern "C" int kc_convert_awq_int4(const int32_t* d_qweight, const int32_t* d_qzeros,
                                   const uint16_t* d_scales_f16, int K, int N, int group_size,
                                   uint8_t* d_packed, float* d_scales, uint8_t* d_zeros,
                                   kc_stream_t stream) {
    return convert<true>("kc_convert_awq_int4", d_qweight, d_qzeros, d_scales_f16, nullptr, K, N,
                         group_size, 0, d_packed, d_scales, d_zeros, stream);
}
