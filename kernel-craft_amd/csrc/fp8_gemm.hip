// fp8_gemm.hip -- W8A8 FP8 GEMM on gfx950 matrix cores: the consumer of the
// FP8 quantizers (fp8_quant.hip).
//
//   Y[m, n] = sx[m] * sw[n] * sum_k e4m3(qx[m, k]) * e4m3(qw[n, k])
//
// qx [M, K] are per-token E4M3 codes of the activations with scales sx [M]
// (kc_quantize_fp8_per_token_* / _smooth_div_*), qw [N, K] per-output-channel
// codes of the weights with scales sw [N] (kc_quantize_fp8_per_token_* /
// _smooth_mul_bf16 on W).  The reference has no FP8 GEMM; its example
// dequantizes the codes and multiplies in fp32
// (examples/python/transformer/fp8_quant.py:55-60), which is what the tests'
// oracle does in fp64.
//
// Products of two E4M3 values are exact in fp32 (4-bit significands).  The
// matrix core (v_mfma_scale_f32_16x16x128_f8f6f4, block scales fixed at 2^0)
// does not accumulate them as IEEE fp32 adds: measured on MI355X, the
// products of each block of 8 consecutive k are aligned to the block's
// largest and truncated toward zero 14 bits below its leading bit before the
// block sum joins the fp32 accumulator; E4M3 subnormals are exact.  Integer
// valued codes (|v| <= 16) therefore come out exact, and in general each
// output is within 2^-10 sum_k |product| of the exact sum.  The scales are
// applied once per output: (acc * sx) * sw.
//
// Tiling.  A 512-thread workgroup (8 waves) computes a 256 x 256 tile of Y;
// wave w owns the 128 x 64 block (w / 4, w % 4) as 8 x 4 MFMA tiles of
// 16 x 16 (128 fp32 accumulators per lane).  K advances 128 at a time: the
// workgroup's 256 rows of qx and 256 rows of qw for a step (32 KB each) go
// from global memory straight into LDS (global_load_lds_dwordx4, no
// registers in between), double-buffered: step s + 1's loads are issued
// right after the step's barrier, before step s is multiplied.  Each wave
// reads its operands from LDS: lane (i, kb) of an A or B operand holds bytes
// 32 kb .. 32 kb + 31 of row i of a 16-row block -- the same byte slots for
// both operands, so each product pairs equal k.  Within a step the four B
// blocks and the first two A blocks are read first, then each A block two
// groups of four MFMAs ahead of its use, in a pinned order.
//
// LDS rows are 128 bytes with the 16-byte chunks XOR-swizzled by the row
// (chunk c of row r at slot c ^ ((r / 2) % 8)): a wave's load instruction
// fills 1 KB = 8 whole rows, and the operand reads (16 consecutive rows, one
// chunk pair per lane group) measure free of bank conflicts.
//
// Tails.  Rows past M (N) load row M - 1 (N - 1): they only feed outputs
// that are not stored.  In a last step with K % 128 != 0, the chunks past K
// load the last valid chunk and the operand registers holding them are
// zeroed before the MFMA, in both operands (so that a NaN code there cannot
// reach a stored output).
//
// Order.  Workgroup b runs on XCD b % 8; each XCD takes a contiguous share
// of the tile list, which is ordered in groups of kGroupM row tiles walked
// column by column, so that the 32 tiles an XCD holds at once form a 4 x 8
// block whose qx and qw rows its L2 shares.
//
// Output.  The MFMAs take the qw block as A and the qx block as B, so a
// lane's four accumulators of a 16 x 16 tile are four neighbouring columns
// of one row (the products and their summation are the same either way).
// With bf16 Y each wave stages its 128 x 64 block in its own 16 KB of LDS and
// writes 128-byte row pieces, 16 bytes per lane, with nontemporal stores;
// otherwise each lane writes its four columns at once (8 or 16 bytes).  Every
// workgroup of the grid finishes its tile at about the same time, so the
// stores go out as one burst with the matrix cores idle: the earlier
// epilogue, one 2-byte store per output, cost cfg4's shape 4153 against
// 3681 us, and the staged rows save another 2 % (3749 against 3835 us).
#include <algorithm>

#include "kc_common.hpp"

namespace {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

constexpr int kThreads = 512;
constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kTileBytes = kBM * kBK;            // one operand, one step
constexpr int kStageBytes = 2 * kTileBytes;      // qx rows then qw rows
constexpr int kScaleOff = 2 * kStageBytes;       // double buffer: 128 KB
constexpr int kLdsBytes = kScaleOff + (kBM + kBN) * 4;  // + the tile's sx and sw
constexpr int kGroupM = 4;
constexpr int kE8M0One = 127;                    // block scale 2^0
// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedMfma = 0x008, kSchedDsRead = 0x100;

__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 7; }

// One global_load_lds_dwordx4: 16 bytes per lane from `g` into LDS at
// lds_base + 16 * lane.  Written as inline assembly so that the compiler's
// LDS-wait bookkeeping does not see it: with such a load in flight the
// compiler cannot count the ordinary LDS reads and drains them all before
// every use.  The kernel waits for these loads itself (vmcnt(0) before the
// barrier that publishes the buffer), and the "memory" clobber keeps LDS
// reads and writes on their side of it.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_address(const uint8_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<size_t>((lds_void*)p));
}

// Issue the loads of one operand's 256 x 128-byte step tile into LDS.  Wave
// w fills rows 32 w .. 32 w + 31 with four 1-KB instructions; lane l of
// instruction i carries row 32 w + 8 i + l / 8 into slot l % 8, i.e. chunk
// (l % 8) ^ swizzle(row).  Rows past the end load the last row, chunks past
// K the last valid chunk (their operand bytes are masked before use).
__device__ __forceinline__ void load_tile_lds(const int8_t* src, int64_t rows, int64_t K, int64_t r0,
                                              int64_t k0, uint8_t* tile, int wave, int lane) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_address(tile + 32 * wave * kBK));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 32 * wave + 8 * i + (lane >> 3);
        const int chunk = (lane & 7) ^ swizzle(row);
        const int64_t k = min(k0 + 16 * chunk, K - 16);
        const int64_t r = min(r0 + row, rows - 1);
        lds_dma16(src + r * K + k, base + 8 * i * kBK);
    }
}

__device__ __forceinline__ void load_stage(const int8_t* qx, const int8_t* qw, int64_t M, int64_t N,
                                           int64_t K, int64_t m0, int64_t n0, int64_t k0,
                                           uint8_t* stage, int wave, int lane) {
    load_tile_lds(qx, M, K, m0, k0, stage, wave, lane);
    load_tile_lds(qw, N, K, n0, k0, stage + kTileBytes, wave, lane);
}

// Operand of the 16-row block at tile row r0: lane (i, kb) gets bytes
// 32 kb .. 32 kb + 31 of row r0 + i; with kvalid < 128 the 16-byte halves at
// or past kvalid read as zeros.
template <bool TAIL>
__device__ __forceinline__ i32x8 read_operand(const uint8_t* tile, int r0, int lane, int kvalid) {
    const int row = r0 + (lane & 15), kb = lane >> 4, sw = swizzle(row);
    const uint8_t* p = tile + row * kBK;
    u32x4 lo = *reinterpret_cast<const u32x4*>(p + 16 * ((2 * kb) ^ sw));
    u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16 * ((2 * kb + 1) ^ sw));
    if constexpr (TAIL) {
        if (32 * kb >= kvalid) lo = u32x4{0u, 0u, 0u, 0u};
        if (32 * kb + 16 >= kvalid) hi = u32x4{0u, 0u, 0u, 0u};
    }
    return i32x8{static_cast<int32_t>(lo.x), static_cast<int32_t>(lo.y), static_cast<int32_t>(lo.z),
                 static_cast<int32_t>(lo.w), static_cast<int32_t>(hi.x), static_cast<int32_t>(hi.y),
                 static_cast<int32_t>(hi.z), static_cast<int32_t>(hi.w)};
}

template <bool TAIL>
__device__ __forceinline__ void mfma_step(const uint8_t* stage, int wm, int wn, int lane, int kvalid,
                                          f32x4 (&acc)[8][4]) {
    const uint8_t* at = stage;
    const uint8_t* bt = stage + kTileBytes;
    // One A operand is read ahead of the four MFMAs that use the previous
    // one; the scheduling fences keep the compiler from hoisting all eight
    // reads (which would not fit beside the accumulators).
    i32x8 b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = read_operand<TAIL>(bt, 64 * wn + 16 * j, lane, kvalid);
    i32x8 a = read_operand<TAIL>(at, 128 * wm, lane, kvalid);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        i32x8 a_next = a;
        if (i + 1 < 8) a_next = read_operand<TAIL>(at, 128 * wm + 16 * (i + 1), lane, kvalid);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b[j], a, acc[i][j], 0, 0, 0,
                                                                         kE8M0One, 0, kE8M0One);
        __builtin_amdgcn_sched_barrier(0);
        a = a_next;
    }
}

// One full step (no tail masks) with the A blocks read two groups ahead of
// their four MFMAs, in a pinned order: B blocks and A blocks 0, 1 first,
// then (read A block i + 2, MFMAs of A block i) for i = 0 .. 7.
__device__ __forceinline__ void mfma_step_full(const uint8_t* stage, int wm, int wn, int lane,
                                               f32x4 (&acc)[8][4]) {
    const uint8_t* at = stage;
    const uint8_t* bt = stage + kTileBytes;
    i32x8 b[4], a[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = read_operand<false>(bt, 64 * wn + 16 * j, lane, kBK);
    a[0] = read_operand<false>(at, 128 * wm, lane, kBK);
    a[1] = read_operand<false>(at, 128 * wm + 16, lane, kBK);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (i + 2 < 8) a[i + 2] = read_operand<false>(at, 128 * wm + 16 * (i + 2), lane, kBK);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b[j], a[i], acc[i][j], 0, 0, 0,
                                                                         kE8M0One, 0, kE8M0One);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 12, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (i + 2 < 8) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
    }
}

template <bool YBF16>
__global__ __launch_bounds__(kThreads) void gemm_fp8_kernel(
    const int8_t* __restrict__ qx, const float* __restrict__ sx, const int8_t* __restrict__ qw,
    const float* __restrict__ sw, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int tiles_m, int tiles_n, bool vec, bool lds_out) {
    extern __shared__ __align__(16) uint8_t lds[];  // [2 steps][qx tile, qw tile]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 2, wn = wave & 3;

    const int b = blockIdx.x, nb = gridDim.x;
    const int x = b % 8, q = nb / 8, r = nb % 8;
    const int lin = x * q + min(x, r) + b / 8;      // a bijection of [0, nb)
    const int per_group = kGroupM * tiles_n;
    const int first_m = (lin / per_group) * kGroupM;
    const int group_m = min(tiles_m - first_m, kGroupM);
    const int tm = first_m + (lin % per_group) % group_m;
    const int tn = (lin % per_group) / group_m;
    const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One barrier per step, at its end: after it, every wave's loads of step
    // s + 1 are in LDS and every wave has finished reading step s's buffer,
    // which then receives step s + 2 while step s + 1 is multiplied.  Full
    // steps run in the loop, a partial last step (K % 128 != 0) after it, so
    // that the loop body has one code path for the accumulators.
    // Settle the scalar loads of the epilogue's pointers here: a scalar load
    // still in flight in the loop would make every LDS wait a full drain
    // (scalar loads return out of order on the same counter).
    asm volatile("" ::"s"(y), "s"(sx), "s"(sw));
    const int full = static_cast<int>(K / kBK);
    const int steps = static_cast<int>((K + kBK - 1) / kBK);
    // The tile's row and column scales wait in LDS for the epilogue: thread
    // t < 256 loads sx of row m0 + t, the others sw of column n0 + t - 256 (0
    // past the end), ahead of the first operand loads, and stores the value
    // once those have landed.
    float* scl = reinterpret_cast<float*>(lds + kScaleOff);  // [kBM sx][kBN sw]
    const int tt = static_cast<int>(threadIdx.x);
    const int64_t si = tt < kBM ? m0 + tt : n0 + (tt - kBM);
    const float sval = tt < kBM ? (si < M ? sx[si] : 0.0f) : (si < N ? sw[si] : 0.0f);
    load_stage(qx, qw, M, N, K, m0, n0, 0, lds, wave, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    scl[tt] = sval;
    for (int s = 0; s < full; ++s) {
        if (s + 1 < steps)
            load_stage(qx, qw, M, N, K, m0, n0, static_cast<int64_t>(s + 1) * kBK,
                       lds + ((s + 1) & 1) * kStageBytes, wave, lane);
        mfma_step_full(lds + (s & 1) * kStageBytes, wm, wn, lane, acc);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (full < steps) {
        mfma_step<true>(lds + (full & 1) * kStageBytes, wm, wn, lane,
                        static_cast<int>(K - static_cast<int64_t>(full) * kBK), acc);
        __syncthreads();
    }
    // Here every wave has read its last operands and the scales are in LDS.

    // D layout of a 16 x 16 tile (the qw block as A, the qx block as B):
    // lane (j, g) holds columns n = 4g + v (v < 4) of row m = j, so each lane
    // writes four neighbouring outputs at once.
    const int j = lane & 15, g = lane >> 4;
    if constexpr (YBF16) {
        if (lds_out) {
            // Each wave stages its 128 x 64 bf16 block in its own 16 KB of LDS
            // (128-byte rows, 16-byte chunks XOR-swizzled by row % 8), then
            // writes whole 128-byte row pieces, 16 bytes per lane, nontemporal.
            uint8_t* wl = lds + wave * (kBM / 2) * (kBN / 4) * 2;
#pragma unroll
            for (int mi = 0; mi < 8; ++mi) {
                const int row = 16 * mi + j;
                const float sxm = scl[128 * wm + row];
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const f32x4 s4 = *reinterpret_cast<const f32x4*>(scl + kBM + 64 * wn + 16 * ni + 4 * g);
                    const uint32_t lo = kc::f32_to_bf16((acc[mi][ni][0] * sxm) * s4.x) |
                                        static_cast<uint32_t>(kc::f32_to_bf16((acc[mi][ni][1] * sxm) * s4.y)) << 16;
                    const uint32_t hi = kc::f32_to_bf16((acc[mi][ni][2] * sxm) * s4.z) |
                                        static_cast<uint32_t>(kc::f32_to_bf16((acc[mi][ni][3] * sxm) * s4.w)) << 16;
                    const int c = (2 * ni + (g >> 1)) ^ (row & 7);
                    *reinterpret_cast<u32x2*>(wl + row * 128 + 16 * c + 8 * (g & 1)) = u32x2{lo, hi};
                }
            }
            // lane l: chunk l % 8 of block row 8 it + l / 8
#pragma unroll
            for (int it = 0; it < 16; ++it) {
                const int row = 8 * it + (lane >> 3), c = lane & 7;
                const u32x4 v = *reinterpret_cast<const u32x4*>(wl + row * 128 + 16 * (c ^ (row & 7)));
                const int64_t m = m0 + 128 * wm + row, n = n0 + 64 * wn + 8 * c;
                if (m < M && n < N)
                    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + m * N + n));
            }
            return;
        }
    }
#pragma unroll
    for (int mi = 0; mi < 8; ++mi) {
        const int64_t m = m0 + 128 * wm + 16 * mi + j;
        if (m >= M) continue;
        const float sxm = scl[128 * wm + 16 * mi + j];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int nl = 64 * wn + 16 * ni + 4 * g;
            const int64_t n = n0 + nl;
            if (vec && n + 3 < N) {
                const f32x4 s4 = *reinterpret_cast<const f32x4*>(scl + kBM + nl);
                const float r0 = (acc[mi][ni][0] * sxm) * s4.x, r1 = (acc[mi][ni][1] * sxm) * s4.y;
                const float r2 = (acc[mi][ni][2] * sxm) * s4.z, r3 = (acc[mi][ni][3] * sxm) * s4.w;
                if constexpr (YBF16) {
                    const uint32_t lo = kc::f32_to_bf16(r0) | static_cast<uint32_t>(kc::f32_to_bf16(r1)) << 16;
                    const uint32_t hi = kc::f32_to_bf16(r2) | static_cast<uint32_t>(kc::f32_to_bf16(r3)) << 16;
                    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(y) + m * N + n) = u32x2{lo, hi};
                } else {
                    *reinterpret_cast<f32x4*>(static_cast<float*>(y) + m * N + n) = f32x4{r0, r1, r2, r3};
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (n + v >= N) break;
                    const float rv = (acc[mi][ni][v] * sxm) * scl[kBM + nl + v];
                    if constexpr (YBF16) static_cast<uint16_t*>(y)[m * N + n + v] = kc::f32_to_bf16(rv);
                    else static_cast<float*>(y)[m * N + n + v] = rv;
                }
            }
        }
    }
}

// Y = 0 for an empty contraction (K == 0): the GEMM kernel's prologue
// always loads its first K step, so it is never launched with K == 0.
template <typename T>
__global__ void fill_zero_kernel(T* y, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        y[i] = T(0);
}

template <bool YBF16>
int gemm_fp8(const char* fn, const int8_t* qx, const float* sx, const int8_t* qw, const float* sw,
             void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: negative shape", fn);
    if (M == 0 || N == 0) return KC_SUCCESS;
    if (K % 16 != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: K=%lld must be a multiple of 16", fn,
                             (long long)K);
    if (K == 0) {  // qx and qw hold no bytes and may be null
        if (!y) return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
        const int64_t n = M * N;
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 4096));
        if constexpr (YBF16)
            fill_zero_kernel<<<blocks, 256, 0, stream>>>(static_cast<uint16_t*>(y), n);
        else
            fill_zero_kernel<<<blocks, 256, 0, stream>>>(static_cast<float*>(y), n);
        return kc::check_launch(fn);
    }
    if (!qx || !sx || !qw || !sw || !y)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    if (!kc::aligned(qx, 16) || !kc::aligned(qw, 16))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: qx and qw must be 16-byte aligned", fn);
    const int64_t tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
    if (tm * tn > INT32_MAX)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: too many tiles", fn);
    static bool attr_set = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_fp8_kernel<YBF16>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes) == hipSuccess;
    }();
    if (!attr_set) return kc::set_error(KC_ERR_HIP, "%s: cannot raise the LDS limit", fn);
    gemm_fp8_kernel<YBF16><<<static_cast<unsigned>(tm * tn), kThreads, kLdsBytes, stream>>>(
        qx, sx, qw, sw, y, M, N, K, static_cast<int>(tm), static_cast<int>(tn),
        N % 4 == 0 && kc::aligned(y, YBF16 ? 8 : 16), YBF16 && N % 8 == 0 && kc::aligned(y, 16));
    return kc::check_launch(fn);
}

}  // namespace

extern "C" int kc_gemm_fp8_w8a8_bf16(const int8_t* d_qx, const float* d_sx, const int8_t* d_qw,
                                     const float* d_sw, uint16_t* d_y, int64_t M, int64_t N,
                                     int64_t K, kc_stream_t stream) {
    return gemm_fp8<true>("kc_gemm_fp8_w8a8_bf16", d_qx, d_sx, d_qw, d_sw, d_y, M, N, K, stream);
}

extern "C" int kc_gemm_fp8_w8a8_f32(const int8_t* d_qx, const float* d_sx, const int8_t* d_qw,
                                    const float* d_sw, float* d_y, int64_t M, int64_t N, int64_t K,
                                    kc_stream_t stream) {
    return gemm_fp8<false>("kc_gemm_fp8_w8a8_f32", d_qx, d_sx, d_qw, d_sw, d_y, M, N, K, stream);
}
