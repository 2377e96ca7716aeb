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
// contraction.  A 128-k block ("T-block") of a 16-row tile is one 16-byte
// load per lane (lane (i, kb) reads bytes 16*kb .. 16*kb+15 of the block of
// row i, 32 nibbles); MFMA step t (t = 0..3) takes dword t, whose 8 nibbles
// become the bf16 pairs (k0,k4) (k1,k5) (k2,k6) (k3,k7) -- exact values
// 128 + (q ^ 8), one bitwise op each -- so the B operand holds X in the same
// pair order.
//
// A T-block lies inside one quantization group (gs a multiple of 128), so
// its MFMA sum C is folded into the fp32 accumulator as
//     acc += s * C + c2 * sum_k X[m, k],   c2 = -s * (136 + z)
// which removes the +128 encoding offset, the +8 of q ^ 8 and the zero point
// exactly as the GEMV does.  Groups smaller than 128 fall back to the GEMV
// per activation row.
//
// Kernels, by M (kc_gemm_int4_bf16 at the bottom picks one):
//   M 2..64   gemm_int4_kslds_kernel: K split over the four waves of a CU, X
//             and the weights streamed into LDS by direct-to-LDS loads; on
//             the reference layout at M <= 48 with K a multiple of 1024 the
//             weights come in pairs of T-blocks (whole 128-byte rows; K up to
//             12288 / 9216 / 12288 at M <= 16 / 32 / 48), otherwise one T-block at a
//             time (K up to 16384 / 13824 / 11776 / 9216 at M <= 16 / 32 /
//             48 / 64), and on the reference layout at M <= 8 only in the
//             pair form;
//   M 2..8    gemm_int4_xres_kernel (reference layout, where the pair form
//             does not apply): X resident in LDS, one wave per 16-row weight
//             tile over all of K;
//   M 9..64   gemm_int4_kslice_kernel (X from the cache into registers)
//             where gemm_int4_kslds_kernel's LDS does not fit;
//   fallbacks gemm_int4_xres_kernel (M 2..16), gemm_int4_xbig_kernel
//             (M 33..64) and gemm_int4_mfma_kernel (below) when the K-split
//             kernels' coefficients do not fit in LDS (K above about 20000).
//
// gemm_int4_mfma_kernel work split.  A workgroup of NW waves owns
// 16*RT*NW consecutive weight rows and the whole K; wave w owns row tiles
// w*RT .. w*RT+RT-1.  K is walked in chunks of TPC T-blocks, software
// pipelined:
//   * X of the next chunk is loaded, rearranged into the B-operand layout
//     (with its T-block sums) and written to the other half of a
//     double-buffered LDS area, together with that chunk's fold coefficients
//     (s, c2) for the workgroup's rows -- one barrier per chunk;
//   * X and the fold coefficients are loaded two chunks ahead and the
//     weights one chunk ahead, so no load is waited for before a whole chunk
//     period has passed.
// Each B operand read from LDS serves RT row tiles, each decoded A operand
// MT activation tiles.
#include <algorithm>
#include <type_traits>

#include "kc_common.hpp"

namespace {

using kc::kWave;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kTBlock = 128;  // k per T-block: 64 bytes of each W row

// The weight bytes lane (i, kb) feeds to the matrix core for T-block T of
// the 16-row tile that starts at row r0 (a multiple of 16): 16 bytes, 32
// nibbles.
//   reference layout: bytes 64 T + 16 kb of row r0 + i (rows past N read
//     row N - 1);
//   shuffled layout (kc_shuffle_int4_mfma): the tile's T-blocks are 1 KB
//     blocks in T order, tiles one after another, lane l's 16 bytes at byte
//     16 l of a block -- one wave-wide load then reads 1 KB in address order
//     instead of 64 bytes of each of 16 rows 2-8 KB apart.
// tile_lane_ptr points at T-block 0; T-block T is kTStep<SHUF> u32x4 on.
template <bool SHUF>
constexpr int kTStep = SHUF ? 64 : 4;

template <bool SHUF>
__device__ __forceinline__ const u32x4* tile_lane_ptr(const uint8_t* packed, int r0, int N, int K,
                                                      int lane) {
    if constexpr (SHUF)  // tiles past the last (rows past the pad) read the last tile
        return reinterpret_cast<const u32x4*>(packed + static_cast<int64_t>(min(r0 >> 4, (N + 15) / 16 - 1)) *
                                                           (K / kTBlock) * 1024) + lane;
    else
        return reinterpret_cast<const u32x4*>(packed + static_cast<int64_t>(min(r0 + (lane & 15), N - 1)) * (K >> 1)) +
               (lane >> 4);
}

// Nibble-decode constants in VGPRs (an SGPR operand halves VALU issue rate on
// gfx950); the asm makes them opaque to the compiler.
struct NibConsts {
    uint32_t mask, magic;
};

__device__ __forceinline__ NibConsts nib_consts() {
    NibConsts k;
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(k.mask));
    asm volatile("v_mov_b32 %0, 0x43084308" : "=v"(k.magic));
    return k;
}

// ((d ^ 0x00080008) & 0x000F000F) | 0x43004300 == (d & 0x000F000F) ^ 0x43084308
__device__ __forceinline__ uint32_t nib_pair(uint32_t d, NibConsts k) { return (d & k.mask) ^ k.magic; }

__device__ __forceinline__ bf16x8_t a_operand(uint32_t d, NibConsts k) {
    const u32x4 p{nib_pair(d, k), nib_pair(d >> 4, k), nib_pair(d >> 8, k), nib_pair(d >> 12, k)};
    return __builtin_bit_cast(bf16x8_t, p);
}

__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// Workgroup shape.  64 weight rows (4 row tiles of 16) per workgroup; the
// K dimension is split KW ways across its waves.  Wave w owns K part
// q = w / (4/RT) and row tiles (w % (4/RT))*RT .. +RT-1.
template <int MT, int RT, int KW, int TPC>
struct GemmShape {
    static constexpr int kRowGroups = 4 / RT;               // waves per K part
    static constexpr int kNW = kRowGroups * KW;             // waves per workgroup
    static constexpr int kThreadsWG = kNW * kWave;
    static constexpr int kRowsWG = 64;
    // LDS per chunk buffer
    static constexpr int kXSlots = KW * MT * TPC * 4 * kWave;  // 16-byte B-operand slots
    static constexpr int kXsum = KW * MT * TPC * 16;           // T-block sums of X per row
    static constexpr int kCoef = KW * TPC * kRowsWG;           // s (and c2) per T-block and row
    static constexpr int kBufBytes = kXSlots * 16 + kXsum * 4 + 2 * kCoef * 4;
    // staging work per thread: X groups of 4 slots (one (q, t, mt, lane)
    // each: the 4 MFMA steps of a T-block, 64 contiguous bytes of one X row)
    // and fold coefficients
    static constexpr int kXGroups = KW * MT * TPC * kWave;
    static constexpr int kXItems = (kXGroups + kThreadsWG - 1) / kThreadsWG;
    static constexpr int kCItems = (kCoef + kThreadsWG - 1) / kThreadsWG;
    static_assert(TPC % 2 == 0, "T-blocks are computed in pairs");
};

// One chunk buffer in LDS.
template <class S>
struct ChunkLds {
    u32x4* x;       // [KW][MT][TPC][4][64] B-operand slots
    float* xsum;    // [KW][MT][TPC][16]
    float* cs;      // [KW][TPC][64 rows]   s
    float* cz;      // [KW][TPC][64 rows]   c2
    __device__ ChunkLds(char* base) {
        x = reinterpret_cast<u32x4*>(base);
        xsum = reinterpret_cast<float*>(base + S::kXSlots * 16);
        cs = xsum + S::kXsum;
        cz = cs + S::kCoef;
    }
};

// Raw loads of one chunk's X groups and fold coefficients (registers).
template <class S>
struct ChunkRaw {
    u32x4 x[S::kXItems][4];
    float s[S::kCItems];
    uint32_t zb[S::kCItems];
};

// Position of the chunk's T-block t of K part q in the row.
struct KSplit {
    int nT;    // T-blocks per row
    int nTq;   // T-blocks per K part
    __device__ int T(int q, int T0, int t) const { return min(q * nTq + min(T0 + t, nTq - 1), nT - 1); }
};

// X group g -> (K part q, T-block t, m-tile mt, B lane l = j + 16*kb).  A
// wave's 64 consecutive groups are the 64 lanes of one (q, t, mt): each of
// its 4 LDS stores covers 64 consecutive 16-byte slots (no bank conflicts),
// and the 4 lanes of one activation row (kb = 0..3) are lanes j, j+16, j+32,
// j+48.
template <int MT, int TPC>
__device__ __forceinline__ void x_group(int g, int& q, int& t, int& mt, int& j, int& kb) {
    const int l = g & (kWave - 1);
    j = l & 15;
    kb = l >> 4;
    int r = g >> 6;
    mt = r % MT;
    r /= MT;
    t = r % TPC;
    q = r / TPC;
}

template <int MT, int RT, int KW, int TPC>
__device__ __forceinline__ void load_chunk_raw(ChunkRaw<GemmShape<MT, RT, KW, TPC>>& raw,
                                               const uint16_t* __restrict__ X,
                                               const float* __restrict__ scales,
                                               const uint8_t* __restrict__ zeros, int M, int N,
                                               int K, int T0, KSplit ks, int nbase, int G,
                                               int gshift) {
    using S = GemmShape<MT, RT, KW, TPC>;
#pragma unroll
    for (int u = 0; u < S::kXItems; ++u) {
        const int g = threadIdx.x + u * S::kThreadsWG;
        if (g >= S::kXGroups) break;  // uniform per wave: kXGroups is a multiple of 64
        int q, t, mt, j, kb;
        x_group<MT, TPC>(g, q, t, mt, j, kb);
        const int m = 16 * mt + j;
        const u32x4* src = reinterpret_cast<const u32x4*>(
            X + static_cast<int64_t>(min(m, M - 1)) * K + ks.T(q, T0, t) * kTBlock + 32 * kb);
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) raw.x[u][w4] = m < M ? src[w4] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < S::kCItems; ++u) {
        const int it = min(static_cast<int>(threadIdx.x) + u * S::kThreadsWG, S::kCoef - 1);
        const int rw = it % S::kRowsWG, t = (it / S::kRowsWG) % TPC, q = it / (S::kRowsWG * TPC);
        const int g = ks.T(q, T0, t) >> gshift;
        const int64_t row = min(nbase + rw, N - 1);
        raw.s[u] = scales[row * G + g];
        raw.zb[u] = zeros[row * (G >> 1) + (g >> 1)];
    }
}

template <int MT, int RT, int KW, int TPC>
__device__ __forceinline__ void stage_chunk(const ChunkRaw<GemmShape<MT, RT, KW, TPC>>& raw,
                                            ChunkLds<GemmShape<MT, RT, KW, TPC>> L, int T0,
                                            KSplit ks, int gshift) {
    using S = GemmShape<MT, RT, KW, TPC>;
    uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs
    asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
    asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
    const uint32_t ones = 0x3F803F80u;
#pragma unroll
    for (int u = 0; u < S::kXItems; ++u) {
        const int g = threadIdx.x + u * S::kThreadsWG;
        if (g >= S::kXGroups) break;
        int q, t, mt, j, kb;
        x_group<MT, TPC>(g, q, t, mt, j, kb);
        const int tile = (q * MT + mt) * TPC + t;
        float sm = 0.0f;
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) {
            const u32x4 d = raw.x[u][w4];
            const uint32_t d0 = d.x, d1 = d.y, d2 = d.z, d3 = d.w;
            u32x4 p;
            p.x = __builtin_amdgcn_perm(d2, d0, sel_lo);  // (x0, x4)
            p.y = __builtin_amdgcn_perm(d2, d0, sel_hi);  // (x1, x5)
            p.z = __builtin_amdgcn_perm(d3, d1, sel_lo);  // (x2, x6)
            p.w = __builtin_amdgcn_perm(d3, d1, sel_hi);  // (x3, x7)
            L.x[(tile * 4 + w4) * kWave + j + 16 * kb] = p;
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d0), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d1), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d2), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d3), as_bf16x2(ones), sm, false);
        }
        sm += __shfl_xor(sm, 16, kWave);  // the 4 k-quarters of the row's T-block
        sm += __shfl_xor(sm, 32, kWave);
        if (kb == 0) L.xsum[tile * 16 + j] = sm;
    }
#pragma unroll
    for (int u = 0; u < S::kCItems; ++u) {
        const int it = threadIdx.x + u * S::kThreadsWG;
        if (it < S::kCoef) {
            const int t = (it / S::kRowsWG) % TPC, q = it / (S::kRowsWG * TPC);
            const int g = ks.T(q, T0, t) >> gshift;
            const uint32_t z = (g & 1) ? (raw.zb[u] >> 4) : (raw.zb[u] & 0xFu);
            L.cs[it] = raw.s[u];
            L.cz[it] = -raw.s[u] * static_cast<float>(136u + z);
        }
    }
}

template <int MT, int RT>
struct Acc {
    f32x4 v[RT][MT];
};

// B operands of one T-block (4 MFMA steps x MT tiles) from LDS.
template <int MT, int TPC>
__device__ __forceinline__ void read_b(bf16x8_t (&b)[4][MT], const u32x4* x, int q, int t, int lane) {
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            b[w4][mt] = __builtin_bit_cast(bf16x8_t, x[(((q * MT + mt) * TPC + t) * 4 + w4) * kWave + lane]);
}

// One chunk of MFMA work for this wave: weights w[rt][t] from registers, X
// and coefficients from LDS.  T-blocks go in pairs so that two independent
// accumulation chains interleave on the matrix core.
template <int MT, int RT, int KW, int TPC>
__device__ __forceinline__ void compute_chunk(Acc<MT, RT>& acc, const u32x4 (&w)[RT][TPC],
                                              ChunkLds<GemmShape<MT, RT, KW, TPC>> L, int T0,
                                              int nTq, int q, int rg, int lane, NibConsts nk) {
    using S = GemmShape<MT, RT, KW, TPC>;
    const int j = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int tp = 0; tp < TPC; tp += 2) {
        if (T0 + tp >= nTq) break;  // uniform: past the end of this K part
        const bool second = T0 + tp + 1 < nTq;
        bf16x8_t b[2][4][MT];
        read_b<MT, TPC>(b[0], L.x, q, tp, lane);
        read_b<MT, TPC>(b[1], L.x, q, tp + 1, lane);
        f32x4 d[2][RT][MT];
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const u32x4 wv = w[rt][tp + h];
                    const uint32_t wd = w4 == 0 ? wv.x : w4 == 1 ? wv.y : w4 == 2 ? wv.z : wv.w;
                    const bf16x8_t a = a_operand(wd, nk);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        d[h][rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            a, b[h][w4][mt], w4 == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[h][rt][mt], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (h == 1 && !second) break;
            const int t = tp + h;
            float xs[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) xs[mt] = L.xsum[((q * MT + mt) * TPC + t) * 16 + j];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int rw = (rg * RT + rt) * 16 + 4 * kb;
                const int ci = (q * TPC + t) * S::kRowsWG + rw;
                const f32x4 s4 = *reinterpret_cast<const f32x4*>(L.cs + ci);
                const f32x4 z4 = *reinterpret_cast<const f32x4*>(L.cz + ci);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f32x4 a = acc.v[rt][mt];
                    const f32x4 c = d[h][rt][mt];
                    a.x = fmaf(s4.x, c.x, fmaf(z4.x, xs[mt], a.x));
                    a.y = fmaf(s4.y, c.y, fmaf(z4.y, xs[mt], a.y));
                    a.z = fmaf(s4.z, c.z, fmaf(z4.z, xs[mt], a.z));
                    a.w = fmaf(s4.w, c.w, fmaf(z4.w, xs[mt], a.w));
                    acc.v[rt][mt] = a;
                }
            }
        }
    }
}

template <int RT, int TPC, bool SHUF>
__device__ __forceinline__ void load_weights(u32x4 (&w)[RT][TPC], const uint8_t* __restrict__ packed,
                                             int N, int64_t rbytes, int nbase, int rg, int q,
                                             int lane, int T0, KSplit ks) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const u32x4* prow = tile_lane_ptr<SHUF>(packed, nbase + (rg * RT + rt) * 16, N,
                                                static_cast<int>(2 * rbytes), lane);
#pragma unroll
        for (int t = 0; t < TPC; ++t)
            w[rt][t] = __builtin_nontemporal_load(prow + ks.T(q, T0, t) * kTStep<SHUF>);
    }
}

template <int MT, int RT, int KW, int TPC, bool SHUF>
__global__ __launch_bounds__((4 / RT) * KW * kWave) void gemm_int4_mfma_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int M, int N, int K, int gshift) {
    using S = GemmShape<MT, RT, KW, TPC>;
    extern __shared__ __align__(16) char lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int q = wave / S::kRowGroups;             // K part
    const int rg = wave % S::kRowGroups;            // row-tile group
    const int nbase = blockIdx.x * S::kRowsWG;
    KSplit ks;
    ks.nT = K / kTBlock;
    ks.nTq = ks.nT / KW;                            // the launcher checks KW divides nT
    const int G = ks.nT >> gshift;                  // groups per row (gs = 128 << gshift)
    const int64_t rbytes = K >> 1;
    const int nchunks = (ks.nTq + TPC - 1) / TPC;
    ChunkLds<S> buf[2] = {ChunkLds<S>(lds), ChunkLds<S>(lds + S::kBufBytes)};

    Acc<MT, RT> acc;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc.v[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Pipeline: in iteration c the wave computes chunk c, while X (with the
    // fold coefficients) of chunk c+2 and the weights of chunk c+1 are in
    // flight; chunk c+1's X, loaded during iteration c-1, is staged into
    // LDS at the end of the iteration.  Every load has a whole chunk period
    // to arrive before anything waits for it.  Two iterations per loop trip
    // let the register buffers alternate without copies.
    ChunkRaw<S> raw0, raw1;
    u32x4 w0[RT][TPC], w1[RT][TPC];
    load_chunk_raw<MT, RT, KW, TPC>(raw0, X, scales, zeros, M, N, K, 0, ks, nbase, G, gshift);
    if (nchunks > 1)
        load_chunk_raw<MT, RT, KW, TPC>(raw1, X, scales, zeros, M, N, K, TPC, ks, nbase, G, gshift);
    load_weights<RT, TPC, SHUF>(w0, packed, N, rbytes, nbase, rg, q, lane, 0, ks);
    stage_chunk<MT, RT, KW, TPC>(raw0, buf[0], 0, ks, gshift);
    __syncthreads();
    const NibConsts nk = nib_consts();

    for (int c = 0; c < nchunks; c += 2) {
        // chunk c: w0 / buf[0]; chunk c+1 staged from raw1; chunk c+2 -> raw0
        const int T0 = c * TPC, T1 = T0 + TPC, T2 = T1 + TPC, T3 = T2 + TPC;
        if (c + 2 < nchunks)
            load_chunk_raw<MT, RT, KW, TPC>(raw0, X, scales, zeros, M, N, K, T2, ks, nbase, G, gshift);
        if (c + 1 < nchunks) load_weights<RT, TPC, SHUF>(w1, packed, N, rbytes, nbase, rg, q, lane, T1, ks);
        compute_chunk<MT, RT, KW, TPC>(acc, w0, buf[0], T0, ks.nTq, q, rg, lane, nk);
        if (c + 1 >= nchunks) break;
        stage_chunk<MT, RT, KW, TPC>(raw1, buf[1], T1, ks, gshift);
        __syncthreads();
        // chunk c+1: w1 / buf[1]; chunk c+2 staged from raw0; chunk c+3 -> raw1
        if (c + 3 < nchunks)
            load_chunk_raw<MT, RT, KW, TPC>(raw1, X, scales, zeros, M, N, K, T3, ks, nbase, G, gshift);
        if (c + 2 < nchunks) load_weights<RT, TPC, SHUF>(w0, packed, N, rbytes, nbase, rg, q, lane, T2, ks);
        compute_chunk<MT, RT, KW, TPC>(acc, w1, buf[1], T1, ks.nTq, q, rg, lane, nk);
        if (c + 2 >= nchunks) break;
        stage_chunk<MT, RT, KW, TPC>(raw0, buf[0], T2, ks, gshift);
        __syncthreads();
    }

    // Sum the KW K parts in a fixed order (part 0 + part 1 + ...) through LDS.
    if constexpr (KW > 1) {
        __syncthreads();  // every wave is done reading the chunk buffers
        f32x4* red = reinterpret_cast<f32x4*>(lds);   // [KW-1][row groups][RT*MT][64]
        if (q > 0) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    red[(((q - 1) * S::kRowGroups + rg) * RT * MT + rt * MT + mt) * kWave + lane] = acc.v[rt][mt];
        }
        __syncthreads();
        if (q > 0) return;
        for (int p = 1; p < KW; ++p) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc.v[rt][mt] += red[(((p - 1) * S::kRowGroups + rg) * RT * MT + rt * MT + mt) * kWave + lane];
        }
    }

    // lane (j, kb) holds Y[m = 16*mt + j][n = tile + 4*kb + v]
    const int j = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + j;
            if (m >= M) continue;
            const f32x4 a = acc.v[rt][mt];
            const float vals[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = nbase + (rg * RT + rt) * 16 + 4 * kb + v;
                if (n < N) Y[static_cast<int64_t>(m) * N + n] = kc::f32_to_bf16(vals[v]);
            }
        }
    }
}

template <int MT, int RT, int KW, int TPC, bool SHUF>
int launch_mfma(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                const uint16_t* X, uint16_t* Y, int M, int N, int K, int gshift,
                hipStream_t stream) {
    using S = GemmShape<MT, RT, KW, TPC>;
    constexpr size_t kLds = std::max<size_t>(2 * static_cast<size_t>(S::kBufBytes),
                                             (KW - 1) * S::kRowGroups * RT * MT * kWave * 16);
    static bool attr_set = false;  // launches above 64 KB of LDS need the attribute
    if (kLds > 65536 && !attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_int4_mfma_kernel<MT, RT, KW, TPC, SHUF>),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(kLds)) != hipSuccess)
            return kc::set_error(KC_ERR_HIP, "%s: cannot reserve %zu bytes of LDS", fn, kLds);
        attr_set = true;
    }
    const unsigned grid = static_cast<unsigned>((N + S::kRowsWG - 1) / S::kRowsWG);
    gemm_int4_mfma_kernel<MT, RT, KW, TPC, SHUF><<<grid, S::kThreadsWG, kLds, stream>>>(
        packed, scales, zeros, X, Y, M, N, K, gshift);
    return kc::check_launch(fn);
}

// ---------------------------------------------------------------------------
// Small M (2..16): X resident in LDS.  Each wave streams one 16-row weight
// tile over the whole of K with no barrier in its loop: X (all M rows) is
// staged in the B-operand pair layout with its T-block sums -- all of K at
// once when it fits, else in P phases of K / P (one restaging, between two
// barriers, per phase) -- and each wave stages the fold coefficients
// (s and c2 = -s * (136 + z)) of its 16 rows for every group once.  The wave
// keeps D T-blocks of its weights in flight in a register ring (16 bytes per
// lane per T-block, issued D T-blocks ahead of their use), across phases.
// A workgroup of W waves owns W consecutive row tiles; W = 7 gives one
// workgroup per CU at N = 28672.
//
// LDS: X slots [T of the phase][step w4][m][kb] (16 bytes each), X sums
// [T of the phase][m] (padded to 16 bytes), then per wave cs[g][16 rows],
// cz[g][16 rows].
// ---------------------------------------------------------------------------
constexpr int kXresMaxM = 16;  // the kernel's limit; kc_gemm_int4_bf16 uses it up to kXresBestM
constexpr int kXresBestM = 8;  // M 9..16 are faster on the K-split kernel (K 8192, N 28672: M 12 35.9 against 37.6 us, M 16 37.4 against 41.0)

// Sum over each 16-lane row of the wave with DPP rotations (VALU only).
template <int CTRL>
__device__ __forceinline__ float dpp_ror(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_ror<0x128>(v);  // row_ror:8
    v += dpp_ror<0x124>(v);  // row_ror:4
    v += dpp_ror<0x122>(v);  // row_ror:2
    v += dpp_ror<0x121>(v);  // row_ror:1
    return v;
}

__host__ __device__ constexpr size_t xres_lds_bytes(int M, int K, int G, int W, int P) {
    return static_cast<size_t>(K / kTBlock / P) * 4 * M * 4 * 16 +   // X slots of a phase
           static_cast<size_t>((K / kTBlock / P * M + 3) & ~3) * 4 +  // X sums, padded to 16 bytes
           static_cast<size_t>(W) * 2 * G * 16 * 4;                  // cs, cz per wave
}

template <int W, int D, bool SHUF>
__global__ __launch_bounds__(W * kWave) void gemm_int4_xres_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int M, int N, int K, int gshift, int P) {
    extern __shared__ __align__(16) char lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int nT = K / kTBlock;
    const int nTp = nT / P;                         // T-blocks per phase (the launcher: D divides it)
    const int G = nT >> gshift;
    u32x4* xslot = reinterpret_cast<u32x4*>(lds);
    float* xsum = reinterpret_cast<float*>(xslot + static_cast<size_t>(nTp) * 16 * M);
    float* cs = xsum + ((nTp * M + 3) & ~3) + wave * 2 * G * 16;  // 16-byte aligned
    float* cz = cs + G * 16;
    const int ntiles = (N + 15) / 16;
    const int tile = min(static_cast<int>(blockIdx.x) * W + wave, ntiles - 1);  // spare waves redo the last tile's math, store nothing
    const bool owner = static_cast<int>(blockIdx.x) * W + wave < ntiles;
    const int row0 = tile * 16;
    const int i = lane & 15, kb = lane >> 4;

    // This lane's weights: row row0 + i, bytes 16 kb .. 16 kb + 15 of each
    // T-block (64 bytes of the row); a ring of the next D T-blocks.
    const u32x4* wrow = tile_lane_ptr<SHUF>(packed, row0, N, K, lane);
    u32x4 w[D];

    // Staging of a phase's X: piece p of row m is X[m][8 p .. 8 p + 7] of the
    // phase: the B operand of T-block p / 16, step p % 4, lane kb = (p / 4) %
    // 4; 16 consecutive pieces (one T-block of one row) sit in 16 consecutive
    // lanes, which sum them with DPP.  Every load of a batch (kXBatch pieces
    // per thread) is issued before the first is used, so that a batch costs
    // one memory round trip; (idx + 0.5) / ppr in fp32 gives the row exactly
    // (idx < 2^24, and the quotient is never within 0.5 / ppr of an integer).
    // With the first phase the wave also stages its coefficients,
    // cs[g][row] = s, cz[g][row] = -s * (136 + z) (16 rows per lane, lane
    // g + 64 j of each row), and fills its weight ring.
    constexpr int kXBatch = 10;  // 4480 pieces per pass: M 16 x 2048 k, or M 4 x 8192 k
    const int ppr = nTp * 16;                       // X pieces per row and phase
    const int npieces = M * ppr;
    const float inv_ppr = 1.0f / static_cast<float>(ppr);
    const int cpasses = (G + kWave - 1) / kWave;
    auto stage = [&](int phase) {
        for (int xbase = 0; xbase < npieces; xbase += kXBatch * W * kWave) {
            u32x4 dv[kXBatch];
#pragma unroll
            for (int b = 0; b < kXBatch; ++b) {
                const int idx = min(xbase + b * W * kWave + static_cast<int>(threadIdx.x), npieces - 1);
                const int m = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_ppr);
                const int p = idx - m * ppr;
                dv[b] = *reinterpret_cast<const u32x4*>(X + static_cast<int64_t>(m) * K +
                                                        8 * (static_cast<int64_t>(phase) * ppr + p));
            }
            if (phase == 0 && xbase == 0) {
                for (int j = 0; j < cpasses; ++j) {
                    const int g = min(lane + kWave * j, G - 1);
                    float sv[16];
                    uint32_t zb[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = min(row0 + r, N - 1);
                        sv[r] = scales[row * G + g];
                        zb[r] = zeros[row * (G >> 1) + (g >> 1)];
                    }
                    if (lane + kWave * j < G) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const uint32_t z = (g & 1) ? (zb[r] >> 4) : (zb[r] & 0xFu);
                            cs[g * 16 + r] = sv[r];  // [g][row]: a lane's 4 rows are one 16-byte read
                            cz[g * 16 + r] = -sv[r] * static_cast<float>(136u + z);
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < D; ++u) w[u] = wrow[min(u, nT - 1) * kTStep<SHUF>];
            }
            uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs
            asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
            asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
            const uint32_t ones = 0x3F803F80u;
#pragma unroll
            for (int b = 0; b < kXBatch; ++b) {
                const int idx0 = xbase + b * W * kWave + static_cast<int>(threadIdx.x);
                const bool valid = idx0 < npieces;
                const int idx = valid ? idx0 : 0;
                const int m = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_ppr);
                const int p = idx - m * ppr;
                const u32x4 d = valid ? dv[b] : u32x4{0u, 0u, 0u, 0u};
                u32x4 q;
                q.x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);  // (x0, x4)
                q.y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);  // (x1, x5)
                q.z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);  // (x2, x6)
                q.w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);  // (x3, x7)
                float sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), 0.0f, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), sm, false);
                sm = row16_sum(sm);  // the T-block's 16 pieces, in one 16-lane row
                if (valid) {
                    const int T = p >> 4, w4 = p & 3, pkb = (p >> 2) & 3;
                    xslot[((T * 4 + w4) * M + m) * 4 + pkb] = q;
                    if ((p & 15) == 0) xsum[T * M + m] = sm;
                }
            }
        }
    };
    stage(0);
    __syncthreads();

    // Stream the weights: T-block T's four MFMA steps with X from LDS,
    // folded into acc (rows 4 kb + v of the tile, activation row i).
    const NibConsts nk = nib_consts();
    // lanes of activation rows past M read row M - 1: their output columns
    // are never stored, and no branch or zero fill is needed per T-block
    const int ib = min(i, M - 1);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int ph = 0; ph < P; ++ph) {
        for (int T0 = ph * nTp; T0 < (ph + 1) * nTp; T0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int T = T0 + u;
                const int Tl = T - ph * nTp;
                bf16x8_t b[4];
#pragma unroll
                for (int w4 = 0; w4 < 4; ++w4)
                    b[w4] = __builtin_bit_cast(bf16x8_t, xslot[((Tl * 4 + w4) * M + ib) * 4 + kb]);
                const float xs = xsum[Tl * M + ib];
                const int g = T >> gshift;
                const f32x4 s4 = *reinterpret_cast<const f32x4*>(cs + g * 16 + 4 * kb);  // rows 4 kb .. 4 kb + 3
                const f32x4 z4 = *reinterpret_cast<const f32x4*>(cz + g * 16 + 4 * kb);
                const u32x4 wv = w[u];
                f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_operand(wv.x, nk), b[0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_operand(wv.y, nk), b[1], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_operand(wv.z, nk), b[2], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_operand(wv.w, nk), b[3], d, 0, 0, 0);
                acc.x = fmaf(s4.x, d.x, fmaf(z4.x, xs, acc.x));
                acc.y = fmaf(s4.y, d.y, fmaf(z4.y, xs, acc.y));
                acc.z = fmaf(s4.z, d.z, fmaf(z4.z, xs, acc.z));
                acc.w = fmaf(s4.w, d.w, fmaf(z4.w, xs, acc.w));
                // refill the ring slot: T-block T + D (past the end: the last one again)
                w[u] = wrow[min(T + D, nT - 1) * kTStep<SHUF>];
                // issued here, right after its slot's last use: left to the
                // scheduler, the D refills sink to the end of the unrolled
                // body and the ring drains every D T-blocks (M 4 / 8: 31.6 /
                // 35.0 -> 31.2 / 32.7 us at K 8192, N 28672)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (ph + 1 < P) {  // uniform: restage X for the next phase
            __syncthreads();
            stage(ph + 1);
            __syncthreads();
        }
    }

    // lane (i, kb) holds Y[m = i][n = row0 + 4 kb + v]
    if (owner && i < M) {
        const float vals[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = row0 + 4 * kb + v;
            if (n < N) Y[static_cast<int64_t>(i) * N + n] = kc::f32_to_bf16(vals[v]);
        }
    }
}

// Phases of K for the X-resident kernel: the fewest (1, 2, 4, ...) whose LDS
// fits, with D dividing the T-blocks of a phase; 0 when none does.
constexpr int kXresW = 7, kXresD = 8;

inline int xres_phases(int M, int K, int G) {
    const int nT = K / kTBlock;
    for (int P = 1; P <= nT; P *= 2) {
        if (nT % P != 0 || (nT / P) % kXresD != 0) break;
        if (xres_lds_bytes(M, K, G, kXresW, P) <= 160 * 1024) return P;
    }
    return 0;
}

template <int W, int D, bool SHUF>
int launch_xres(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                const uint16_t* X, uint16_t* Y, int M, int N, int K, int gshift, int P,
                hipStream_t stream) {
    const int G = (K / kTBlock) >> gshift;
    const size_t lds = xres_lds_bytes(M, K, G, W, P);
    static bool attr_set = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_int4_xres_kernel<W, D, SHUF>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    }();
    if (!attr_set) return kc::set_error(KC_ERR_HIP, "%s: cannot raise the LDS limit", fn);
    const int ntiles = (N + 15) / 16;
    const unsigned grid = static_cast<unsigned>((ntiles + W - 1) / W);
    gemm_int4_xres_kernel<W, D, SHUF><<<grid, W * kWave, lds, stream>>>(packed, scales, zeros, X, Y, M, N, K,
                                                                   gshift, P);
    return kc::check_launch(fn);
}

// ---------------------------------------------------------------------------
// M 33..64 when the K-split kernel below does not apply (K above about
// 20000): X resident in LDS, four activation tiles.  Each wave owns RT
// 16-row weight tiles (consecutive) over the whole of K and every
// activation row: per T-block it decodes each tile's A operands once and
// runs them against the MT = 4 activation tiles' B operands from LDS (each
// B read serves the RT weight tiles).  X is too large to hold whole (64 x
// 8192 bf16 = 1 MB), so it passes through LDS in phases of NTP T-blocks,
// double-buffered: the next phase's X is loaded into registers at the start
// of a phase and written to the other buffer after the phase's math, with
// one barrier per phase.  Weights stream through a D-deep register ring
// (D a multiple of NTP, so phase switches sit at fixed places of the ring).
// Coefficients per wave: scales [row][g] and zero nibbles [row][g] bytes.
// ---------------------------------------------------------------------------
constexpr int kXbigMT = 4;

__host__ __device__ constexpr size_t xbig_lds_bytes(int M, int G, int W, int RT, int NTP) {
    return 2 * static_cast<size_t>(NTP) * 4 * M * 4 * 16 +          // X slots, two phases
           2 * static_cast<size_t>((NTP * M + 3) & ~3) * 4 +         // X sums, two phases
           static_cast<size_t>(W) * RT * 16 * G * 5 +                // scales + zero bytes per wave
           16;                                                        // alignment slack
}

template <int W, int RT, int NTP, int D, bool SHUF>
__global__ __launch_bounds__(W * kWave) void gemm_int4_xbig_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int M, int N, int K, int gshift) {
    static_assert(D % NTP == 0, "phase switches at fixed ring positions");
    constexpr int MT = kXbigMT;
    extern __shared__ __align__(16) char lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int nT = K / kTBlock;
    const int G = nT >> gshift;
    const int slots = NTP * 16 * M;                 // u32x4 per phase buffer
    const int sums = (NTP * M + 3) & ~3;
    u32x4* xslot0 = reinterpret_cast<u32x4*>(lds);
    float* xsum0 = reinterpret_cast<float*>(xslot0 + 2 * static_cast<size_t>(slots));
    float* csw = xsum0 + 2 * sums + wave * RT * 16 * G;                // [RT*16 rows][G]
    uint8_t* zsw = reinterpret_cast<uint8_t*>(xsum0 + 2 * sums + W * RT * 16 * G) + wave * RT * 16 * G;
    const int ntiles = (N + 15) / 16;
    const int tile0 = min((static_cast<int>(blockIdx.x) * W + wave) * RT, ntiles - 1);
    const int i = lane & 15, kb = lane >> 4;

    // weight rows of this lane: row 16 (tile0 + rt) + i
    const u32x4* wrow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        wrow[rt] = tile_lane_ptr<SHUF>(packed, 16 * (tile0 + rt), N, K, lane);
    u32x4 w[D][RT];

    // X staging (see gemm_int4_xres_kernel): piece p of row m within a phase
    constexpr int kXB = (NTP * 16 * 64 + W * kWave - 1) / (W * kWave);  // pieces per thread, M <= 64
    const int ppr = NTP * 16;
    const int npieces = M * ppr;
    const float inv_ppr = 1.0f / static_cast<float>(ppr);
    auto load_x = [&](int phase, u32x4 (&dv)[kXB]) {
#pragma unroll
        for (int b = 0; b < kXB; ++b) {
            const int idx = min(b * W * kWave + static_cast<int>(threadIdx.x), npieces - 1);
            const int m = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_ppr);
            const int p = idx - m * ppr;
            dv[b] = *reinterpret_cast<const u32x4*>(X + static_cast<int64_t>(m) * K +
                                                    8 * (static_cast<int64_t>(phase) * ppr + p));
        }
    };
    auto write_x = [&](int buf, const u32x4 (&dv)[kXB]) {
        u32x4* xs = xslot0 + buf * slots;
        float* xm = xsum0 + buf * sums;
        uint32_t sel_lo, sel_hi;
        asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
        asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
        const uint32_t ones = 0x3F803F80u;
#pragma unroll
        for (int b = 0; b < kXB; ++b) {
            const int idx0 = b * W * kWave + static_cast<int>(threadIdx.x);
            const bool valid = idx0 < npieces;
            const int idx = valid ? idx0 : 0;
            const int m = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_ppr);
            const int p = idx - m * ppr;
            const u32x4 d = valid ? dv[b] : u32x4{0u, 0u, 0u, 0u};
            u32x4 q;
            q.x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);
            q.y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);
            q.z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);
            q.w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);
            float sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), 0.0f, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), sm, false);
            sm = row16_sum(sm);
            if (valid) {
                const int T = p >> 4, w4 = p & 3, pkb = (p >> 2) & 3;
                xs[((T * 4 + w4) * M + m) * 4 + pkb] = q;
                if ((p & 15) == 0) xm[T * M + m] = sm;
            }
        }
    };

    // prologue: phase 0's X, this wave's coefficients, the weight ring
    {
        u32x4 dv[kXB];
        load_x(0, dv);
        const int cpasses = (G + kWave - 1) / kWave;
        for (int j = 0; j < cpasses; ++j) {
            const int g = min(lane + kWave * j, G - 1);
#pragma unroll
            for (int r = 0; r < 16 * RT; ++r) {
                const int64_t row = min(16 * tile0 + r, N - 1);
                const float sv = scales[row * G + g];
                const uint32_t zb = zeros[row * (G >> 1) + (g >> 1)];
                if (lane + kWave * j < G) {
                    csw[r * G + g] = sv;
                    zsw[r * G + g] = static_cast<uint8_t>((g & 1) ? (zb >> 4) : (zb & 0xFu));
                }
            }
        }
#pragma unroll
        for (int u = 0; u < D; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) w[u][rt] = wrow[rt][min(u, nT - 1) * kTStep<SHUF>];
        write_x(0, dv);
    }
    __syncthreads();

    const NibConsts nk = nib_consts();
    f32x4 acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 nx[kXB];
    for (int T0 = 0; T0 < nT; T0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int T = T0 + u;
            if (T >= nT) continue;                    // uniform
            const int ph = T / NTP, Tl = T - ph * NTP;
            const int buf = ph & 1;
            if (Tl == 0 && ph + 1 < nT / NTP) load_x(ph + 1, nx);   // next phase's X in flight
            const u32x4* xs = xslot0 + buf * slots;
            const float* xm = xsum0 + buf * sums;
            const int g = T >> gshift;
            bf16x8_t a[RT][4];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const u32x4 wv = w[u][rt];
                a[rt][0] = a_operand(wv.x, nk);
                a[rt][1] = a_operand(wv.y, nk);
                a[rt][2] = a_operand(wv.z, nk);
                a[rt][3] = a_operand(wv.w, nk);
                w[u][rt] = wrow[rt][min(T + D, nT - 1) * kTStep<SHUF>];   // refill the ring slot
            }
            f32x4 s4[RT], z4[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const float* cr = csw + (16 * rt + 4 * kb) * G + g;
                const uint8_t* zr = zsw + (16 * rt + 4 * kb) * G + g;
                s4[rt] = f32x4{cr[0], cr[G], cr[2 * G], cr[3 * G]};
                z4[rt] = f32x4{-s4[rt].x * static_cast<float>(136u + zr[0]),
                               -s4[rt].y * static_cast<float>(136u + zr[G]),
                               -s4[rt].z * static_cast<float>(136u + zr[2 * G]),
                               -s4[rt].w * static_cast<float>(136u + zr[3 * G])};
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = 16 * mt + i;
                bf16x8_t b[4];
                float xsv = 0.0f;
#pragma unroll
                for (int w4 = 0; w4 < 4; ++w4) b[w4] = bf16x8_t{};
                if (m < M) {
#pragma unroll
                    for (int w4 = 0; w4 < 4; ++w4)
                        b[w4] = __builtin_bit_cast(bf16x8_t, xs[((Tl * 4 + w4) * M + m) * 4 + kb]);
                    xsv = xm[Tl * M + m];
                }
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rt][0], b[0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rt][1], b[1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rt][2], b[2], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rt][3], b[3], d, 0, 0, 0);
                    f32x4 ac = acc[rt][mt];
                    ac.x = fmaf(s4[rt].x, d.x, fmaf(z4[rt].x, xsv, ac.x));
                    ac.y = fmaf(s4[rt].y, d.y, fmaf(z4[rt].y, xsv, ac.y));
                    ac.z = fmaf(s4[rt].z, d.z, fmaf(z4[rt].z, xsv, ac.z));
                    ac.w = fmaf(s4[rt].w, d.w, fmaf(z4[rt].w, xsv, ac.w));
                    acc[rt][mt] = ac;
                }
            }
            if (Tl == NTP - 1 && ph + 1 < nT / NTP) {  // uniform: publish the next phase
                write_x(buf ^ 1, nx);
                __syncthreads();
            }
        }
    }

    // lane (i, kb) holds Y[m = 16 mt + i][n = 16 (tile0 + rt) + 4 kb + v]
    const int first = (static_cast<int>(blockIdx.x) * W + wave) * RT;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (first + rt >= ntiles) continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = 16 * mt + i;
            if (m >= M) continue;
            const float vals[4] = {acc[rt][mt].x, acc[rt][mt].y, acc[rt][mt].z, acc[rt][mt].w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = 16 * (first + rt) + 4 * kb + v;
                if (n < N) Y[static_cast<int64_t>(m) * N + n] = kc::f32_to_bf16(vals[v]);
            }
        }
    }
}

template <int W, int RT, int NTP, int D, bool SHUF>
int launch_xbig(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                const uint16_t* X, uint16_t* Y, int M, int N, int K, int gshift, hipStream_t stream) {
    const int G = (K / kTBlock) >> gshift;
    const size_t lds = xbig_lds_bytes(M, G, W, RT, NTP);
    if (lds > 160 * 1024) return -1;
    static bool attr_set = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_int4_xbig_kernel<W, RT, NTP, D, SHUF>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    }();
    if (!attr_set) return kc::set_error(KC_ERR_HIP, "%s: cannot raise the LDS limit", fn);
    const int ntiles = (N + 15) / 16;
    const int per_wg = W * RT;
    const unsigned grid = static_cast<unsigned>((ntiles + per_wg - 1) / per_wg);
    gemm_int4_xbig_kernel<W, RT, NTP, D, SHUF><<<grid, W * kWave, lds, stream>>>(packed, scales, zeros, X, Y, M, N, K, gshift);
    return kc::check_launch(fn);
}


// ---------------------------------------------------------------------------
// M 17..64: K split across the waves of a workgroup, X straight from the
// cache into registers.
//
// A workgroup of four waves (one per SIMD) owns RT = 7 consecutive 16-row
// weight tiles (112 rows: N = 28672 gives 256 workgroups, one per CU); wave
// w owns the T-blocks [w nT / 4, (w + 1) nT / 4) of K for all seven tiles
// and all MT activation tiles.  Per T-block a wave loads the MT B operands
// of its K range from X (every wave reads a different quarter of X, so no
// activation byte passes through LDS or is read twice by a CU), decodes each
// weight tile's A operands once and runs them against the MT activation
// tiles, and folds the T-block into its accumulators with the coefficients
// (s, c2) staged in LDS at the start.  The weights stream through a D-deep
// ring of T-blocks in registers, X one T-block ahead.  At the end the four
// K parts of each output tile are summed through LDS in a fixed order.
//
// Against the X-resident kernels, where every wave runs over all of K and
// all waves of a CU share X through LDS, the B-operand LDS traffic (each
// wave re-reading all of X) and the restaging of X by phases are gone; the
// cost is 4 x RT x MT accumulators per wave and a final cross-wave sum.
// ---------------------------------------------------------------------------
constexpr int kKsWaves = 4;
constexpr int kKsRT = 7, kKsD = 2;

__device__ __forceinline__ float swap32_sum(float a) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a),
                                                    __builtin_bit_cast(unsigned, a), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float swap16_sum(float a) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a),
                                                    __builtin_bit_cast(unsigned, a), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

// LDS: the coefficients cs[t][row], cz[t][row] of every wave's K range, later
// reused for the cross-wave sum (one f32x4 per lane, tile and wave).
// (a wave's range rounded up to whole ring turns of D T-blocks)
__host__ __device__ constexpr size_t kslice_lds_bytes(int MT, int RT, int D, int nT) {
    const size_t coef = static_cast<size_t>(kKsWaves) * (((nT + kKsWaves - 1) / kKsWaves + D - 1) / D * D) * 16 * RT * 8;
    const size_t red = static_cast<size_t>(kKsWaves) * RT * MT * kWave * 16;
    return coef > red ? coef : red;
}

template <int MT, int RT, int D, bool SHUF>
__global__ __launch_bounds__(kKsWaves * kWave) void gemm_int4_kslice_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int M, int N, int K, int gshift) {
    extern __shared__ __align__(16) char lds[];
    constexpr int kRows = 16 * RT;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int i = lane & 15, kb = lane >> 4;
    const int nT = K / kTBlock;
    const int G = nT >> gshift;
    const int ntmax = ((nT + kKsWaves - 1) / kKsWaves + D - 1) / D * D;  // whole ring turns
    const int t0 = (wave * nT) / kKsWaves, t1 = ((wave + 1) * nT) / kKsWaves;
    const int nt = t1 - t0;  // 0 for some waves when nT < 4
    const int ntp = (nt + D - 1) / D * D;  // the loop's T-blocks: nt, padded to whole ring turns
    const int tl = max(t1 - 1, 0);
    const int row_base = blockIdx.x * kRows;
    float* cs = reinterpret_cast<float*>(lds) + static_cast<size_t>(wave) * ntmax * kRows * 2;
    float* cz = cs + ntmax * kRows;

    // Byte offsets of this lane's weight rows (row_base + 16 rt + i, bytes
    // 16 kb .. 16 kb + 15 of each T-block) and X rows (16 c + i, bytes
    // 64 kb .. 64 kb + 63 of each T-block): 32 bits, the launcher checks that
    // both operands are smaller than 4 GiB.  Rows past the end are clamped.
    uint32_t woff[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        woff[rt] = SHUF ? static_cast<uint32_t>(min(row_base / 16 + rt, (N + 15) / 16 - 1)) * static_cast<uint32_t>(nT * 1024) + 16u * lane
                        : static_cast<uint32_t>(min(row_base + 16 * rt + i, N - 1)) * static_cast<uint32_t>(K >> 1) + 16u * kb;
    uint32_t xoff[MT];
#pragma unroll
    for (int c = 0; c < MT; ++c)
        xoff[c] = static_cast<uint32_t>(min(16 * c + i, M - 1)) * static_cast<uint32_t>(2 * K) + 64u * kb;
    const uint8_t* xbytes = reinterpret_cast<const uint8_t*>(X);
    auto wload = [&](int rt, int T) {
        return *reinterpret_cast<const u32x4*>(packed + (static_cast<uint32_t>(16 * kTStep<SHUF> * min(T, tl)) + woff[rt]));
    };
    auto xload = [&](int c, int T, int s) {
        return *reinterpret_cast<const u32x4*>(xbytes + (static_cast<uint32_t>(256 * min(T, tl) + 16 * s) + xoff[c]));
    };

    u32x4 wr[D][RT];  // weight ring: T-blocks T .. T + D - 1
    u32x4 xb[MT][4];  // X of the next T-block
#pragma unroll
    for (int u = 0; u < D; ++u)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) wr[u][rt] = wload(rt, t0 + u);
#pragma unroll
    for (int c = 0; c < MT; ++c)
#pragma unroll
        for (int s = 0; s < 4; ++s) xb[c][s] = xload(c, t0, s);

    // Fold coefficients of this wave's K range, cs[t][row] = s and
    // cz[t][row] = -s (136 + z): every load of a pass is issued before the
    // first is used (one memory round trip per pass); item idx = (row, t)
    // with t fastest, row = (idx + 0.5) / nt in fp32 (exact: idx < 2^24 and
    // the quotient is never within 0.5 / nt of an integer).
    {
        constexpr int kBatch = 28;  // 16 T-blocks x 112 rows in one pass
        const int items = nt * kRows;
        const float inv_nt = 1.0f / static_cast<float>(max(nt, 1));
        for (int base = 0; base < items; base += kBatch * kWave) {
            float sv[kBatch];
            uint32_t zb[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int idx = min(base + b * kWave + lane, items - 1);
                const int r = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_nt);
                const int g = (t0 + idx - r * nt) >> gshift;
                const int64_t row = min(row_base + r, N - 1);
                sv[b] = scales[row * G + g];
                zb[b] = zeros[row * (G >> 1) + (g >> 1)];
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int idx = base + b * kWave + lane;
                if (idx < items) {
                    const int r = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_nt);
                    const int t = idx - r * nt;
                    const int g = (t0 + t) >> gshift;
                    const uint32_t z = (g & 1) ? (zb[b] >> 4) : (zb[b] & 0xFu);
                    cs[t * kRows + r] = sv[b];
                    cz[t * kRows + r] = -sv[b] * static_cast<float>(136u + z);
                }
            }
        }
        // padding T-blocks fold with zero coefficients
        for (int idx = nt * kRows + lane; idx < ntp * kRows; idx += kWave) {
            cs[idx] = 0.0f;
            cz[idx] = 0.0f;
        }
    }
    __syncthreads();

    const NibConsts nk = nib_consts();
    uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs
    asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
    asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
    const uint32_t ones = 0x3F803F80u;
    f32x4 acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int c = 0; c < MT; ++c) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    // A whole number of ring turns, so the body has no branch (a guarded
    // iteration would make the compiler's load-count waits conservative):
    // padding T-blocks past the range reload the last one and fold with the
    // zero coefficients staged for them.
    const int tend = t0 + ntp;
    for (int T0 = t0; T0 < tend; T0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int T = T0 + u;
            // B operands in pair order, and the T-block sums of X: lane
            // (i, kb) sums its 32 values, the four kb lanes are added with
            // permlane swaps.
            bf16x8_t b[MT][4];
            float xs[MT];
#pragma unroll
            for (int c = 0; c < MT; ++c) {
                float sm = 0.0f;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const u32x4 d = xb[c][s];
                    u32x4 q;
                    q.x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);  // (x0, x4)
                    q.y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);  // (x1, x5)
                    q.z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);  // (x2, x6)
                    q.w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);  // (x3, x7)
                    b[c][s] = __builtin_bit_cast(bf16x8_t, q);
                    sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), sm, false);
                    sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), sm, false);
                    sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), sm, false);
                    sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), sm, false);
                }
                xs[c] = swap16_sum(swap32_sum(sm));
            }
#pragma unroll
            for (int c = 0; c < MT; ++c)
#pragma unroll
                for (int s = 0; s < 4; ++s) xb[c][s] = xload(c, T + 1, s);
            const int tt = T - t0;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const u32x4 wv = wr[u][rt];
                const bf16x8_t a0 = a_operand(wv.x, nk), a1 = a_operand(wv.y, nk);
                const bf16x8_t a2 = a_operand(wv.z, nk), a3 = a_operand(wv.w, nk);
                wr[u][rt] = wload(rt, T + D);
                const f32x4 s4 = *reinterpret_cast<const f32x4*>(cs + tt * kRows + 16 * rt + 4 * kb);
                const f32x4 z4 = *reinterpret_cast<const f32x4*>(cz + tt * kRows + 16 * rt + 4 * kb);
#pragma unroll
                for (int c = 0; c < MT; ++c) {
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[c][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[c][1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[c][2], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b[c][3], d, 0, 0, 0);
                    f32x4& a = acc[rt][c];
                    a.x = fmaf(s4.x, d.x, fmaf(z4.x, xs[c], a.x));
                    a.y = fmaf(s4.y, d.y, fmaf(z4.y, xs[c], a.y));
                    a.z = fmaf(s4.z, d.z, fmaf(z4.z, xs[c], a.z));
                    a.w = fmaf(s4.w, d.w, fmaf(z4.w, xs[c], a.w));
                }
                // one weight tile at a time: without this fence the scheduler
                // interleaves the tiles and the register demand spills
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // Sum the four K parts of every output tile through LDS (waves in a
    // fixed order), wave w finishing tiles w, w + 4, ...; lane (i, kb) of
    // tile (rt, c) holds Y[m = 16 c + i][n = row_base + 16 rt + 4 kb + v].
    __syncthreads();  // every wave is done with the coefficients
    f32x4* red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int c = 0; c < MT; ++c) red[((wave * RT + rt) * MT + c) * kWave + lane] = acc[rt][c];
    __syncthreads();
    for (int tile = wave; tile < RT * MT; tile += kKsWaves) {
        const int rt = tile / MT, c = tile - rt * MT;
        f32x4 v = red[(rt * MT + c) * kWave + lane];
#pragma unroll
        for (int w = 1; w < kKsWaves; ++w) {
            const f32x4 o = red[((w * RT + rt) * MT + c) * kWave + lane];
            v.x += o.x;
            v.y += o.y;
            v.z += o.z;
            v.w += o.w;
        }
        const int m = 16 * c + i;
        const int n0 = row_base + 16 * rt + 4 * kb;
        if (m < M) {
            const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n0 + e < N) Y[static_cast<int64_t>(m) * N + n0 + e] = kc::f32_to_bf16(vals[e]);
        }
    }
}

// Returns -1 when the kernel does not apply (LDS or 32-bit offsets).
template <int MT, bool SHUF>
int launch_kslice(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                  const uint16_t* X, uint16_t* Y, int M, int N, int K, int gshift, hipStream_t stream) {
    const size_t lds = kslice_lds_bytes(MT, kKsRT, kKsD, K / kTBlock);
    if (lds > 160 * 1024 || static_cast<uint64_t>((N + 15) / 16) * 16 * (K / 2) >= (uint64_t{1} << 32) ||
        static_cast<uint64_t>(M) * K * 2 >= (uint64_t{1} << 32))
        return -1;
    static bool attr_set = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_int4_kslice_kernel<MT, kKsRT, kKsD, SHUF>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    }();
    if (!attr_set) return kc::set_error(KC_ERR_HIP, "%s: cannot raise the LDS limit", fn);
    const unsigned grid = static_cast<unsigned>((N + 16 * kKsRT - 1) / (16 * kKsRT));
    gemm_int4_kslice_kernel<MT, kKsRT, kKsD, SHUF><<<grid, kKsWaves * kWave, lds, stream>>>(
        packed, scales, zeros, X, Y, M, N, K, gshift);
    return kc::check_launch(fn);
}

// ---------------------------------------------------------------------------
// M 9..64 with both operands streamed through LDS: gemm_int4_kslds_kernel.
//
// The work split of gemm_int4_kslice_kernel (four waves per CU, wave w owns
// K quarter w of RT = 7 row tiles for all MT activation tiles, the four K
// parts summed through LDS at the end), with the operands brought in by
// direct-to-LDS loads instead of through registers:
//   * X: per T-block the wave's 16 MT rows x 256 bytes, in 1-KB blocks of
//     four rows, each block one load instruction that reads its 1 KB in one
//     piece (the register kernel's B-operand loads touch 32 cache lines per
//     instruction).  Lane l of block j carries chunk u of local row
//     r = l / 16, u = (l - 4 (j mod 4) - r) mod 16, so chunk u of row r sits
//     in slot 16 r + ((u + 4 (j mod 4) + r) mod 16): a B-operand read (lane
//     (i, kb), step s: chunk 4 kb + s of row 16 c + i, rotated by i) gives
//     the 16 lanes of each kb 16 different 16-byte bank groups.
//   * W: per T-block and row tile the wave-wide 1-KB load of the register
//     kernel, lane l's 16 bytes in slot l.  On the reference layout that
//     load reads 64 bytes from each of 16 rows, and 16 neighbouring lanes
//     touch 16 cache lines; with K a multiple of 1024 and M <= 48 (the LDS
//     for 2-KB slots; at M 33..48 the zero points kept as bytes) the weights
//     instead come per pair of T-blocks,
//     two loads per tile of 8 whole 128-byte rows each (8 lanes per row).
//     The first T-block of the pair reads both halves of every tile and
//     keeps the second T-block's in registers; it then requests the next
//     pair's rows 0-7 of the tile and the second T-block its rows 8-15.
// One T-block (pair) of each is resident per wave.  X of the next T-block is
// requested once the current one has been read out, each row tile's next
// weights right after that tile's decode, so every load has about one
// T-block to arrive; the last T-block requests nothing.  The waits are
// explicit (loads complete in order: vmcnt(7) before X, vmcnt(22) before
// each weight tile, counting the loads issued since).  With no operand ring
// in registers, the accumulators, the B operands and the matrix-core results
// fit the 256 VGPRs.  With three or four activation tiles the fold keeps only
// its scale FMA per T-block; the zero-point terms of four T-blocks at a time
// go through one fp32 MFMA (16 x 16 x 4) per output tile.
// ---------------------------------------------------------------------------
constexpr int kKlRT = 7;
// Coefficient table row stride: 112 rows padded to 116 floats, so that the
// staging writes (64 lanes, T-block fastest: 116 t + r) fall in 64 different
// banks instead of 4, and a 4-row read stays 16-byte aligned (464 bytes).
constexpr int kKlCS = 16 * kKlRT + 4;

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<size_t>((lds_void_t*)p));
}

// One global_load_lds_dwordx4: 16 bytes per lane from sbase + voff into LDS
// at lds_base + 16 lane.  `after` is a register the load is made to depend
// on (a value computed from the last LDS read of the slot it overwrites), so
// it is issued after that read has returned.
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t lds_base, uint32_t after) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base),
                 "v"(after)
                 : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_waitcnt vmcnt(n), n a constant once the caller's loop is unrolled.
__device__ __forceinline__ void wait_vmcnt_n(int n) {
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        case 7: wait_vmcnt<7>(); break;
        case 8: wait_vmcnt<8>(); break;
        case 9: wait_vmcnt<9>(); break;
        case 10: wait_vmcnt<10>(); break;
        case 11: wait_vmcnt<11>(); break;
        case 12: wait_vmcnt<12>(); break;
        case 13: wait_vmcnt<13>(); break;
        case 14: wait_vmcnt<14>(); break;
        case 15: wait_vmcnt<15>(); break;
        case 16: wait_vmcnt<16>(); break;
        case 17: wait_vmcnt<17>(); break;
        case 18: wait_vmcnt<18>(); break;
        case 19: wait_vmcnt<19>(); break;
        case 20: wait_vmcnt<20>(); break;
        case 21: wait_vmcnt<21>(); break;
        case 22: wait_vmcnt<22>(); break;
        case 23: wait_vmcnt<23>(); break;
        case 24: wait_vmcnt<24>(); break;
        case 25: wait_vmcnt<25>(); break;
        case 26: wait_vmcnt<26>(); break;
        case 27: wait_vmcnt<27>(); break;
        default: wait_vmcnt<0>(); break;
    }
}

// Zero points kept as bytes (c2 = -s (136 + z) formed where it is read):
// pairs of T-blocks with three activation tiles, where only the zero-point
// pass on the fp32 matrix core reads them, once per four T-blocks.
template <int MT, bool PAIR>
constexpr bool kKslZBytes = PAIR && MT >= 3;

// Per-wave LDS: X (4 MT KB), weights (RT KB, or 2 RT KB for a pair of
// T-blocks), fold coefficients of the wave's quarter (ceil(nT / 4) T-blocks
// x kKlCS x (s, c2), or (s, z) with z a byte, the byte table rounded to 16).
template <int MT, bool PAIR>
__host__ __device__ constexpr size_t kslds_wave_bytes(int nT) {
    const size_t nq = static_cast<size_t>((nT + kKsWaves - 1) / kKsWaves);
    const size_t coef = kKslZBytes<MT, PAIR> ? nq * kKlCS * 4 + (nq * kKlCS + 15) / 16 * 16 : nq * kKlCS * 8;
    return static_cast<size_t>(4 * MT + (PAIR ? 2 : 1) * kKlRT) * 1024 + coef;
}

template <int MT, bool PAIR>
__host__ __device__ constexpr size_t kslds_lds_bytes(int nT) {
    const size_t ops = kKsWaves * kslds_wave_bytes<MT, PAIR>(nT);
    const size_t red = static_cast<size_t>(kKsWaves) * kKlRT * MT * kWave * 16;
    return ops > red ? ops : red;
}

template <int MT, bool SHUF, bool PAIR>
__global__ __launch_bounds__(kKsWaves * kWave) void gemm_int4_kslds_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int M, int N, int K, int gshift) {
    extern __shared__ __align__(16) char lds[];
    constexpr int RT = kKlRT;
    constexpr int kRows = 16 * RT;
    constexpr int kCS = kKlCS;  // coefficient row stride (floats per T-block)
    constexpr int kXB = 4 * MT;  // X blocks of four rows per T-block
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int i = lane & 15, kb = lane >> 4;
    const int nT = K / kTBlock;
    const int G = nT >> gshift;
    const int ntmax = (nT + kKsWaves - 1) / kKsWaves;
    const int t0 = (wave * nT) / kKsWaves, t1 = ((wave + 1) * nT) / kKsWaves;
    const int nt = t1 - t0;  // 0 for some waves when nT < 4
    const int tl = max(t1 - 1, 0);
    const int row_base = blockIdx.x * kRows;
    char* xl = lds + static_cast<size_t>(wave) * kslds_wave_bytes<MT, PAIR>(nT);
    char* wl = xl + kXB * 1024;
    float* cs = reinterpret_cast<float*>(wl + (PAIR ? 2 : 1) * RT * 1024);
    float* cz = cs + ntmax * kCS;
    constexpr bool kZB = kKslZBytes<MT, PAIR>;
    uint8_t* czb = reinterpret_cast<uint8_t*>(cz);  // zero points, when kZB
    const uint32_t x_lds = lds_addr(xl), w_lds = lds_addr(wl);

    // DMA offsets.  X block j, lane l: row 4 j + r (r = l / 16), chunk u.
    // Rows below 16 (MT - 1) exist (M > 16 (MT - 1)): blocks j < 4 MT - 4
    // take lane offset xg[j & 3] and 8 K j bytes on the scalar base; the last
    // tile's four blocks clamp their rows to M - 1 per lane (xe).
    uint32_t xg[4], xe[4];
    {
        const int r = lane >> 4;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            xg[q] = static_cast<uint32_t>(r) * static_cast<uint32_t>(2 * K) + 16u * (((lane & 15) - 4 * q - r) & 15);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = kXB - 4 + q;
            xe[q] = static_cast<uint32_t>(min(4 * j + r, M - 1)) * static_cast<uint32_t>(2 * K) +
                    16u * (((lane & 15) - 4 * q - r) & 15);
        }
    }
    uint32_t woff[RT];
    if constexpr (!PAIR) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            woff[rt] = SHUF ? static_cast<uint32_t>(min(row_base / 16 + rt, (N + 15) / 16 - 1)) * static_cast<uint32_t>(nT * 1024) + 16u * lane
                            : static_cast<uint32_t>(min(row_base + 16 * rt + i, N - 1)) * static_cast<uint32_t>(K >> 1) + 16u * kb;
    }
    // Pairs of T-blocks (reference layout): tile rt's 16 rows x 128 bytes
    // (T-blocks 2 p and 2 p + 1) in two loads of 8 whole rows, h = 0 / 1 for
    // rows 8 h .. 8 h + 7.  Lane l = 8 r + pos of load h carries chunk
    // c = (pos - (r xor h)) mod 8 of row 8 h + r into slot
    // 2048 rt + 1024 h + 16 l, so chunk c of that row sits at position
    // (c + (r xor h)) mod 8 of its 128 bytes: the 16 rows of one chunk fall
    // in 16 different 16-byte bank groups, each 8 of them in 8.
    uint32_t woffp[PAIR ? RT : 1][2];
    if constexpr (PAIR) {
        const int r = lane >> 3, pos = lane & 7;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                woffp[rt][h] = static_cast<uint32_t>(min(row_base + 16 * rt + 8 * h + r, N - 1)) * static_cast<uint32_t>(K >> 1) +
                               16u * static_cast<uint32_t>((pos - (r ^ h)) & 7);
    }
    const uint8_t* xbytes = reinterpret_cast<const uint8_t*>(X);
    auto issue_x = [&](int T, uint32_t after) {
        const uint8_t* base = xbytes + 256 * min(T, tl);
#pragma unroll
        for (int j = 0; j < kXB - 4; ++j)
            dma16(xg[j & 3], base + static_cast<size_t>(8 * j) * K, x_lds + 1024 * j, after);
#pragma unroll
        for (int e = 0; e < 4; ++e) dma16(xe[e], base, x_lds + 1024 * (kXB - 4 + e), after);
    };
    auto issue_w = [&](int rt, int T, uint32_t after) {
        dma16(woff[rt], packed + 16 * kTStep<SHUF> * min(T, tl), w_lds + 1024 * rt, after);
    };
    // load h of tile rt for the pair of T-blocks 2 p, 2 p + 1
    auto issue_wh = [&](int rt, int p, int h, uint32_t after) {
        dma16(woffp[rt][h], packed + 128 * min(p, tl >> 1), w_lds + 2048 * rt + 1024 * h, after);
    };
    auto issue_wp = [&](int rt, int p, uint32_t after) {
        issue_wh(rt, p, 0, after);
        issue_wh(rt, p, 1, after);
    };
    // A-operand read offsets in a pair slot: lane (i, kb) of T-block parity t
    // reads chunk 4 t + kb of row i (h = i / 8, r = i % 8).
    uint32_t wrd[PAIR ? 2 : 1];
    if constexpr (PAIR) {
        const int h = i >> 3, r = i & 7;
#pragma unroll
        for (int t = 0; t < 2; ++t)
            wrd[t] = 1024u * h + 16u * static_cast<uint32_t>(8 * r + ((4 * t + kb + (r ^ h)) & 7));
    }
    // B-operand read offsets: lane (i, kb), step s reads chunk 4 kb + s of
    // row 16 c + i (block 4 c + i / 4, local row i % 4, rotation
    // 4 (i / 4) + i % 4 = i) at xrd[s] + 4096 c.
    uint32_t xrd[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) xrd[s] = 1024u * (i >> 2) + 256u * (i & 3) + 16u * ((4 * kb + s + i) & 15);

    constexpr int kWL = (PAIR ? 2 : 1) * RT;  // weight loads per T-block, per pair when PAIR
    auto issue_first = [&]() {
        issue_x(t0, 0u);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if constexpr (PAIR) issue_wp(rt, t0 >> 1, 0u);
            else issue_w(rt, t0, 0u);
        }
    };

    // Fold coefficients of this wave's K range, cs[t][row] = s and
    // cz[t][row] = -s (136 + z).
    //
    // One group per T-block, whole quads of T-blocks and aligned tables (the
    // usual case, e.g. K 8192 with groups of 128): lane item (row, quad q)
    // reads the four scales of T-blocks 4 q .. 4 q + 3 with one 16-byte load
    // and their four zero points with one 2-byte load; the first pass (all of
    // a 16-T-block quarter) is requested before this T-block's operand loads
    // and waited for with them still in flight.  Otherwise one item per
    // (row, T-block), as in gemm_int4_kslice_kernel.
    const bool quad = gshift == 0 && (nT & 15) == 0 && (reinterpret_cast<uintptr_t>(scales) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(zeros) & 1) == 0;
    if (quad) {
        constexpr int kQB = 7;  // 112 rows x 4 quads in one pass
        const int nq = nt >> 2;
        const int items = kRows * nq;
        const float inv_nq = 1.0f / static_cast<float>(max(nq, 1));
        const float* srow = scales + static_cast<size_t>(row_base) * G + t0;
        const uint8_t* zrow = zeros + static_cast<size_t>(row_base) * (G >> 1) + (t0 >> 1);
        auto item = [&](int idx, int& r, int& q) {
            r = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_nq);
            q = idx - r * nq;
        };
        auto store = [&](int base, const u32x4 (&sq)[kQB], const uint32_t (&zq)[kQB]) {
#pragma unroll
            for (int b = 0; b < kQB; ++b) {
                const int idx = base + b * kWave + lane;
                if (idx < items) {
                    int r, q;
                    item(idx, r, q);
                    // the whole vector is cast: this compiler reads component 0
                    // for a bit cast of any single component of an ext-vector
                    const f32x4 sf = __builtin_bit_cast(f32x4, sq[b]);
                    const float sv[4] = {sf.x, sf.y, sf.z, sf.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t z = (zq[b] >> (4 * e)) & 0xFu;
                        cs[(4 * q + e) * kCS + r] = sv[e];
                        if constexpr (kZB) czb[(4 * q + e) * kCS + r] = static_cast<uint8_t>(z);
                        else cz[(4 * q + e) * kCS + r] = -sv[e] * static_cast<float>(136u + z);
                    }
                }
            }
        };
        // 32-bit offsets from the workgroup's first row (rows past N - 1 read row N - 1)
        auto offsets = [&](int base, int b, uint32_t& so, uint32_t& zo) {
            int r, q;
            item(min(base + b * kWave + lane, items - 1), r, q);
            const uint32_t rr = static_cast<uint32_t>(min(row_base + r, N - 1) - row_base);
            so = (rr * static_cast<uint32_t>(G) + 4u * q) * 4u;
            zo = rr * static_cast<uint32_t>(G >> 1) + 2u * q;
        };
        {
            u32x4 sq[kQB];
            uint32_t zq[kQB];
#pragma unroll
            for (int b = 0; b < kQB; ++b) {
                uint32_t so, zo;
                offsets(0, b, so, zo);
                asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(sq[b]) : "v"(so), "s"(srow));
                asm volatile("global_load_ushort %0, %1, %2" : "=v"(zq[b]) : "v"(zo), "s"(zrow));
            }
            issue_first();
            // the 2 kQB loads above have landed once only this T-block's
            // kXB + kWL operand loads can remain
            asm volatile("s_waitcnt vmcnt(%14)"
                         : "+v"(sq[0]), "+v"(sq[1]), "+v"(sq[2]), "+v"(sq[3]), "+v"(sq[4]), "+v"(sq[5]), "+v"(sq[6]),
                           "+v"(zq[0]), "+v"(zq[1]), "+v"(zq[2]), "+v"(zq[3]), "+v"(zq[4]), "+v"(zq[5]), "+v"(zq[6])
                         : "n"(kXB + kWL)
                         : "memory");
            store(0, sq, zq);
        }
        for (int base = kQB * kWave; base < items; base += kQB * kWave) {
            u32x4 sq[kQB];
            uint32_t zq[kQB];
#pragma unroll
            for (int b = 0; b < kQB; ++b) {
                uint32_t so, zo;
                offsets(base, b, so, zo);
                sq[b] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(srow) + so);
                zq[b] = *reinterpret_cast<const uint16_t*>(zrow + zo);
            }
            store(base, sq, zq);
        }
    } else {
        issue_first();
        constexpr int kBatch = 28;  // 16 T-blocks x 112 rows in one pass
        const int items = nt * kRows;
        const float inv_nt = 1.0f / static_cast<float>(max(nt, 1));
        for (int base = 0; base < items; base += kBatch * kWave) {
            float sv[kBatch];
            uint32_t zb[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int idx = min(base + b * kWave + lane, items - 1);
                const int r = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_nt);
                const int g = (t0 + idx - r * nt) >> gshift;
                const int64_t row = min(row_base + r, N - 1);
                sv[b] = scales[row * G + g];
                zb[b] = zeros[row * (G >> 1) + (g >> 1)];
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int idx = base + b * kWave + lane;
                if (idx < items) {
                    const int r = static_cast<int>((static_cast<float>(idx) + 0.5f) * inv_nt);
                    const int t = idx - r * nt;
                    const int g = (t0 + t) >> gshift;
                    const uint32_t z = (g & 1) ? (zb[b] >> 4) : (zb[b] & 0xFu);
                    cs[t * kCS + r] = sv[b];
                    if constexpr (kZB) czb[t * kCS + r] = static_cast<uint8_t>(z);
                    else cz[t * kCS + r] = -sv[b] * static_cast<float>(136u + z);
                }
            }
        }
    }

    const NibConsts nk = nib_consts();
    uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs
    asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
    asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
    const uint32_t ones = 0x3F803F80u;
    f32x4 acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int c = 0; c < MT; ++c) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    // With three or four activation tiles the zero-point half of the fold,
    // cz[t][n] xs[t][m], is left to the fp32 matrix core, four T-blocks at a
    // time: xsb[c] holds xs of T-block g0 + kb of the current group of four.
    constexpr bool kZmf = MT >= 3;
    float xsb[kZmf ? MT : 1];
    if constexpr (kZmf) {
#pragma unroll
        for (int c = 0; c < MT; ++c) xsb[c] = 0.0f;
    }

    // Pairs of T-blocks: the first T-block of a pair reads both halves of
    // every tile and keeps the second T-block's half here, so the slot is
    // free once it has been read: the first T-block requests the next pair's
    // rows 0-7 of the tile, the second T-block its rows 8-15 (seven loads per
    // T-block, each with one or two T-blocks to arrive), and the second
    // T-block reads no weights from LDS.
    u32x4 wv1[PAIR ? RT : 1];

    // One T-block; the last one issues no loads for a next one, so its
    // waits count only its own remaining weight tiles.  kPar < 0: one
    // T-block per weight slot; else bit 0: second T-block of a pair, bit 1:
    // the first pair (the prologue's loads), bit 2: the last pair (no
    // weights for a next pair).
    auto tblock = [&](int T, auto last_tag, auto par_tag) {
        constexpr bool kLast = decltype(last_tag)::value;
        constexpr int kPar = decltype(par_tag)::value;
        constexpr bool kPair = kPar >= 0;
        constexpr bool kSecond = kPair && (kPar & 1) != 0;
        constexpr bool kFirstPair = kPair && (kPar & 2) != 0;
        constexpr bool kLastPair = kPair && (kPar & 4) != 0;
        constexpr bool kEnd = kPair ? kSecond && kLastPair : kLast;  // no X for a next T-block
        const int tt = T - t0;
        // X of this T-block: issued before the 7 weight loads of this
        // T-block (in a pair, the previous T-block's 7), the prologue's 14,
        // or none (second T-block of the last pair).
        if constexpr (!kPair) wait_vmcnt<RT>();
        else if constexpr (!kSecond && kFirstPair) wait_vmcnt<2 * RT>();
        else if constexpr (kSecond && kLastPair) wait_vmcnt<0>();
        else wait_vmcnt<RT>();
        // all X reads in flight at once (the previous T-block's B operands
        // are dead), then the permutation and sums as they return
        u32x4 xr[MT][4];
#pragma unroll
        for (int c = 0; c < MT; ++c)
#pragma unroll
            for (int s = 0; s < 4; ++s) xr[c][s] = *reinterpret_cast<const u32x4*>(xl + xrd[s] + 4096 * c);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8_t b[MT][4];
        float xs[MT];
#pragma unroll
        for (int c = 0; c < MT; ++c) {
            float sm = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const u32x4 d = xr[c][s];
                u32x4 q;
                q.x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);  // (x0, x4)
                q.y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);  // (x1, x5)
                q.z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);  // (x2, x6)
                q.w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);  // (x3, x7)
                b[c][s] = __builtin_bit_cast(bf16x8_t, q);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), sm, false);
            }
            xs[c] = swap16_sum(swap32_sum(sm));
        }
        if constexpr (kZmf) {
#pragma unroll
            for (int c = 0; c < MT; ++c) xsb[c] = kb == (tt & 3) ? xs[c] : xsb[c];
        }
        if constexpr (!kEnd) {
            // every X read has returned once the sums exist
            uint32_t xdone = __builtin_bit_cast(uint32_t, xs[0]);
#pragma unroll
            for (int c = 1; c < MT; ++c) xdone ^= __builtin_bit_cast(uint32_t, xs[c]);
            issue_x(T + 1, xdone);
        }
        // Each tile's weights are read from LDS one tile ahead.  Tile rt's
        // load was issued before the 6 - rt later tiles of this T-block and,
        // unless this is the last T-block, the next T-block's X (kXB) and the
        // rt next-T-block tiles issued before the read: RT - 1 + kXB younger
        // loads, or RT - 1 - rt in the last T-block.
        // In a pair, tile rt's rows 8-15 were followed by the rows 8-15 of
        // the 6 - rt later tiles (the rows 0-7 and 8-15 of each, in the
        // prologue's first pair), the kXB of X(T + 1) and the rows 0-7 of
        // the next pair's tiles requested so far.
        u32x4 wv;
        if constexpr (!kPair) {
            if constexpr (kLast) wait_vmcnt<RT - 1>();
            else wait_vmcnt<RT - 1 + kXB>();
            wv = *reinterpret_cast<const u32x4*>(wl + 16 * lane);
        } else if constexpr (!kSecond) {
            if constexpr (kFirstPair) wait_vmcnt<2 * (RT - 1) + kXB>();
            else wait_vmcnt<RT - 1 + kXB>();
            wv = *reinterpret_cast<const u32x4*>(wl + wrd[0]);
            wv1[0] = *reinterpret_cast<const u32x4*>(wl + wrd[1]);
        } else {
            wv = wv1[0];
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const bf16x8_t a0 = a_operand(wv.x, nk), a1 = a_operand(wv.y, nk);
            const bf16x8_t a2 = a_operand(wv.z, nk), a3 = a_operand(wv.w, nk);
            if constexpr (!kPair) {
                if constexpr (!kLast) issue_w(rt, T + 1, __builtin_bit_cast(u32x4, a3).w ^ __builtin_bit_cast(u32x4, a0).x);
                if (rt + 1 < RT) {
                    if constexpr (kLast) wait_vmcnt_n(RT - 2 - rt);
                    else wait_vmcnt<RT - 1 + kXB>();
                    wv = *reinterpret_cast<const u32x4*>(wl + 1024 * (rt + 1) + 16 * lane);
                }
            } else if constexpr (!kSecond) {
                // both halves of slot rt have been read: the next pair's rows
                // 0-7 of the tile
                if constexpr (!kLastPair)
                    issue_wh(rt, (T >> 1) + 1, 0,
                             __builtin_bit_cast(u32x4, a3).w ^ __builtin_bit_cast(u32x4, a0).x ^ wv1[rt].x);
                if (rt + 1 < RT) {
                    constexpr int kNext = kLastPair ? 0 : 1;
                    if constexpr (kFirstPair) wait_vmcnt_n(kXB + 2 * (RT - 2 - rt) + kNext * (rt + 1));
                    else wait_vmcnt_n(kXB + (RT - 2 - rt) + kNext * (rt + 1));
                    wv = *reinterpret_cast<const u32x4*>(wl + 2048 * (rt + 1) + wrd[0]);
                    wv1[rt + 1] = *reinterpret_cast<const u32x4*>(wl + 2048 * (rt + 1) + wrd[1]);
                }
            } else {
                // the next pair's rows 8-15 of tile rt
                if constexpr (!kLastPair)
                    issue_wh(rt, (T >> 1) + 1, 1, __builtin_bit_cast(u32x4, a3).w ^ __builtin_bit_cast(u32x4, a0).x);
                if (rt + 1 < RT) wv = wv1[rt + 1];
            }
            const f32x4 s4 = *reinterpret_cast<const f32x4*>(cs + tt * kCS + 16 * rt + 4 * kb);
            if constexpr (kZmf) {
#pragma unroll
                for (int c = 0; c < MT; ++c) {
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[c][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[c][1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[c][2], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b[c][3], d, 0, 0, 0);
                    f32x4& a = acc[rt][c];
                    a.x = fmaf(s4.x, d.x, a.x);
                    a.y = fmaf(s4.y, d.y, a.y);
                    a.z = fmaf(s4.z, d.z, a.z);
                    a.w = fmaf(s4.w, d.w, a.w);
                }
            } else {
                const f32x4 z4 = *reinterpret_cast<const f32x4*>(cz + tt * kCS + 16 * rt + 4 * kb);
#pragma unroll
                for (int c = 0; c < MT; ++c) {
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[c][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[c][1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[c][2], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b[c][3], d, 0, 0, 0);
                    f32x4& a = acc[rt][c];
                    a.x = fmaf(s4.x, d.x, fmaf(z4.x, xs[c], a.x));
                    a.y = fmaf(s4.y, d.y, fmaf(z4.y, xs[c], a.y));
                    a.z = fmaf(s4.z, d.z, fmaf(z4.z, xs[c], a.z));
                    a.w = fmaf(s4.w, d.w, fmaf(z4.w, xs[c], a.w));
                }
            }
            // one weight tile at a time (register demand)
            __builtin_amdgcn_sched_barrier(0);
        }
        // zero points of the group of four T-blocks ending here, on the fp32
        // matrix core: acc[n][m] += sum_kb cz[g0 + kb][n] xs[g0 + kb][m]
        if constexpr (kZmf) {
            if ((tt & 3) == 3 || kEnd) {
                const int g0 = tt & ~3;
                const int tz = min(g0 + kb, nt - 1);  // lanes past the range hold xs = 0
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    float av;
                    if constexpr (kZB)  // the staging's c2, formed the same way
                        av = -cs[tz * kCS + 16 * rt + i] * static_cast<float>(136u + czb[tz * kCS + 16 * rt + i]);
                    else
                        av = cz[tz * kCS + 16 * rt + i];
#pragma unroll
                    for (int c = 0; c < MT; ++c) acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, xsb[c], acc[rt][c], 0, 0, 0);
                }
#pragma unroll
                for (int c = 0; c < MT; ++c) xsb[c] = 0.0f;
            }
        }
    };
    if constexpr (PAIR) {
        // t0 and nt even, nt >= 2 (the launch requires nT a multiple of 8)
        using F = std::false_type;
        using first = std::integral_constant<int, 0>;
        using second = std::integral_constant<int, 1>;
        using first_of_first = std::integral_constant<int, 2>;
        using first_of_last = std::integral_constant<int, 4>;
        using second_of_last = std::integral_constant<int, 5>;
        using first_of_only = std::integral_constant<int, 6>;
        if (nt == 2) {
            tblock(t0, F{}, first_of_only{});
            tblock(t0 + 1, F{}, second_of_last{});
        } else {
            tblock(t0, F{}, first_of_first{});
            tblock(t0 + 1, F{}, second{});
            for (int T = t0 + 2; T + 2 < t1; T += 2) {
                tblock(T, F{}, first{});
                tblock(T + 1, F{}, second{});
            }
            tblock(t1 - 2, F{}, first_of_last{});
            tblock(t1 - 1, F{}, second_of_last{});
        }
    } else {
        using single = std::integral_constant<int, -1>;
        for (int T = t0; T + 1 < t1; ++T) tblock(T, std::false_type{}, single{});
        if (nt > 0) tblock(t1 - 1, std::true_type{}, single{});
    }

    // Sum the four K parts of every output tile through LDS, as in
    // gemm_int4_kslice_kernel, once the last loads into LDS have landed.
    wait_vmcnt<0>();
    __syncthreads();
    f32x4* red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int c = 0; c < MT; ++c) red[((wave * RT + rt) * MT + c) * kWave + lane] = acc[rt][c];
    __syncthreads();
    const bool y8 = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 7) == 0;
    for (int tile = wave; tile < RT * MT; tile += kKsWaves) {
        const int rt = tile / MT, c = tile - rt * MT;
        f32x4 v = red[(rt * MT + c) * kWave + lane];
#pragma unroll
        for (int w = 1; w < kKsWaves; ++w) {
            const f32x4 o = red[((w * RT + rt) * MT + c) * kWave + lane];
            v.x += o.x;
            v.y += o.y;
            v.z += o.z;
            v.w += o.w;
        }
        const int m = 16 * c + i;
        const int n0 = row_base + 16 * rt + 4 * kb;
        if (m < M) {
            uint16_t* yp = Y + static_cast<int64_t>(m) * N + n0;
            if (y8 && n0 + 3 < N) {
                // four consecutive outputs, 8-byte aligned: one store
                const uint32_t lo = kc::f32_to_bf16(v.x) | (static_cast<uint32_t>(kc::f32_to_bf16(v.y)) << 16);
                const uint32_t hi = kc::f32_to_bf16(v.z) | (static_cast<uint32_t>(kc::f32_to_bf16(v.w)) << 16);
                *reinterpret_cast<uint2*>(yp) = make_uint2(lo, hi);
            } else {
                const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n0 + e < N) yp[e] = kc::f32_to_bf16(vals[e]);
            }
        }
    }
}

// Returns -1 when the kernel does not apply (LDS or 32-bit offsets; for the
// pair form, the shuffled layout or K not a multiple of 1024).
template <int MT, bool SHUF, bool PAIR>
int launch_kslds(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                 const uint16_t* X, uint16_t* Y, int M, int N, int K, int gshift, hipStream_t stream) {
    const int nT = K / kTBlock;
    if (PAIR && (SHUF || MT > 3 || nT % (2 * kKsWaves) != 0)) return -1;
    const size_t lds = kslds_lds_bytes<MT, PAIR>(nT);
    if (lds > 160 * 1024 || static_cast<uint64_t>((N + 15) / 16) * 16 * (K / 2) >= (uint64_t{1} << 32) ||
        static_cast<uint64_t>(M) * K * 2 >= (uint64_t{1} << 32))
        return -1;
    static bool attr_set = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_int4_kslds_kernel<MT, SHUF, PAIR>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    }();
    if (!attr_set) return kc::set_error(KC_ERR_HIP, "%s: cannot raise the LDS limit", fn);
    const unsigned grid = static_cast<unsigned>((N + 16 * kKlRT - 1) / (16 * kKlRT));
    gemm_int4_kslds_kernel<MT, SHUF, PAIR><<<grid, kKsWaves * kWave, lds, stream>>>(packed, scales, zeros, X, Y,
                                                                                     M, N, K, gshift);
    return kc::check_launch(fn);
}

// ---------------------------------------------------------------------------
// M = 1 on the shuffled layout: x is the A operand, the same 32 values in
// every row of the 16 x 32 block (a broadcast), the weight tile the B
// operand, so every row m of D = A B holds the 16 dot products and lane
// (i, kb)'s first accumulator is row i's.  A workgroup of KW waves owns one
// 16-row tile; wave w takes T-blocks TPW w .. TPW w + TPW - 1
// (K = 128 TPW KW, TPW 4 or 8) and issues all their loads at once: 1 KB in
// address order each.  Per wave the x of its range is staged in LDS in the decode's pair
// order with its T-block sums (no workgroup barrier), and each T-block is
// folded with its scale and zero point as in the other kernels.  Measured
// at K 4096 / 14336 against the reference-layout GEMV (bf16, rotating
// weights): gate/up 11.9-12.0 against 12.1-12.2 us, down 7.9 against 8.6,
// O 3.96 against 3.97, QKV 4.93 against 4.75.
// ---------------------------------------------------------------------------
template <int KW, int TPW, bool G128>
// (the waves-per-EU floor caps the registers at 85: without it the compiler
// takes 100, and fewer waves fit beside each other)
__global__ __launch_bounds__(KW * kWave) __attribute__((amdgpu_waves_per_eu(6))) void gemv_int4_shuf_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
    int rows, int cols, int gshift) {
    static_assert(TPW == 4 || TPW == 8 || TPW == 16, "T-blocks per wave");
    constexpr int kQ = TPW * 16;         // x quads (8 bf16) of a wave's range
    constexpr int kQPL = kQ / kWave;     // per lane
    __shared__ u32x4 xsh[KW][kQ];
    __shared__ float xsum[KW][TPW];
    __shared__ float part[KW][16];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int n = lane & 15, kb = lane >> 4;
    const int row0 = static_cast<int>(blockIdx.x) * 16;
    const int row = min(row0 + n, rows - 1);
    const int nT = cols / kTBlock;
    const int G = nT >> gshift;
    const int t0 = wave * TPW;

    // loads: x of the wave's range, this lane's scales and zero bytes, then
    // the weights (vector loads complete in order)
    u32x4 xr[kQPL];
    const u32x4* xq = reinterpret_cast<const u32x4*>(x) + t0 * 16;
#pragma unroll
    for (int u = 0; u < kQPL; ++u) xr[u] = xq[lane + kWave * u];
    float sv[TPW];
    uint32_t zv[TPW];
    if constexpr (G128) {  // one group per T-block: TPW scales and TPW / 2 zero bytes in a row
        const f32x4* sp = reinterpret_cast<const f32x4*>(scales + static_cast<int64_t>(row) * G + t0);
#pragma unroll
        for (int i = 0; i < TPW / 4; ++i) {
            const f32x4 s4 = sp[i];
            sv[4 * i] = s4.x; sv[4 * i + 1] = s4.y; sv[4 * i + 2] = s4.z; sv[4 * i + 3] = s4.w;
        }
        const uint8_t* zp = zeros + static_cast<int64_t>(row) * (G >> 1) + (t0 >> 1);
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            if constexpr (TPW == 4) zv[t] = *reinterpret_cast<const uint16_t*>(zp);
            else zv[t] = reinterpret_cast<const uint32_t*>(zp)[t / 8];
        }
    } else {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const int g = (t0 + t) >> gshift;
            sv[t] = scales[static_cast<int64_t>(row) * G + g];
            zv[t] = zeros[static_cast<int64_t>(row) * (G >> 1) + (g >> 1)];
        }
    }
    u32x4 w[TPW];
    const u32x4* wp = tile_lane_ptr<true>(packed, row0, rows, cols, lane) + t0 * kTStep<true>;
#pragma unroll
    for (int t = 0; t < TPW; ++t) w[t] = __builtin_nontemporal_load(wp + t * kTStep<true>);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before any use

    {   // x in the pair order (x0,x4)(x1,x5)(x2,x6)(x3,x7) of each 8, and T-block sums
        uint32_t sel_lo, sel_hi;
        asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
        asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
        const uint32_t ones = 0x3F803F80u;
#pragma unroll
        for (int u = 0; u < kQPL; ++u) {
            const u32x4 d = xr[u];
            u32x4 q;
            q.x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);
            q.y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);
            q.z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);
            q.w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);
            xsh[wave][lane + kWave * u] = q;
            float sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), 0.0f, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), sm, false);
            sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), sm, false);
            sm = row16_sum(sm);  // quad lane + 64 u lies in T-block 4 u + lane / 16
            if ((lane & 15) == 0) xsum[wave][4 * u + kb] = sm;
        }
    }
    // this wave's LDS writes before its own reads (no other wave reads them)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const NibConsts nk = nib_consts();
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const u32x4* xa = &xsh[wave][16 * t + 4 * kb];
        const u32x4 wv = w[t];
        const uint32_t w0 = wv.x, w1 = wv.y, w2 = wv.z, w3 = wv.w;
        f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[0]), a_operand(w0, nk),
                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[1]), a_operand(w1, nk), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[2]), a_operand(w2, nk), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[3]), a_operand(w3, nk), d, 0, 0, 0);
        const int g = (t0 + t) >> gshift;
        const uint32_t z = G128 ? (zv[t] >> (4 * (t % 8))) & 0xFu : ((g & 1) ? (zv[t] >> 4) : (zv[t] & 0xFu));
        const float c2 = -sv[t] * (136.0f + static_cast<float>(z));
        const float dx = d.x;
        acc = fmaf(sv[t], dx, fmaf(c2, xsum[wave][t], acc));
    }
    if (kb == 0) part[wave][n] = acc;
    __syncthreads();
    if (wave == 0 && lane < 16) {
        float tot = part[0][lane];
#pragma unroll
        for (int k = 1; k < KW; ++k) tot += part[k][lane];
        if (row0 + lane < rows) y[row0 + lane] = kc::f32_to_bf16(tot);
    }
}

template <int KW, int TPW>
int launch_gemv_shuf(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
                     const uint16_t* x, uint16_t* y, int rows, int cols, int gshift, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>((rows + 15) / 16);
    // 8 scales of a row at once: 16-byte aligned when the row's scales are
    // (G = K / 128 a multiple of 8) and the array is
    if (gshift == 0 && kc::aligned(scales, 16) && kc::aligned(zeros, 4))
        gemv_int4_shuf_kernel<KW, TPW, true><<<grid, KW * kWave, 0, stream>>>(packed, scales, zeros, x, y, rows,
                                                                          cols, gshift);
    else
        gemv_int4_shuf_kernel<KW, TPW, false><<<grid, KW * kWave, 0, stream>>>(packed, scales, zeros, x, y, rows,
                                                                           cols, gshift);
    return kc::check_launch(fn);
}

// Up to N = 8192 (and K = 8192) four T-blocks per wave, twice the waves:
// QKV 5.16 -> 4.93 us, O 4.14 -> 3.96 us; the same elsewhere.
constexpr int kGvSmallRows = 8192;

// -1 when the kernel does not apply (K not 128 TPW KW with KW <= 16).
int gemv_shuf(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
              const uint16_t* x, uint16_t* y, int rows, int cols, int gshift, hipStream_t stream) {
#define KC_GV(KWV, TPWV) \
    case KWV: return launch_gemv_shuf<KWV, TPWV>(fn, packed, scales, zeros, x, y, rows, cols, gshift, stream);
    if (rows <= kGvSmallRows && cols % 512 == 0 && cols / 512 <= 16) {
        switch (cols / 512) {
            KC_GV(1, 4) KC_GV(2, 4) KC_GV(3, 4) KC_GV(4, 4) KC_GV(5, 4) KC_GV(6, 4) KC_GV(7, 4) KC_GV(8, 4)
            KC_GV(9, 4) KC_GV(10, 4) KC_GV(11, 4) KC_GV(12, 4) KC_GV(13, 4) KC_GV(14, 4) KC_GV(15, 4) KC_GV(16, 4)
            default: break;
        }
    }
    if (cols % 1024 != 0) return -1;
    switch (cols / 1024) {
        KC_GV(1, 8) KC_GV(2, 8) KC_GV(3, 8) KC_GV(4, 8) KC_GV(5, 8) KC_GV(6, 8) KC_GV(7, 8) KC_GV(8, 8)
        KC_GV(9, 8) KC_GV(10, 8) KC_GV(11, 8) KC_GV(12, 8) KC_GV(13, 8) KC_GV(14, 8) KC_GV(15, 8) KC_GV(16, 8)
        default: return -1;
    }
#undef KC_GV
}

template <bool SHUF>
int gemm_int4(const char* fn, const uint8_t* d_packed, const float* d_scales,
              const uint8_t* d_zeros, const uint16_t* d_x, uint16_t* d_y, int m, int rows,
              int cols, int group_size, hipStream_t stream) {
    if (m < 0 || m > 64)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: m=%d must be in [0, 64]", fn, m);
    if (rows < 0 || cols < 0 || group_size <= 0 || cols % 2 != 0 || cols % group_size != 0)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                             "%s: invalid shape rows=%d cols=%d group_size=%d", fn, rows, cols,
                             group_size);
    if (m == 0 || rows == 0) return KC_SUCCESS;
    if (!d_y || (cols > 0 && (!d_packed || !d_scales || !d_zeros || !d_x)))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    const bool fast = cols > 0 && cols % kTBlock == 0 && group_size % kTBlock == 0 &&
                      kc::is_pow2(group_size) && kc::aligned(d_packed, 16) &&
                      kc::aligned(d_x, 16);
    if constexpr (SHUF) {
        // K = 0: Y = 0, as on the reference layout (the per-row GEMV below
        // writes zeros and reads no weights)
        if (cols == 0) {
            for (int i = 0; i < m; ++i) {
                const int st = kc_gemv_int4_bf16(d_packed, d_scales, d_zeros, d_x,
                                                 d_y + static_cast<int64_t>(i) * rows, rows, 0,
                                                 group_size, stream);
                if (st != KC_SUCCESS) return st;
            }
            return KC_SUCCESS;
        }
        // only the matrix-core kernels read the shuffled layout
        if (!fast)
            return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                                 "%s: the shuffled layout needs cols a multiple of 128, group_size a "
                                 "power of two >= 128, and 16-byte aligned weights and x (cols=%d "
                                 "group_size=%d)",
                                 fn, cols, group_size);
        if (m == 1) {
            const int st = gemv_shuf(fn, d_packed, d_scales, d_zeros, d_x, d_y, rows, cols,
                                     kc::ilog2(group_size) - 7, stream);
            if (st >= 0) return st;  // else the X-resident kernel below, at M = 1
        }
    } else if (!fast || m == 1) {
        // One GEMV per activation row: same results, no matrix cores (and for
        // a single row the GEMV streams the weights faster: K 8192, N 28672,
        // 20.4 us against 28.3 us for the X-resident kernel below).
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
    // M <= 8 on the reference layout: the K-split kernel below in its pair
    // form where that applies (K a multiple of 1024, up to 12288), else the
    // X-resident kernel when its LDS fits in some number of phases of K.  On
    // the shuffled layout the K-split kernel below from M = 2.  (K 8192,
    // N 28672, MI355X: M 2 / 4 / 8 in 25.3 / 25.1 / 25.3 us on the reference
    // layout against 30.3 / 30.6 / 32.0 for the X-resident kernel; 25.4 /
    // 25.4 / 25.2 on the shuffled layout against 27.5 / 27.3 / 28.2.)
    if (m <= kXresBestM && !SHUF) {
        const int st = launch_kslds<1, SHUF, true>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift,
                                                  stream);
        if (st >= 0) return st;
        const int P = xres_phases(m, cols, (cols / kTBlock) >> gshift);
        if (P > 0)
            return launch_xres<kXresW, kXresD, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols,
                                               gshift, P, stream);
    }
    // M 9..64: the K-split kernels, operands through LDS where they fit (on
    // the reference layout in pairs of T-blocks up to M 48 where K allows),
    // else through registers (K 8192, N 28672, MI355X, reference layout:
    // M 16 / 32 / 48 / 64 in 26 / 31 / 38 / 47 us through LDS, 37 / 48 / 58 /
    // 69 us through registers, 41 / 77 / 95 / 101 us for the kernels below,
    // which remain for shapes neither takes: K above about 20000, where the
    // coefficient stage does not fit in LDS, or operands of 4 GiB).
    if (m > kXresBestM || SHUF) {
        int st = -1;
        if constexpr (!SHUF) {
            switch ((m + 15) / 16) {
                case 1: st = launch_kslds<1, SHUF, true>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
                case 2: st = launch_kslds<2, SHUF, true>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
                case 3: st = launch_kslds<3, SHUF, true>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
                default: break;  // four activation tiles: one T-block at a time (faster there)
            }
            if (st >= 0) return st;
        }
        switch ((m + 15) / 16) {
            case 1: st = launch_kslds<1, SHUF, false>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
            case 2: st = launch_kslds<2, SHUF, false>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
            case 3: st = launch_kslds<3, SHUF, false>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
            default: st = launch_kslds<4, SHUF, false>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
        }
        if (st >= 0) return st;
        switch ((m + 15) / 16) {
            case 1: st = launch_kslice<1, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
            case 2: st = launch_kslice<2, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
            case 3: st = launch_kslice<3, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
            default: st = launch_kslice<4, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream); break;
        }
        if (st >= 0) return st;
    }
    if (m <= kXresMaxM) {
        const int P = xres_phases(m, cols, (cols / kTBlock) >> gshift);
        if (P > 0)
            return launch_xres<kXresW, kXresD, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols,
                                               gshift, P, stream);
    }
    // M 33..64: the four-tile X-resident kernel when its LDS fits (K 8192,
    // N 28672: M 33 / 48 / 64 in 86 / 90 / 94 us against 105 / 119 / 125 us
    // below; at M 17..32 the kernel below is faster, 65-77 us against 80-85)
    if (m > 32 && (cols / kTBlock) % 8 == 0) {
        const int st = launch_xbig<7, 1, 2, 8, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols,
                                               gshift, stream);
        if (st >= 0) return st;
    }
    // m-tiles of 16 activation rows; with more of them each B operand read
    // from LDS is reused across two weight row tiles.
    // (KW = 1: measured on MI355X at K 8192, N 28672, splitting K across the
    // waves of a workgroup was slower for every M.)
    switch ((m + 15) / 16) {
        case 1: return launch_mfma<1, 1, 1, 8, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream);
        case 2: return launch_mfma<2, 1, 1, 4, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream);
        case 3: return launch_mfma<3, 2, 1, 2, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream);
        default: return launch_mfma<4, 2, 1, 2, SHUF>(fn, d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols, gshift, stream);
    }
}

}  // namespace

extern "C" int kc_gemm_int4_bf16(const uint8_t* d_packed, const float* d_scales,
                                 const uint8_t* d_zeros, const uint16_t* d_x, uint16_t* d_y,
                                 int m, int rows, int cols, int group_size, kc_stream_t stream) {
    return gemm_int4<false>("kc_gemm_int4_bf16", d_packed, d_scales, d_zeros, d_x, d_y, m, rows, cols,
                            group_size, stream);
}

extern "C" int kc_gemm_int4_bf16_shuffled(const uint8_t* d_packed_shuffled, const float* d_scales,
                                          const uint8_t* d_zeros, const uint16_t* d_x, uint16_t* d_y,
                                          int m, int rows, int cols, int group_size, kc_stream_t stream) {
    return gemm_int4<true>("kc_gemm_int4_bf16_shuffled", d_packed_shuffled, d_scales, d_zeros, d_x, d_y,
                           m, rows, cols, group_size, stream);
}
