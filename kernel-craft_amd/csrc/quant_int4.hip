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
// LDS (gemv_int4_fast_kernel), or once per lane for the one chunk it owns
// (gemv_int4_xl_kernel, K = 2048 x 2..8: no LDS staging).  With bf16 x each nibble becomes the exact bf16 (128 + n') by one
// bitwise op, ((d ^ 0x00080008) & 0x000F000F) | 0x43004300 (v_bitop3_b32), and
// pairs of them meet pairs of x in v_dot2_f32_bf16 (exact products, fp32
// accumulation); the extra 128 * sum x is removed with the zero point.  With
// fp32 x (the reference ABI) each nibble goes through v_cvt_f32_ubyteN and an
// fp32 FMA, so every product is exact before its single rounding.
#include <algorithm>
#include <cstdlib>

#include "int4_decode.hpp"
#include "kc_common.hpp"

namespace {

using kc::kWave;
using namespace kc::int4;


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

// 1 / sqrt(sum h^2 / K + eps) of a bf16 vector, summed by one wave (the
// RMSNorm in front of a fused GEMV; the arithmetic of rmsnorm.hip).
__device__ __forceinline__ float rms_inverse(const uint16_t* h, int64_t K, float eps, int lane) {
    float ss = 0.0f;
    for (int64_t k = lane; k < K; k += kWave) {
        const float v = kc::bf16_to_f32(h[k]);
        ss = fmaf(v, v, ss);
    }
    ss = kc::wave_sum(ss);
    return 1.0f / sqrtf(ss / static_cast<float>(K) + eps);
}

// ---------------------------------------------------------------------------
// Generic GEMV: any even K and any group size dividing K.  One wave per row,
// lanes stride over bytes with the reference's own index arithmetic
// (quant_int4.cu:143-164), dequantizing each weight to fp32 as the reference
// does before the FMA.
// ---------------------------------------------------------------------------
template <bool XBF16, bool YBF16, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_int4_generic_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const void* __restrict__ x, void* __restrict__ y,
    int64_t rows, int64_t cols, int64_t gs, const uint16_t* __restrict__ gamma, float eps) {
    static_assert(!NORM || XBF16, "the fused RMSNorm takes bf16 x");
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t nbytes = cols >> 1;
    const int64_t G = cols / gs;
    const uint8_t* prow = packed + row * nbytes;
    float rms_inv = 1.0f;
    if constexpr (NORM) rms_inv = rms_inverse(static_cast<const uint16_t*>(x), cols, eps, lane);
    // x[k] as the GEMV sees it: bf16(gamma[k] * h[k]) when fused (the row
    // sum is scaled by rms_inv at the end)
    auto xin = [&](int64_t k) {
        if constexpr (NORM)
            return kc::bf16_to_f32(kc::f32_to_bf16(kc::bf16_to_f32(gamma[k]) * load_x<true>(x, k)));
        else
            return load_x<XBF16>(x, k);
    };
    float acc = 0.0f;
    for (int64_t b = lane; b < nbytes; b += kWave) {
        const int64_t c0 = 2 * b;
        const uint32_t p = prow[b];
        const int64_t g0 = c0 / gs, g1 = (c0 + 1) / gs;
        const float w0 =
            static_cast<float>(sext4(p) - zero_nibble(zeros, row, G, g0)) * scales[row * G + g0];
        const float w1 =
            static_cast<float>(sext4(p >> 4) - zero_nibble(zeros, row, G, g1)) * scales[row * G + g1];
        acc = fmaf(w0, xin(c0), acc);
        acc = fmaf(w1, xin(c0 + 1), acc);
    }
    acc = kc::wave_sum(acc) * rms_inv;
    if (lane == 0) store_y<YBF16>(y, row, acc);
}

// ---------------------------------------------------------------------------
// Fast GEMV.
//
// A row is split into chunks of 32 k (16 bytes of packed weights); lane l of
// a wave owns chunks j*64 + l (j < CPL) of every row it computes, so each
// wave-wide load reads 1 KB of one row.  A workgroup of WPB waves computes
// R*WPB consecutive rows, R per wave, and shares one copy of x in LDS:
//
//   1. every thread issues its x loads first, then the scale/zero loads of
//      its wave's rows, then all R*CPL weight loads (vector loads return in
//      order, so x arrives first and the weights are all in flight at once);
//   2. the workgroup writes x to LDS in the order the nibble decode needs
//      (bf16: k-block quads rearranged to the pairs (x0,x4)(x1,x5)(x2,x6)
//      (x3,x7) with v_perm_b32; fp32: as is) together with each chunk's
//      fp32 sum of x;
//   3. after one barrier each wave reads its chunks of x from LDS as it
//      reaches them, decodes and multiplies, and reduces its R rows across
//      the wave with permlane swaps and DPP row rotations.
//
// Per workgroup the x staging is done once instead of once per wave, and no
// wave holds more than one chunk of x in registers.
// ---------------------------------------------------------------------------
// The fold of one chunk's dot product into the row sum:
//     acc += c1 * dot + c2 * sum(x),   c1 = s,  c2 = -s * (off + z)
// off = 136 for the bf16 encoding 128 + (q ^ 8), 8 for fp32.
template <int R, int CPL, int SLOT, int WPB, bool XBF16, bool YBF16, bool NORM>
__global__ __launch_bounds__(WPB * kWave) void gemv_int4_fast_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const void* __restrict__ x, void* __restrict__ y,
    int rows, int cols, int gshift, const uint16_t* __restrict__ gamma, float eps) {
    static_assert(!NORM || XBF16, "the fused RMSNorm takes bf16 x");
    using SM = SlotMap<SLOT>;
    constexpr int kSlots = R * CPL;
    constexpr int kRegs = (kSlots + SM::kPerReg - 1) / SM::kPerReg;
    constexpr int kQuadsPerChunk = XBF16 ? 4 : 8;
    constexpr int kThreadsWG = WPB * kWave;
    constexpr int kMaxQuads = CPL * 64 * kQuadsPerChunk;
    constexpr int kQPT = (kMaxQuads + kThreadsWG - 1) / kThreadsWG;  // x quads per thread
    extern __shared__ u32x4 xl[];                                    // x quads, then chunk sums

    __builtin_amdgcn_s_setprio(kIssuePrio);  // until the loads are out
    const int lane = threadIdx.x & (kWave - 1);
    // wave-uniform: row bases and K offsets stay in SGPRs, so the loads
    // address with a scalar base and one shared lane offset
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int cpr = cols >> 5;                      // chunks per row
    const int nquads = cpr * kQuadsPerChunk;
    float* xsum = reinterpret_cast<float*>(xl + nquads);
    const int row0 = (blockIdx.x * WPB + wave) * R;
    const int64_t rbytes = cols >> 1;
    const int G = cols >> (5 + gshift);             // groups per row
    const int ng = gshift >= 6 ? 1 : (64 >> gshift);  // groups per chunk slot

    // 1a. x, raw
    u32x4 xr[kQPT];
    u32x4 gr[NORM ? kQPT : 1];
    {
        const u32x4* src = static_cast<const u32x4*>(x);
#pragma unroll
        for (int u = 0; u < kQPT; ++u)
            xr[u] = src[min(static_cast<int>(threadIdx.x) + u * kThreadsWG, nquads - 1)];
        if constexpr (NORM) {
            const u32x4* gsrc = reinterpret_cast<const u32x4*>(gamma);
#pragma unroll
            for (int u = 0; u < kQPT; ++u)
                gr[u] = gsrc[min(static_cast<int>(threadIdx.x) + u * kThreadsWG, nquads - 1)];
        }
    }
    // 1b. scale and zero byte of every item this lane holds
    float s_it[kRegs];
    uint32_t z_it[kRegs];
#pragma unroll
    for (int q = 0; q < kRegs; ++q) {
        const int s = min(q * SM::kPerReg + lane / SLOT, kSlots - 1);
        const int gi = min(lane % SLOT, ng - 1);
        const int r = s / CPL, j = s % CPL;
        const int g = min(((j * 64) >> gshift) + gi, G - 1);
        const int64_t rr = min(row0 + r, rows - 1);
        s_it[q] = scales[rr * G + g];
        z_it[q] = zeros[rr * (G >> 1) + (g >> 1)];
    }
    // 1c. weights (chunks past the end of a row read chunk 0 and are masked)
    u32x4 w[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t rr = min(row0 + r, rows - 1);
        const u32x4* prow = reinterpret_cast<const u32x4*>(packed + rr * rbytes);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = j * 64 + lane;
            w[r][j] = __builtin_nontemporal_load(prow + (c < cpr ? c : 0));
        }
    }
    // keep every load above this point: the compiler otherwise sinks weight
    // loads towards their uses, leaving one row in flight at a time
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);

    // 1d. fused RMSNorm: x = bf16(gamma h) is staged in place of h, and each
    // wave's sum of h^2 (every quad once: the clamped duplicates past the
    // end are skipped) goes to LDS; after the staging barrier every wave adds
    // the partial sums in a fixed order and scales its row sums by
    // rms_inv = 1 / sqrt(sum h^2 / K + eps).  No barrier of its own.
    [[maybe_unused]] float* part = xsum + cpr;  // WPB partial sums after the chunk sums
    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < kQPT; ++u) {
            const bool valid = static_cast<int>(threadIdx.x) + u * kThreadsWG < nquads;
            const uint32_t w4[4] = {xr[u].x, xr[u].y, xr[u].z, xr[u].w};
            const uint32_t g4[4] = {gr[u].x, gr[u].y, gr[u].z, gr[u].w};
            uint32_t o4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = __uint_as_float(w4[j] << 16), hi = __uint_as_float(w4[j] & 0xFFFF0000u);
                if (valid)  // lo^2 + hi^2 + ss, exact products
                    ss = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w4[j]), as_bf16x2(w4[j]), ss, false);
                o4[j] = kc::pack_bf16x2(__uint_as_float(g4[j] << 16) * lo,
                                        __uint_as_float(g4[j] & 0xFFFF0000u) * hi);
            }
            xr[u] = u32x4{o4[0], o4[1], o4[2], o4[3]};
        }
        ss = kc::wave_sum(ss);
        if (lane == 0) part[wave] = ss;
    }

    // 2. stage x in LDS
    {
        const uint32_t ones = 0x3F803F80u;
        uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs (see nib_consts)
        asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
        asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
#pragma unroll
        for (int u = 0; u < kQPT; ++u) {
            const int i = threadIdx.x + u * kThreadsWG;
            const u32x4 d = xr[u];
            const uint32_t d0 = d.x, d1 = d.y, d2 = d.z, d3 = d.w;
            u32x4 p;
            float sm;
            if constexpr (XBF16) {
                p.x = __builtin_amdgcn_perm(d2, d0, sel_lo);   // (x0, x4)
                p.y = __builtin_amdgcn_perm(d2, d0, sel_hi);   // (x1, x5)
                p.z = __builtin_amdgcn_perm(d3, d1, sel_lo);   // (x2, x6)
                p.w = __builtin_amdgcn_perm(d3, d1, sel_hi);   // (x3, x7)
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d0), as_bf16x2(ones), 0.0f, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d1), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d2), as_bf16x2(ones), sm, false);
                sm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d3), as_bf16x2(ones), sm, false);
                sm += __shfl_xor(sm, 1, kWave);  // 4 consecutive quads form a chunk
                sm += __shfl_xor(sm, 2, kWave);
            } else {
                p = d;
                sm = (__uint_as_float(d0) + __uint_as_float(d1)) +
                     (__uint_as_float(d2) + __uint_as_float(d3));
                sm += __shfl_xor(sm, 1, kWave);  // 8 consecutive quads form a chunk
                sm += __shfl_xor(sm, 2, kWave);
                sm += __shfl_xor(sm, 4, kWave);
            }
            if (i < nquads) {
                xl[i] = p;
                if (i % kQuadsPerChunk == 0) xsum[i / kQuadsPerChunk] = sm;
            }
        }
    }
    __syncthreads();

    // 3. decode, multiply, fold, reduce
    float c1[kRegs], c2[kRegs];
#pragma unroll
    for (int q = 0; q < kRegs; ++q) {
        const int s = min(q * SM::kPerReg + lane / SLOT, kSlots - 1);
        const int gi = min(lane % SLOT, ng - 1);
        const int j = s % CPL;
        const int g = min(((j * 64) >> gshift) + gi, G - 1);
        const uint32_t z = (g & 1) ? (z_it[q] >> 4) : (z_it[q] & 0xFu);
        c1[q] = s_it[q];
        c2[q] = -s_it[q] * static_cast<float>((XBF16 ? 136u : 8u) + z);
    }
    const NibConsts nk = nib_consts();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = j * 64 + lane;
        const bool act = c < cpr;
        const int cc = act ? c : 0;
        const u32x4* xc = xl + cc * kQuadsPerChunk;
        const float xs = xsum[cc];
        // this lane's group within the slot
        const int gi = ((j * 64 + lane) >> gshift) - ((j * 64) >> gshift);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int s = r * CPL + j;
            const int src = (SM::base_lane(s) + gi) << 2;
            float m1 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, c1[SM::reg(s)])));
            float m2 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, c2[SM::reg(s)])));
            m1 = act ? m1 : 0.0f;
            m2 = act ? m2 : 0.0f;
            acc[r] = fmaf(m1, chunk_dot<XBF16>(w[r][j], xc, nk), fmaf(m2, xs, acc[r]));
        }
    }
    float t = wave_reduce_rows<R>(acc);
    if constexpr (NORM) {
        float tot = part[0];
#pragma unroll
        for (int w = 1; w < WPB; ++w) tot += part[w];
        t *= 1.0f / sqrtf(tot / static_cast<float>(cols) + eps);
    }
    constexpr int kGroup = kWave / R;
    const int r = lane / kGroup;
    if ((lane & (kGroup - 1)) == 0 && row0 + r < rows) store_y<YBF16>(y, row0 + r, t);
}


// ---------------------------------------------------------------------------
// GEMV with K split across waves and x in registers per lane (K a multiple of
// 2048; bf16 x and y, or fp32 x and y below N = 8192).
//
// A workgroup of KW x RGW waves computes RGW groups of R rows; wave (kw, rg)
// takes chunk c = 64 kw + lane (32 k) of each of its R rows.  A lane holds
// its own chunk of x (64 bytes), permutes it into the decode's pair order and
// sums it once, and reuses both for all R rows.  With one row group per
// workgroup the lane loads its chunk itself and no barrier stands between a
// wave's loads and its arithmetic; with RGW > 1 the workgroup copies x into
// LDS once (direct-to-LDS loads issued before the weights) and its waves read
// their chunks after one barrier that waits for the copies only, the weights
// staying in flight.  Each wave reduces its R row sums across its lanes; the
// KW partial sums of a row meet in LDS after the last barrier.  Measured against the
// LDS-staged kernel (K 14336 down projection: 8.8 -> 8.0 us; K 4096 with
// N <= 6144 a few per cent; K 16384 / 8192 with N 4096: 9.8 -> 8.6, 5.6 ->
// 5.4 us); the gate/up shape (K 4096, N 28672) keeps the staged kernel.
// With NORM, x = bf16(gamma h) and each wave adds its lanes' sums of h^2 to
// the partials, so the row sums are scaled by rms_inv at the end.  With fp32
// x a lane loads its chunk's 32 values (128 bytes) in their own order and
// folds with offset 8, as the staged kernel's fp32 decode does.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

// One global_load_lds_dwordx4: 16 bytes per lane from g into LDS at
// lds_base + 16 lane.  Inline assembly, so that the compiler's LDS-wait
// bookkeeping does not see it; the kernel waits for these loads itself.
__device__ __forceinline__ void x_dma16(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(n) for n in [0, 7] (a constant once the caller's loop is
// unrolled).  The wait reads and writes `after` (a value the caller computes
// just before, e.g. the previous row's sum), so it is not hoisted above that
// work; an empty asm then reads and writes v, so v counts as produced after
// the wait and nothing reads its register before it.
__device__ __forceinline__ void wait_vmcnt_tied(int n, u32x4& v, float& after) {
    switch (n) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" : "+v"(after)::"memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(1)" : "+v"(after)::"memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(2)" : "+v"(after)::"memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(3)" : "+v"(after)::"memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(4)" : "+v"(after)::"memory"); break;
        case 5: asm volatile("s_waitcnt vmcnt(5)" : "+v"(after)::"memory"); break;
        case 6: asm volatile("s_waitcnt vmcnt(6)" : "+v"(after)::"memory"); break;
        default: asm volatile("s_waitcnt vmcnt(7)" : "+v"(after)::"memory"); break;
    }
    asm volatile("" : "+v"(v));
}

template <int R, int KW, int RGW, bool NORM, bool BF16 = true>
__global__ __launch_bounds__(KW * RGW * kWave) void gemv_int4_xl_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const void* __restrict__ x, void* __restrict__ y,
    int rows, int cols, int gshift, const uint16_t* __restrict__ gamma, float eps) {
    static_assert(R % 4 == 0, "rows are reduced across the wave four at a time");
    static_assert(R <= 8, "weight-load waits count up to 7 younger loads");
    static_assert(BF16 || !NORM, "the fused RMSNorm takes bf16 x");
    constexpr int kXQ = BF16 ? 4 : 8;  // 16-byte quads of x per 32-k chunk
    __shared__ float part[RGW][KW][R + 1];  // row sums, then the sum of h^2
    __builtin_amdgcn_s_setprio(kIssuePrio);  // until the loads are out
    const int lane = threadIdx.x & (kWave - 1);
    // wave-uniform: row bases and K offsets stay in SGPRs, so the loads
    // address with a scalar base and one shared lane offset
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int kw = wave % KW, rg = wave / KW;
    const int row0 = (blockIdx.x * RGW + rg) * R;
    const int c = kw * kWave + lane;  // cols == KW * 2048: every lane has a chunk
    const int G = cols >> (5 + gshift);
    const int g = c >> gshift;
    const int64_t rbytes = cols >> 1;

    // loads: x (and gamma), then scales and zero bytes, then weights.  With
    // more than one row group per workgroup, x is copied into LDS once per
    // workgroup (global_load_lds, no registers) instead of once per wave:
    // LDS slot (t, l), t = kw' kXQ + j, holds quad j of chunk 64 kw' + l, so
    // that a wave's reads of quad j are 64 consecutive slots.
    constexpr bool kShare = !NORM && RGW > 1;
    static_assert(!kShare || (KW * kXQ) % (KW * RGW) == 0, "x copies split evenly over the waves");
    __shared__ u32x4 xsh[kShare ? KW * kXQ * kWave : 1];
    u32x4 xq[kXQ], gq[NORM ? 4 : 1];
    const u32x4* xs = static_cast<const u32x4*>(x) + c * kXQ;
    if constexpr (!kShare) {
#pragma unroll
        for (int q = 0; q < kXQ; ++q) xq[q] = xs[q];
    }
    if constexpr (NORM) {
        const u32x4* gsrc = reinterpret_cast<const u32x4*>(gamma) + c * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) gq[q] = gsrc[q];
    }
    float sv[R];
    uint32_t zb[R];
    u32x4 w[R];
    if constexpr (kShare) {
        // x is copied into LDS with direct-to-LDS loads, then come the R
        // scale, R zero-byte and R weight loads of this wave's rows; all are
        // written out as instructions here, so that exactly 3R vector loads
        // are issued after the last copy.  Vector loads complete in order:
        // once no more than 3R are outstanding, every copy has landed,
        // whatever the compiler emits elsewhere (a load it added in between
        // would only make the wait stricter).  The barrier then publishes
        // every wave's part while the rest stays in flight; the values these
        // loads produce are tied to explicit waits before their first use.
        const uint32_t base = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_void_t*)xsh));
#pragma unroll
        for (int t0 = 0; t0 < KW * kXQ; t0 += KW * RGW) {
            const int t = t0 + wave;
            const int kwp = t / kXQ, j = t - kwp * kXQ;
            x_dma16(static_cast<const u32x4*>(x) + (kwp * kWave + lane) * kXQ + j,
                    __builtin_amdgcn_readfirstlane(base + t * kWave * 16));
        }
        const uint32_t soff = static_cast<uint32_t>(g) * 4u, zoff = static_cast<uint32_t>(g >> 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t rr = min(row0 + r, rows - 1);
            const float* srow = scales + rr * G;
            const uint8_t* zrow = zeros + rr * (G >> 1);
            asm volatile("global_load_dword %0, %1, %2" : "=v"(sv[r]) : "v"(soff), "s"(srow)
                         : "memory");
            asm volatile("global_load_ubyte %0, %1, %2" : "=v"(zb[r]) : "v"(zoff), "s"(zrow)
                         : "memory");
        }
        const uint32_t voff = static_cast<uint32_t>(c) * 16u;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t rr = min(row0 + r, rows - 1);
            const uint8_t* prow = packed + rr * rbytes;
            asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(w[r]) : "v"(voff), "s"(prow)
                         : "memory");
        }
        __builtin_amdgcn_s_setprio(0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * R) : "memory");
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int q = 0; q < kXQ; ++q) xq[q] = xsh[(kw * kXQ + q) * kWave + lane];
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t rr = min(row0 + r, rows - 1);
            sv[r] = scales[rr * G + g];
            zb[r] = zeros[rr * (G >> 1) + (g >> 1)];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t rr = min(row0 + r, rows - 1);
            w[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(packed + rr * rbytes) + c);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load above issued before any use
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
    }

    uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs
    asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
    asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
    const uint32_t ones = 0x3F803F80u;
    float hss = 0.0f;  // this lane's sum of h^2 (NORM)
    u32x4 xp[4];
    float xsm = 0.0f;
#pragma unroll
    for (int q = 0; q < (BF16 ? 4 : 0); ++q) {
        u32x4 d = xq[q];
        if constexpr (NORM) {
            const uint32_t h4[4] = {d.x, d.y, d.z, d.w};
            const uint32_t g4[4] = {gq[q].x, gq[q].y, gq[q].z, gq[q].w};
            uint32_t o4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hss = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(h4[j]), as_bf16x2(h4[j]), hss, false);
                o4[j] = kc::pack_bf16x2(__uint_as_float(g4[j] << 16) * __uint_as_float(h4[j] << 16),
                                        __uint_as_float(g4[j] & 0xFFFF0000u) * __uint_as_float(h4[j] & 0xFFFF0000u));
            }
            d = u32x4{o4[0], o4[1], o4[2], o4[3]};
        }
        xp[q].x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);  // (x0, x4)
        xp[q].y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);  // (x1, x5)
        xp[q].z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);  // (x2, x6)
        xp[q].w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);  // (x3, x7)
        xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), xsm, false);
        xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), xsm, false);
        xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), xsm, false);
        xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), xsm, false);
    }
    if constexpr (!BF16) {  // fp32 x: raw order, offset 8 (dot8_f32)
#pragma unroll
        for (int q = 0; q < kXQ; ++q)
            xsm += (__uint_as_float(xq[q].x) + __uint_as_float(xq[q].y)) +
                   (__uint_as_float(xq[q].z) + __uint_as_float(xq[q].w));
    }
    const NibConsts nk = nib_consts();
    constexpr float kOff = BF16 ? 136.0f : 8.0f;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // weights loaded by explicit instructions are not tracked by the
        // compiler's waits: wait until row r's load has landed (at most
        // R - 1 - r younger loads outstanding) and tie w[r] to that wait, so
        // that no use of it can be placed before
        if constexpr (kShare) {
            wait_vmcnt_tied(R - 1 - r, w[r], r == 0 ? xsm : acc[r > 0 ? r - 1 : 0]);
            if (r == 0) {  // every scale and zero byte is older than the first weight load
#pragma unroll
                for (int q = 0; q < R; ++q) asm volatile("" : "+v"(sv[q]), "+v"(zb[q]));
            }
        }
        const uint32_t z = (g & 1) ? (zb[r] >> 4) : (zb[r] & 0xFu);
        const float dot = BF16 ? chunk_dot<true>(w[r], xp, nk) : chunk_dot<false>(w[r], xq, nk);
        acc[r] = fmaf(sv[r], dot, -sv[r] * (kOff + static_cast<float>(z)) * xsm);
    }
#pragma unroll
    for (int r4 = 0; r4 < R; r4 += 4) {
        const float v4[4] = {acc[r4], acc[r4 + 1], acc[r4 + 2], acc[r4 + 3]};
        const float t = wave_reduce_rows<4>(v4);  // lane 16 j holds row r4 + j
        if ((lane & 15) == 0) part[rg][kw][r4 + (lane >> 4)] = t;
    }
    if constexpr (NORM) {
        hss = kc::wave_sum(hss);
        if (lane == 0) part[rg][kw][R] = hss;
    }
    __syncthreads();
    if (kw == 0 && lane < R) {
        float t = part[rg][0][lane];
#pragma unroll
        for (int k = 1; k < KW; ++k) t += part[rg][k][lane];
        if constexpr (NORM) {
            float ss = part[rg][0][R];
#pragma unroll
            for (int k = 1; k < KW; ++k) ss += part[rg][k][R];
            t *= 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
        }
        if (row0 + lane < rows) store_y<BF16>(y, row0 + lane, t);
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

// The staged kernel's LDS ceiling: all of a CU's 160 KB.  Beyond the 64 KB a
// launch gets by default (fp32 x at K > 15872) the kernel is opted in once.
constexpr int kDefaultLds = 64 * 1024;
constexpr int kMaxFastLds = 160 * 1024;

int device_max_lds() {
    static const int v = [] {
        int dev = 0, lds = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            lds <= 0)
            lds = kDefaultLds;
        return std::min(lds, kMaxFastLds);
    }();
    return v;
}

// Launch arguments shared by every GEMV variant; gamma and eps are used by
// the fused RMSNorm only.
struct GemvArgs {
    const uint8_t* packed;
    const float* scales;
    const uint8_t* zeros;
    const void* x;
    void* y;
    const uint16_t* gamma;
    float eps;
};

// False (nothing launched) when the kernel cannot be given the LDS it needs.
template <int R, int CPL, int SLOT, int WPB, bool XB, bool YB, bool NORM>
bool launch_fast(const GemvArgs& a, int rows, int cols, int gshift, size_t lds, hipStream_t stream) {
    const auto kernel = gemv_int4_fast_kernel<R, CPL, SLOT, WPB, XB, YB, NORM>;
    if (lds > static_cast<size_t>(kDefaultLds)) {
        static const bool opted_in = [&] {
            const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                                kMaxFastLds) == hipSuccess;
            if (!ok) (void)hipGetLastError();  // the caller takes another kernel
            return ok;
        }();
        if (!opted_in) return false;
    }
    const int wave_blocks = (rows + R - 1) / R;
    const unsigned grid = static_cast<unsigned>((wave_blocks + WPB - 1) / WPB);
    kernel<<<grid, WPB * kWave, lds, stream>>>(a.packed, a.scales, a.zeros, a.x, a.y, rows, cols,
                                               gshift, a.gamma, a.eps);
    return true;
}

// Rows per wave and waves per workgroup: 2 rows and 4 waves up to K = 16384
// (at most 8 weight chunks per row and lane), 1 row and 8 waves beyond; 4 rows
// when each lane holds 2 or 4 whole chunks per row and N is large enough
// (K = 4096 from N = 4096, K = 8192 from N = 8192) -- measured 4-26 % faster
// there (gate/up 13.0 -> 11.8 us), and 2-20 % slower at N <= 1024 or with a
// part-filled chunk (K = 5120, 14336).
template <int CPL, bool XB, bool YB, bool NORM>
bool launch_fast_cpl(int slot, const GemvArgs& a, int rows, int cols, int gshift, size_t lds,
                     hipStream_t stream) {
    constexpr int R = CPL <= 8 ? 2 : 1;
    constexpr int WPB = CPL <= 8 ? 4 : 8;
    if constexpr (CPL == 2 || CPL == 4) {
        const bool four = cols == CPL * 2048 && rows >= CPL * 2048;
        if (four && slot == 16) return launch_fast<4, CPL, 16, 4, XB, YB, NORM>(a, rows, cols, gshift, lds, stream);
        if (four) return launch_fast<4, CPL, 64, 4, XB, YB, NORM>(a, rows, cols, gshift, lds, stream);
    }
    if (slot == 16) return launch_fast<R, CPL, 16, WPB, XB, YB, NORM>(a, rows, cols, gshift, lds, stream);
    return launch_fast<R, CPL, 64, WPB, XB, YB, NORM>(a, rows, cols, gshift, lds, stream);
}

// The per-lane-x kernel for GEMVs whose K is 2048 x KW (KW 2..8):
// R = 4 rows per wave (8 for KW >= 3 with at least 24 MiB of packed
// weights), two row groups per workgroup at KW = 2; at KW = 2 only up to
// N = 16384 (the staged kernel is as fast or faster on the larger K = 4096
// shapes).  False when it does not apply.
template <bool NORM, bool BF16>
bool launch_xl(const GemvArgs& a, int64_t rows, int64_t cols, int gshift, hipStream_t stream) {
    if (cols % 2048 != 0 || rows > INT32_MAX) return false;
    const int kw = static_cast<int>(cols / 2048);
    if (kw < 2 || kw > 8 || (kw == 2 && rows > 16384)) return false;
    // fp32 x: 3-18 % faster than the staged kernel up to N = 6144 (cfg0 5.27
    // -> 5.12 us, K 14336 14.8 -> 12.9, K 16384 16.7 -> 13.8), slower from
    // N = 14336 (the staged kernel's 4 rows per wave)
    if (!BF16 && rows >= 8192) return false;
    const int r = static_cast<int>(rows), c = static_cast<int>(cols);
    // Eight rows per wave halve the waves and the x loads per weight byte:
    // faster from about 24 MiB of weights (N 4096: K 14336 7.60 -> 7.45 us,
    // K 16384 8.21 -> 7.99; N 8192 K 8192 8.23 -> 8.00), even at 14-16 MiB,
    // slower below (N 4096 K 6144 4.39 -> 4.60).  Same outputs either way.
    const bool wide = kw >= 3 && static_cast<int64_t>(rows) * (cols / 2) >= (int64_t{24} << 20);
#define KC_XL(KWV, RV, RGWV)                                                                     \
    gemv_int4_xl_kernel<RV, KWV, RGWV, NORM, BF16><<<static_cast<unsigned>((r + RV * RGWV - 1) / (RV * RGWV)), \
                                               KWV * RGWV * kWave, 0, stream>>>(                 \
        a.packed, a.scales, a.zeros, a.x, a.y, r, c, gshift, a.gamma, a.eps)
#define KC_XL_CASE(KWV)                  \
    case KWV:                            \
        if (wide) KC_XL(KWV, 8, 1);      \
        else KC_XL(KWV, 4, 1);           \
        break;
    // K = 4096: two row groups per workgroup sharing x (bf16: QKV 4.49 ->
    // 4.38 us, O 3.95 -> 3.92 against x per wave), four with fp32 x, whose
    // per-wave copies were a third of the kernel (cfg0 4.88 -> 4.01 us).
    // Sharing x between the two row groups of K = 14336 (down) was slower
    // (7.9 -> 10.0 us), so K above 4096 keeps one row group per workgroup.
    switch (kw) {
        case 2:
            if (BF16) KC_XL(2, 4, 2);
            else KC_XL(2, 4, 4);
            break;
        KC_XL_CASE(3) KC_XL_CASE(4) KC_XL_CASE(5) KC_XL_CASE(6) KC_XL_CASE(7) KC_XL_CASE(8)
        default: return false;
    }
#undef KC_XL_CASE
#undef KC_XL
    return true;
}

template <bool XB, bool YB, bool NORM = false>
int gemv_int4(const char* fn, const uint8_t* packed, const float* scales, const uint8_t* zeros,
              const void* x, void* y, int64_t rows, int64_t cols, int64_t gs,
              hipStream_t stream, const uint16_t* gamma = nullptr, float eps = 0.0f) {
    int st = check_int4_args(fn, packed, scales, zeros, x, y, rows, cols, gs);
    if (st != KC_SUCCESS) return st;
    if (NORM && rows > 0 && cols > 0 && !gamma)
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: null device pointer", fn);
    if (rows == 0) return KC_SUCCESS;
    const int64_t cpr = cols >> 5;
    const int64_t cpl = (cpr + 63) / 64;
    // x and its chunk sums in LDS (and the waves' partial sums of squares)
    const size_t lds = static_cast<size_t>(cpr) * (XB ? 64 : 128) + static_cast<size_t>(cpr) * 4 +
                       (NORM ? 8 * sizeof(float) : 0);
    const bool fast = cols > 0 && gs >= 32 && kc::is_pow2(gs) && cpl <= 16 &&
                      rows <= INT32_MAX && kc::aligned(packed, 16) && kc::aligned(x, 16) &&
                      (!NORM || kc::aligned(gamma, 16)) &&
                      lds <= static_cast<size_t>(device_max_lds());
    const GemvArgs a{packed, scales, zeros, x, y, gamma, eps};
    if constexpr (XB == YB) {
        if (fast && launch_xl<NORM, XB>(a, rows, cols, kc::ilog2(gs) - 5, stream)) return kc::check_launch(fn);
    }
    bool launched = false;
    if (fast) {
        const int gshift = kc::ilog2(gs) - 5;
        const int slot = gshift >= 2 ? 16 : 64;
        const int r = static_cast<int>(rows), c = static_cast<int>(cols);
#define KC_FAST_CASE(N)                                                                   \
    case N:                                                                               \
        launched = launch_fast_cpl<N, XB, YB, NORM>(slot, a, r, c, gshift, lds, stream);  \
        break;
        switch (cpl) {
            KC_FAST_CASE(1) KC_FAST_CASE(2) KC_FAST_CASE(3) KC_FAST_CASE(4)
            KC_FAST_CASE(5) KC_FAST_CASE(6) KC_FAST_CASE(7) KC_FAST_CASE(8)
            KC_FAST_CASE(9) KC_FAST_CASE(10) KC_FAST_CASE(11) KC_FAST_CASE(12)
            KC_FAST_CASE(13) KC_FAST_CASE(14) KC_FAST_CASE(15) KC_FAST_CASE(16)
            default: break;
        }
#undef KC_FAST_CASE
    }
    if (!launched) {
        const int64_t grid = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
        if (grid > INT32_MAX)
            return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: rows=%lld too large", fn,
                                 (long long)rows);
        gemv_int4_generic_kernel<XB, YB, NORM><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(
            packed, scales, zeros, x, y, rows, cols, gs, gamma, eps);
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

// y = rms_inv * (W bf16(gamma h)): the RMSNorm in front of a decoder GEMV
// (rmsnorm.cu:40-70 followed by quant_int4.cu:126-175), folded into the
// GEMV.  Every workgroup sums the squares of h itself (K bf16 values from
// the cache) while it stages bf16(gamma h) as x, and scales its row sums by
// rms_inv at the end, so the normalized vector is never written and the
// staging needs no barrier of its own.
extern "C" int kc_rmsnorm_gemv_int4_bf16(const uint16_t* d_h, const uint16_t* d_gamma, float eps,
                                         const uint8_t* d_packed, const float* d_scales,
                                         const uint8_t* d_zeros, uint16_t* d_y, int rows, int cols,
                                         int group_size, kc_stream_t stream) {
    return gemv_int4<true, true, true>("kc_rmsnorm_gemv_int4_bf16", d_packed, d_scales, d_zeros, d_h,
                                       d_y, rows, cols, group_size, stream, d_gamma, eps);
}
