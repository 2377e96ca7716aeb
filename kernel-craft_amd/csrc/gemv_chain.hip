// gemv_chain.hip -- a decode step's INT4 GEMVs from one call.
//
// kc_gemv_int4_bf16_chain computes a list of bf16 INT4 GEMVs in order, so
// that an op may read what earlier ops wrote (its x may be an earlier op's
// y), and a caller crosses the FFI boundary once per decode step instead of
// once per projection (the reference's decode loop calls launch_gemv_int4
// once per projection, quant_int4.cu:221-234).
//
// The list is cut into runs at dependencies: a run is a maximal sequence of
// consecutive ops none of which depends on another op of the run (reads its
// y, or writes what it reads or writes).  A run of two or more ops whose
// shapes the fused tile takes is ONE launch (gemv_run_kernel): the grid holds
// every op's tiles in op order, so the weight stream runs across the ops
// without the drain and ramp of a launch boundary between them.  Other runs
// launch kc_gemv_int4_bf16 per op.  Runs follow each other on the stream.
//
// Dependent ops are not fused into one launch with a wait inside it: on
// MI355X a tile that waits for another op's y must see that y across XCDs
// (write-through stores, their acknowledgement, a counter, a coherent poll,
// coherent loads of x), and under a full weight stream each of those memory
// round trips waits behind the stream (about 5 us with 32 MB in flight),
// while the waiting tiles hold their CU slots.  Measured on the Llama-3-8B
// decode layer wired QKV -> O -> gate/up -> down: 67 us per call in one launch
// with the waits, against 28.6 us launch by launch.
#include <algorithm>
#include <cstddef>

#include "int4_decode.hpp"
#include "kc_common.hpp"

namespace {

using kc::kWave;
using namespace kc::int4;

int validate_ops(const char* fn, const kc_gemv_op* ops, int n_ops) {
    if (n_ops < 0 || n_ops > KC_GEMV_CHAIN_MAX_OPS || (n_ops > 0 && !ops))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: n_ops=%d (at most %d, ops non-null)",
                             fn, n_ops, KC_GEMV_CHAIN_MAX_OPS);
    for (int i = 0; i < n_ops; ++i) {
        const kc_gemv_op& o = ops[i];
        if (o.rows < 0 || o.cols < 0 || o.group_size <= 0 || o.cols % 2 != 0 ||
            (o.cols > 0 && o.cols % o.group_size != 0))
            return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                                 "%s: op %d: rows=%d cols=%d group_size=%d", fn, i, o.rows,
                                 o.cols, o.group_size);
        if (o.rows > 0 && (!o.y || (o.cols > 0 && (!o.packed || !o.scales || !o.zeros || !o.x))))
            return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: op %d: null device pointer", fn, i);
    }
    return KC_SUCCESS;
}

// ---------------------------------------------------------------------------
// The fused tile: the per-lane-x GEMV of quant_int4.hip in 512-thread
// workgroups.  K = 2048 KW (KW 2..8); wave (kw, rg) owns chunk 64 kw + lane
// (32 k) of the R rows of row group rg; RGW = 8 / KW row groups (4 at KW 2,
// 2 at KW 3-4, 1 above; waves past KW RGW idle through the barriers) share
// one copy of x, which the workgroup copies into LDS with direct-to-LDS
// loads ahead of its scale, zero-byte and weight loads.  Per row the
// arithmetic is the per-lane-x kernel's: each wave folds its chunk with the
// group's scale and zero point and reduces its rows across its lanes, and
// the KW partial sums of a row are added in kw order.
// ---------------------------------------------------------------------------
constexpr int kRunWaves = 8;
constexpr int kRunThreads = kRunWaves * kWave;
constexpr int kXQ = 4;  // 16-byte quads of bf16 x per 32-k chunk
constexpr int kMaxRunLds = 4 * kXQ * kWave * 16 + 8 * 4 * 8 * 4;

constexpr int row_groups(int kw) { return kw == 2 ? 4 : (kw <= 4 ? 2 : 1); }


// One op of a run: 64 bytes, so that a workgroup fetches all of its fields
// with one scalar load (s_load_dwordx16).
struct __attribute__((aligned(64))) RunOp {
    const uint8_t* packed;
    const float* scales;
    const uint8_t* zeros;
    const uint16_t* x;
    uint16_t* y;
    int rows, cols, gshift, kw;
    int pad_[2];
};
static_assert(sizeof(RunOp) == 64, "one s_load_dwordx16 per op");
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

// Pointers read from the op table are generic; loads through them would be
// flat loads, which count on the LDS counter too and so leave the compiler
// only full waits.  Every pointer of an op is global memory.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gbl(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gbl(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}

// The op table.  The first workgroup of ops 1..7 (INT32_MAX for unused ops)
// and the ops' KW (4 bits each) are passed as scalar arguments ahead of it:
// the first 16 dwords of the arguments are preloaded into SGPRs at wave
// launch, so a workgroup finds its op and its tile code without a memory
// round trip; the op's fields then take one scalar load.
struct RunParams {
    int tile0[KC_GEMV_CHAIN_MAX_OPS];
    int n_ops;
    RunOp op[KC_GEMV_CHAIN_MAX_OPS];
};


__device__ __forceinline__ void x_dma16(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(n), n a constant once the caller's loop is unrolled; the
// wait reads and writes `after` (work the caller does just before), so it is
// not hoisted above it.
__device__ __forceinline__ void wait_vm(int n, float& after) {
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
}

// An op's fields, from the argument segment with one scalar load; the load
// is issued where the compiler likes (at the top) and waited for at the
// first use of a field.
__device__ __forceinline__ RunOp load_op(const RunOp* op) {
    const u32x16 d = *reinterpret_cast<const u32x16*>(op);
    const uint32_t w[16] = {d[0], d[1], d[2],  d[3],  d[4],  d[5],  d[6],  d[7],
                            d[8], d[9], d[10], d[11], d[12], d[13], d[14], d[15]};
    RunOp o;
    __builtin_memcpy(&o, w, sizeof o);
    return o;
}

// One tile: loads in the order x (copies into LDS, or this lane's 64 bytes),
// R scale, R zero-byte and R weight loads.  K = 2048 KW is a constant of the
// tile code.
template <int KW, int R>
__device__ __forceinline__ void run_tile(const RunOp* op, int tile, char* lds) {
    constexpr int RGW = row_groups(KW);
    constexpr bool kShare = RGW > 1;
    constexpr int kActive = KW * RGW;
    constexpr int cols = KW * 2048;
    constexpr int64_t rbytes = cols / 2;
    static_assert(kActive <= kRunWaves && R % 4 == 0 && R <= 8, "tile shape");
    u32x4* xsh = reinterpret_cast<u32x4*>(lds);                                    // [KW kXQ][64]
    float* part = reinterpret_cast<float*>(lds + (kShare ? KW * kXQ * kWave * 16 : 0));  // [RGW][KW][R]

    const RunOp o = load_op(op);
    const int rows = o.rows;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const bool active = wave < kActive;
    const int kw = wave % KW, rg = active ? wave / KW : 0;
    const int row0 = (tile * RGW + rg) * R;
    const int c = kw * kWave + lane;
    const int gshift = o.gshift;
    const int G = cols >> (5 + gshift);
    const int g = c >> gshift;

    // With x in LDS the loads are written out as instructions, so that the
    // wait for the copies counts exactly the 3R loads issued after them
    // (vector loads complete in order, and the compiler does not count
    // direct-to-LDS loads); with x per lane the compiler issues and waits for
    // them itself.  The op's pointers are read as global-memory pointers.
    u32x4 xq[kXQ];
    float sv[R];
    uint32_t zb[R];
    u32x4 w[R];
    if (active) {
        if constexpr (kShare) {
            const uint32_t base = static_cast<uint32_t>(reinterpret_cast<size_t>(
                (__attribute__((address_space(3))) void*)xsh));
#pragma unroll
            for (int t0 = 0; t0 < KW * kXQ; t0 += kActive) {
                const int t = t0 + wave;
                const int kwp = t / kXQ, j = t - kwp * kXQ;
                x_dma16(o.x + ((kwp * kWave + lane) * kXQ + j) * 8,
                        __builtin_amdgcn_readfirstlane(base + t * kWave * 16));
            }
            const uint32_t soff = static_cast<uint32_t>(g) * 4u, zoff = static_cast<uint32_t>(g >> 1);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t rr = min(row0 + r, rows - 1);
                const float* srow = o.scales + rr * G;
                const uint8_t* zrow = o.zeros + rr * (G >> 1);
                asm volatile("global_load_dword %0, %1, %2" : "=v"(sv[r]) : "v"(soff), "s"(srow)
                             : "memory");
                asm volatile("global_load_ubyte %0, %1, %2" : "=v"(zb[r]) : "v"(zoff), "s"(zrow)
                             : "memory");
            }
            const uint32_t voff = static_cast<uint32_t>(c) * 16u;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t rr = min(row0 + r, rows - 1);
                const uint8_t* prow = o.packed + rr * rbytes;
                asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(w[r]) : "v"(voff), "s"(prow)
                             : "memory");
            }
            __builtin_amdgcn_s_setprio(0);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * R) : "memory");  // x has landed
        } else {
            const auto xs = gbl(reinterpret_cast<const u32x4*>(o.x)) + c * kXQ;
#pragma unroll
            for (int q = 0; q < kXQ; ++q) xq[q] = xs[q];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t rr = min(row0 + r, rows - 1);
                sv[r] = gbl(o.scales + rr * G)[g];
                zb[r] = gbl(o.zeros + rr * (G >> 1))[g >> 1];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t rr = min(row0 + r, rows - 1);
                w[r] = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x4*>(o.packed + rr * rbytes)) + c);
            }
            __builtin_amdgcn_sched_barrier(0);  // every load above issued before any use
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_s_setprio(0);  // the waves that issue no loads
    if constexpr (kShare) {
        __builtin_amdgcn_s_barrier();  // every wave's copies of x, in LDS
        if (active) {
#pragma unroll
            for (int q = 0; q < kXQ; ++q) xq[q] = xsh[(kw * kXQ + q) * kWave + lane];
        }
    }

    if (active) {
        if constexpr (kShare) asm volatile("" : "+v"(xq[0]), "+v"(xq[1]), "+v"(xq[2]), "+v"(xq[3]));
        uint32_t sel_lo, sel_hi;  // v_perm_b32 selectors, in VGPRs
        asm volatile("v_mov_b32 %0, 0x05040100" : "=v"(sel_lo));
        asm volatile("v_mov_b32 %0, 0x07060302" : "=v"(sel_hi));
        const uint32_t ones = 0x3F803F80u;
        u32x4 xp[4];
        float xsm = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 d = xq[q];
            xp[q].x = __builtin_amdgcn_perm(d.z, d.x, sel_lo);  // (x0, x4)
            xp[q].y = __builtin_amdgcn_perm(d.z, d.x, sel_hi);  // (x1, x5)
            xp[q].z = __builtin_amdgcn_perm(d.w, d.y, sel_lo);  // (x2, x6)
            xp[q].w = __builtin_amdgcn_perm(d.w, d.y, sel_hi);  // (x3, x7)
            xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.x), as_bf16x2(ones), xsm, false);
            xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.y), as_bf16x2(ones), xsm, false);
            xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.z), as_bf16x2(ones), xsm, false);
            xsm = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(d.w), as_bf16x2(ones), xsm, false);
        }
        const NibConsts nk = nib_consts();
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // explicit loads: row r's weights have landed once at most
            // R - 1 - r younger loads are outstanding; the values the loads
            // produced count as produced by the wait
            if constexpr (kShare) {
                wait_vm(R - 1 - r, r == 0 ? xsm : acc[r > 0 ? r - 1 : 0]);
                asm volatile("" : "+v"(w[r]));
                if (r == 0) {
#pragma unroll
                    for (int q = 0; q < R; ++q) asm volatile("" : "+v"(sv[q]), "+v"(zb[q]));
                }
            }
            const uint32_t z = (g & 1) ? (zb[r] >> 4) : (zb[r] & 0xFu);
            const float dot = chunk_dot<true>(w[r], xp, nk);
            acc[r] = fmaf(sv[r], dot, -sv[r] * (136.0f + static_cast<float>(z)) * xsm);
        }
#pragma unroll
        for (int r4 = 0; r4 < R; r4 += 4) {
            const float v4[4] = {acc[r4], acc[r4 + 1], acc[r4 + 2], acc[r4 + 3]};
            const float t = wave_reduce_rows<4>(v4);  // lane 16 j holds row r4 + j
            if ((lane & 15) == 0) part[(rg * KW + kw) * R + r4 + (lane >> 4)] = t;
        }
    }
    __syncthreads();

    // wave 0 adds the KW partial sums of every row of the tile (kw order)
    if (wave != 0) return;
    constexpr int kTileRows = R * RGW;
    const int tr = lane < kTileRows ? lane : 0;
    float sum = part[(tr / R) * KW * R + (tr % R)];
#pragma unroll
    for (int k = 1; k < KW; ++k) sum += part[((tr / R) * KW + k) * R + (tr % R)];
    const int row = tile * kTileRows + lane;
    if (lane < kTileRows && row < rows) gbl(o.y)[row] = kc::f32_to_bf16(sum);
}

// The run kernel: the tile starts of ops 1..7 (INT32_MAX for unused ops) and
// the ops' KW (4 bits each) come as scalar arguments, which the hardware
// preloads into SGPRs, so a workgroup finds its op and its tile code with no
// memory access; the op's fields then take one scalar load.  A wave issues
// its tile's loads at a raised priority and computes at the normal one.
template <int R>
__global__ __launch_bounds__(kRunThreads) void gemv_run_kernel(int t1, int t2, int t3, int t4,
                                                               int t5, int t6, int t7, uint32_t kws,
                                                               RunParams p) {
    __shared__ __attribute__((aligned(16))) char lds[kMaxRunLds];
    __builtin_amdgcn_s_setprio(kIssuePrio);  // until this tile's loads are out
    const int b = static_cast<int>(blockIdx.x);
    const int ts[KC_GEMV_CHAIN_MAX_OPS] = {0, t1, t2, t3, t4, t5, t6, t7};
    int i = 0, t0 = 0;
#pragma unroll
    for (int j = 1; j < KC_GEMV_CHAIN_MAX_OPS; ++j)
        if (b >= ts[j]) {
            i = j;
            t0 = ts[j];
        }
    const int kw = (kws >> (4 * i)) & 0xF;
    const RunOp* op = &p.op[i];
    const int tile = b - t0;
    switch (kw) {
        case 2: run_tile<2, R>(op, tile, lds); break;
        case 3: run_tile<3, R>(op, tile, lds); break;
        case 4: run_tile<4, R>(op, tile, lds); break;
        case 5: run_tile<5, R>(op, tile, lds); break;
        case 6: run_tile<6, R>(op, tile, lds); break;
        case 7: run_tile<7, R>(op, tile, lds); break;
        default: run_tile<8, R>(op, tile, lds); break;
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct Span {
    uintptr_t lo, hi;  // [lo, hi)
};

bool overlap(Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; }

Span span_of(const void* p, int64_t bytes) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    return {lo, lo + static_cast<uintptr_t>(std::max<int64_t>(bytes, 1))};
}

// The memory an op reads (weights, scales, zero bytes, x) and writes (y).
struct OpSpans {
    Span in[4];
    Span out;
};

OpSpans spans_of(const kc_gemv_op& o) {
    const int64_t G = o.cols / o.group_size;
    return {{span_of(o.packed, int64_t{o.rows} * (o.cols / 2)),
             span_of(o.scales, int64_t{o.rows} * G * 4),
             span_of(o.zeros, int64_t{o.rows - 1} * (G / 2) + (G - 1) / 2 + 1),
             span_of(o.x, int64_t{o.cols} * 2)},
            span_of(o.y, int64_t{o.rows} * 2)};
}

// Op i depends on op j < i when it reads j's output or writes what j reads
// or writes.
bool depends(const OpSpans& j, const OpSpans& i) {
    if (overlap(j.out, i.out)) return true;
    for (const Span& s : i.in)
        if (overlap(j.out, s)) return true;
    for (const Span& s : j.in)
        if (overlap(s, i.out)) return true;
    return false;
}

// Whether an op with rows > 0 fits the fused tile: K = 2048 KW with KW
// 2..8, a power-of-two group of at least 32, 16-byte aligned weights and x.
bool fused_shape(const kc_gemv_op& o) {
    return o.cols % 2048 == 0 && o.cols / 2048 >= 2 && o.cols / 2048 <= 8 &&
           o.group_size >= 32 && kc::is_pow2(o.group_size) && kc::aligned(o.packed, 16) &&
           kc::aligned(o.x, 16);
}

constexpr int kRunRows = 4;  // rows per wave

// ops [first, last) as one launch: every op fits the fused tile and none
// depends on another, so their tiles may go in any order.  Ops with the
// longest rows (largest K) go first and the short-K tiles fill the end of
// the launch, then more rows first (decode layer, one launch: QKV, O,
// gate/up, down in the caller's order 22.2 us; down, gate/up first 21.8 us).
int launch_run(const char* fn, const kc_gemv_op* ops, int first, int last, hipStream_t stream) {
    int order[KC_GEMV_CHAIN_MAX_OPS];
    const int n = last - first;
    for (int i = 0; i < n; ++i) order[i] = first + i;
    std::stable_sort(order, order + n, [&](int a, int b) {
        if (ops[a].cols != ops[b].cols) return ops[a].cols > ops[b].cols;
        return ops[a].rows > ops[b].rows;
    });
    RunParams p{};
    for (int& t : p.tile0) t = INT32_MAX;
    uint32_t kws = 0;
    int64_t tiles = 0;
    for (int k = 0; k < n; ++k) {
        const kc_gemv_op& o = ops[order[k]];
        RunOp& f = p.op[p.n_ops++];
        f.packed = o.packed;
        f.scales = o.scales;
        f.zeros = o.zeros;
        f.x = o.x;
        f.y = o.y;
        f.rows = o.rows;
        f.cols = o.cols;
        f.gshift = kc::ilog2(o.group_size) - 5;
        f.kw = o.cols / 2048;
        kws |= static_cast<uint32_t>(f.kw) << (4 * (p.n_ops - 1));
        p.tile0[p.n_ops - 1] = static_cast<int>(tiles);
        const int per_tile = kRunRows * row_groups(f.kw);
        tiles += (int64_t{o.rows} + per_tile - 1) / per_tile;
        if (tiles > INT32_MAX)
            return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: %lld tiles in one launch", fn,
                                 (long long)tiles);
    }
    gemv_run_kernel<kRunRows><<<static_cast<unsigned>(tiles), kRunThreads, 0, stream>>>(
        p.tile0[1], p.tile0[2], p.tile0[3], p.tile0[4], p.tile0[5], p.tile0[6], p.tile0[7], kws, p);
    return kc::check_launch(fn);
}

}  // namespace

extern "C" int kc_gemv_int4_bf16_chain(const kc_gemv_op* ops, int n_ops, kc_stream_t stream) {
    const char* fn = "kc_gemv_int4_bf16_chain";
    int st = validate_ops(fn, ops, n_ops);
    if (st != KC_SUCCESS) return st;
    // the live ops (an op with no rows reads and writes nothing), cut into runs
    kc_gemv_op live[KC_GEMV_CHAIN_MAX_OPS];
    OpSpans sp[KC_GEMV_CHAIN_MAX_OPS];
    int n = 0;
    for (int i = 0; i < n_ops; ++i)
        if (ops[i].rows > 0) {
            live[n] = ops[i];
            sp[n] = spans_of(ops[i]);
            ++n;
        }
    int first = 0;
    while (first < n) {
        int last = first + 1;
        if (live[first].cols > 0 && fused_shape(live[first])) {
            while (last < n && live[last].cols > 0 && fused_shape(live[last])) {
                bool dep = false;
                for (int j = first; j < last && !dep; ++j) dep = depends(sp[j], sp[last]);
                if (dep) break;
                ++last;
            }
        }
        if (last - first >= 2) {
            st = launch_run(fn, live, first, last, stream);
        } else {
            const kc_gemv_op& o = live[first];
            st = kc_gemv_int4_bf16(o.packed, o.scales, o.zeros, o.x, o.y, o.rows, o.cols,
                                   o.group_size, stream);
        }
        if (st != KC_SUCCESS) return st;
        first = last;
    }
    return KC_SUCCESS;
}
