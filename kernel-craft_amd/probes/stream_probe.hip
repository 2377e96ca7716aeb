// stream_probe.hip -- measurement kernels for bench.py (libkc_probes.so), not
// part of libkernels.so.
//
// They give the floors the path's kernels are compared with on the same
// machine: how fast a plain stream of a given number of bytes can be read
// from HBM (the INT4 GEMVs read their weights once), and how fast a stream
// can be read while 1/2 or 1/4 of its size is written back (the FP8
// quantizers' traffic: bf16 -> E4M3 is 2:1, fp32 -> E4M3 is 4:1).  The caller
// sweeps the grid size and the loads in flight per thread and keeps the best.
//
// Every access stays inside the buffers: thread t of a grid of G x 256
// threads reads 16-byte units t, t + 256 G, ... below n16 and writes the unit
// of the same index in the output; the read kernel writes its sink word only
// when its checksum hits a value the caller's data never produce, and the sink
// holds one word per thread in any case.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr uint32_t kNever = 0x9E3779B9u;

__device__ __forceinline__ uint32_t fold(const u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

template <int U>
__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                        uint32_t* __restrict__ sink) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    uint32_t acc = 0;
    int64_t i = t;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        u32x4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= fold(r[u]);
    }
    for (; i < n16; i += stride) acc ^= fold(__builtin_nontemporal_load(src + i));
    if (acc == kNever) sink[t] = acc;
}

// 16 bytes in, 16 / R bytes out per unit (R = 2: bf16 -> FP8, R = 4: fp32 -> FP8).
template <int R, int U>
__global__ __launch_bounds__(kThreads) void copy_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                        void* __restrict__ dst) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    auto put = [&](int64_t j, const u32x4 v) {
        if constexpr (R == 4)
            __builtin_nontemporal_store(fold(v), static_cast<uint32_t*>(dst) + j);
        else
            __builtin_nontemporal_store(u32x2{v.x ^ v.y, v.z ^ v.w}, static_cast<u32x2*>(dst) + j);
    };
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        u32x4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) put(i + u * stride, r[u]);
    }
    for (; i < n16; i += stride) put(i, __builtin_nontemporal_load(src + i));
}

__global__ void empty_kernel() {}

}  // namespace

// Reads `bytes` (a multiple of 16) from src; sink holds grid * 256 words.
// unroll: loads in flight per thread, 1, 4, 8 or 16.  Returns a hipError_t.
extern "C" int kcp_stream_read(const void* src, int64_t bytes, uint32_t* sink, int grid, int unroll,
                               hipStream_t stream) {
    if (bytes < 0 || bytes % 16 != 0 || grid <= 0 || !src || !sink) return hipErrorInvalidValue;
    const u32x4* s = static_cast<const u32x4*>(src);
    const int64_t n = bytes / 16;
    switch (unroll) {
        case 1: read_kernel<1><<<grid, kThreads, 0, stream>>>(s, n, sink); break;
        case 4: read_kernel<4><<<grid, kThreads, 0, stream>>>(s, n, sink); break;
        case 8: read_kernel<8><<<grid, kThreads, 0, stream>>>(s, n, sink); break;
        case 16: read_kernel<16><<<grid, kThreads, 0, stream>>>(s, n, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Reads `bytes` (a multiple of 16) from src and writes bytes / ratio to dst
// (ratio 2 or 4).  unroll 1, 4 or 8.
extern "C" int kcp_stream_copy(const void* src, int64_t bytes, void* dst, int ratio, int grid,
                               int unroll, hipStream_t stream) {
    if (bytes < 0 || bytes % 16 != 0 || grid <= 0 || !src || !dst) return hipErrorInvalidValue;
    const u32x4* s = static_cast<const u32x4*>(src);
    const int64_t n = bytes / 16;
#define KCP_COPY(R, U) copy_kernel<R, U><<<grid, kThreads, 0, stream>>>(s, n, dst)
    if (ratio == 2 && unroll == 1) KCP_COPY(2, 1);
    else if (ratio == 2 && unroll == 4) KCP_COPY(2, 4);
    else if (ratio == 2 && unroll == 8) KCP_COPY(2, 8);
    else if (ratio == 4 && unroll == 1) KCP_COPY(4, 1);
    else if (ratio == 4 && unroll == 4) KCP_COPY(4, 4);
    else if (ratio == 4 && unroll == 8) KCP_COPY(4, 8);
    else return hipErrorInvalidValue;
#undef KCP_COPY
    return hipGetLastError();
}

// An empty launch: the per-launch cost the back-to-back kernels pay.
extern "C" int kcp_empty(int grid, hipStream_t stream) {
    if (grid <= 0) return hipErrorInvalidValue;
    empty_kernel<<<grid, kThreads, 0, stream>>>();
    return hipGetLastError();
}
