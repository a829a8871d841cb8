// probe.hip -- HBM streaming probe: the bandwidth a plain streaming kernel
// reaches on this device for the RMSNorm path's traffic mixes (one read + one
// write, as the forward; two reads + one write, as the backward; reads only),
// with and without the non-temporal cache policy the row kernels use.  It is
// the practical ceiling the row kernels are measured against, next to the
// vendor peak.  No reference counterpart; part of the benchmark's own library
// (libagk_bench.so), not of the kernel library.
//
// Two access patterns.  Grid-stride: each lane moves 16-byte slots in a
// grid-stride loop with four independent slots in flight per iteration.
// Chunked: each workgroup moves one contiguous 16 KiB chunk of each buffer
// (four slots per lane, all loads issued before any store), one workgroup per
// chunk, which is how the row kernels touch memory (a row or a band of rows
// per workgroup).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "agk_bench.h"
#include "rowcommon.hpp"

namespace agk {

constexpr int kProbeBlock = 256;
constexpr int kProbeUnroll = 4;

template <bool NT>
__device__ __forceinline__ u32x4 probe_load(const u32x4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}
template <bool NT>
__device__ __forceinline__ void probe_store(u32x4* p, u32x4 v) {
    if constexpr (NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

// READS in {1, 2}, WRITES in {0, 1, 2} (c = the value, d = the value + 1).  n = slots per buffer, a multiple of
// kProbeUnroll * kProbeBlock * gridDim.x is not required: the tail is guarded.
template <int READS, int WRITES, bool NT>
__global__ __launch_bounds__(kProbeBlock) void probe_stream_kernel(const u32x4* __restrict__ a,
                                                                   const u32x4* __restrict__ b,
                                                                   u32x4* __restrict__ c,
                                                                   u32x4* __restrict__ d,
                                                                   int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeBlock;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeBlock + threadIdx.x;
    u32x4 sink = u32x4{0u, 0u, 0u, 0u};
    for (; i + (kProbeUnroll - 1) * stride < n; i += kProbeUnroll * stride) {
        u32x4 v[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) v[u] = probe_load<NT>(a + i + u * stride);
        if constexpr (READS == 2) {
#pragma unroll
            for (int u = 0; u < kProbeUnroll; ++u) v[u] ^= probe_load<NT>(b + i + u * stride);
        }
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            if constexpr (WRITES >= 1)
                probe_store<NT>(c + i + u * stride, v[u]);
            else
                sink ^= v[u];
            if constexpr (WRITES == 2) probe_store<NT>(d + i + u * stride, v[u] + 1u);
        }
    }
    for (; i < n; i += stride) {
        u32x4 v = probe_load<NT>(a + i);
        if constexpr (READS == 2) v ^= probe_load<NT>(b + i);
        if constexpr (WRITES >= 1)
            probe_store<NT>(c + i, v);
        else
            sink ^= v;
        if constexpr (WRITES == 2) probe_store<NT>(d + i, v + 1u);
    }
    if constexpr (WRITES == 0) {
        // Keeps the loads: a store that the data decides on (all-ones XOR of
        // every slot this lane read), written to slot 0 of c, which the
        // caller provides.
        if (sink.x == 0xffffffffu && sink.y == 0xffffffffu && sink.z == 0xffffffffu &&
            sink.w == 0xffffffffu)
            c[0] = sink;
    }
}

template <int READS, int WRITES, bool NT>
__global__ __launch_bounds__(kProbeBlock) void probe_chunk_kernel(const u32x4* __restrict__ a,
                                                                  const u32x4* __restrict__ b,
                                                                  u32x4* __restrict__ c,
                                                                  u32x4* __restrict__ d,
                                                                  int64_t n) {
    constexpr int64_t kChunk = static_cast<int64_t>(kProbeBlock) * kProbeUnroll;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
    u32x4 v[kProbeUnroll];
    u32x4 sink = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
        const int64_t i = base + u * kProbeBlock;
        v[u] = i < n ? probe_load<NT>(a + i) : u32x4{0u, 0u, 0u, 0u};
        if constexpr (READS == 2) v[u] ^= i < n ? probe_load<NT>(b + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
        const int64_t i = base + u * kProbeBlock;
        if constexpr (WRITES >= 1) {
            if (i < n) probe_store<NT>(c + i, v[u]);
        } else {
            sink ^= v[u];
        }
        if constexpr (WRITES == 2) {
            if (i < n) probe_store<NT>(d + i, v[u] + 1u);
        }
    }
    if constexpr (WRITES == 0) {
        if (sink.x == 0xffffffffu && sink.y == 0xffffffffu && sink.z == 0xffffffffu &&
            sink.w == 0xffffffffu)
            c[0] = sink;
    }
}

}  // namespace agk

extern "C" int agk_probe_stream(const void* a, const void* b, void* c, void* d, int64_t bytes,
                                int reads, int writes, int nontemporal, int grid,
                                agk_stream_t stream) {
    using namespace agk;
    if (bytes < 0 || (bytes & 15) != 0 || grid < 0) return AGK_EINVAL;
    if (reads != 1 && reads != 2) return AGK_EINVAL;
    if (writes < 0 || writes > 2) return AGK_EINVAL;
    if (!a || !c || (reads == 2 && !b) || (writes == 2 && !d)) return AGK_EINVAL;
    if (bytes == 0) return AGK_OK;
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const u32x4* pa = static_cast<const u32x4*>(a);
    const u32x4* pb = static_cast<const u32x4*>(b);
    u32x4* pc = static_cast<u32x4*>(c);
    u32x4* pd = static_cast<u32x4*>(d);
    const int64_t n = bytes / 16;
    const int64_t chunks = (n + kProbeBlock * kProbeUnroll - 1) / (kProbeBlock * kProbeUnroll);
    if (grid == 0 && chunks > 0x7fffffffLL) return AGK_EINVAL;
    const dim3 g(static_cast<unsigned>(grid == 0 ? chunks : grid)), blk(kProbeBlock);
#define AGK_PROBE(R, W, NT)                                                                   \
    do {                                                                                      \
        if (grid == 0)                                                                        \
            hipLaunchKernelGGL((probe_chunk_kernel<R, W, NT>), g, blk, 0, st, pa, pb, pc, pd,  \
                               n);                                                            \
        else                                                                                  \
            hipLaunchKernelGGL((probe_stream_kernel<R, W, NT>), g, blk, 0, st, pa, pb, pc, pd, \
                               n);                                                            \
    } while (0)
#define AGK_PROBE_NT(R, W)          \
    do {                            \
        if (nontemporal)            \
            AGK_PROBE(R, W, true);  \
        else                        \
            AGK_PROBE(R, W, false); \
    } while (0)
    switch ((reads - 1) * 3 + writes) {
        case 0: AGK_PROBE_NT(1, 0); break;
        case 1: AGK_PROBE_NT(1, 1); break;
        case 2: AGK_PROBE_NT(1, 2); break;
        case 3: AGK_PROBE_NT(2, 0); break;
        case 4: AGK_PROBE_NT(2, 1); break;
        default: AGK_PROBE_NT(2, 2); break;
    }
#undef AGK_PROBE_NT
#undef AGK_PROBE
    return check_launch();
}
