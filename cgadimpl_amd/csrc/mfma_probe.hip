// mfma_probe.hip -- what the matrix cores sustain on this device when they run
// the bf16 GEMM's inner loop with no global loads and no barriers, as a
// function of the operand data.  Part of the benchmark's own library
// (libagk_bench.so, cgadimpl_amd/csrc/agk_bench.h); no reference counterpart.
//
// Each workgroup is the GEMM's (gemm.hip, gemm_nt_direct_kernel): 4 waves,
// each holding a 128 x 128 block of C as 4 x 4 v_mfma_f32_32x32x16_bf16
// accumulators in AGPRs, the operand tile a 64-deep stage of 256 A rows and
// 256 B rows in LDS (128-byte rows, 16-byte chunks XOR-swizzled as in the
// GEMM).  A k-step is four 16-deep substeps of 16 MFMAs.
//   mode 0: every substep reads its 8 fragments from LDS one substep ahead of
//           the MFMAs (the GEMM's LDS traffic and schedule, minus the loads
//           and the end-of-step barrier);
//   mode 1: two fragment sets are read once; the loop is MFMAs only.
//   modes 2 and 3: modes 0 and 1 on v_mfma_f32_16x16x32_bf16 (the same
//           128 x 128 block per wave as 8 x 8 accumulators of 16 x 16, the
//           same fragment bytes per k: eight 16-byte fragments per 32-deep
//           half step), to compare the two instructions at the power limit.
// Wave 0 reads the shader clock counter (s_memtime) and the constant 100 MHz
// counter (s_memrealtime) around its loop, so the host can report the shader
// clock the loop ran at.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "agk_bench.h"
#include "rowcommon.hpp"

namespace agk_mfma_probe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

constexpr int kLanes = 256;
constexpr int kRowElems = 64;               // bf16 per LDS row (one 64-deep k-step)
constexpr int kTileElems = 512 * kRowElems;  // 256 A rows + 256 B rows: 64 KiB

__device__ __forceinline__ int lds_off(int row, int c) {
    return row * kRowElems + ((c ^ (row & 7) ^ ((row >> 3) & 7)) << 3);
}
__device__ __forceinline__ bf16x8 frag(const uint16_t* lds, int row, int k) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4v*>(lds + lds_off(row, k >> 3)));
}

struct Frags {
    bf16x8 a[4], b[4];
};

__device__ __forceinline__ void read_frags(Frags& f, const uint16_t* lds, int s, int wm, int wn,
                                           int frow, int fk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[i] = frag(lds, wm * 128 + i * 32 + frow, s * 16 + fk);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.b[j] = frag(lds, 256 + wn * 128 + j * 32 + frow, s * 16 + fk);
}

__device__ __forceinline__ void mfma_sub(const Frags& f, f32x16 (&acc)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// 16x16x32: operand lane l holds row (column) l % 16, k 8 (l / 16) .. + 7.
typedef float f32x4 __attribute__((ext_vector_type(4)));
struct Frags16 {
    bf16x8 a[8], b[8];
};
__device__ __forceinline__ void read_frags16(Frags16& f, const uint16_t* lds, int h, int wm, int wn,
                                             int lane) {
    const int r = lane & 15, k = h * 32 + (lane >> 4) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) f.a[i] = frag(lds, wm * 128 + i * 16 + r, k);
#pragma unroll
    for (int j = 0; j < 8; ++j) f.b[j] = frag(lds, 256 + wn * 128 + j * 16 + r, k);
}
__device__ __forceinline__ void mfma_half16(const Frags16& f, f32x4 (&acc)[8][8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// one fragment read, two MFMAs; eight of them cover a substep
#define AGK_PROBE_RM                                    \
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#define AGK_PROBE_X8(g) g g g g g g g g

template <int MODE>
__global__ __launch_bounds__(kLanes) void mfma_probe_kernel(const uint16_t* __restrict__ src,
                                                            float* __restrict__ out,
                                                            uint64_t* __restrict__ clocks,
                                                            int steps) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[kTileElems];
    const u32x4v* s16 = reinterpret_cast<const u32x4v*>(src);
    u32x4v* l16 = reinterpret_cast<u32x4v*>(lds);
    for (int i = threadIdx.x; i < kTileElems / 8; i += kLanes) l16[i] = s16[i];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int frow = lane & 31, fk = (lane >> 5) * 8;
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    Frags f0, f1;
    read_frags(f0, lds, 0, wm, wn, frow, fk);
    read_frags(f1, lds, 1, wm, wn, frow, fk);
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    for (int t = 0; t < steps; ++t) {
        if constexpr (MODE == 0) {
            // substep s multiplies while substep s + 1's fragments are read
            mfma_sub(f0, acc);
            read_frags(f1, lds, 1, wm, wn, frow, fk);
            AGK_PROBE_X8(AGK_PROBE_RM)
            __builtin_amdgcn_sched_barrier(0);
            mfma_sub(f1, acc);
            read_frags(f0, lds, 2, wm, wn, frow, fk);
            AGK_PROBE_X8(AGK_PROBE_RM)
            __builtin_amdgcn_sched_barrier(0);
            mfma_sub(f0, acc);
            read_frags(f1, lds, 3, wm, wn, frow, fk);
            AGK_PROBE_X8(AGK_PROBE_RM)
            __builtin_amdgcn_sched_barrier(0);
            mfma_sub(f1, acc);
            read_frags(f0, lds, 0, wm, wn, frow, fk);
            AGK_PROBE_X8(AGK_PROBE_RM)
            __builtin_amdgcn_sched_barrier(0);
        } else {
            mfma_sub(f0, acc);
            mfma_sub(f1, acc);
            mfma_sub(f0, acc);
            mfma_sub(f1, acc);
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();

    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) sum += acc[i][j][e];
    if (lane == 0) out[blockIdx.x * 4 + wave] = sum;
    if (clocks != nullptr && threadIdx.x == 0) {
        uint64_t* c = clocks + static_cast<int64_t>(blockIdx.x) * 4;
        c[0] = t0;
        c[1] = t1;
        c[2] = r0;
        c[3] = r1;
    }
}

// Modes 2 (fragments from LDS, one 32-deep half step ahead) and 3 (registers
// only) on v_mfma_f32_16x16x32_bf16: 128 MFMAs per 64-deep k-step.
template <int MODE>
__global__ __launch_bounds__(kLanes) void mfma_probe16_kernel(const uint16_t* __restrict__ src,
                                                              float* __restrict__ out,
                                                              uint64_t* __restrict__ clocks,
                                                              int steps) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[kTileElems];
    const u32x4v* s16 = reinterpret_cast<const u32x4v*>(src);
    u32x4v* l16 = reinterpret_cast<u32x4v*>(lds);
    for (int i = threadIdx.x; i < kTileElems / 8; i += kLanes) l16[i] = s16[i];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;

    Frags16 f0, f1;
    read_frags16(f0, lds, 0, wm, wn, lane);
    read_frags16(f1, lds, 1, wm, wn, lane);
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    for (int t = 0; t < steps; ++t) {
        if constexpr (MODE == 2) {
            mfma_half16(f0, acc);
            read_frags16(f1, lds, 1, wm, wn, lane);
            AGK_PROBE_X8(AGK_PROBE_X8(AGK_PROBE_RM))
            __builtin_amdgcn_sched_barrier(0);
            mfma_half16(f1, acc);
            read_frags16(f0, lds, 0, wm, wn, lane);
            AGK_PROBE_X8(AGK_PROBE_X8(AGK_PROBE_RM))
            __builtin_amdgcn_sched_barrier(0);
        } else {
            mfma_half16(f0, acc);
            mfma_half16(f1, acc);
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();

    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) sum += acc[i][j][e];
    if (lane == 0) out[blockIdx.x * 4 + wave] = sum;
    if (clocks != nullptr && threadIdx.x == 0) {
        uint64_t* c = clocks + static_cast<int64_t>(blockIdx.x) * 4;
        c[0] = t0;
        c[1] = t1;
        c[2] = r0;
        c[3] = r1;
    }
}

}  // namespace agk_mfma_probe

extern "C" int agk_probe_mfma(const void* src, float* out, uint64_t* clocks, int workgroups,
                              int steps, int mode, agk_stream_t stream) {
    using namespace agk_mfma_probe;
    if (!src || !out || workgroups <= 0 || steps < 0 || mode < 0 || mode > 3) return AGK_EINVAL;
    if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0) return AGK_EINVAL;
    agk::clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(workgroups)), block(kLanes);
    const uint16_t* s = static_cast<const uint16_t*>(src);
    if (mode == 0)
        hipLaunchKernelGGL(mfma_probe_kernel<0>, grid, block, 0, st, s, out, clocks, steps);
    else if (mode == 1)
        hipLaunchKernelGGL(mfma_probe_kernel<1>, grid, block, 0, st, s, out, clocks, steps);
    else if (mode == 2)
        hipLaunchKernelGGL(mfma_probe16_kernel<2>, grid, block, 0, st, s, out, clocks, steps);
    else
        hipLaunchKernelGGL(mfma_probe16_kernel<3>, grid, block, 0, st, s, out, clocks, steps);
    return agk::check_launch();
}
