// rmsnorm.hip -- CDNA4 (gfx950) kernels and C ABI for cgadimpl's RMSNorm
// layer path: forward y = x * rsqrt(mean(x^2) + eps) * gamma, backward
// (dx, dgamma), plus the broadcast multiply used when the layer is written
// unfused as ag::rms(x) * gamma.
//
// Reference behaviour replaced here (paths relative to the reference tree):
//   rms_nodeops        cgadimpl/src/ops/normalization.cpp:23-35
//   mul_nodeops        cgadimpl/src/ops/arithmetic.cpp:31-39
//   vjp_Mul            cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:54-59
//   reduce_for_broadcast  autodiff_vjp_ops.cpp:15-35
//   vjp_RMSNorm        autodiff_vjp_ops.cpp:368-377
//   accumulate_grad    cgadimpl/src/core/graph.cpp:44-47
// The reference runs these as ~30 separate tensor-library launches that
// materialise every intermediate; here the forward is one kernel (one read of
// x, one write of y, r saved per row) and the backward is one kernel (one read
// each of x and dy, one write of dx, dgamma partials per row block) plus a
// small fixed-order column reduction for dgamma.
//
// Kernel shapes.  A row of `cols` elements is owned by a group of TPR lanes:
// TPR <= 64 packs 64/TPR rows into each wave (narrow rows, e.g. 128-wide
// per-head norms), TPR == 64 is one wave per row, TPR > 64 spreads one row
// over several waves of a workgroup (wide rows) and combines the per-wave
// sums through LDS.  Each lane keeps NV 16-byte slots of the row in registers
// between the reduction and the elementwise pass, so x (and dy) are read from
// HBM exactly once.  Rows whose pointers are not 16-byte aligned, whose width
// is not a multiple of the vector width, or that are too wide for registers
// take a looped kernel that re-reads the row (from cache) instead.
//
// dgamma is deterministic: each workgroup of the backward owns a fixed set of
// rows (dealt round-robin in the register-resident kernel, a contiguous run in
// the looped one) and sums dy*xhat for them in a fixed order into one row of
// fp32 partials; dgamma_finalize then sums the partial rows in a fixed order
// in fp64.  No floating-point atomics are used anywhere.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "agk_rmsnorm.h"
#include "rowcommon.hpp"

namespace agk {

// ---- register-resident forward ---------------------------------------------
// y[row] = (x[row] * r) * gamma, r = 1 / sqrt(sum(x^2)/cols + eps); inv_rms[row] = r.
// A workgroup of TPR*G lanes normalises G rows, one per TPR-lane group; each
// lane holds NV 16-byte slots of its row (columns (t + k*TPR)*W .. +W).
// gamma == nullptr: no scale.  Requires 16-byte aligned x/y/gamma,
// cols % S::kVec == 0 and cols <= TPR * NV * kVec.
//
// MUL: the broadcast multiply y = x * gamma on the same launch shape (the
// unfused layer's Mul): no row sum, no inv_rms.
// EARLY_G: gamma's slots are loaded with x's, before the row sum, so that
// their latency overlaps it: for grids of at most one workgroup per CU with
// short rows (at most 1024 16-byte slots), where the call is latency-bound.
// Measured (graph replays, one box): [512, 512] fp32 2.57-2.61 -> 2.36-2.38 us;
// but [51, 13824] fp32 4.19-4.21 -> 4.38-4.39 us (a long row's gamma loads
// compete with its x loads before the sum) and many rows lose ~3 % (live
// registers).  Same arithmetic either way.
template <class S, int TPR, int NV, int G, bool MUL = false, bool EARLY_G = false>
__global__ __launch_bounds__(TPR * G) void rms_fwd_resident(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    typename S::T* __restrict__ y, float* __restrict__ inv_rms, int64_t rows, int cols,
    float eps) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    __shared__ float red[2][TPR > 64 ? G * (TPR / 64) : 1];

    const int t = threadIdx.x % TPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * G + threadIdx.x / TPR;
    const bool active = row < rows;
    const T* xr = x + (active ? row : 0) * static_cast<int64_t>(cols);

    u32x4 xv[NV];
    float part[W];
#pragma unroll
    for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = (t + k * TPR) * W;
        xv[k] = (active && col < cols) ? load16_stream<S>(xr + col) : u32x4{0u, 0u, 0u, 0u};
    }
    [[maybe_unused]] u32x4 gv[EARLY_G ? NV : 1];
    if constexpr (EARLY_G) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            gv[k] = (active && col < cols) ? load16<S>(gamma + col) : u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float f[W];
        S::unpack(xv[k], f);
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] += f[e] * f[e];
    }
    float r = 1.0f;
    if constexpr (!MUL) {
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < W; ++e) ss += part[e];
        ss = row_sum<TPR, G>(ss, red, 0);
        const float ms = ss / static_cast<float>(cols);
        r = 1.0f / sqrtf(ms + eps);
    } else {
        (void)red;
        (void)eps;
    }
    if (!active) return;
    if (!MUL && t == 0) inv_rms[row] = r;

    T* yr = y + row * static_cast<int64_t>(cols);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = (t + k * TPR) * W;
        if (col < cols) {
            float f[W];
            S::unpack(xv[k], f);
            if (MUL) {
                float gm[W];
                S::unpack(load16<S>(gamma + col), gm);
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = f[e] * gm[e];
            } else if (EARLY_G) {
                float gm[W];
                S::unpack(gv[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = (f[e] * r) * gm[e];
            } else if (gamma) {
                float gm[W];
                S::unpack(load16<S>(gamma + col), gm);
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = (f[e] * r) * gm[e];
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = f[e] * r;
            }
            store16_stream<S>(yr + col, S::pack(f));
        }
    }
}

// ---- register-resident backward --------------------------------------------
// The grid has nblk workgroups (one fp32 partial row of dgamma each); group q
// of workgroup b takes rows b*G + q + k*nblk*G, k = 0, 1, ... (about rows/nblk
// rows per workgroup).  Rows are dealt round-robin so that at any moment the
// whole grid works on one contiguous band of rows, which streams from HBM
// faster than one run of rows per workgroup.  Per row:
//   g = dy*gamma, dot = sum(g*x), dx (+)= r*(g - x*(r*r*dot/cols))
// and each lane accumulates dy*(x*r) for the columns it owns.  At the end the
// G groups' sums are added in group order (through LDS) into partials[b][*],
// one fp32 row per workgroup.  gamma is read once and kept in registers.
//
// Memory access is branch-free, through buffer resources: a wave's rows of a
// step get a resource sized to the rows that exist (zero for a step past the
// last row), and a slot past the row end gets an out-of-range offset.  Such
// loads return zeros, which add nothing to dot or dgamma, and such stores are
// dropped.  dx's old values (accumulate) are read the same way, through a
// resource of size zero when dx is not wanted.  The old values are loaded
// (and held in registers) only in the accumulating instantiation (ACC).
//
// With NSET > 1 register sets the loop is software-pipelined: the loads of
// step s+NSET go into a set as soon as step s has stored from it, so NSET
// steps' loads are in flight while a step reduces and stores.  The first NSET
// steps are peeled so that the loop is entered with the same memory
// operations outstanding as at its back edge; the compiler then waits for
// exactly the set being processed and never for the stores just issued or the
// other sets' loads.  With one set (narrow rows, and wide shapes whose second
// set would not fit in registers) each step loads and then processes.
template <class S, int NV, bool ACC>
struct BwdSet {
    u32x4 xv[NV], dv[NV];   // x, dy
    u32x4 ov[ACC ? NV : 1]; // old dx (accumulate)
    float r;
};

// What one instantiation of the skeleton computes (template argument KIND):
//   kBwdRms     the RMSNorm VJP above (gamma optional);
//   kBwdMul     the broadcast multiply's VJP (x = a, gamma = b, dy = gy):
//               da = gy*b, db += gy*a, no row reduction and no inv_rms (r = 1);
//   kBwdRmsMul  both VJPs of the composition y = rms(x) * gamma, back to back:
//               g = gy*gamma rounded to storage (written to dr, the gradient
//               of rms(x)), dx (+)= r*(g - x*(r*r*sum(g*x)/cols)), and
//               dgamma += gy*h with h = x*r rounded to storage (rms(x) as the
//               forward stored it).  Every value and every summation order is
//               the one the two separate calls produce;
//   kBwdColSum  column sums of dy alone (the bias gradient of a linear
//               layer): partials += dy, no row reduction, nothing stored.
enum : int { kBwdRms = 0, kBwdMul = 1, kBwdRmsMul = 2, kBwdColSum = 3 };

template <class S, int TPR, int NV, int G, bool ACC, int KIND>
struct BwdCtx {
    using T = typename S::T;
    static constexpr int W = S::kVec;
    static constexpr int RPW = TPR >= 64 ? 1 : 64 / TPR;  // rows a wave holds per step
    const T* x;
    const T* gamma;
    const float* inv_rms;
    const T* dy;
    T* dx;
    T* dr;  // kBwdRmsMul: the gradient of rms(x)
    int64_t rows, first, stride;
    int cols, wgrp0;
    uint32_t row_bytes, x_bytes, old_bytes, dx_bytes, dr_bytes, roff;
    uint32_t off[NV];
    float inv_cols;

    // First row of the wave's rows at `step` (clamped into range) and how many exist.
    __device__ __forceinline__ void wave_rows(int64_t step, int64_t& r0, uint32_t& n) const {
        const int64_t w0 = first + wgrp0 + step * stride;
        int64_t cnt = rows - w0;
        cnt = cnt < 0 ? 0 : (cnt > RPW ? RPW : cnt);
        r0 = w0 < rows ? w0 : rows - 1;
        n = static_cast<uint32_t>(cnt);
    }

    __device__ __forceinline__ void issue(BwdSet<S, NV, ACC>& b, int64_t step) const {
        int64_t r0;
        uint32_t n;
        wave_rows(step, r0, n);
        const int64_t e0 = r0 * static_cast<int64_t>(cols);
        const rsrc_t rx = make_rsrc(x ? x + e0 : x, n * x_bytes);
        const rsrc_t rd = make_rsrc(dy + e0, n * row_bytes);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            b.xv[k] = bload16_stream(rx, off[k]);
            b.dv[k] = bload16_stream(rd, off[k]);
        }
        if constexpr (ACC) {
            const rsrc_t ro = make_rsrc(dx ? dx + e0 : dx, n * old_bytes);
#pragma unroll
            for (int k = 0; k < NV; ++k) b.ov[k] = bload16_stream(ro, off[k]);
        }
        if constexpr (KIND == kBwdMul || KIND == kBwdColSum)
            b.r = 1.0f;
        else
            b.r = bload_f32(make_rsrc(inv_rms + r0, n * 4u), roff);
    }
};

// g = dy*gamma for kBwdRmsMul: rounded to storage and kept out of any fused
// multiply-add, as the separate multiply's VJP stores it.
template <class S>
__device__ __forceinline__ void stored_product(float (&f)[S::kVec], const float (&gm)[S::kVec],
                                               u32x4& q) {
    constexpr int W = S::kVec;
#pragma unroll
    for (int e = 0; e < W; ++e) f[e] = f[e] * gm[e];
    q = S::pack(f);
    S::unpack(q, f);
#pragma unroll
    for (int e = 0; e < W; ++e) asm("" : "+v"(f[e]));
}

template <class S, int TPR, int NV, int G, bool ACC, int KIND>
__device__ __forceinline__ void bwd_process(const BwdCtx<S, TPR, NV, G, ACC, KIND>& c,
                                            BwdSet<S, NV, ACC>& b,
                                            int64_t step, int parity, const u32x4 (&gv)[NV],
                                            bool has_gamma, float (&dg)[NV][S::kVec],
                                            float (*red)[TPR > 64 ? G * (TPR / 64) : 1]) {
    constexpr int W = S::kVec;
    const float r = b.r;
    float s = 0.0f;
    constexpr bool MUL = KIND == kBwdMul;
    constexpr bool COMP = KIND == kBwdRmsMul;
    if constexpr (KIND == kBwdColSum) {
        (void)c;
        (void)step;
        (void)parity;
        (void)red;
        (void)gv;
        (void)has_gamma;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fd[W];
            S::unpack(b.dv[k], fd);
#pragma unroll
            for (int e = 0; e < W; ++e) dg[k][e] += fd[e];
        }
        return;
    }
    if constexpr (!MUL) {
        float part[W];
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fx[W], fd[W];
            S::unpack(b.xv[k], fx);
            S::unpack(b.dv[k], fd);
            if constexpr (COMP) {
                float gm[W];
                u32x4 q;
                S::unpack(gv[k], gm);
                stored_product<S>(fd, gm, q);
            } else if (has_gamma) {
                float gm[W];
                S::unpack(gv[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) fd[e] = fd[e] * gm[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] += fd[e] * fx[e];
        }
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < W; ++e) dot += part[e];
        dot = row_sum<TPR, G>(dot, red, parity);
        s = (r * r * dot) * c.inv_cols;
        // Re-derive the unpacked values from the raw slots after the reduction
        // instead of keeping both copies live across it.
#pragma unroll
        for (int k = 0; k < NV; ++k) opaque(b.xv[k], b.dv[k]);
    } else {
        (void)parity;
        (void)red;
    }

    int64_t r0;
    uint32_t n;
    c.wave_rows(step, r0, n);
    const rsrc_t rdx = make_rsrc(c.dx ? c.dx + r0 * static_cast<int64_t>(c.cols) : c.dx,
                                 n * c.dx_bytes);
    const rsrc_t rdr = make_rsrc(c.dr ? c.dr + r0 * static_cast<int64_t>(c.cols) : c.dr,
                                 n * c.dr_bytes);  // used by kBwdRmsMul only
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float fx[W], fd[W], gk[W], o[W];
        S::unpack(b.xv[k], fx);
        S::unpack(b.dv[k], fd);
        if constexpr (COMP) {
            float gm[W];
            u32x4 q;
            S::unpack(gv[k], gm);
#pragma unroll
            for (int e = 0; e < W; ++e) gk[e] = fd[e];
            stored_product<S>(gk, gm, q);
            bstore16_stream(rdr, c.off[k], q);
        } else if (has_gamma) {
            float gm[W];
            S::unpack(gv[k], gm);
#pragma unroll
            for (int e = 0; e < W; ++e) gk[e] = fd[e] * gm[e];
        } else {
#pragma unroll
            for (int e = 0; e < W; ++e) gk[e] = fd[e];
        }
        if constexpr (MUL) {
#pragma unroll
            for (int e = 0; e < W; ++e) o[e] = gk[e];
        } else {
#pragma unroll
            for (int e = 0; e < W; ++e) o[e] = r * (gk[e] - fx[e] * s);
        }
        if constexpr (ACC) {
            float old[W];
            S::unpack(b.ov[k], old);
#pragma unroll
            for (int e = 0; e < W; ++e) o[e] = acc_add(old[e], o[e]);
        }
        bstore16_stream(rdx, c.off[k], S::pack(o));
        if constexpr (MUL) {
#pragma unroll
            for (int e = 0; e < W; ++e) dg[k][e] += fd[e] * fx[e];
        } else if constexpr (COMP) {
            float h[W];
#pragma unroll
            for (int e = 0; e < W; ++e) h[e] = fx[e] * r;
            S::unpack(S::pack(h), h);
#pragma unroll
            for (int e = 0; e < W; ++e) dg[k][e] += fd[e] * h[e];
        } else {
#pragma unroll
            for (int e = 0; e < W; ++e) dg[k][e] += fd[e] * (fx[e] * r);
        }
    }
}

// Runs steps 0 .. steps-1 of c's row sequence with NSET (1, 2 or 3) register
// sets, adding each lane's dgamma terms into dg.
template <class S, int TPR, int NV, int G, int NSET, bool ACC, int KIND>
__device__ __forceinline__ void bwd_segment(const BwdCtx<S, TPR, NV, G, ACC, KIND>& c, int64_t steps,
                                            const u32x4 (&gv)[NV], bool has_gamma,
                                            float (&dg)[NV][S::kVec],
                                            float (*red)[TPR > 64 ? G * (TPR / 64) : 1]) {
    if constexpr (NSET == 1) {
        BwdSet<S, NV, ACC> A;
        for (int64_t s = 0; s < steps; ++s) {
            c.issue(A, s);
            bwd_process(c, A, s, static_cast<int>(s & 1), gv, has_gamma, dg, red);
        }
    } else if constexpr (NSET == 2) {
        BwdSet<S, NV, ACC> A, B;
        c.issue(A, 0);
        c.issue(B, 1);
        bwd_process(c, A, 0, 0, gv, has_gamma, dg, red);
        c.issue(A, 2);
        bwd_process(c, B, 1, 1, gv, has_gamma, dg, red);
        c.issue(B, 3);
        for (int64_t s = 2; s < steps; s += 2) {  // steps is uniform
            bwd_process(c, A, s, 0, gv, has_gamma, dg, red);
            c.issue(A, s + 2);
            bwd_process(c, B, s + 1, 1, gv, has_gamma, dg, red);
            c.issue(B, s + 3);
        }
    } else {
        // Three sets: the parity of the LDS reduction row still alternates
        // step by step, so it is taken from the step, not from the set.
        static_assert(NSET == 3, "one, two or three register sets");
        BwdSet<S, NV, ACC> A, B, C;
        c.issue(A, 0);
        c.issue(B, 1);
        c.issue(C, 2);
        bwd_process(c, A, 0, 0, gv, has_gamma, dg, red);
        c.issue(A, 3);
        bwd_process(c, B, 1, 1, gv, has_gamma, dg, red);
        c.issue(B, 4);
        bwd_process(c, C, 2, 0, gv, has_gamma, dg, red);
        c.issue(C, 5);
        for (int64_t s = 3; s < steps; s += 3) {  // steps is uniform
            const int par = static_cast<int>(s & 1);
            bwd_process(c, A, s, par, gv, has_gamma, dg, red);
            c.issue(A, s + 3);
            bwd_process(c, B, s + 1, par ^ 1, gv, has_gamma, dg, red);
            c.issue(B, s + 4);
            bwd_process(c, C, s + 2, par, gv, has_gamma, dg, red);
            c.issue(C, s + 5);
        }
    }
}

// Writes one partial row of dgamma: the G groups' sums (each group's in its
// own LDS row) added in group order, column by column.  Ends with a barrier
// so the LDS rows can be written again.
template <class S, int TPR, int NV, int G>
__device__ __forceinline__ void bwd_write_partial(float* __restrict__ prow, int cols, int t,
                                                  int grp, const float (&dg)[NV][S::kVec],
                                                  float* lds_part) {
    constexpr int W = S::kVec;
    if constexpr (G == 1) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            if (col < cols) {
#pragma unroll
                for (int e = 0; e < W; ++e) prow[col + e] = dg[k][e];
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            if (col < cols) {
#pragma unroll
                for (int e = 0; e < W; ++e) lds_part[grp * cols + col + e] = dg[k][e];
            }
        }
        __syncthreads();
        for (int c2 = threadIdx.x; c2 < cols; c2 += TPR * G) {
            float v = lds_part[c2];
            for (int q = 1; q < G; ++q) v += lds_part[q * cols + c2];
            prow[c2] = v;
        }
        __syncthreads();
    }
}

// The skeleton's per-lane context for workgroup blk of a grid of nblk row
// workgroups (group q of workgroup blk takes rows blk*G + q + k*nblk*G), and
// the lane's slots of gamma.
template <class S, int TPR, int NV, int G, bool ACC, int KIND>
__device__ __forceinline__ void bwd_setup(BwdCtx<S, TPR, NV, G, ACC, KIND>& c, u32x4 (&gv)[NV],
                                          const typename S::T* x, const typename S::T* gamma,
                                          const float* inv_rms, const typename S::T* dy,
                                          typename S::T* dx, typename S::T* dr, int64_t rows,
                                          int cols, int64_t blk, int64_t nblk) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int RPW = TPR >= 64 ? 1 : 64 / TPR;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int t = threadIdx.x % TPR;
    const int sub = TPR >= 64 ? 0 : lane / TPR;  // the lane's row among the wave's rows
    c.x = x;
    c.gamma = gamma;
    c.inv_rms = inv_rms;
    c.dy = dy;
    c.dx = dx;
    c.dr = dr;
    c.rows = rows;
    c.first = blk * G;
    c.stride = nblk * G;
    c.cols = cols;
    c.wgrp0 = TPR >= 64 ? wave / (TPR / 64) : wave * RPW;
    c.row_bytes = static_cast<uint32_t>(cols) * static_cast<uint32_t>(sizeof(T));
    c.x_bytes = x ? c.row_bytes : 0u;
    c.old_bytes = dx ? c.row_bytes : 0u;
    c.dx_bytes = dx ? c.row_bytes : 0u;
    c.dr_bytes = dr ? c.row_bytes : 0u;
    c.roff = static_cast<uint32_t>(sub) * 4u;
    c.inv_cols = 1.0f / static_cast<float>(cols);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = (t + k * TPR) * W;
        c.off[k] = col < cols ? (static_cast<uint32_t>(sub) * static_cast<uint32_t>(cols) +
                                 static_cast<uint32_t>(col)) * static_cast<uint32_t>(sizeof(T))
                              : kOffOut;
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = (t + k * TPR) * W;
        gv[k] = (gamma != nullptr && col < cols) ? load16<S>(gamma + col) : u32x4{0u, 0u, 0u, 0u};
    }
}

// Rows are dealt round-robin to the gridDim.x workgroups; workgroup b writes
// partial row b.
template <class S, int TPR, int NV, int G, int NSET, bool ACC, int KIND>
__device__ __forceinline__ void bwd_resident_body(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, typename S::T* __restrict__ dr, float* __restrict__ partials,
    int64_t rows, int cols, float (*red)[TPR > 64 ? G * (TPR / 64) : 1], float* lds_part) {
    constexpr int W = S::kVec;
    const int t = threadIdx.x % TPR;
    const int grp = threadIdx.x / TPR;

    BwdCtx<S, TPR, NV, G, ACC, KIND> c;
    u32x4 gv[NV];
    bwd_setup(c, gv, x, gamma, inv_rms, dy, dx, dr, rows, cols, blockIdx.x, gridDim.x);
    const bool has_gamma = gamma != nullptr;
    float dg[NV][W];
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < W; ++e) dg[k][e] = 0.0f;

    const int64_t steps = c.first < rows ? (rows - c.first + c.stride - 1) / c.stride : 0;
    bwd_segment<S, TPR, NV, G, NSET, ACC, KIND>(c, steps, gv, has_gamma, dg, red);
    if (partials)
        bwd_write_partial<S, TPR, NV, G>(partials + static_cast<int64_t>(blockIdx.x) * cols, cols,
                                         t, grp, dg, lds_part);
}

// RMSNorm backward: dx (+)= r*(dy*gamma - x*r*r*dot/cols), dgamma partials.
template <class S, int TPR, int NV, int G, int NSET, bool ACC>
__global__ __launch_bounds__(TPR * G) void rms_bwd_resident(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, float* __restrict__ partials, int64_t rows, int cols) {
    __shared__ float red[2][TPR > 64 ? G * (TPR / 64) : 1];
    extern __shared__ float lds_part[];  // [G][cols] when G > 1 and partials
    bwd_resident_body<S, TPR, NV, G, NSET, ACC, kBwdRms>(x, gamma, inv_rms, dy, dx, nullptr,
                                                         partials, rows, cols, red, lds_part);
}

// The composition y = rms(x) * gamma (kBwdRmsMul): dr = gy*gamma, dx (+)=
// the RMSNorm VJP of dr, dgamma partials of gy*rms(x).  gamma is required.
template <class S, int TPR, int NV, int G, int NSET, bool ACC>
__global__ __launch_bounds__(TPR * G) void rms_mul_bwd_resident(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ gy,
    typename S::T* __restrict__ dx, typename S::T* __restrict__ dr, float* __restrict__ partials,
    int64_t rows, int cols) {
    __shared__ float red[2][TPR > 64 ? G * (TPR / 64) : 1];
    extern __shared__ float lds_part[];  // [G][cols] when G > 1 and partials
    bwd_resident_body<S, TPR, NV, G, NSET, ACC, kBwdRmsMul>(x, gamma, inv_rms, gy, dx, dr,
                                                            partials, rows, cols, red, lds_part);
}

// Broadcast multiply backward (vjp_Mul with reduce_for_broadcast): da (+)=
// gy*b, db partials of gy*a.  a, b, da may be null when not needed.
template <class S, int TPR, int NV, int G, int NSET, bool ACC>
__global__ __launch_bounds__(TPR * G) void mul_rowbcast_bwd_resident(
    const typename S::T* __restrict__ a, const typename S::T* __restrict__ b,
    const typename S::T* __restrict__ gy, typename S::T* __restrict__ da,
    float* __restrict__ partials, int64_t rows, int cols) {
    __shared__ float red[2][TPR > 64 ? G * (TPR / 64) : 1];
    extern __shared__ float lds_part[];  // [G][cols] when G > 1 and partials
    bwd_resident_body<S, TPR, NV, G, NSET, ACC, kBwdMul>(a, b, nullptr, gy, da, nullptr, partials,
                                                         rows, cols, red, lds_part);
}

// Column sums (kBwdColSum): partial rows of sum_rows x, as the backward's dgamma.
template <class S, int TPR, int NV, int G, int NSET>
__global__ __launch_bounds__(TPR * G) void sum_rows_resident(const typename S::T* __restrict__ x,
                                                             float* __restrict__ partials,
                                                             int64_t rows, int cols) {
    __shared__ float red[2][TPR > 64 ? G * (TPR / 64) : 1];
    extern __shared__ float lds_part[];  // [G][cols] when G > 1
    bwd_resident_body<S, TPR, NV, G, NSET, false, kBwdColSum>(nullptr, nullptr, nullptr, x,
                                                              nullptr, nullptr, partials, rows,
                                                              cols, red, lds_part);
}

// ---- few rows: row workgroups beside column workgroups -------------------------
// With fewer rows than the resident backward has workgroups (kBwdBlocks), most
// CUs would sit idle and the dgamma partial rows plus their finalize launch
// would cost as much as the rows themselves.  Here one launch runs two kinds
// of workgroup side by side:
//  - row workgroups [0, nrow_blocks): one step of the resident skeleton over
//    G rows (dx, and dr for the composition; the same arithmetic as the
//    resident kernel, so dx is bit-identical to it);
//  - column workgroups: 64 slots of columns each (kFewQuads lanes x kVec
//    columns), split over kFewGroups row groups of one wave.  Row group q sums
//    rows q, q + kFewGroups, ... in increasing order in fp64; the groups' sums
//    are then added in group order and written to dgamma directly.  dgamma
//    needs no row dot product, so these workgroups do not wait for the rows.
// No partial rows, no finalize launch, no atomics; the summation order
// depends only on rows.  The column term per KIND is the one the resident
// kernel adds: dy*(x*r), dy*stored(x*r) (composition), gy*a (broadcast
// multiply) or dy (column sums).
constexpr int64_t kFewRowsMax = 255;  // rows below the resident backward's kBwdBlocks
constexpr int kFewQuads = 64;         // column slots per column workgroup
constexpr int kFewGroups = 16;        // row groups of a 1024-lane column workgroup
constexpr int kFewBatch = 8;          // rows per group loaded before they are added

template <class S, int TPR, int NV, int G, bool ACC, int KIND>
__global__ __launch_bounds__(TPR * G) void bwd_fewrows(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, typename S::T* __restrict__ dr, float* __restrict__ dgamma,
    int64_t rows, int cols, int64_t nrow_blocks, int acc_dg) {
    static_assert(TPR * G == kFewGroups * 64, "column workgroups are 16 waves");
    using T = typename S::T;
    constexpr int W = S::kVec;
    __shared__ float red[2][TPR > 64 ? G * (TPR / 64) : 1];
    __shared__ double cred[kFewGroups][kFewQuads * 4];
    if (static_cast<int64_t>(blockIdx.x) < nrow_blocks) {  // workgroup-uniform
        BwdCtx<S, TPR, NV, G, ACC, KIND> c;
        u32x4 gv[NV];
        bwd_setup(c, gv, x, gamma, inv_rms, dy, dx, dr, rows, cols, blockIdx.x, nrow_blocks);
        float dg[NV][W];  // unused: dgamma comes from the column workgroups
#pragma unroll
        for (int k = 0; k < NV; ++k)
#pragma unroll
            for (int e = 0; e < W; ++e) dg[k][e] = 0.0f;
        BwdSet<S, NV, ACC> A;
        c.issue(A, 0);
        bwd_process(c, A, 0, 0, gv, gamma != nullptr, dg, red);
        return;
    }
    // column workgroup
    const int lane = threadIdx.x & 63;
    const int grp = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t cb = static_cast<int64_t>(blockIdx.x) - nrow_blocks;
    const int col = static_cast<int>((cb * kFewQuads + lane) * W);
    const uint32_t off = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    double acc[W];
#pragma unroll
    for (int e = 0; e < W; ++e) acc[e] = 0.0;
    for (int64_t r0 = grp; r0 < rows; r0 += static_cast<int64_t>(kFewGroups) * kFewBatch) {
        u32x4 xv[kFewBatch], dv[kFewBatch];
        float rr[kFewBatch];
#pragma unroll
        for (int u = 0; u < kFewBatch; ++u) {
            // The wave's row of this batch entry: a resource of zero bytes past
            // the last row, so its loads return zeros and its terms add +0.0.
            const int64_t row = r0 + static_cast<int64_t>(u) * kFewGroups;
            const uint32_t n = row < rows ? 1u : 0u;
            const int64_t e0 = (row < rows ? row : 0) * static_cast<int64_t>(cols);
            dv[u] = bload16_stream(make_rsrc(dy + e0, n * row_bytes), off);
            if constexpr (KIND != kBwdColSum)
                xv[u] = bload16_stream(make_rsrc(x + e0, n * row_bytes), off);
            if constexpr (KIND == kBwdRms || KIND == kBwdRmsMul)
                rr[u] = bload_f32(make_rsrc(inv_rms + (row < rows ? row : 0), n * 4u), 0);
        }
#pragma unroll
        for (int u = 0; u < kFewBatch; ++u) {
            float fd[W];
            S::unpack(dv[u], fd);
            float term[W];
            if constexpr (KIND == kBwdColSum) {
#pragma unroll
                for (int e = 0; e < W; ++e) term[e] = fd[e];
            } else {
                float fx[W];
                S::unpack(xv[u], fx);
                if constexpr (KIND == kBwdMul) {
#pragma unroll
                    for (int e = 0; e < W; ++e) term[e] = fd[e] * fx[e];
                } else if constexpr (KIND == kBwdRmsMul) {
                    float h[W];
#pragma unroll
                    for (int e = 0; e < W; ++e) h[e] = fx[e] * rr[u];
                    S::unpack(S::pack(h), h);
#pragma unroll
                    for (int e = 0; e < W; ++e) term[e] = fd[e] * h[e];
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) term[e] = fd[e] * (fx[e] * rr[u]);
                }
            }
#pragma unroll
            for (int e = 0; e < W; ++e) acc[e] += static_cast<double>(term[e]);
        }
    }
    // Groups' sums in group order, 4 columns per lane at a time (bf16 lanes
    // hold 8 columns: two rounds).
#pragma unroll
    for (int h = 0; h < W; h += 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) cred[grp][lane * 4 + i] = acc[h + i];
        __syncthreads();
        if (threadIdx.x < kFewQuads * 4) {
            const int l = static_cast<int>(threadIdx.x) >> 2, i = static_cast<int>(threadIdx.x) & 3;
            double tot = cred[0][threadIdx.x];
#pragma unroll
            for (int q = 1; q < kFewGroups; ++q) tot += cred[q][threadIdx.x];
            const int64_t c = (cb * kFewQuads + l) * W + h + i;
            if (c < cols) {
                const float v = static_cast<float>(tot);
                dgamma[c] = acc_dg ? dgamma[c] + v : v;
            }
        }
        __syncthreads();
    }
}

// ---- looped kernels (any alignment, any width) --------------------------------
// One workgroup per row (forward) or per row block (backward); element-wise
// accesses; the row is read twice (second read normally hits L2).  In the
// backward, lane c % kBlock exclusively owns column c of this block's partial
// row, so the per-row read-modify-write of the partial row needs no atomics.
template <class S>
__global__ __launch_bounds__(kBlock) void rms_fwd_looped(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    typename S::T* __restrict__ y, float* __restrict__ inv_rms, int64_t rows, int cols,
    float eps) {
    __shared__ float red[2][kBlock / 64];
    const int64_t row = blockIdx.x;
    if (row >= rows) return;  // block-uniform
    const int64_t off = row * static_cast<int64_t>(cols);
    float ss = 0.0f;
    for (int c = threadIdx.x; c < cols; c += kBlock) {
        const float v = S::get(x + off + c);
        ss += v * v;
    }
    ss = row_sum<kBlock, 1>(ss, red, 0);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    if (threadIdx.x == 0) inv_rms[row] = r;
    for (int c = threadIdx.x; c < cols; c += kBlock) {
        float v = S::get(x + off + c) * r;
        if (gamma) v = v * S::get(gamma + c);
        S::put(y + off + c, v);
    }
}

// With dr (the composition y = rms(x) * gamma, gamma required): g = dy*gamma
// rounded to storage is written to dr, and the dgamma term is dy*h with
// h = x*r rounded to storage, as the separate multiply's VJP computes them.
template <class S>
__global__ __launch_bounds__(kBlock) void rms_bwd_looped(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, typename S::T* __restrict__ dr, float* __restrict__ partials,
    int64_t rows, int cols, int64_t rpb, int acc_dx) {
    __shared__ float red[2][kBlock / 64];
    const int64_t row_begin = static_cast<int64_t>(blockIdx.x) * rpb;
    const int64_t row_end = row_begin + rpb < rows ? row_begin + rpb : rows;
    const float inv_cols = 1.0f / static_cast<float>(cols);
    float* prow = partials ? partials + static_cast<int64_t>(blockIdx.x) * cols : nullptr;
    int parity = 0;
    for (int64_t row = row_begin; row < row_end; ++row, parity ^= 1) {
        const int64_t off = row * static_cast<int64_t>(cols);
        const float r = inv_rms[row];
        float s = 0.0f;
        if (dx) {  // block-uniform
            float dot = 0.0f;
            for (int c = threadIdx.x; c < cols; c += kBlock) {
                float g = S::get(dy + off + c);
                if (gamma) g = g * S::get(gamma + c);
                if (dr) g = S::stored(g);
                dot += g * S::get(x + off + c);
            }
            dot = row_sum<kBlock, 1>(dot, red, parity);
            s = (r * r * dot) * inv_cols;
        }
        const bool first = row == row_begin;
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            const float xv = S::get(x + off + c);
            const float d = S::get(dy + off + c);
            float g = gamma ? d * S::get(gamma + c) : d;
            if (dr) {
                g = S::stored(g);
                S::put(dr + off + c, g);
            }
            if (dx) {
                float o = r * (g - xv * s);
                if (acc_dx) o = acc_add(S::get(dx + off + c), o);
                S::put(dx + off + c, o);
            }
            if (prow) {
                const float t = d * (dr ? S::stored(xv * r) : xv * r);
                prow[c] = first ? t : acc_add(prow[c], t);
            }
        }
    }
}

// ---- broadcast multiply (unfused ag::rms(x) * gamma) -------------------------
// Both looped kernels split a row into column chunks of `chunk` elements
// (blockIdx.y), so that few long rows (an equal-shape product is one row of
// numel columns) still spread over many workgroups.  chunk is a multiple of
// kBlock * kVec.
__host__ __device__ inline int64_t chunk_end(int64_t c0, int64_t chunk, int cols) {
    return c0 + chunk < cols ? c0 + chunk : cols;
}

// Column chunk for rows x cols: about kChunkBlocks workgroups in all, at most
// 65535 chunks per row, a multiple of kBlock * vec elements.
inline int64_t mul_chunk(int64_t rows_or_blocks, int cols, int vec) {
    constexpr int64_t kChunkBlocks = 4096;
    const int64_t step = static_cast<int64_t>(kBlock) * vec;
    const int64_t per_row =
        rows_or_blocks >= kChunkBlocks ? 1 : (kChunkBlocks + rows_or_blocks - 1) / rows_or_blocks;
    int64_t chunk = (cols + per_row - 1) / per_row;
    const int64_t min_chunk = (cols + 65534) / 65535;
    if (chunk < min_chunk) chunk = min_chunk;
    return (chunk + step - 1) / step * step;
}

template <class S>
__global__ __launch_bounds__(kBlock) void mul_rowbcast_fwd_kernel(
    const typename S::T* __restrict__ a, const typename S::T* __restrict__ b,
    typename S::T* __restrict__ y, int64_t rows, int cols, int vec, int64_t chunk) {
    // vec: 1 when a/b/y are 16-byte aligned and cols % kVec == 0.
    constexpr int W = S::kVec;
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const int64_t off = row * static_cast<int64_t>(cols);
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * chunk;
    const int64_t c1 = chunk_end(c0, chunk, cols);
    if (vec) {
        for (int64_t c = c0 + threadIdx.x * W; c < c1; c += kBlock * W) {
            float fa[W], fb[W];
            S::unpack(load16_stream<S>(a + off + c), fa);
            S::unpack(load16<S>(b + c), fb);
#pragma unroll
            for (int e = 0; e < W; ++e) fa[e] = fa[e] * fb[e];
            store16_stream<S>(y + off + c, S::pack(fa));
        }
    } else {
        for (int64_t c = c0 + threadIdx.x; c < c1; c += kBlock)
            S::put(y + off + c, S::get(a + off + c) * S::get(b + c));
    }
}

// da (+)= gy*b; partial row of this row block (+)= gy*a for the block's
// column chunk (owned-column RMW: the chunks are disjoint, and within one the
// lane (c - c0) % kBlock owns column c).  Each column still sums the block's
// rows in row order, whatever the chunking.
// vec: every pointer 16-byte aligned and cols % kVec == 0 (chunk is then a
// multiple of kBlock * kVec): each lane takes kVec consecutive columns, with
// the same arithmetic per element and the same order per column.
template <class S>
__global__ __launch_bounds__(kBlock) void mul_rowbcast_bwd_kernel(
    const typename S::T* __restrict__ gy, const typename S::T* __restrict__ a,
    const typename S::T* __restrict__ b, typename S::T* __restrict__ da,
    float* __restrict__ partials, int64_t rows, int cols, int64_t rpb, int acc_da,
    int64_t chunk, int vec) {
    constexpr int W = S::kVec;
    const int64_t row_begin = static_cast<int64_t>(blockIdx.x) * rpb;
    const int64_t row_end = row_begin + rpb < rows ? row_begin + rpb : rows;
    float* prow = partials ? partials + static_cast<int64_t>(blockIdx.x) * cols : nullptr;
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * chunk;
    const int64_t c1 = chunk_end(c0, chunk, cols);
    if (vec) {
        for (int64_t row = row_begin; row < row_end; ++row) {
            const int64_t off = row * static_cast<int64_t>(cols);
            const bool first = row == row_begin;
            for (int64_t c = c0 + threadIdx.x * W; c < c1; c += kBlock * W) {
                float g[W];
                S::unpack(load16_stream<S>(gy + off + c), g);
                if (da) {
                    float bb[W], o[W];
                    S::unpack(load16<S>(b + c), bb);
#pragma unroll
                    for (int e = 0; e < W; ++e) o[e] = g[e] * bb[e];
                    if (acc_da) {
                        float old[W];
                        S::unpack(load16_stream<S>(da + off + c), old);
#pragma unroll
                        for (int e = 0; e < W; ++e) o[e] = acc_add(old[e], o[e]);
                    }
                    store16_stream<S>(da + off + c, S::pack(o));
                }
                if (prow) {
                    float t[W];
                    if (a) {
                        float aa[W];
                        S::unpack(load16_stream<S>(a + off + c), aa);
#pragma unroll
                        for (int e = 0; e < W; ++e) t[e] = g[e] * aa[e];
                    } else {
#pragma unroll
                        for (int e = 0; e < W; ++e) t[e] = g[e];
                    }
#pragma unroll
                    for (int e = 0; e < W; ++e) prow[c + e] = first ? t[e] : acc_add(prow[c + e], t[e]);
                }
            }
        }
        return;
    }
    for (int64_t row = row_begin; row < row_end; ++row) {
        const int64_t off = row * static_cast<int64_t>(cols);
        const bool first = row == row_begin;
        for (int64_t c = c0 + threadIdx.x; c < c1; c += kBlock) {
            const float g = S::get(gy + off + c);
            if (da) {
                float o = g * S::get(b + c);
                if (acc_da) o = acc_add(S::get(da + off + c), o);
                S::put(da + off + c, o);
            }
            if (prow) {  // a == nullptr: column sums of gy
                const float t = a ? g * S::get(a + off + c) : g;
                prow[c] = first ? t : acc_add(prow[c], t);
            }
        }
    }
}

// ---- dgamma: fixed-order column sum of the partial rows ------------------------
// Workgroup: kFinCols columns x kFinSplits row splits.  Split s sums partial
// rows s, s + kFinSplits, ... in increasing order in fp64; the split sums are
// then added in split order.  The order depends only on nblk, never on timing
// or on the path taken.  Each lane loads kFinBatch partial rows before it adds
// any of them: the partials were just written by other XCDs' workgroups, so
// every load misses this XCD's L2, and at the resident backward's 256 partial
// rows one round trip covers all of them.  Narrow column chunks give one
// workgroup per 32 columns (128 at 4096 columns), so the partials stream in
// over half the CUs rather than a few of them, and each workgroup reads whole
// 128-byte lines of every partial row: with 16 columns, two workgroups on
// different XCDs each fetched half of every line, doubling the bytes read and
// costing c2's finalize 0.8 us, 1.3 us at 5120 columns and 2.6 us at 11008.
// VEC: a lane sums 4 adjacent columns with 16-byte loads (cols % 4 == 0 and
// partials 16-byte aligned, so every partial row's quads are aligned);
// otherwise a lane sums one column with 4-byte loads (16 columns per
// workgroup, 1024 lanes).  Same order either way.
constexpr int kFinSplits = 64;
constexpr int kFinBatch = 4;
constexpr int fin_cols(bool vec) { return vec ? 32 : 16; }  // columns per workgroup

template <bool VEC>
__global__ __launch_bounds__((VEC ? fin_cols(VEC) / 4 : fin_cols(VEC)) * kFinSplits) void
dgamma_finalize(const float* __restrict__ partials, float* __restrict__ dgamma, int64_t nblk,
                int cols, int accumulate) {
    constexpr int kFinCols = fin_cols(VEC);
    constexpr int CPL = VEC ? 4 : 1;              // columns per lane
    constexpr int LANES = kFinCols / CPL;         // lanes per split
    __shared__ double red[kFinSplits][kFinCols];
    const int q = threadIdx.x % LANES;
    const int split = threadIdx.x / LANES;
    const int c0 = blockIdx.x * kFinCols + q * CPL;
    const bool in = c0 < cols;  // VEC: the whole quad is in (cols % 4 == 0)
    // Loads are unconditional (a row or column past the end reads the last
    // valid one instead) and the values are selected afterwards: loads behind
    // branches would each wait for all earlier loads to return.  A skipped
    // term adds +0.0, which leaves the sum unchanged (it starts at +0.0 and
    // round-to-nearest never makes it -0.0).
    const int cl = in ? c0 : cols - CPL;
    double acc[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) acc[i] = 0.0;
    for (int64_t base = split; base < nblk; base += static_cast<int64_t>(kFinSplits) * kFinBatch) {
        float v[kFinBatch][CPL];
#pragma unroll
        for (int u = 0; u < kFinBatch; ++u) {
            const int64_t b = base + static_cast<int64_t>(u) * kFinSplits;
            const float* p = partials + (b < nblk ? b : nblk - 1) * cols + cl;
            if constexpr (VEC) {
                const float4 t = *reinterpret_cast<const float4*>(p);
                v[u][0] = t.x;
                v[u][CPL > 1 ? 1 : 0] = t.y;
                v[u][CPL > 2 ? 2 : 0] = t.z;
                v[u][CPL > 3 ? 3 : 0] = t.w;
            } else {
                v[u][0] = *p;
            }
        }
#pragma unroll
        for (int u = 0; u < kFinBatch; ++u) {
            const bool take = in && base + static_cast<int64_t>(u) * kFinSplits < nblk;
#pragma unroll
            for (int i = 0; i < CPL; ++i) acc[i] += take ? v[u][i] : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) red[split][q * CPL + i] = acc[i];
    __syncthreads();
    if (threadIdx.x < kFinCols) {
        const int c = blockIdx.x * kFinCols + static_cast<int>(threadIdx.x);
        if (c < cols) {
            double tot = red[0][threadIdx.x];
#pragma unroll
            for (int s2 = 1; s2 < kFinSplits; ++s2) tot += red[s2][threadIdx.x];
            const float v = static_cast<float>(tot);
            dgamma[c] = accumulate ? dgamma[c] + v : v;
        }
    }
}

// dgamma from at most kFinSplits partial rows: one lane per column, the
// partial rows added in order in fp64 from +0.0, kFewFinBatch rows loaded
// before any is added.  With nblk <= kFinSplits every split of
// dgamma_finalize holds at most one row, so its sum is this sum bit for bit
// (its split sums are +0.0 + p_s, added in split order, and the empty splits
// add +0.0 to a sum that is never -0.0); this kernel spreads over the columns
// instead of launching a workgroup per 16 columns for a few rows.
constexpr int kFewFinBatch = 16;
__global__ __launch_bounds__(kBlock) void dgamma_finalize_few(
    const float* __restrict__ partials, float* __restrict__ dgamma, int64_t nblk, int cols,
    int accumulate) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= cols) return;
    double tot = 0.0;
    for (int64_t b0 = 0; b0 < nblk; b0 += kFewFinBatch) {
        float v[kFewFinBatch];
#pragma unroll
        for (int u = 0; u < kFewFinBatch; ++u) {
            const int64_t b = b0 + u < nblk ? b0 + u : nblk - 1;  // in range; dropped below
            v[u] = partials[b * cols + c];
        }
#pragma unroll
        for (int u = 0; u < kFewFinBatch; ++u)
            if (b0 + u < nblk) tot += v[u];
    }
    const float v = static_cast<float>(tot);
    dgamma[c] = accumulate ? dgamma[c] + v : v;
}

__global__ __launch_bounds__(kBlock) void fill_zero_f32(float* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}


// (TPR, NV, G, register sets).  Every shape is a 1024-lane workgroup (TPR * G =
// 1024).  Rows of up to 1024 slots take one slot per lane (TPR = the width
// rounded up to a power of two, G = 1024 / TPR rows per step); wider rows take
// 2 or 4 slots per lane on 1024 lanes.  Narrow rows (TPR <= 64) and the
// widest shape process one register set at a time; the others prefetch.
// Measured on MI355X (c2 f32 [65536, 4096], c3 bf16 [65536, 8192],
// c4a [7161, 5120], c4b [1048576, 128]) against 256- to 1024-lane and
// 1- to 4-slot alternatives, with and without prefetch.
#define AGK_BWD_SHAPES(X)                                                                  \
    X(1, 1, 1024, 1) X(2, 1, 512, 1) X(4, 1, 256, 1) X(8, 1, 128, 1) X(16, 1, 64, 1)       \
    X(32, 1, 32, 1) X(64, 1, 16, 1) X(128, 1, 8, 2) X(256, 1, 4, 2) X(512, 1, 2, 2)       \
    X(1024, 1, 1, 2) X(1024, 2, 1, 2) X(1024, 4, 1, 1)

// Backward shapes that are not built for a storage type: bf16 unpacks to
// twice the floats per slot, and the widest shape would spill registers.
template <class S>
constexpr bool bwd_shape_enabled(int tpr, int nv) {
    return !(std::is_same<S, BF16>::value && tpr == 1024 && nv == 4);
}
// Register sets of a shape for a storage type: bf16 with two slots per lane
// holds one (two would spill).
template <class S>
constexpr int bwd_sets(int nv, int sets) {
    return (std::is_same<S, BF16>::value && nv >= 2) ? 1 : sets;
}
// The composition's backward (kBwdRmsMul) does more arithmetic per slot than
// the others (two products rounded to storage, an extra store stream), so its
// one-slot shapes keep a third row's loads in flight while a row computes.
template <class S>
constexpr int rms_mul_sets(int nv, int sets) {
    return (nv == 1 && sets == 2) ? 3 : bwd_sets<S>(nv, sets);
}

template <class S>
inline Plan bwd_plan(int64_t nslot) {
    Plan p;
    if (nslot <= 1024) {
        p.tpr = pow2_at_least(nslot);
        p.nv = 1;
    } else if (nslot <= 2048) {
        p.tpr = 1024;
        p.nv = 2;
    } else if (nslot <= 4096) {
        p.tpr = 1024;
        p.nv = 4;
    } else {
        return Plan{};
    }
    p.g = 1024 / p.tpr;
    if (!bwd_shape_enabled<S>(p.tpr, p.nv)) return Plan{};
    return p;
}

// Row blocking of the resident backward: min(kBwdBlocks, rows) workgroups,
// about one per CU, so the whole grid runs in one generation and finishes
// together; workgroup b takes rows b*G + q + k*nblk*G (round-robin, so the
// grid streams through one band of rows at a time) and writes one partial
// row of dgamma.  A grid of more workgroups than fit at once finishes in a
// ragged last generation, measured 3-15 % slower at the configurations above.
// Depends only on rows, so the dgamma summation order is fixed by the shape.
constexpr int64_t kBwdBlocks = 256;
inline int64_t bwd_resident_blocks(int64_t rows) { return rows < kBwdBlocks ? rows : kBwdBlocks; }

// Row blocking of the looped backward (unaligned or too-wide rows): about
// kTargetBlocks workgroups, each summing a run of rpb consecutive rows into
// one partial row (at least kMinRowsPerBlockLarge rows once there are enough
// rows, so the partial rows stay a small fraction of the traffic).  Never
// fewer blocks than the resident blocking, so it also sizes the workspace.
inline int64_t bwd_rows_per_block(int64_t rows) {
    int64_t rpb = (rows + kTargetBlocks - 1) / kTargetBlocks;
    if (rows >= kLargeRows / 8 && rpb < kMinRowsPerBlockLarge) rpb = kMinRowsPerBlockLarge;
    return rpb < 1 ? 1 : rpb;
}
inline int64_t bwd_num_blocks(int64_t rows) {
    if (rows <= 0) return 0;
    const int64_t rpb = bwd_rows_per_block(rows);
    return (rows + rpb - 1) / rpb;
}

#include "rmsnorm_wide.hpp"

// Forward grids of at most this many workgroups (one per CU), over rows of at
// most kFwdEarlyGammaSlots 16-byte slots per row shape, load gamma with x.
constexpr int64_t kFwdEarlyGammaGrid = 256;
constexpr int64_t kFwdEarlyGammaSlots = 1024;

template <class S>
int launch_fwd_plan(const Plan& p, const void* x, const void* gamma, void* y, float* inv_rms,
                    int64_t rows, int cols, float eps, hipStream_t st) {
    using T = typename S::T;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    T* yp = static_cast<T*>(y);
    if (p.tpr == 0) {
        if (rows > 0x7fffffffLL) return AGK_EINVAL;
        hipLaunchKernelGGL(rms_fwd_looped<S>, dim3(static_cast<unsigned>(rows)), dim3(kBlock), 0,
                           st, xp, gp, yp, inv_rms, rows, cols, eps);
        return check_launch();
    }
    const int64_t grid = (rows + p.g - 1) / p.g;
    if (grid > 0x7fffffffLL) return AGK_EINVAL;
    // one generation of workgroups over short rows, with gamma: gamma loaded beside x
    const bool early_g = gp != nullptr && grid <= kFwdEarlyGammaGrid &&
                         static_cast<int64_t>(p.tpr) * p.nv <= kFwdEarlyGammaSlots;
#define AGK_X(a, b, c)                                                                       \
    if (p.tpr == a && p.nv == b && p.g == c) {                                               \
        if (early_g)                                                                          \
            hipLaunchKernelGGL((rms_fwd_resident<S, a, b, c, false, true>),                  \
                               dim3(static_cast<unsigned>(grid)), dim3(a * c), 0, st, xp, gp, \
                               yp, inv_rms, rows, cols, eps);                                \
        else                                                                                  \
            hipLaunchKernelGGL((rms_fwd_resident<S, a, b, c>), dim3(static_cast<unsigned>(grid)), \
                               dim3(a * c), 0, st, xp, gp, yp, inv_rms, rows, cols, eps);    \
        return check_launch();                                                               \
    }
    AGK_FWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

bool team_fwd_enabled();

// ws: the team forward's slots (nullptr: none), at least
// fwd_team_ws_bytes(rows, cols) bytes and 8-byte aligned (checked by the caller).
template <class S>
int launch_fwd(const void* x, const void* gamma, void* y, float* inv_rms, int64_t rows,
               int cols, float eps, void* ws, hipStream_t st) {
    const bool vec = (cols % S::kVec) == 0 && aligned16(x) && aligned16(y) &&
                     (gamma == nullptr || aligned16(gamma));
    Plan p;
    if (vec) p = fwd_plan(cols / S::kVec, rows);
    if (wide_fwd_eligible<S>(x, gamma, y, rows, cols, p.tpr != 0)) {
        if (ws && team_fwd_enabled() && fwd_team_shape_ok(rows, cols))
            return launch_wide_team_fwd<S>(x, gamma, y, inv_rms, ws, rows, cols, eps, st);
        return launch_wide_fwd<S>(x, gamma, y, inv_rms, rows, cols, eps, st);
    }
    return launch_fwd_plan<S>(p, x, gamma, y, inv_rms, rows, cols, eps, st);
}

// y = a * b (b broadcast over rows): the forward's resident launch shape when
// rows are aligned and fit, else one workgroup per row.
template <class S>
int launch_mul_fwd(const void* a, const void* b, void* y, int64_t rows, int cols,
                   hipStream_t st) {
    using T = typename S::T;
    const T* ap = static_cast<const T*>(a);
    const T* bp = static_cast<const T*>(b);
    T* yp = static_cast<T*>(y);
    const bool vec = (cols % S::kVec) == 0 && aligned16(a) && aligned16(b) && aligned16(y);
    Plan p;
    if (vec) p = fwd_plan(cols / S::kVec, rows);
    if (p.tpr == 0) {
        if (rows > 0x7fffffffLL) return AGK_EINVAL;
        const int64_t chunk = mul_chunk(rows, cols, vec ? S::kVec : 1);
        const int64_t nchunk = (cols + chunk - 1) / chunk;
        hipLaunchKernelGGL(mul_rowbcast_fwd_kernel<S>,
                           dim3(static_cast<unsigned>(rows), static_cast<unsigned>(nchunk)),
                           dim3(kBlock), 0, st, ap, bp, yp, rows, cols, vec ? 1 : 0, chunk);
        return check_launch();
    }
    const int64_t grid = (rows + p.g - 1) / p.g;
    if (grid > 0x7fffffffLL) return AGK_EINVAL;
#define AGK_X(a_, b_, c_)                                                                 \
    if (p.tpr == a_ && p.nv == b_ && p.g == c_) {                                         \
        hipLaunchKernelGGL((rms_fwd_resident<S, a_, b_, c_, true>),                       \
                           dim3(static_cast<unsigned>(grid)), dim3(a_ * c_), 0, st, ap, bp, \
                           yp, nullptr, rows, cols, 0.0f);                                \
        return check_launch();                                                            \
    }
    AGK_FWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

template <class S, bool ACC>
int launch_bwd_resident(const Plan& p, int64_t nblk, const void* x, const void* gamma,
                        const float* inv_rms, const void* dy, void* dx, float* partials,
                        int64_t rows, int cols, hipStream_t st) {
    using T = typename S::T;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* dyp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    const size_t lds = (partials && p.g > 1) ? static_cast<size_t>(p.g) * cols * 4 : 0;
#define AGK_X(a, b, c, d)                                                                  \
    if constexpr (bwd_shape_enabled<S>(a, b)) {                                            \
        if (p.tpr == a && p.nv == b && p.g == c) {                                         \
            hipLaunchKernelGGL((rms_bwd_resident<S, a, b, c, bwd_sets<S>(b, d), ACC>),     \
                               dim3(static_cast<unsigned>(nblk)), dim3(a * c), lds, st, xp, \
                               gp, inv_rms, dyp, dxp, partials, rows, cols);                \
            return check_launch();                                                         \
        }                                                                                  \
    }
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

template <class S, bool ACC>
int launch_mul_bwd_resident(const Plan& p, int64_t nblk, const void* a, const void* b,
                            const void* gy, void* da, float* partials, int64_t rows, int cols,
                            hipStream_t st) {
    using T = typename S::T;
    const T* ap = static_cast<const T*>(a);
    const T* bp = static_cast<const T*>(b);
    const T* gp = static_cast<const T*>(gy);
    T* dap = static_cast<T*>(da);
    const size_t lds = (partials && p.g > 1) ? static_cast<size_t>(p.g) * cols * 4 : 0;
#define AGK_X(a_, b_, c_, d_)                                                              \
    if constexpr (bwd_shape_enabled<S>(a_, b_)) {                                          \
        if (p.tpr == a_ && p.nv == b_ && p.g == c_) {                                      \
            hipLaunchKernelGGL((mul_rowbcast_bwd_resident<S, a_, b_, c_,                   \
                                                          bwd_sets<S>(b_, d_), ACC>),      \
                               dim3(static_cast<unsigned>(nblk)), dim3(a_ * c_), lds, st,   \
                               ap, bp, gp, dap, partials, rows, cols);                     \
            return check_launch();                                                         \
        }                                                                                  \
    }
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

template <class S>
int launch_sum_rows_resident(const Plan& p, int64_t nblk, const void* x, float* partials,
                             int64_t rows, int cols, hipStream_t st) {
    using T = typename S::T;
    const T* xp = static_cast<const T*>(x);
    const size_t lds = p.g > 1 ? static_cast<size_t>(p.g) * cols * 4 : 0;
#define AGK_X(a_, b_, c_, d_)                                                              \
    if constexpr (bwd_shape_enabled<S>(a_, b_)) {                                          \
        if (p.tpr == a_ && p.nv == b_ && p.g == c_) {                                      \
            hipLaunchKernelGGL((sum_rows_resident<S, a_, b_, c_, bwd_sets<S>(b_, d_)>),    \
                               dim3(static_cast<unsigned>(nblk)), dim3(a_ * c_), lds, st,   \
                               xp, partials, rows, cols);                                  \
            return check_launch();                                                         \
        }                                                                                  \
    }
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

// The shape and row blocking a backward call of these sizes takes; nblk is
// the number of dgamma partial rows it writes.
template <class S>
inline Plan bwd_plan_for(const void* x, const void* gamma, const void* dy, const void* dx,
                         int64_t rows, int cols, int64_t& nblk, int64_t& rpb) {
    const bool vec = (cols % S::kVec) == 0 && aligned16(x) && aligned16(dy) &&
                     (dx == nullptr || aligned16(dx)) && (gamma == nullptr || aligned16(gamma));
    Plan p;
    if (vec) p = bwd_plan<S>(cols / S::kVec);
    // the per-group partial rows must fit in LDS
    if (p.tpr != 0 && p.g > 1 && static_cast<int64_t>(p.g) * cols * 4 > 64 * 1024) p = Plan{};
    if (p.tpr != 0) {
        nblk = bwd_resident_blocks(rows);
        rpb = (rows + nblk - 1) / nblk;
    } else {
        rpb = bwd_rows_per_block(rows);
        nblk = bwd_num_blocks(rows);
    }
    return p;
}

template <class S, bool ACC>
int launch_rms_mul_bwd_resident(const Plan& p, int64_t nblk, const void* x, const void* gamma,
                                const float* inv_rms, const void* gy, void* dx, void* dr,
                                float* partials, int64_t rows, int cols, hipStream_t st) {
    using T = typename S::T;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* gyp = static_cast<const T*>(gy);
    T* dxp = static_cast<T*>(dx);
    T* drp = static_cast<T*>(dr);
    const size_t lds = (partials && p.g > 1) ? static_cast<size_t>(p.g) * cols * 4 : 0;
#define AGK_X(a, b, c, d)                                                                  \
    if constexpr (bwd_shape_enabled<S>(a, b)) {                                            \
        if (p.tpr == a && p.nv == b && p.g == c) {                                         \
            hipLaunchKernelGGL((rms_mul_bwd_resident<S, a, b, c, rms_mul_sets<S>(b, d),    \
                                                     ACC>),                                \
                               dim3(static_cast<unsigned>(nblk)), dim3(a * c), lds, st, xp, \
                               gp, inv_rms, gyp, dxp, drp, partials, rows, cols);           \
            return check_launch();                                                         \
        }                                                                                  \
    }
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

// The few-rows backward (bwd_fewrows) of KIND for a resident plan p with
// rows <= kFewRowsMax: row workgroups when dx or dr is wanted, column
// workgroups when dgamma is; dgamma is written (or added into, acc_dg)
// directly.
template <class S, int KIND>
int launch_fewrows(const Plan& p, const void* x, const void* gamma, const float* inv_rms,
                   const void* dy, void* dx, void* dr, float* dgamma, int64_t rows, int cols,
                   int acc_dx, int acc_dg, hipStream_t st) {
    using T = typename S::T;
    const int64_t nrow_blocks = (dx != nullptr || dr != nullptr) ? (rows + p.g - 1) / p.g : 0;
    const int64_t ncol_blocks =
        dgamma != nullptr ? (cols / S::kVec + kFewQuads - 1) / kFewQuads : 0;
    const int64_t grid = nrow_blocks + ncol_blocks;
    if (grid == 0) return AGK_OK;
    if (grid > 0x7fffffffLL) return AGK_EINVAL;
    const bool acc = acc_dx && dx != nullptr;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* dyp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    T* drp = static_cast<T*>(dr);
#define AGK_X(a, b, c, d)                                                                   \
    if constexpr (bwd_shape_enabled<S>(a, b)) {                                             \
        if (p.tpr == a && p.nv == b && p.g == c) {                                          \
            if constexpr (KIND != kBwdColSum) {                                             \
                if (acc) {                                                                  \
                    hipLaunchKernelGGL((bwd_fewrows<S, a, b, c, true, KIND>),               \
                                       dim3(static_cast<unsigned>(grid)), dim3(a * c), 0, st, \
                                       xp, gp, inv_rms, dyp, dxp, drp, dgamma, rows, cols,  \
                                       nrow_blocks, acc_dg);                                \
                    return check_launch();                                                  \
                }                                                                           \
            }                                                                               \
            hipLaunchKernelGGL((bwd_fewrows<S, a, b, c, false, KIND>),                      \
                               dim3(static_cast<unsigned>(grid)), dim3(a * c), 0, st, xp, gp, \
                               inv_rms, dyp, dxp, drp, dgamma, rows, cols, nrow_blocks,     \
                               acc_dg);                                                     \
            return check_launch();                                                          \
        }                                                                                   \
    }
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

// dr == nullptr: the RMSNorm VJP (gamma optional); dr != nullptr: the
// composition rms(x) * gamma (gamma required), dr receiving gy*gamma.
// Rows that fit the resident shapes but are fewer than kFewRowsMax take the
// few-rows kernel, which writes dgamma itself: nblk is then 0 (no partial
// rows to finalize).  Otherwise nblk is the number of dgamma partial rows
// written to `partials`.
template <class S>
int launch_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
               void* dx, void* dr, float* partials, float* dgamma, int64_t rows, int cols,
               int accumulate, int acc_dg, hipStream_t st, int64_t& nblk) {
    using T = typename S::T;
    int64_t rpb = 0;
    Plan p = bwd_plan_for<S>(x, gamma, dy, dx, rows, cols, nblk, rpb);
    if (dr && p.tpr != 0 && !aligned16(dr)) {  // the looped kernel, with its own row blocking
        p = Plan{};
        rpb = bwd_rows_per_block(rows);
        nblk = bwd_num_blocks(rows);
    }
    if (p.tpr != 0 && rows <= kFewRowsMax) {
        nblk = 0;
        return dr ? launch_fewrows<S, kBwdRmsMul>(p, x, gamma, inv_rms, dy, dx, dr, dgamma, rows,
                                                  cols, accumulate, acc_dg, st)
                  : launch_fewrows<S, kBwdRms>(p, x, gamma, inv_rms, dy, dx, nullptr, dgamma,
                                               rows, cols, accumulate, acc_dg, st);
    }
    if (nblk > 0x7fffffffLL) return AGK_EINVAL;
    if (p.tpr == 0) {
        hipLaunchKernelGGL(rms_bwd_looped<S>, dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0,
                           st, static_cast<const T*>(x), static_cast<const T*>(gamma), inv_rms,
                           static_cast<const T*>(dy), static_cast<T*>(dx), static_cast<T*>(dr),
                           partials, rows, cols, rpb, accumulate);
        return check_launch();
    }
    if (dr) {
        if (accumulate && dx)
            return launch_rms_mul_bwd_resident<S, true>(p, nblk, x, gamma, inv_rms, dy, dx, dr,
                                                        partials, rows, cols, st);
        return launch_rms_mul_bwd_resident<S, false>(p, nblk, x, gamma, inv_rms, dy, dx, dr,
                                                     partials, rows, cols, st);
    }
    if (accumulate && dx)
        return launch_bwd_resident<S, true>(p, nblk, x, gamma, inv_rms, dy, dx, partials, rows,
                                            cols, st);
    return launch_bwd_resident<S, false>(p, nblk, x, gamma, inv_rms, dy, dx, partials, rows,
                                         cols, st);
}

inline int launch_finalize(const float* partials, float* dgamma, int64_t nblk, int cols,
                           int accumulate, hipStream_t st) {
    if (nblk <= kFinSplits) {  // same sums, spread over the columns
        const unsigned g = static_cast<unsigned>((cols + kBlock - 1) / kBlock);
        hipLaunchKernelGGL(dgamma_finalize_few, dim3(g), dim3(kBlock), 0, st, partials, dgamma,
                           nblk, cols, accumulate);
        return check_launch();
    }
    if (cols % 4 == 0 && aligned16(partials)) {
        constexpr int fc = fin_cols(true);
        hipLaunchKernelGGL(dgamma_finalize<true>, dim3(static_cast<unsigned>((cols + fc - 1) / fc)),
                           dim3(fc / 4 * kFinSplits), 0, st, partials, dgamma, nblk, cols,
                           accumulate);
    } else {
        constexpr int fc = fin_cols(false);
        hipLaunchKernelGGL(dgamma_finalize<false>,
                           dim3(static_cast<unsigned>((cols + fc - 1) / fc)),
                           dim3(fc * kFinSplits), 0, st, partials, dgamma, nblk, cols, accumulate);
    }
    return check_launch();
}

inline int zero_fill(float* p, int64_t n, hipStream_t st) {
    if (n <= 0) return AGK_OK;
    const int64_t grid = (n + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(fill_zero_f32, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, st, p,
                       n);
    return check_launch();
}

// Polls of a team's wait before a missing segment sum is recomputed
// (agk_set_exchange_wait_limit).
std::atomic<int> g_team_wait_polls{kTeamWaitPolls};
int team_wait_polls() { return g_team_wait_polls.load(std::memory_order_relaxed); }
// Whether the team kernel may be taken (agk_set_team_backward).
std::atomic<int> g_team_enabled{1};
inline bool team_enabled() { return g_team_enabled.load(std::memory_order_relaxed) != 0; }
// Whether the team forward may be taken (agk_set_team_forward).
std::atomic<int> g_team_fwd_enabled{1};
bool team_fwd_enabled() { return g_team_fwd_enabled.load(std::memory_order_relaxed) != 0; }

// Bytes of dgamma partial rows the backward writes for these pointers and
// sizes (the path launch_bwd takes): none for the few-rows kernel, 256 rows
// for the resident kernel, the looped kernel's row blocks otherwise.
template <class S>
inline size_t bwd_partials_bytes(const void* x, const void* gamma, const void* dy,
                                 const void* dx, int64_t rows, int cols) {
    int64_t nblk = 0, rpb = 0;
    const Plan p = bwd_plan_for<S>(x, gamma, dy, dx, rows, cols, nblk, rpb);
    if (p.tpr != 0 && rows <= kFewRowsMax) return 0;
    return static_cast<size_t>(nblk) * static_cast<size_t>(cols) * sizeof(float);
}

// Whether the backward takes the wide path for these arguments, given a
// 16-byte aligned workspace of at least wide_ws_bytes(rows, cols, false).
template <class S>
inline bool bwd_wide_possible(const void* x, const void* gamma, const void* dy, const void* dx,
                              int64_t rows, int cols) {
    int64_t nblk = 0, rpb = 0;
    const Plan p = bwd_plan_for<S>(x, gamma, dy, dx, rows, cols, nblk, rpb);
    return wide_bwd_eligible<S>(x, gamma, dy, dx, cols, p.tpr != 0);
}
// Whether the one-pass kernel for rows of up to 32768 columns takes these
// arguments (dr: the composition's output, or nullptr).
template <class S>
inline bool bwd_res_wide_possible(const void* x, const void* gamma, const void* dy,
                                  const void* dx, const void* dr, int64_t rows, int cols) {
    int64_t nblk = 0, rpb = 0;
    const Plan p = bwd_plan_for<S>(x, gamma, dy, dx, rows, cols, nblk, rpb);
    return wide_res_eligible<S>(x, gamma, dy, dx, dr, rows, cols, p.tpr != 0);
}
inline bool bwd_takes_res_wide(const void* x, const void* gamma, const void* dy, const void* dx,
                               const void* dr, int64_t rows, int cols, int dtype) {
    return dtype == AGK_F32 ? bwd_res_wide_possible<F32>(x, gamma, dy, dx, dr, rows, cols)
                            : bwd_res_wide_possible<BF16>(x, gamma, dy, dx, dr, rows, cols);
}
// dgamma partial rows the one-pass kernel writes (its workspace need).
inline size_t bwd_res_wide_bytes(int64_t rows, int cols, bool comp) {
    int64_t nblk = 0, rpb = 0;
    wide_res_blocking(rows, comp, nblk, rpb);
    return static_cast<size_t>(nblk) * static_cast<size_t>(cols) * 4u;
}

// Whether the team kernel (one pass, a row over several workgroups) takes
// these arguments.
template <class S>
inline bool bwd_team_possible(const void* x, const void* gamma, const void* dy, const void* dx,
                              int64_t rows, int cols) {
    int64_t nblk = 0, rpb = 0;
    const Plan p = bwd_plan_for<S>(x, gamma, dy, dx, rows, cols, nblk, rpb);
    return team_enabled() && team_eligible<S>(x, gamma, dy, dx, rows, cols, p.tpr != 0);
}

// The workspace the wide paths need: the dgamma partial rows only when dgamma
// is wanted (the team path takes the split path's regions).
inline bool wide_ws_ok(int64_t rows, int cols, const void* ws, size_t ws_bytes,
                       bool want_dgamma) {
    const size_t need =
        want_dgamma ? wide_ws_bytes(rows, cols, false) : wide_ws_stats_bytes(rows, cols);
    return ws && aligned16(ws) && ws_bytes >= need;
}
inline bool bwd_takes_team(const void* x, const void* gamma, const void* dy, const void* dx,
                           int64_t rows, int cols, int dtype, const void* ws, size_t ws_bytes,
                           bool want_dgamma) {
    if (!wide_ws_ok(rows, cols, ws, ws_bytes, want_dgamma)) return false;
    return dtype == AGK_F32 ? bwd_team_possible<F32>(x, gamma, dy, dx, rows, cols)
                            : bwd_team_possible<BF16>(x, gamma, dy, dx, rows, cols);
}

// The workspace must hold the dgamma partial rows only when dgamma is wanted.
inline bool bwd_takes_wide(const void* x, const void* gamma, const void* dy, const void* dx,
                           int64_t rows, int cols, int dtype, const void* ws, size_t ws_bytes,
                           bool want_dgamma) {
    if (!wide_ws_ok(rows, cols, ws, ws_bytes, want_dgamma)) return false;
    return dtype == AGK_F32 ? bwd_wide_possible<F32>(x, gamma, dy, dx, rows, cols)
                            : bwd_wide_possible<BF16>(x, gamma, dy, dx, rows, cols);
}

// The RMSNorm backward with validated arguments.  Rows too wide for the
// resident shapes take the team kernel (up to 1M columns) or the split path
// when `ws` (16-byte aligned, ws_bytes long) holds wide_ws_bytes(rows, cols,
// false) (wide_ws_stats_bytes when dgamma is NULL); otherwise dgamma partials
// go to `partials` (which must hold bwd_partials_bytes when dgamma != NULL).
inline int rmsnorm_bwd_run(const void* x, const void* gamma, const float* inv_rms,
                           const void* dy, void* dx, float* dgamma, float* partials, void* ws,
                           size_t ws_bytes, int64_t rows, int cols, int dtype, int acc_dx,
                           int acc_dg, hipStream_t st) {
    if (bwd_takes_res_wide(x, gamma, dy, dx, nullptr, rows, cols, dtype))
        return dtype == AGK_F32
                   ? launch_wide_res_bwd<F32>(x, gamma, inv_rms, dy, dx, nullptr, partials, dgamma,
                                              rows, cols, acc_dx, acc_dg, st)
                   : launch_wide_res_bwd<BF16>(x, gamma, inv_rms, dy, dx, nullptr, partials,
                                               dgamma, rows, cols, acc_dx, acc_dg, st);
    if (bwd_takes_team(x, gamma, dy, dx, rows, cols, dtype, ws, ws_bytes, dgamma != nullptr))
        return dtype == AGK_F32
                   ? launch_wide_team_bwd<F32>(x, gamma, inv_rms, dy, dx, dgamma, ws, rows, cols,
                                               acc_dx, acc_dg, st)
                   : launch_wide_team_bwd<BF16>(x, gamma, inv_rms, dy, dx, dgamma, ws, rows,
                                                cols, acc_dx, acc_dg, st);
    if (bwd_takes_wide(x, gamma, dy, dx, rows, cols, dtype, ws, ws_bytes, dgamma != nullptr))
        return dtype == AGK_F32
                   ? launch_wide_bwd<F32>(x, gamma, inv_rms, dy, dx, nullptr, dgamma, ws, rows,
                                          cols, acc_dx, acc_dg, st)
                   : launch_wide_bwd<BF16>(x, gamma, inv_rms, dy, dx, nullptr, dgamma, ws, rows,
                                           cols, acc_dx, acc_dg, st);
    int64_t nblk = 0;
    int rc = dtype == AGK_F32 ? launch_bwd<F32>(x, gamma, inv_rms, dy, dx, nullptr, partials,
                                                dgamma, rows, cols, acc_dx, acc_dg, st, nblk)
                              : launch_bwd<BF16>(x, gamma, inv_rms, dy, dx, nullptr, partials,
                                                 dgamma, rows, cols, acc_dx, acc_dg, st, nblk);
    if (rc != AGK_OK || !dgamma || nblk == 0) return rc;
    return launch_finalize(partials, dgamma, nblk, cols, acc_dg, st);
}

}  // namespace agk

// ---- scratch of the entry point that allocates nothing ---------------------------
// agk_rmsnorm_bwd_noalloc keeps its dgamma partial rows here instead of in a
// caller workspace.  Every device the library runs on holds one copy for the
// life of the process; every call on that device shares it (overlapping calls
// on one device race).  The kernels write every partial row they later read,
// so nothing in it needs clearing between calls.  Host code must not pass the
// name to a kernel (on the host it is a stand-in, not a device address): it
// uses the address hipGetSymbolAddress gives for the device, kept per device.
static __device__ __align__(256) float scratch[AGK_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace agk {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on the device `stream` runs on (the current
// device for the null stream), looked up once per device with that device
// current.
inline int scratch_on_device(hipStream_t stream, float** out) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return status_from_hip(e);
    int dev = cur;
    if (stream != nullptr) {
        hipDevice_t d = 0;
        e = hipStreamGetDevice(stream, &d);
        if (e != hipSuccess) return status_from_hip(e);
        dev = static_cast<int>(d);
    }
    if (dev < 0 || dev >= kMaxDevices) return AGK_EINVAL;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return status_from_hip(e);
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess) return status_from_hip(e);
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return AGK_OK;
}

}  // namespace agk

// ---- C ABI ----------------------------------------------------------------------

extern "C" {

int agk_rmsnorm_fwd(const void* x, const void* gamma, void* y, float* inv_rms, int64_t rows,
                    int64_t cols, float eps, int dtype, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (rows == 0 || cols == 0) return AGK_OK;
    if (!x || !y || !inv_rms) return AGK_EINVAL;
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == AGK_F32)
        return launch_fwd<F32>(x, gamma, y, inv_rms, rows, static_cast<int>(cols), eps, nullptr,
                               st);
    return launch_fwd<BF16>(x, gamma, y, inv_rms, rows, static_cast<int>(cols), eps, nullptr,
                            st);
}

size_t agk_rmsnorm_fwd_workspace_bytes(int64_t rows, int64_t cols) {
    if (agk::check_sizes(rows, cols) != AGK_OK) return 0;
    return agk::fwd_team_ws_bytes(rows, cols);
}

int agk_rmsnorm_fwd_ws(const void* x, const void* gamma, void* y, float* inv_rms,
                       void* workspace, size_t workspace_bytes, int64_t rows, int64_t cols,
                       float eps, int dtype, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (rows == 0 || cols == 0) return AGK_OK;
    if (!x || !y || !inv_rms) return AGK_EINVAL;
    if (workspace) {
        if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return AGK_EINVAL;
        if (workspace_bytes < fwd_team_ws_bytes(rows, cols)) return AGK_EWORKSPACE;
    }
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == AGK_F32)
        return launch_fwd<F32>(x, gamma, y, inv_rms, rows, static_cast<int>(cols), eps,
                               workspace, st);
    return launch_fwd<BF16>(x, gamma, y, inv_rms, rows, static_cast<int>(cols), eps, workspace,
                            st);
}

size_t agk_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
    if (agk::check_sizes(rows, cols) != AGK_OK || rows == 0 || cols == 0) return 0;
    const size_t looped =
        static_cast<size_t>(agk::bwd_num_blocks(rows)) * static_cast<size_t>(cols) * 4u;
    const size_t wide = agk::wide_ws_bytes(rows, cols, false);
    const size_t comp = agk::wide_ws_bytes(rows, cols, true);
    const size_t split = wide > comp ? wide : comp;
    return split > looped ? split : looped;
}

int agk_rmsnorm_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
                    void* dx, float* dgamma, void* workspace, size_t workspace_bytes,
                    int64_t rows, int64_t cols, int dtype, int accumulate,
                    agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    clear_pending_error();
    if (accumulate & ~AGK_ACCUM_ALL) return AGK_EINVAL;
    const int acc_dx = (accumulate & AGK_ACCUM_DX) != 0;
    const int acc_dg = (accumulate & AGK_ACCUM_DGAMMA) != 0;
    if (rows == 0 || cols == 0) {
        if (dgamma && !acc_dg && cols > 0) return zero_fill(dgamma, cols, st);
        return AGK_OK;
    }
    if (!x || !inv_rms || !dy) return AGK_EINVAL;
    if (!dx && !dgamma) return AGK_OK;  // nothing requested
    float* partials = nullptr;
    if (dgamma) {
        const size_t need = agk_rmsnorm_bwd_workspace_bytes(rows, cols);
        if (!workspace || workspace_bytes < need) return AGK_EWORKSPACE;
        partials = static_cast<float*>(workspace);
    }
    return rmsnorm_bwd_run(x, gamma, inv_rms, dy, dx, dgamma, partials, workspace,
                           workspace ? workspace_bytes : 0, rows, static_cast<int>(cols), dtype,
                           acc_dx, acc_dg, st);
}

int agk_rmsnorm_bwd_noalloc(const void* x, const void* gamma, const float* inv_rms,
                            const void* dy, void* dx, float* dgamma, int64_t rows, int64_t cols,
                            int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    clear_pending_error();
    if (accumulate & ~AGK_ACCUM_ALL) return AGK_EINVAL;
    const int acc_dx = (accumulate & AGK_ACCUM_DX) != 0;
    const int acc_dg = (accumulate & AGK_ACCUM_DGAMMA) != 0;
    if (rows == 0 || cols == 0) {
        if (dgamma && !acc_dg && cols > 0) return zero_fill(dgamma, cols, st);
        return AGK_OK;
    }
    if (!x || !inv_rms || !dy) return AGK_EINVAL;
    if (!dx && !dgamma) return AGK_OK;  // nothing requested
    const int c = static_cast<int>(cols);
    // Rows of up to 32768 columns, at least 256 of them: the one-pass kernel,
    // its partial rows in the scratch array.
    if (bwd_takes_res_wide(x, gamma, dy, dx, nullptr, rows, c, dtype)) {
        float* ws = nullptr;
        if (dgamma) {
            if (bwd_res_wide_bytes(rows, c, false) > AGK_NOALLOC_SCRATCH_BYTES)
                return AGK_EWORKSPACE;
            if (int rc = scratch_on_device(st, &ws)) return rc;
        }
        return rmsnorm_bwd_run(x, gamma, inv_rms, dy, dx, dgamma, ws, nullptr, 0, rows, c, dtype,
                               acc_dx, acc_dg, st);
    }
    // Rows too wide for the resident shapes: the wide path with the scratch
    // array as its workspace, as agk_rmsnorm_bwd takes it with the workspace
    // agk_rmsnorm_bwd_workspace_bytes asks for (with dgamma NULL, only the
    // row statistics must fit).
    const bool wide = dtype == AGK_F32 ? bwd_wide_possible<F32>(x, gamma, dy, dx, rows, c)
                                       : bwd_wide_possible<BF16>(x, gamma, dy, dx, rows, c);
    if (wide) {
        const size_t need = dgamma ? wide_ws_bytes(rows, c, false) : wide_ws_stats_bytes(rows, c);
        if (need > AGK_NOALLOC_SCRATCH_BYTES) return AGK_EWORKSPACE;
        float* ws = nullptr;
        if (int rc = scratch_on_device(st, &ws)) return rc;
        return rmsnorm_bwd_run(x, gamma, inv_rms, dy, dx, dgamma, ws, ws,
                               AGK_NOALLOC_SCRATCH_BYTES, rows, c, dtype, acc_dx, acc_dg, st);
    }
    float* partials = nullptr;
    if (dgamma) {
        const size_t need = dtype == AGK_F32 ? bwd_partials_bytes<F32>(x, gamma, dy, dx, rows, c)
                                             : bwd_partials_bytes<BF16>(x, gamma, dy, dx, rows, c);
        if (need > AGK_NOALLOC_SCRATCH_BYTES) return AGK_EWORKSPACE;
        if (need > 0) {
            if (int rc = scratch_on_device(st, &partials)) return rc;
        }
    }
    return rmsnorm_bwd_run(x, gamma, inv_rms, dy, dx, dgamma, partials, nullptr, 0, rows, c,
                           dtype, acc_dx, acc_dg, st);
}

int agk_rms_mul_bwd(const void* x, const void* gamma, const float* inv_rms, const void* gy,
                    void* dr, void* dx, float* dgamma, void* workspace, size_t workspace_bytes,
                    int64_t rows, int64_t cols, int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    clear_pending_error();
    if (accumulate & ~AGK_ACCUM_ALL) return AGK_EINVAL;
    const int acc_dx = (accumulate & AGK_ACCUM_DX) != 0;
    const int acc_dg = (accumulate & AGK_ACCUM_DGAMMA) != 0;
    if (rows == 0 || cols == 0) {
        if (dgamma && !acc_dg && cols > 0) return zero_fill(dgamma, cols, st);
        return AGK_OK;
    }
    if (!x || !gamma || !inv_rms || !gy || !dr) return AGK_EINVAL;
    float* partials = nullptr;
    if (dgamma) {
        const size_t need = agk_rmsnorm_bwd_workspace_bytes(rows, cols);
        if (!workspace || workspace_bytes < need) return AGK_EWORKSPACE;
        partials = static_cast<float*>(workspace);
    }
    const int c = static_cast<int>(cols);
    // Rows of up to 32768 columns and at least 256 rows: the one-pass kernel,
    // whose outputs are the two separate calls' (agk_rmsnorm_bwd takes the
    // same kernel for them, agk_mul_rowbcast_bwd the looped one).
    if (bwd_takes_res_wide(x, gamma, gy, dx, dr, rows, c, dtype))
        return dtype == AGK_F32 ? launch_wide_res_bwd<F32>(x, gamma, inv_rms, gy, dx, dr, partials,
                                                           dgamma, rows, c, acc_dx, acc_dg, st)
                                : launch_wide_res_bwd<BF16>(x, gamma, inv_rms, gy, dx, dr,
                                                            partials, dgamma, rows, c, acc_dx,
                                                            acc_dg, st);
    // Rows too wide for the resident shapes, with a workspace: the split
    // path, whose outputs are the two separate calls' on their split paths.
    if (workspace && aligned16(workspace) && aligned16(dr) &&
        workspace_bytes >= wide_ws_bytes(rows, c, true) &&
        (dtype == AGK_F32 ? bwd_wide_possible<F32>(x, gamma, gy, dx, rows, c)
                          : bwd_wide_possible<BF16>(x, gamma, gy, dx, rows, c)))
        return dtype == AGK_F32 ? launch_wide_bwd<F32>(x, gamma, inv_rms, gy, dx, dr, dgamma,
                                                       workspace, rows, c, acc_dx, acc_dg, st)
                                : launch_wide_bwd<BF16>(x, gamma, inv_rms, gy, dx, dr, dgamma,
                                                        workspace, rows, c, acc_dx, acc_dg, st);
    int64_t nblk = 0;
    int rc = dtype == AGK_F32 ? launch_bwd<F32>(x, gamma, inv_rms, gy, dx, dr, partials, dgamma,
                                                rows, c, acc_dx, acc_dg, st, nblk)
                              : launch_bwd<BF16>(x, gamma, inv_rms, gy, dx, dr, partials, dgamma,
                                                 rows, c, acc_dx, acc_dg, st, nblk);
    if (rc != AGK_OK || !dgamma || nblk == 0) return rc;
    return launch_finalize(partials, dgamma, nblk, c, acc_dg, st);
}

int agk_mul_rowbcast_fwd(const void* a, const void* b, void* y, int64_t rows, int64_t cols,
                         int dtype, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (rows == 0 || cols == 0) return AGK_OK;
    if (!a || !b || !y) return AGK_EINVAL;
    if (rows > 0x7fffffffLL) return AGK_EINVAL;
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int c = static_cast<int>(cols);
    return dtype == AGK_F32 ? launch_mul_fwd<F32>(a, b, y, rows, c, st)
                            : launch_mul_fwd<BF16>(a, b, y, rows, c, st);
}

size_t agk_mul_rowbcast_bwd_workspace_bytes(int64_t rows, int64_t cols) {
    return agk_rmsnorm_bwd_workspace_bytes(rows, cols);
}

int agk_mul_rowbcast_bwd(const void* gy, const void* a, const void* b, void* da, float* db,
                         void* workspace, size_t workspace_bytes, int64_t rows, int64_t cols,
                         int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    clear_pending_error();
    if (accumulate & ~AGK_ACCUM_ALL) return AGK_EINVAL;
    const int acc_da = (accumulate & AGK_ACCUM_DX) != 0;
    const int acc_db = (accumulate & AGK_ACCUM_DGAMMA) != 0;
    if (rows == 0 || cols == 0) {
        if (db && !acc_db && cols > 0) return zero_fill(db, cols, st);
        return AGK_OK;
    }
    if (!gy || (da && !b) || (db && !a)) return AGK_EINVAL;
    if (!da && !db) return AGK_OK;
    float* partials = nullptr;
    if (db) {
        const size_t need = agk_mul_rowbcast_bwd_workspace_bytes(rows, cols);
        if (!workspace || workspace_bytes < need) return AGK_EWORKSPACE;
        partials = static_cast<float*>(workspace);
    }
    const int c = static_cast<int>(cols);
    int64_t nblk = 0, rpb = 0;
    const Plan p = dtype == AGK_F32 ? bwd_plan_for<F32>(a, b, gy, da, rows, c, nblk, rpb)
                                    : bwd_plan_for<BF16>(a, b, gy, da, rows, c, nblk, rpb);
    if (nblk > 0x7fffffffLL) return AGK_EINVAL;
    if (p.tpr != 0 && rows <= kFewRowsMax)  // few rows: db written directly
        return dtype == AGK_F32
                   ? launch_fewrows<F32, kBwdMul>(p, a, b, nullptr, gy, da, nullptr, db, rows, c,
                                                  acc_da, acc_db, st)
                   : launch_fewrows<BF16, kBwdMul>(p, a, b, nullptr, gy, da, nullptr, db, rows, c,
                                                   acc_da, acc_db, st);
    if (p.tpr != 0) {  // register-resident, as the RMSNorm backward
        const bool acc = acc_da && da;
        int rc = dtype == AGK_F32
                     ? (acc ? launch_mul_bwd_resident<F32, true>(p, nblk, a, b, gy, da, partials,
                                                                 rows, c, st)
                            : launch_mul_bwd_resident<F32, false>(p, nblk, a, b, gy, da, partials,
                                                                  rows, c, st))
                     : (acc ? launch_mul_bwd_resident<BF16, true>(p, nblk, a, b, gy, da,
                                                                  partials, rows, c, st)
                            : launch_mul_bwd_resident<BF16, false>(p, nblk, a, b, gy, da,
                                                                   partials, rows, c, st));
        if (rc != AGK_OK || !db) return rc;
        return launch_finalize(partials, db, nblk, c, acc_db, st);
    }
    const int w = dtype == AGK_F32 ? F32::kVec : BF16::kVec;
    const int vec = c % w == 0 && aligned16(gy) && (!a || aligned16(a)) && (!b || aligned16(b)) &&
                    (!da || aligned16(da));
    const int64_t chunk = mul_chunk(nblk, c, vec ? w : 1);
    const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>((c + chunk - 1) / chunk));
    if (dtype == AGK_F32) {
        hipLaunchKernelGGL(mul_rowbcast_bwd_kernel<F32>, grid, dim3(kBlock), 0, st,
                           static_cast<const float*>(gy), static_cast<const float*>(a),
                           static_cast<const float*>(b), static_cast<float*>(da), partials, rows,
                           c, rpb, acc_da, chunk, vec);
    } else {
        hipLaunchKernelGGL(mul_rowbcast_bwd_kernel<BF16>, grid, dim3(kBlock), 0, st,
                           static_cast<const uint16_t*>(gy), static_cast<const uint16_t*>(a),
                           static_cast<const uint16_t*>(b), static_cast<uint16_t*>(da), partials,
                           rows, c, rpb, acc_da, chunk, vec);
    }
    int rc = check_launch();
    if (rc != AGK_OK || !db) return rc;
    return launch_finalize(partials, db, nblk, c, acc_db, st);
}

size_t agk_sum_rows_workspace_bytes(int64_t rows, int64_t cols) {
    return agk_rmsnorm_bwd_workspace_bytes(rows, cols);
}

int agk_sum_rows(const void* x, float* out, void* workspace, size_t workspace_bytes,
                 int64_t rows, int64_t cols, int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    clear_pending_error();
    if (accumulate != 0 && accumulate != 1) return AGK_EINVAL;
    if (cols == 0) return AGK_OK;
    if (!out) return AGK_EINVAL;
    if (rows == 0) return accumulate ? AGK_OK : zero_fill(out, cols, st);
    if (!x) return AGK_EINVAL;
    const size_t need = agk_sum_rows_workspace_bytes(rows, cols);
    if (!workspace || workspace_bytes < need) return AGK_EWORKSPACE;
    float* partials = static_cast<float*>(workspace);
    const int c = static_cast<int>(cols);
    int64_t nblk = 0, rpb = 0;
    const Plan p = dtype == AGK_F32 ? bwd_plan_for<F32>(x, nullptr, x, nullptr, rows, c, nblk, rpb)
                                    : bwd_plan_for<BF16>(x, nullptr, x, nullptr, rows, c, nblk,
                                                         rpb);
    if (nblk > 0x7fffffffLL) return AGK_EINVAL;
    if (p.tpr != 0 && rows <= kFewRowsMax)  // few rows: out written directly
        return dtype == AGK_F32
                   ? launch_fewrows<F32, kBwdColSum>(p, nullptr, nullptr, nullptr, x, nullptr,
                                                     nullptr, out, rows, c, 0, accumulate, st)
                   : launch_fewrows<BF16, kBwdColSum>(p, nullptr, nullptr, nullptr, x, nullptr,
                                                      nullptr, out, rows, c, 0, accumulate, st);
    int rc;
    if (p.tpr != 0) {
        rc = dtype == AGK_F32 ? launch_sum_rows_resident<F32>(p, nblk, x, partials, rows, c, st)
                              : launch_sum_rows_resident<BF16>(p, nblk, x, partials, rows, c, st);
    } else {
        const int w = dtype == AGK_F32 ? F32::kVec : BF16::kVec;
        const int vec = c % w == 0 && aligned16(x);
        const int64_t chunk = mul_chunk(nblk, c, vec ? w : 1);
        const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>((c + chunk - 1) / chunk));
        if (dtype == AGK_F32)
            hipLaunchKernelGGL(mul_rowbcast_bwd_kernel<F32>, grid, dim3(kBlock), 0, st,
                               static_cast<const float*>(x), nullptr, nullptr, nullptr, partials,
                               rows, c, rpb, 0, chunk, vec);
        else
            hipLaunchKernelGGL(mul_rowbcast_bwd_kernel<BF16>, grid, dim3(kBlock), 0, st,
                               static_cast<const uint16_t*>(x), nullptr, nullptr, nullptr,
                               partials, rows, c, rpb, 0, chunk, vec);
        rc = check_launch();
    }
    if (rc != AGK_OK) return rc;
    return launch_finalize(partials, out, nblk, c, accumulate, st);
}

int agk_set_exchange_wait_limit(int polls) {
    const int prev = agk::g_team_wait_polls.load(std::memory_order_relaxed);
    if (polls >= 0) agk::g_team_wait_polls.store(polls, std::memory_order_relaxed);
    return prev;
}

int agk_set_team_backward(int enabled) {
    const int prev = agk::g_team_enabled.load(std::memory_order_relaxed);
    if (enabled >= 0) agk::g_team_enabled.store(enabled != 0 ? 1 : 0, std::memory_order_relaxed);
    return prev;
}

int agk_set_team_forward(int enabled) {
    const int prev = agk::g_team_fwd_enabled.load(std::memory_order_relaxed);
    if (enabled >= 0)
        agk::g_team_fwd_enabled.store(enabled != 0 ? 1 : 0, std::memory_order_relaxed);
    return prev;
}

int agk_rmsnorm_launch_plan(int64_t rows, int64_t cols, int dtype, int backward,
                            int32_t* plan) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (!plan) return AGK_EINVAL;
    if (backward < 0 || backward > 2) return AGK_EINVAL;
    const bool fwd_ws = backward == 2;  // a forward given a workspace
    if (fwd_ws) backward = 0;
    const int w = dtype == AGK_F32 ? F32::kVec : BF16::kVec;
    Plan p;
    int64_t nblk = 0, rpb = 0;
    if (!backward) {
        if (cols > 0 && cols % w == 0) p = fwd_plan(cols / w, rows);
    } else if (cols > 0 && cols <= 0x7fffffffLL) {
        // aligned stand-in pointers: the plan depends only on alignment
        const void* a = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
        const int c = static_cast<int>(cols);
        p = dtype == AGK_F32 ? bwd_plan_for<F32>(a, a, a, a, rows, c, nblk, rpb)
                             : bwd_plan_for<BF16>(a, a, a, a, rows, c, nblk, rpb);
        if (p.tpr != 0 && rows <= kFewRowsMax) rpb = nblk = 0;  // few rows: no partial rows
    }
    plan[0] = p.tpr;
    plan[1] = p.nv;
    plan[2] = p.g;
    plan[3] = static_cast<int32_t>(rpb);
    plan[4] = static_cast<int32_t>(nblk);
    if (p.tpr == 0 && backward && cols > 0 && cols <= 0x7fffffffLL) {
        // the one-pass kernel for rows of up to 32768 columns
        const void* a = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
        const int c = static_cast<int>(cols);
        const bool res = dtype == AGK_F32
                             ? wide_res_eligible<F32>(a, a, a, a, nullptr, rows, c, false)
                             : wide_res_eligible<BF16>(a, a, a, a, nullptr, rows, c, false);
        if (res) {
            int64_t wb = 0, wr = 0;
            wide_res_blocking(rows, false, wb, wr);
            plan[0] = kWideResLanes;
            plan[1] = kWideResMaxCols / (w * kWideResLanes);
            plan[2] = 1;
            plan[3] = static_cast<int32_t>((rows + wb - 1) / wb);
            plan[4] = static_cast<int32_t>(wb);
            return AGK_OK;
        }
    }
    if (p.tpr == 0 && backward && cols > 0 && cols <= 0x7fffffffLL) {
        // the team kernel: a row over `parts` workgroups of 256 lanes
        const void* a = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
        const int c = static_cast<int>(cols);
        const bool team = team_enabled() &&
                          (dtype == AGK_F32 ? team_eligible<F32>(a, a, a, a, rows, c, false)
                                            : team_eligible<BF16>(a, a, a, a, rows, c, false));
        if (team) {
            const int segs = team_segs_for(dtype, rows, c);
            const TeamPlan tp = team_plan(rows, c, segs);
            plan[0] = static_cast<int32_t>(tp.parts * kWideLanes);
            plan[1] = segs * kWideSegCols / (w * kWideLanes);
            plan[2] = 0;
            plan[3] = static_cast<int32_t>((rows + tp.teams - 1) / tp.teams);
            plan[4] = static_cast<int32_t>(tp.teams);
            return AGK_OK;
        }
    }
    if (p.tpr == 0 && fwd_ws && cols > 0 && cols <= 0x7fffffffLL && team_fwd_enabled() &&
        fwd_team_shape_ok(rows, cols) &&
        (dtype == AGK_F32 ? wide_fwd_shape_ok<F32>(rows, static_cast<int>(cols), false)
                          : wide_fwd_shape_ok<BF16>(rows, static_cast<int>(cols), false))) {
        // the team forward: a row over `parts` workgroups of 256 lanes
        const int segs = fwd_team_segs_for(dtype, rows, cols);
        const TeamPlan tp = fwd_team_plan(rows, static_cast<int>(cols), segs);
        plan[0] = static_cast<int32_t>(tp.parts * kWideLanes);
        plan[1] = segs * kWideSegCols / (w * kWideLanes);
        plan[2] = 0;
        plan[3] = static_cast<int32_t>((rows + tp.teams - 1) / tp.teams);
        plan[4] = static_cast<int32_t>(tp.teams);
        return AGK_OK;
    }
    if (p.tpr == 0 && cols > 0 && cols <= 0x7fffffffLL) {
        // aligned stand-in pointers, and for the forward a y apart from x
        const void* a = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
        const int c = static_cast<int>(cols);
        const bool split =
            backward ? (dtype == AGK_F32 ? wide_bwd_eligible<F32>(a, a, a, a, c, false)
                                         : wide_bwd_eligible<BF16>(a, a, a, a, c, false))
                     : (dtype == AGK_F32 ? wide_fwd_shape_ok<F32>(rows, c, false)
                                         : wide_fwd_shape_ok<BF16>(rows, c, false));
        if (split) {
            const WidePlan w = wide_plan(rows, c);
            plan[1] = static_cast<int32_t>(w.nseg);
            plan[2] = static_cast<int32_t>(w.nch);
            plan[3] = backward ? static_cast<int32_t>(w.rb) : 0;
            plan[4] = backward && w.nrb > 1 ? static_cast<int32_t>(w.nrb) : 0;
        }
    }
    return AGK_OK;
}

const char* agk_status_str(int status) {
    switch (status) {
        case AGK_OK: return "AGK_OK: success";
        case AGK_EINVAL: return "AGK_EINVAL: invalid argument (null pointer or bad size)";
        case AGK_EDTYPE: return "AGK_EDTYPE: unsupported storage dtype";
        case AGK_EWORKSPACE: return "AGK_EWORKSPACE: workspace missing or too small";
        case AGK_EHIP: return "AGK_EHIP: HIP runtime or launch failure";
        default: return "unknown agk status";
    }
}

const char* agk_last_error(void) {
    return agk::t_last_hip_error == hipSuccess ? "no HIP error"
                                               : hipGetErrorString(agk::t_last_hip_error);
}

const char* agk_version(void) { return "agk_rmsnorm 0.2 gfx950"; }

}  // extern "C"
