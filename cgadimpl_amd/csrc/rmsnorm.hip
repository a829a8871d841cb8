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
// dgamma is deterministic: each workgroup of the backward owns a contiguous
// block of rows and sums dy*xhat for them in a fixed order into one row of
// fp32 partials; dgamma_finalize then sums the partial rows in a fixed order
// in fp64.  No floating-point atomics are used anywhere.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <type_traits>

#include "agk_rmsnorm.h"

namespace agk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;          // threads per workgroup (TPR <= 256)
constexpr int kTargetBlocks = 1024;  // backward row blocks (sets partial rows)
constexpr int kMinRowsPerBlock = 16;

// ---- storage types --------------------------------------------------------

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
        return (u >> 16) | 0x0040u;  // quiet NaN, sign kept
    u += 0x7fffu + ((u >> 16) & 1u); // round to nearest, ties to even
    return u >> 16;
}

struct F32 {
    using T = float;
    static constexpr int kVec = 4;  // elements per 16-byte slot
    __device__ static float get(const T* p) { return *p; }
    __device__ static void put(T* p, float v) { *p = v; }
    __device__ static void unpack(u32x4 v, float (&f)[4]) {
        f[0] = __uint_as_float(v.x);
        f[1] = __uint_as_float(v.y);
        f[2] = __uint_as_float(v.z);
        f[3] = __uint_as_float(v.w);
    }
    __device__ static u32x4 pack(const float (&f)[4]) {
        return u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]),
                     __float_as_uint(f[2]), __float_as_uint(f[3])};
    }
};

struct BF16 {
    using T = uint16_t;
    static constexpr int kVec = 8;
    __device__ static float get(const T* p) {
        return __uint_as_float(static_cast<uint32_t>(*p) << 16);
    }
    __device__ static void put(T* p, float v) {
        *p = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
    __device__ static void unpack(u32x4 v, float (&f)[8]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(v[i] << 16);
            f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
        }
    }
    __device__ static u32x4 pack(const float (&f)[8]) {
        u32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            v[i] = f32_to_bf16_bits(f[2 * i]) | (f32_to_bf16_bits(f[2 * i + 1]) << 16);
        return v;
    }
};

// Makes v opaque to the optimiser at this point, so values derived from it
// earlier are recomputed afterwards rather than held in registers.
__device__ __forceinline__ void opaque(u32x4& a, u32x4& b) {
    asm volatile("" : "+v"(a), "+v"(b));
}

template <class S>
__device__ __forceinline__ u32x4 load16(const typename S::T* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
template <class S>
__device__ __forceinline__ void store16(typename S::T* p, u32x4 v) {
    *reinterpret_cast<u32x4*>(p) = v;
}

// ---- reductions -------------------------------------------------------------

// Sum over the TPR (<= 64) lanes of a row group, butterfly order; every lane
// of the group ends with the same value.
template <int TPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = (TPR < 64 ? TPR : 64) / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Row sum for a row spread over TPR lanes.  For TPR > 64 the per-wave sums go
// through `red` (double-buffered by `parity`, so one barrier per row is
// enough) and are added in wave order.
template <int TPR>
__device__ __forceinline__ float row_sum(float v, float (*red)[16], int parity) {
    v = group_sum<TPR>(v);
    if constexpr (TPR > 64) {
        constexpr int kWaves = TPR / 64;
        const int lane = threadIdx.x & 63;
        const int wave_in_row = (threadIdx.x % TPR) >> 6;
        const int row_slot = threadIdx.x / TPR;  // 0 when TPR >= kBlock
        if (lane == 0) red[parity][row_slot * kWaves + wave_in_row] = v;
        __syncthreads();
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += red[parity][row_slot * kWaves + w];
        v = s;
    }
    return v;
}

// ---- register-resident forward ---------------------------------------------
// y[row] = (x[row] * r) * gamma, r = 1 / sqrt(sum(x^2)/cols + eps); inv_rms[row] = r.
// gamma == nullptr: no scale.  Requires 16-byte aligned x/y/gamma and
// cols % S::kVec == 0, and cols <= TPR * NV * kVec.
template <class S, int TPR, int NV>
__global__ __launch_bounds__(TPR > kBlock ? TPR : kBlock) void rms_fwd_resident(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    typename S::T* __restrict__ y, float* __restrict__ inv_rms, int64_t rows, int cols,
    float eps) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int BLOCK = TPR > kBlock ? TPR : kBlock;
    constexpr int G = BLOCK / TPR;
    __shared__ float red[2][16];

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
        xv[k] = (active && col < cols) ? load16<S>(xr + col) : u32x4{0u, 0u, 0u, 0u};
        float f[W];
        S::unpack(xv[k], f);
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] += f[e] * f[e];
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < W; ++e) ss += part[e];
    ss = row_sum<TPR>(ss, red, 0);

    const float ms = ss / static_cast<float>(cols);
    const float r = 1.0f / sqrtf(ms + eps);
    if (!active) return;
    if (t == 0) inv_rms[row] = r;

    T* yr = y + row * static_cast<int64_t>(cols);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = (t + k * TPR) * W;
        if (col < cols) {
            float f[W];
            S::unpack(xv[k], f);
            if (gamma) {
                float gm[W];
                S::unpack(load16<S>(gamma + col), gm);
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = (f[e] * r) * gm[e];
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = f[e] * r;
            }
            store16<S>(yr + col, S::pack(f));
        }
    }
}

// ---- register-resident backward --------------------------------------------
// Workgroup b owns rows [b*rpb, min(rows, (b+1)*rpb)); its TPR-lane groups
// take rows round-robin.  Per row:
//   g = dy*gamma, dot = sum(g*x), dx (+)= r*(g - x*(r*r*dot/cols))
// and, when partials != nullptr, each lane accumulates dy*(x*r) for the
// columns it owns; the groups' sums are added in group order into
// partials[b][*].
template <class S, int TPR, int NV>
__global__ __launch_bounds__(TPR > kBlock ? TPR : kBlock) void rms_bwd_resident(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, float* __restrict__ partials, int64_t rows, int cols,
    int64_t rpb, int accumulate) {
    constexpr int W = S::kVec;
    constexpr int BLOCK = TPR > kBlock ? TPR : kBlock;
    constexpr int G = BLOCK / TPR;
    __shared__ float red[2][16];
    extern __shared__ float lds_part[];  // [G][cols] when G > 1 and partials

    const int t = threadIdx.x % TPR;
    const int grp = threadIdx.x / TPR;
    const int64_t row_begin = static_cast<int64_t>(blockIdx.x) * rpb;
    const int64_t row_end = row_begin + rpb < rows ? row_begin + rpb : rows;
    const int64_t niter = (row_end - row_begin + G - 1) / G;  // uniform in the block
    const bool want_dg = partials != nullptr;
    const float inv_cols = 1.0f / static_cast<float>(cols);

    float dg[NV][W];
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < W; ++e) dg[k][e] = 0.0f;

    for (int64_t it = 0; it < niter; ++it) {
        const int64_t row = row_begin + it * G + grp;
        const bool active = row < row_end;
        const int64_t off = (active ? row : 0) * static_cast<int64_t>(cols);
        u32x4 xv[NV], dv[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            const bool ok = active && col < cols;
            xv[k] = ok ? load16<S>(x + off + col) : u32x4{0u, 0u, 0u, 0u};
            dv[k] = ok ? load16<S>(dy + off + col) : u32x4{0u, 0u, 0u, 0u};
        }
        const float r = active ? inv_rms[row] : 0.0f;

        float part[W];
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            float fx[W], fd[W];
            S::unpack(xv[k], fx);
            S::unpack(dv[k], fd);
            if (gamma && col < cols) {
                float gm[W];
                S::unpack(load16<S>(gamma + col), gm);
#pragma unroll
                for (int e = 0; e < W; ++e) fd[e] = fd[e] * gm[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] += fd[e] * fx[e];
        }
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < W; ++e) dot += part[e];
        dot = row_sum<TPR>(dot, red, static_cast<int>(it & 1));
        const float s = (r * r * dot) * inv_cols;
        // Re-derive the unpacked values from the raw slots after the
        // reduction instead of keeping both copies live across it.
#pragma unroll
        for (int k = 0; k < NV; ++k) opaque(xv[k], dv[k]);

        if (active) {
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const int col = (t + k * TPR) * W;
                if (col < cols) {
                    float fx[W], fd[W], gk[W];
                    S::unpack(xv[k], fx);
                    S::unpack(dv[k], fd);
                    if (gamma) {
                        float gm[W];
                        S::unpack(load16<S>(gamma + col), gm);
#pragma unroll
                        for (int e = 0; e < W; ++e) gk[e] = fd[e] * gm[e];
                    } else {
#pragma unroll
                        for (int e = 0; e < W; ++e) gk[e] = fd[e];
                    }
                    float o[W];
#pragma unroll
                    for (int e = 0; e < W; ++e) o[e] = r * (gk[e] - fx[e] * s);
                    if (accumulate) {
                        float old[W];
                        S::unpack(load16<S>(dx + off + col), old);
#pragma unroll
                        for (int e = 0; e < W; ++e) o[e] = old[e] + o[e];
                    }
                    store16<S>(dx + off + col, S::pack(o));
                    if (want_dg) {
#pragma unroll
                        for (int e = 0; e < W; ++e) dg[k][e] += fd[e] * (fx[e] * r);
                    }
                }
            }
        }
    }

    if (!want_dg) return;
    float* prow = partials + static_cast<int64_t>(blockIdx.x) * cols;
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
        for (int c = threadIdx.x; c < cols; c += BLOCK) {
            float acc = lds_part[c];
#pragma unroll
            for (int q = 1; q < G; ++q) acc += lds_part[q * cols + c];
            prow[c] = acc;
        }
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
    __shared__ float red[2][16];
    const int64_t row = blockIdx.x;
    if (row >= rows) return;  // block-uniform
    const int64_t off = row * static_cast<int64_t>(cols);
    float ss = 0.0f;
    for (int c = threadIdx.x; c < cols; c += kBlock) {
        const float v = S::get(x + off + c);
        ss += v * v;
    }
    ss = row_sum<kBlock>(ss, red, 0);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    if (threadIdx.x == 0) inv_rms[row] = r;
    for (int c = threadIdx.x; c < cols; c += kBlock) {
        float v = S::get(x + off + c) * r;
        if (gamma) v = v * S::get(gamma + c);
        S::put(y + off + c, v);
    }
}

template <class S>
__global__ __launch_bounds__(kBlock) void rms_bwd_looped(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, float* __restrict__ partials, int64_t rows, int cols,
    int64_t rpb, int accumulate) {
    __shared__ float red[2][16];
    const int64_t row_begin = static_cast<int64_t>(blockIdx.x) * rpb;
    const int64_t row_end = row_begin + rpb < rows ? row_begin + rpb : rows;
    const float inv_cols = 1.0f / static_cast<float>(cols);
    float* prow = partials ? partials + static_cast<int64_t>(blockIdx.x) * cols : nullptr;
    int parity = 0;
    for (int64_t row = row_begin; row < row_end; ++row, parity ^= 1) {
        const int64_t off = row * static_cast<int64_t>(cols);
        float dot = 0.0f;
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            float g = S::get(dy + off + c);
            if (gamma) g = g * S::get(gamma + c);
            dot += g * S::get(x + off + c);
        }
        dot = row_sum<kBlock>(dot, red, parity);
        const float r = inv_rms[row];
        const float s = (r * r * dot) * inv_cols;
        const bool first = row == row_begin;
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            const float xv = S::get(x + off + c);
            const float d = S::get(dy + off + c);
            const float g = gamma ? d * S::get(gamma + c) : d;
            float o = r * (g - xv * s);
            if (accumulate) o = S::get(dx + off + c) + o;
            S::put(dx + off + c, o);
            if (prow) {
                const float t = d * (xv * r);
                prow[c] = first ? t : prow[c] + t;
            }
        }
    }
}

// ---- broadcast multiply (unfused ag::rms(x) * gamma) -------------------------
template <class S>
__global__ __launch_bounds__(kBlock) void mul_rowbcast_fwd_kernel(
    const typename S::T* __restrict__ a, const typename S::T* __restrict__ b,
    typename S::T* __restrict__ y, int64_t rows, int cols, int vec) {
    // vec: 1 when a/b/y are 16-byte aligned and cols % kVec == 0.
    constexpr int W = S::kVec;
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const int64_t off = row * static_cast<int64_t>(cols);
    if (vec) {
        for (int c = threadIdx.x * W; c < cols; c += kBlock * W) {
            float fa[W], fb[W];
            S::unpack(load16<S>(a + off + c), fa);
            S::unpack(load16<S>(b + c), fb);
#pragma unroll
            for (int e = 0; e < W; ++e) fa[e] = fa[e] * fb[e];
            store16<S>(y + off + c, S::pack(fa));
        }
    } else {
        for (int c = threadIdx.x; c < cols; c += kBlock)
            S::put(y + off + c, S::get(a + off + c) * S::get(b + c));
    }
}

// da (+)= gy*b; partial row of this block (+)= gy*a (owned-column RMW).
template <class S>
__global__ __launch_bounds__(kBlock) void mul_rowbcast_bwd_kernel(
    const typename S::T* __restrict__ gy, const typename S::T* __restrict__ a,
    const typename S::T* __restrict__ b, typename S::T* __restrict__ da,
    float* __restrict__ partials, int64_t rows, int cols, int64_t rpb, int accumulate) {
    const int64_t row_begin = static_cast<int64_t>(blockIdx.x) * rpb;
    const int64_t row_end = row_begin + rpb < rows ? row_begin + rpb : rows;
    float* prow = partials ? partials + static_cast<int64_t>(blockIdx.x) * cols : nullptr;
    for (int64_t row = row_begin; row < row_end; ++row) {
        const int64_t off = row * static_cast<int64_t>(cols);
        const bool first = row == row_begin;
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            const float g = S::get(gy + off + c);
            if (da) {
                float o = g * S::get(b + c);
                if (accumulate) o = S::get(da + off + c) + o;
                S::put(da + off + c, o);
            }
            if (prow) {
                const float t = g * S::get(a + off + c);
                prow[c] = first ? t : prow[c] + t;
            }
        }
    }
}

// ---- dgamma: fixed-order column sum of the partial rows ------------------------
// Workgroup: 64 columns x 4 row splits.  Split s sums partial rows s, s+4, ...
// in increasing order in fp64; the 4 split sums are then added in split order.
__global__ __launch_bounds__(kBlock) void dgamma_finalize(const float* __restrict__ partials,
                                                          float* __restrict__ dgamma,
                                                          int64_t nblk, int cols,
                                                          int accumulate) {
    __shared__ double red[4][64];
    const int lane = threadIdx.x & 63;
    const int split = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    double acc = 0.0;
    if (c < cols)
        for (int64_t b = split; b < nblk; b += 4) acc += partials[b * cols + c];
    red[split][lane] = acc;
    __syncthreads();
    if (split == 0 && c < cols) {
        const double tot = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
        const float v = static_cast<float>(tot);
        dgamma[c] = accumulate ? dgamma[c] + v : v;
    }
}

__global__ __launch_bounds__(kBlock) void fill_zero_f32(float* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// ---- launch plans -------------------------------------------------------------

struct RowPlan {
    int tpr = 0;  // lanes per row; 0 = looped kernel
    int nv = 0;   // 16-byte slots per lane
};

// (TPR, NV) pairs with resident instantiations.  Every entry compiles
// without register spills for both storage types (checked with
// -Rpass-analysis=kernel-resource-usage); wider rows take the looped kernels.
#define AGK_FWD_SHAPES(X) \
    X(1, 1) X(2, 1) X(4, 1) X(8, 1) X(16, 1) X(32, 1) X(64, 1) \
    X(64, 2) X(64, 4) X(64, 8) X(64, 16) \
    X(128, 8) X(128, 16) \
    X(256, 8) X(256, 16) \
    X(512, 8) X(512, 16) \
    X(1024, 8)

#define AGK_BWD_SHAPES(X) \
    X(1, 1) X(2, 1) X(4, 1) X(8, 1) X(16, 1) X(32, 1) X(64, 1) \
    X(64, 2) X(64, 4) X(64, 8) \
    X(128, 4) X(128, 8) \
    X(256, 4) X(256, 8) \
    X(512, 4) X(512, 8) \
    X(1024, 4)

struct Shape2 { int tpr, nv; };
constexpr Shape2 kFwdShapes[] = {
#define AGK_X(a, b) {a, b},
    AGK_FWD_SHAPES(AGK_X)
#undef AGK_X
};
constexpr Shape2 kBwdShapes[] = {
#define AGK_X(a, b) {a, b},
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
};

// Pick the resident shape for a row of `nslot` 16-byte slots.  Among shapes
// that fit, prefer the highest slot utilisation, then the smaller TPR (no
// cross-wave exchange).  For the backward, `lds_cap` bounds the
// [groups][cols] fp32 combine buffer.
template <size_t N>
inline RowPlan choose_plan(const Shape2 (&shapes)[N], int64_t nslot, int64_t cols,
                           int64_t lds_cap) {
    RowPlan best;
    double best_util = -1.0;
    for (const Shape2& s : shapes) {
        const int64_t need_nv = (nslot + s.tpr - 1) / s.tpr;
        if (need_nv > s.nv) continue;
        if (s.nv > 1 && need_nv <= s.nv / 2) continue;  // a smaller NV fits
        const int groups = s.tpr >= kBlock ? 1 : kBlock / s.tpr;
        if (lds_cap > 0 && groups > 1 && groups * cols * 4 > lds_cap) continue;
        const double util = static_cast<double>(nslot) / (static_cast<double>(s.tpr) * s.nv);
        if (util > best_util + 1e-9) {
            best_util = util;
            best.tpr = s.tpr;
            best.nv = s.nv;
        }
    }
    return best;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t bwd_rows_per_block(int64_t rows) {
    int64_t rpb = (rows + kTargetBlocks - 1) / kTargetBlocks;
    return rpb < kMinRowsPerBlock ? kMinRowsPerBlock : rpb;
}
inline int64_t bwd_num_blocks(int64_t rows) {
    if (rows <= 0) return 0;
    const int64_t rpb = bwd_rows_per_block(rows);
    return (rows + rpb - 1) / rpb;
}

inline int status_from_hip(hipError_t e) { return e == hipSuccess ? AGK_OK : AGK_EHIP; }

inline int check_launch() { return status_from_hip(hipGetLastError()); }

template <class S>
int launch_fwd(const void* x, const void* gamma, void* y, float* inv_rms, int64_t rows,
               int cols, float eps, hipStream_t st) {
    using T = typename S::T;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    T* yp = static_cast<T*>(y);
    const bool vec = (cols % S::kVec) == 0 && aligned16(x) && aligned16(y) &&
                     (gamma == nullptr || aligned16(gamma));
    RowPlan p;
    if (vec) p = choose_plan(kFwdShapes, cols / S::kVec, cols, 0);
    if (p.tpr == 0) {
        if (rows > 0x7fffffffLL) return AGK_EINVAL;
        hipLaunchKernelGGL(rms_fwd_looped<S>, dim3(static_cast<unsigned>(rows)), dim3(kBlock), 0,
                           st, xp, gp, yp, inv_rms, rows, cols, eps);
        return check_launch();
    }
    const int block = p.tpr > kBlock ? p.tpr : kBlock;
    const int groups = block / p.tpr;
    const int64_t grid = (rows + groups - 1) / groups;
    if (grid > 0x7fffffffLL) return AGK_EINVAL;
#define AGK_X(a, b)                                                                         \
    if (p.tpr == a && p.nv == b) {                                                          \
        hipLaunchKernelGGL((rms_fwd_resident<S, a, b>), dim3(static_cast<unsigned>(grid)),  \
                           dim3(block), 0, st, xp, gp, yp, inv_rms, rows, cols, eps);       \
        return check_launch();                                                              \
    }
    AGK_FWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

template <class S>
int launch_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
               void* dx, float* partials, int64_t rows, int cols, int accumulate,
               hipStream_t st) {
    using T = typename S::T;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* dyp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    const int64_t rpb = bwd_rows_per_block(rows);
    const int64_t nblk = bwd_num_blocks(rows);
    if (nblk > 0x7fffffffLL) return AGK_EINVAL;
    const bool vec = (cols % S::kVec) == 0 && aligned16(x) && aligned16(dy) && aligned16(dx) &&
                     (gamma == nullptr || aligned16(gamma));
    RowPlan p;
    if (vec) p = choose_plan(kBwdShapes, cols / S::kVec, cols, 60 * 1024);
    if (p.tpr == 0) {
        hipLaunchKernelGGL(rms_bwd_looped<S>, dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0,
                           st, xp, gp, inv_rms, dyp, dxp, partials, rows, cols, rpb, accumulate);
        return check_launch();
    }
    const int block = p.tpr > kBlock ? p.tpr : kBlock;
    const int groups = block / p.tpr;
    const size_t lds = (partials && groups > 1) ? static_cast<size_t>(groups) * cols * 4 : 0;
#define AGK_X(a, b)                                                                          \
    if (p.tpr == a && p.nv == b) {                                                           \
        hipLaunchKernelGGL((rms_bwd_resident<S, a, b>), dim3(static_cast<unsigned>(nblk)),   \
                           dim3(block), lds, st, xp, gp, inv_rms, dyp, dxp, partials, rows,  \
                           cols, rpb, accumulate);                                           \
        return check_launch();                                                               \
    }
    AGK_BWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

inline int launch_finalize(const float* partials, float* dgamma, int64_t nblk, int cols,
                           int accumulate, hipStream_t st) {
    const unsigned grid = static_cast<unsigned>((cols + 63) / 64);
    hipLaunchKernelGGL(dgamma_finalize, dim3(grid), dim3(kBlock), 0, st, partials, dgamma, nblk,
                       cols, accumulate);
    return check_launch();
}

inline int zero_fill(float* p, int64_t n, hipStream_t st) {
    if (n <= 0) return AGK_OK;
    const int64_t grid = (n + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(fill_zero_f32, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, st, p,
                       n);
    return check_launch();
}

// Validates sizes common to every entry point.  Returns AGK_OK, or an error.
inline int check_sizes(int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return AGK_EINVAL;
    if (cols > 0x7fffffffLL) return AGK_EINVAL;
    if (cols > 0 && rows > INT64_MAX / cols) return AGK_EINVAL;
    return AGK_OK;
}

inline bool valid_dtype(int dt) { return dt == AGK_F32 || dt == AGK_BF16; }

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
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == AGK_F32)
        return launch_fwd<F32>(x, gamma, y, inv_rms, rows, static_cast<int>(cols), eps, st);
    return launch_fwd<BF16>(x, gamma, y, inv_rms, rows, static_cast<int>(cols), eps, st);
}

size_t agk_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
    if (agk::check_sizes(rows, cols) != AGK_OK || rows == 0 || cols == 0) return 0;
    return static_cast<size_t>(agk::bwd_num_blocks(rows)) * static_cast<size_t>(cols) * 4u;
}

int agk_rmsnorm_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
                    void* dx, float* dgamma, void* workspace, size_t workspace_bytes,
                    int64_t rows, int64_t cols, int dtype, int accumulate,
                    agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (rows == 0 || cols == 0) {
        if (dgamma && !accumulate && cols > 0) return zero_fill(dgamma, cols, st);
        return AGK_OK;
    }
    if (!x || !inv_rms || !dy || !dx) return AGK_EINVAL;
    float* partials = nullptr;
    if (dgamma) {
        const size_t need = agk_rmsnorm_bwd_workspace_bytes(rows, cols);
        if (!workspace || workspace_bytes < need) return AGK_EWORKSPACE;
        partials = static_cast<float*>(workspace);
    }
    const int c = static_cast<int>(cols);
    int rc = dtype == AGK_F32
                 ? launch_bwd<F32>(x, gamma, inv_rms, dy, dx, partials, rows, c, accumulate != 0, st)
                 : launch_bwd<BF16>(x, gamma, inv_rms, dy, dx, partials, rows, c, accumulate != 0, st);
    if (rc != AGK_OK || !dgamma) return rc;
    return launch_finalize(partials, dgamma, bwd_num_blocks(rows), c, accumulate != 0, st);
}

int agk_mul_rowbcast_fwd(const void* a, const void* b, void* y, int64_t rows, int64_t cols,
                         int dtype, agk_stream_t stream) {
    using namespace agk;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (rows == 0 || cols == 0) return AGK_OK;
    if (!a || !b || !y) return AGK_EINVAL;
    if (rows > 0x7fffffffLL) return AGK_EINVAL;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int c = static_cast<int>(cols);
    if (dtype == AGK_F32) {
        const int vec = (c % F32::kVec) == 0 && aligned16(a) && aligned16(b) && aligned16(y);
        hipLaunchKernelGGL(mul_rowbcast_fwd_kernel<F32>, dim3(static_cast<unsigned>(rows)),
                           dim3(kBlock), 0, st, static_cast<const float*>(a),
                           static_cast<const float*>(b), static_cast<float*>(y), rows, c, vec);
    } else {
        const int vec = (c % BF16::kVec) == 0 && aligned16(a) && aligned16(b) && aligned16(y);
        hipLaunchKernelGGL(mul_rowbcast_fwd_kernel<BF16>, dim3(static_cast<unsigned>(rows)),
                           dim3(kBlock), 0, st, static_cast<const uint16_t*>(a),
                           static_cast<const uint16_t*>(b), static_cast<uint16_t*>(y), rows, c,
                           vec);
    }
    return check_launch();
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
    if (rows == 0 || cols == 0) {
        if (db && !accumulate && cols > 0) return zero_fill(db, cols, st);
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
    const int64_t rpb = bwd_rows_per_block(rows);
    const int64_t nblk = bwd_num_blocks(rows);
    if (nblk > 0x7fffffffLL) return AGK_EINVAL;
    const int c = static_cast<int>(cols);
    const int acc = accumulate != 0;
    if (dtype == AGK_F32) {
        hipLaunchKernelGGL(mul_rowbcast_bwd_kernel<F32>, dim3(static_cast<unsigned>(nblk)),
                           dim3(kBlock), 0, st, static_cast<const float*>(gy),
                           static_cast<const float*>(a), static_cast<const float*>(b),
                           static_cast<float*>(da), partials, rows, c, rpb, acc);
    } else {
        hipLaunchKernelGGL(mul_rowbcast_bwd_kernel<BF16>, dim3(static_cast<unsigned>(nblk)),
                           dim3(kBlock), 0, st, static_cast<const uint16_t*>(gy),
                           static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                           static_cast<uint16_t*>(da), partials, rows, c, rpb, acc);
    }
    int rc = check_launch();
    if (rc != AGK_OK || !db) return rc;
    return launch_finalize(partials, db, nblk, c, acc, st);
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

const char* agk_version(void) { return "agk_rmsnorm 0.1 gfx950"; }

}  // extern "C"
