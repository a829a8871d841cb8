// bcast.hip -- element-wise multiply under numpy broadcasting and its VJP:
// mul_nodeops for operands of any broadcast-compatible shapes
// (cgadimpl/src/ops/arithmetic.cpp:31-39, `a->value * b->value`) and vjp_Mul
// (cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:54-59) with reduce_for_broadcast
// (:15-35): the gradient of an operand is gy * other, summed over the axes on
// which that operand was broadcast (axes it lacks, or where its extent is 1
// and the output's is not).
//
// The hot broadcast of the RMSNorm layer (a row vector over the rows) has its
// own kernels in rowops.hip; this file covers every other shape pair, e.g.
// [B, T, D] * [B, 1, D], [R, 1] * [1, C], a scalar times a tensor.
//
// Layout: all operands contiguous, row-major.  Shapes align at the trailing
// axis; after alignment each axis of an operand has the output's extent or 1.
// The host merges adjacent axes that both operands walk contiguously (and
// drops extent-1 output axes), so a launch sees at most 8 axes, usually 2-3.
//
// Forward / full-shape gradient (y (+)= a * b): one workgroup row per run of
// the innermost output axis; its base offsets into a and b are decomposed once
// per run, the lanes walk the run, 16 bytes at a time when the innermost axis
// is contiguous or broadcast in both operands and aligned (element by element
// otherwise).  HBM-bound: reads a and b (b often from cache), writes y.
//
// Reduced gradient (d[j] (+)= sum over the broadcast positions of gy * other),
// accumulating exact products in fp64 and rounding to fp32 once, in an order
// fixed by the shapes (results identical run to run):
//  - the output keeps the innermost axis ([B, T, D] -> [B, 1, D]): a lane per
//    output element, 64 consecutive ones per workgroup, each of its four waves
//    summing a contiguous quarter of the reduced positions (loads contiguous
//    across the lanes); the quarters are added in order;
//  - otherwise (the innermost axis is reduced: [R, C] -> [R, 1]): one wave
//    (short sums) or one 256-lane workgroup (long sums) per output element;
//    lane l takes positions l, l + lanes, ... of the reduced index space in
//    row-major order, and the lanes' partials meet in a fixed tree in LDS.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "agk_rmsnorm.h"
#include "rowcommon.hpp"

namespace agk {

constexpr int kBcastMaxDims = 8;
constexpr int kBcastBlock = 256;

// Output axes (outermost first) with each operand's element stride (0 where it
// is broadcast).
struct BcastGeom {
    int nd;
    int64_t size[kBcastMaxDims];
    int64_t sa[kBcastMaxDims];
    int64_t sb[kBcastMaxDims];
};

// A gradient reduction: the kept axes (extent > 1 in the target, in order,
// so the target's own offset is the row-major index over them) and the
// reduced axes; strides into gy (the output layout) and into the other
// operand for each.
struct BcastRed {
    int nk, nr;
    int64_t ksize[kBcastMaxDims], kgy[kBcastMaxDims], ko[kBcastMaxDims];
    int64_t rsize[kBcastMaxDims], rgy[kBcastMaxDims], ro[kBcastMaxDims];
    int64_t rtotal;  // product of rsize
};

// y[o] (+)= a[.] * b[.] over the output; each block row handles runs of the
// innermost axis (grid-stride over runs).  The product is rounded to storage
// before an accumulating add, as `grad += g` rounds g first.
template <class S>
__global__ __launch_bounds__(kBcastBlock) void bcast_mul_kernel(const typename S::T* __restrict__ a,
                                                               const typename S::T* __restrict__ b,
                                                               typename S::T* __restrict__ y,
                                                               const BcastGeom g, int64_t runs,
                                                               int accumulate) {
    const int last = g.nd - 1;
    const int64_t inner = g.size[last];
    for (int64_t run = blockIdx.y; run < runs; run += gridDim.y) {
        int64_t oa = 0, ob = 0, rem = run;
        for (int d = last - 1; d >= 0; --d) {
            const int64_t c = rem % g.size[d];
            rem /= g.size[d];
            oa += c * g.sa[d];
            ob += c * g.sb[d];
        }
        typename S::T* yr = y + run * inner;
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBcastBlock + threadIdx.x; i < inner;
             i += static_cast<int64_t>(gridDim.x) * kBcastBlock) {
            const float p = S::get(a + oa + i * g.sa[last]) * S::get(b + ob + i * g.sb[last]);
            if (accumulate)
                S::put(yr + i, acc_add(S::get(yr + i), S::stored(p)));
            else
                S::put(yr + i, p);
        }
    }
}

// d[j] (+)= sum over reduced positions of gy * other, fp64, fixed order.
// LANES lanes per element of d (64: one wave; 256: the whole workgroup).
template <class S, int LANES>
__global__ __launch_bounds__(kBcastBlock) void bcast_reduce_kernel(
    const typename S::T* __restrict__ gy, const typename S::T* __restrict__ other,
    float* __restrict__ d, const BcastRed r, int64_t n_out, int accumulate) {
    constexpr int kPer = kBcastBlock / LANES;  // elements of d per workgroup
    __shared__ double part[kBcastBlock];
    const int lane = threadIdx.x % LANES;
    const int slot = threadIdx.x / LANES;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kPer; base < n_out;
         base += static_cast<int64_t>(gridDim.x) * kPer) {
        const int64_t j = base + slot;
        double acc = 0.0;
        if (j < n_out) {
            int64_t og = 0, oo = 0, rem = j;
            for (int k = r.nk - 1; k >= 0; --k) {
                const int64_t c = rem % r.ksize[k];
                rem /= r.ksize[k];
                og += c * r.kgy[k];
                oo += c * r.ko[k];
            }
            // position q = oq * inner_r + i (oq over the outer reduced axes, i
            // along the innermost one); q steps by LANES, and the outer offsets
            // are re-derived only when i leaves the innermost axis
            const int ia = r.nr - 1;
            const int64_t inner_r = r.rsize[ia], sg = r.rgy[ia], so = r.ro[ia];
            auto outer = [&](int64_t oq, int64_t& bg, int64_t& bo) {
                bg = og;
                bo = oo;
                for (int k = ia - 1; k >= 0; --k) {
                    const int64_t c = oq % r.rsize[k];
                    oq /= r.rsize[k];
                    bg += c * r.rgy[k];
                    bo += c * r.ro[k];
                }
            };
            int64_t oq = lane / inner_r, i = lane - oq * inner_r, bg, bo;
            outer(oq, bg, bo);
            for (int64_t q = lane; q < r.rtotal; q += LANES) {
                acc += static_cast<double>(S::get(gy + bg + i * sg)) *
                       static_cast<double>(S::get(other + bo + i * so));
                i += LANES;
                if (i >= inner_r) {
                    oq += i / inner_r;
                    i %= inner_r;
                    outer(oq, bg, bo);
                }
            }
        }
        part[threadIdx.x] = acc;
        __syncthreads();
#pragma unroll
        for (int w = LANES / 2; w > 0; w /= 2) {
            if (lane < w) part[threadIdx.x] += part[threadIdx.x + w];
            __syncthreads();
        }
        if (lane == 0 && j < n_out) {
            const double old = accumulate ? static_cast<double>(d[j]) : 0.0;
            d[j] = static_cast<float>(old + part[threadIdx.x]);
        }
        __syncthreads();
    }
}

// The same product with 16-byte accesses, when the innermost axis is
// contiguous (stride 1) or broadcast (stride 0) in both operands, its extent a
// multiple of the slot width and every base 16-byte aligned.  A run's base
// offsets are computed once per workgroup and a broadcast operand's value once
// per run; the lanes walk the run's slots.  Same roundings as the element-wise
// kernel, so the results are the same bits.
template <class S>
__global__ __launch_bounds__(kBcastBlock) void bcast_mul_vec_kernel(
    const typename S::T* __restrict__ a, const typename S::T* __restrict__ b,
    typename S::T* __restrict__ y, const BcastGeom g, int64_t runs, int accumulate) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    const int last = g.nd - 1;
    const int64_t inner = g.size[last];
    const int64_t nvec = inner / W;
    const bool a_vec = g.sa[last] != 0;
    const bool b_vec = g.sb[last] != 0;
    for (int64_t run = blockIdx.y; run < runs; run += gridDim.y) {
        int64_t oa = 0, ob = 0, rem = run;
        for (int d = last - 1; d >= 0; --d) {
            const int64_t c = rem % g.size[d];
            rem /= g.size[d];
            oa += c * g.sa[d];
            ob += c * g.sb[d];
        }
        const T* ar = a + oa;
        const T* br = b + ob;
        T* yr = y + run * inner;
        const float as = a_vec ? 0.0f : S::get(ar);
        const float bs = b_vec ? 0.0f : S::get(br);
        for (int64_t v = static_cast<int64_t>(blockIdx.x) * kBcastBlock + threadIdx.x; v < nvec;
             v += static_cast<int64_t>(gridDim.x) * kBcastBlock) {
            float fa[W], fb[W], p[W];
            if (a_vec) {
                S::unpack(load16<S>(ar + v * W), fa);
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) fa[e] = as;
            }
            if (b_vec) {
                S::unpack(load16<S>(br + v * W), fb);
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) fb[e] = bs;
            }
#pragma unroll
            for (int e = 0; e < W; ++e) p[e] = fa[e] * fb[e];
            if (accumulate) {
                float old[W];
                S::unpack(load16<S>(yr + v * W), old);
#pragma unroll
                for (int e = 0; e < W; ++e) p[e] = acc_add(old[e], S::stored(p[e]));
            }
            store16_stream<S>(yr + v * W, S::pack(p));
        }
    }
}

// A reduction whose output keeps the innermost axis (e.g. [B, T, D] summed to
// [B, 1, D]): each workgroup takes 64 consecutive outputs, one per lane, so a
// wave's loads are contiguous in gy.  The reduced index space is cut into four
// contiguous quarters, one per wave; a wave walks its quarter along the
// innermost reduced axis (divisions only when it moves to the next outer
// reduced position), accumulating exact products in fp64.  The quarters'
// partials are added in quarter order: a fixed order for the shapes.
template <class S>
__global__ __launch_bounds__(kBcastBlock) void bcast_reduce_cols_kernel(
    const typename S::T* __restrict__ gy, const typename S::T* __restrict__ other,
    float* __restrict__ d, const BcastRed r, int64_t n_out, int accumulate) {
    __shared__ double part[4][64];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int inner_ax = r.nr - 1;
    const int64_t inner_r = r.rsize[inner_ax];
    const int64_t sg = r.rgy[inner_ax], so = r.ro[inner_ax];
    const int64_t q0 = r.rtotal * w / 4, q1 = r.rtotal * (w + 1) / 4;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * 64; base < n_out;
         base += static_cast<int64_t>(gridDim.x) * 64) {
        const int64_t j = base + lane;
        double acc = 0.0;
        if (j < n_out) {
            int64_t og = 0, oo = 0, rem = j;
            for (int k = r.nk - 1; k >= 0; --k) {
                const int64_t c = rem % r.ksize[k];
                rem /= r.ksize[k];
                og += c * r.kgy[k];
                oo += c * r.ko[k];
            }
            for (int64_t q = q0; q < q1;) {
                const int64_t oq = q / inner_r;
                const int64_t i0 = q - oq * inner_r;
                int64_t pg = og, po = oo, qr = oq;
                for (int k = inner_ax - 1; k >= 0; --k) {
                    const int64_t c = qr % r.rsize[k];
                    qr /= r.rsize[k];
                    pg += c * r.rgy[k];
                    po += c * r.ro[k];
                }
                const int64_t i1 = inner_r - i0 < q1 - q ? inner_r : i0 + (q1 - q);
#pragma unroll 4
                for (int64_t i = i0; i < i1; ++i)
                    acc += static_cast<double>(S::get(gy + pg + i * sg)) *
                           static_cast<double>(S::get(other + po + i * so));
                q += i1 - i0;
            }
        }
        part[w][lane] = acc;
        __syncthreads();
        if (w == 0 && j < n_out) {
            const double s = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
            const double old = accumulate ? static_cast<double>(d[j]) : 0.0;
            d[j] = static_cast<float>(old + s);
        }
        __syncthreads();
    }
}

// Zeros n 16-bit words (a kernel rather than a memset node, so that the call
// can be captured into a graph).
__global__ __launch_bounds__(kBcastBlock) void bcast_zero_kernel(uint16_t* __restrict__ p,
                                                                int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBcastBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBcastBlock)
        p[i] = 0;
}

// ---- host side -------------------------------------------------------------------

// Row-major contiguous strides of an operand aligned to nd output axes (its
// missing leading axes and its extent-1 axes get stride 0).
struct Aligned {
    int64_t size[kBcastMaxDims];
    int64_t stride[kBcastMaxDims];
};

inline bool align_operand(const int64_t* shape, int ndim, int nd, Aligned& out) {
    int64_t s = 1;
    for (int i = nd - 1; i >= 0; --i) {
        const int src = i - (nd - ndim);
        const int64_t e = src >= 0 ? shape[src] : 1;
        if (e < 0) return false;
        out.size[i] = e;
        out.stride[i] = e == 1 ? 0 : s;
        if (e > 0 && s > INT64_MAX / e) return false;
        s *= e;
    }
    return true;
}

// The broadcast output shape of a and b; false when incompatible or too many axes.
inline bool broadcast_shape(const int64_t* as, int an, const int64_t* bs, int bn, int& nd,
                            Aligned& a, Aligned& b, int64_t (&osize)[kBcastMaxDims],
                            int64_t& numel) {
    if (an < 0 || bn < 0 || an > kBcastMaxDims || bn > kBcastMaxDims) return false;
    if ((an && !as) || (bn && !bs)) return false;
    nd = an > bn ? an : bn;
    if (!align_operand(as, an, nd, a) || !align_operand(bs, bn, nd, b)) return false;
    numel = 1;
    for (int i = 0; i < nd; ++i) {
        const int64_t x = a.size[i], y = b.size[i];
        if (x != y && x != 1 && y != 1) return false;
        osize[i] = x == 1 ? y : x;
        if (osize[i] > 0 && numel > INT64_MAX / osize[i]) return false;
        numel *= osize[i];
    }
    return true;
}

// Merges adjacent output axes that both operands walk contiguously and drops
// extent-1 axes; at least one axis remains.
inline BcastGeom make_geom(int nd, const int64_t* osize, const Aligned& a, const Aligned& b) {
    BcastGeom g{};
    g.nd = 0;
    for (int i = 0; i < nd; ++i) {
        if (osize[i] == 1) continue;
        const int64_t sa = a.size[i] == 1 ? 0 : a.stride[i];
        const int64_t sb = b.size[i] == 1 ? 0 : b.stride[i];
        if (g.nd > 0) {
            const int p = g.nd - 1;
            if (g.sa[p] == sa * osize[i] && g.sb[p] == sb * osize[i]) {
                g.size[p] *= osize[i];
                g.sa[p] = sa;
                g.sb[p] = sb;
                continue;
            }
        }
        g.size[g.nd] = osize[i];
        g.sa[g.nd] = sa;
        g.sb[g.nd] = sb;
        ++g.nd;
    }
    if (g.nd == 0) {
        g.nd = 1;
        g.size[0] = 1;
        g.sa[0] = g.sb[0] = 0;
    }
    return g;
}

template <class S>
int launch_bcast_mul(const void* a, const void* b, void* y, const BcastGeom& g, int accumulate,
                     hipStream_t st) {
    const int64_t inner = g.size[g.nd - 1];
    int64_t runs = 1;
    for (int d = 0; d + 1 < g.nd; ++d) runs *= g.size[d];
    const int last = g.nd - 1;
    const bool vec = inner % S::kVec == 0 && (g.sa[last] == 0 || g.sa[last] == 1) &&
                     (g.sb[last] == 0 || g.sb[last] == 1) && aligned16(a) && aligned16(b) &&
                     aligned16(y);
    const int64_t per_run = vec ? inner / S::kVec : inner;
    const int64_t bx = (per_run + kBcastBlock - 1) / kBcastBlock;
    const dim3 grid(static_cast<unsigned>(bx < 1024 ? bx : 1024),
                    static_cast<unsigned>(runs < 65535 ? runs : 65535));
    const auto* ap = static_cast<const typename S::T*>(a);
    const auto* bp = static_cast<const typename S::T*>(b);
    auto* yp = static_cast<typename S::T*>(y);
    if (vec)
        hipLaunchKernelGGL(bcast_mul_vec_kernel<S>, grid, dim3(kBcastBlock), 0, st, ap, bp, yp, g,
                           runs, accumulate);
    else
        hipLaunchKernelGGL(bcast_mul_kernel<S>, grid, dim3(kBcastBlock), 0, st, ap, bp, yp, g, runs,
                           accumulate);
    return check_launch();
}

// The reduction that produces the gradient of operand `t` (aligned to the
// output) from gy and the other operand `o`.
inline BcastRed make_red(int nd, const int64_t* osize, const Aligned& t, const Aligned& o,
                         int64_t& n_out) {
    BcastRed r{};
    int64_t sgy[kBcastMaxDims];
    int64_t s = 1;
    for (int i = nd - 1; i >= 0; --i) {
        sgy[i] = s;
        s *= osize[i];
    }
    n_out = 1;
    r.rtotal = 1;
    for (int i = 0; i < nd; ++i) {
        if (osize[i] == 1) continue;
        const int64_t so = o.size[i] == 1 ? 0 : o.stride[i];
        if (t.size[i] == osize[i]) {
            r.ksize[r.nk] = osize[i];
            r.kgy[r.nk] = sgy[i];
            r.ko[r.nk] = so;
            ++r.nk;
            n_out *= osize[i];
        } else {
            r.rsize[r.nr] = osize[i];
            r.rgy[r.nr] = sgy[i];
            r.ro[r.nr] = so;
            ++r.nr;
            r.rtotal *= osize[i];
        }
    }
    return r;
}

template <class S>
int launch_bcast_reduce(const void* gy, const void* other, float* d, const BcastRed& r,
                        int64_t n_out, int accumulate, hipStream_t st) {
    const auto* g = static_cast<const typename S::T*>(gy);
    const auto* o = static_cast<const typename S::T*>(other);
    if (r.nk >= 1 && r.kgy[r.nk - 1] == 1) {  // the output keeps the innermost axis
        const int64_t blocks = (n_out + 63) / 64;
        hipLaunchKernelGGL(bcast_reduce_cols_kernel<S>,
                           dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)),
                           dim3(kBcastBlock), 0, st, g, o, d, r, n_out, accumulate);
        return check_launch();
    }
    const bool wide = r.rtotal >= 4096;
    const int per = wide ? 1 : kBcastBlock / 64;
    const int64_t blocks = (n_out + per - 1) / per;
    const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
    if (wide)
        hipLaunchKernelGGL((bcast_reduce_kernel<S, kBcastBlock>), grid, dim3(kBcastBlock), 0, st,
                           g, o, d, r, n_out, accumulate);
    else
        hipLaunchKernelGGL((bcast_reduce_kernel<S, 64>), grid, dim3(kBcastBlock), 0, st, g, o,
                           d, r, n_out, accumulate);
    return check_launch();
}

// Whether an aligned operand covers the whole output (its gradient is then
// the element-wise product, in the storage dtype).
inline bool is_full(int nd, const int64_t* osize, const Aligned& t) {
    for (int i = 0; i < nd; ++i)
        if (t.size[i] != osize[i]) return false;
    return true;
}

template <class S>
int bcast_bwd_one(const void* gy, const void* other, const Aligned& t, const Aligned& o,
                  const Aligned& gyal, int nd, const int64_t* osize, void* d, int accumulate,
                  hipStream_t st) {
    if (is_full(nd, osize, t)) {
        // d (+)= gy * other: the forward kernel with gy as the full operand
        const BcastGeom g = make_geom(nd, osize, gyal, o);
        return launch_bcast_mul<S>(gy, other, d, g, accumulate, st);
    }
    int64_t n_out = 0;
    const BcastRed r = make_red(nd, osize, t, o, n_out);
    return launch_bcast_reduce<S>(gy, other, static_cast<float*>(d), r, n_out, accumulate, st);
}

}  // namespace agk

namespace agk {

// dst[i] = value for i < n (a grid-stride loop of 256-lane workgroups).
template <class S>
__global__ __launch_bounds__(256) void fill_kernel(typename S::T* __restrict__ dst, int64_t n,
                                                   float value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
        S::put(dst + i, value);
}

}  // namespace agk

extern "C" int agk_fill(void* dst, int64_t n, float value, int dtype, agk_stream_t stream) {
    using namespace agk;
    if (n < 0) return AGK_EINVAL;
    if (dtype != AGK_F32 && dtype != AGK_BF16) return AGK_EDTYPE;
    if (n == 0) return AGK_OK;
    if (!dst) return AGK_EINVAL;
    clear_pending_error();
    const int64_t blocks64 = (n + 255) / 256;
    const unsigned blocks = static_cast<unsigned>(blocks64 < 4096 ? blocks64 : 4096);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == AGK_F32)
        hipLaunchKernelGGL(fill_kernel<F32>, dim3(blocks), dim3(256), 0, st,
                           static_cast<float*>(dst), n, value);
    else
        hipLaunchKernelGGL(fill_kernel<BF16>, dim3(blocks), dim3(256), 0, st,
                           static_cast<uint16_t*>(dst), n, value);
    return check_launch();
}

extern "C" int agk_mul_bcast_shape(const int64_t* a_shape, int a_ndim, const int64_t* b_shape,
                                   int b_ndim, int64_t* out_shape, int* out_ndim) {
    using namespace agk;
    int nd = 0;
    Aligned a, b;
    int64_t osize[kBcastMaxDims];
    int64_t numel = 0;
    if (!out_ndim) return AGK_EINVAL;
    if (!broadcast_shape(a_shape, a_ndim, b_shape, b_ndim, nd, a, b, osize, numel))
        return AGK_EINVAL;
    *out_ndim = nd;
    if (out_shape)
        for (int i = 0; i < nd; ++i) out_shape[i] = osize[i];
    return AGK_OK;
}

extern "C" int agk_mul_bcast_fwd(const void* a, const int64_t* a_shape, int a_ndim,
                                 const void* b, const int64_t* b_shape, int b_ndim, void* y,
                                 int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    int nd = 0;
    Aligned al, bl;
    int64_t osize[kBcastMaxDims];
    int64_t numel = 0;
    if (!broadcast_shape(a_shape, a_ndim, b_shape, b_ndim, nd, al, bl, osize, numel))
        return AGK_EINVAL;
    if (numel == 0) return AGK_OK;
    if (!a || !b || !y) return AGK_EINVAL;
    clear_pending_error();
    const BcastGeom g = make_geom(nd, osize, al, bl);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int acc = accumulate != 0;
    return dtype == AGK_F32 ? launch_bcast_mul<F32>(a, b, y, g, acc, st)
                            : launch_bcast_mul<BF16>(a, b, y, g, acc, st);
}

extern "C" int agk_mul_bcast_bwd(const void* gy, const void* a, const int64_t* a_shape,
                                 int a_ndim, const void* b, const int64_t* b_shape, int b_ndim,
                                 void* da, void* db, int dtype, int accumulate,
                                 agk_stream_t stream) {
    using namespace agk;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (accumulate & ~AGK_ACCUM_ALL) return AGK_EINVAL;
    int nd = 0;
    Aligned al, bl;
    int64_t osize[kBcastMaxDims];
    int64_t numel = 0;
    if (!broadcast_shape(a_shape, a_ndim, b_shape, b_ndim, nd, al, bl, osize, numel))
        return AGK_EINVAL;
    if (!da && !db) return AGK_OK;
    // an empty output: the gradients are empty sums (zeros), or unchanged
    // when accumulating; an empty operand has an empty gradient
    if (numel == 0) {
        if (accumulate == AGK_ACCUM_ALL) return AGK_OK;
        clear_pending_error();
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        for (int w = 0; w < 2; ++w) {
            void* d = w ? db : da;
            const Aligned& t = w ? bl : al;
            if (!d || (accumulate & (w ? AGK_ACCUM_DGAMMA : AGK_ACCUM_DX))) continue;
            int64_t n = 1;
            for (int i = 0; i < nd; ++i) n *= t.size[i];
            if (n == 0) continue;
            const int64_t words = n * (is_full(nd, osize, t) && dtype == AGK_BF16 ? 1 : 2);
            const int64_t blocks = (words + kBcastBlock - 1) / kBcastBlock;
            hipLaunchKernelGGL(bcast_zero_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                               dim3(kBcastBlock), 0, st, static_cast<uint16_t*>(d), words);
            const int rc = check_launch();
            if (rc != AGK_OK) return rc;
        }
        return AGK_OK;
    }
    if (!gy || (da && !b) || (db && !a)) return AGK_EINVAL;
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    Aligned gyal;  // gy in the output layout
    if (!align_operand(osize, nd, nd, gyal)) return AGK_EINVAL;
    int rc = AGK_OK;
    if (da) {
        const int acc = (accumulate & AGK_ACCUM_DX) != 0;
        rc = dtype == AGK_F32 ? bcast_bwd_one<F32>(gy, b, al, bl, gyal, nd, osize, da, acc, st)
                              : bcast_bwd_one<BF16>(gy, b, al, bl, gyal, nd, osize, da, acc, st);
        if (rc != AGK_OK) return rc;
    }
    if (db) {
        const int acc = (accumulate & AGK_ACCUM_DGAMMA) != 0;
        rc = dtype == AGK_F32 ? bcast_bwd_one<F32>(gy, a, bl, al, gyal, nd, osize, db, acc, st)
                              : bcast_bwd_one<BF16>(gy, a, bl, al, gyal, nd, osize, db, acc, st);
    }
    return rc;
}
