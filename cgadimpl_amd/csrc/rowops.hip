// rowops.hip -- CDNA4 (gfx950) kernels and C ABI (include/agk_rowops.h) for
// the row ops that share the RMSNorm layer's row-reduce skeleton: the
// corrected forward-mode product of RMSNorm, LayerNorm, row softmax and row
// log-sum-exp, with their backward (and forward-mode) products.
//
// Reference behaviour replaced here (paths relative to the reference tree):
//   jvp_RMSNorm            cgadimpl/src/autodiff/autodiff_jvp_ops.cpp:366-379
//                          (with its 1/rms-vs-rms error corrected)
//   laynor_nodeops         cgadimpl/src/ops/normalization.cpp:10-22
//   vjp_LayerNorm          cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:351-365
//   softmax_row_nodeops    cgadimpl/src/ops/reduction.cpp:42-53
//   vjp_SoftmaxRow         autodiff_vjp_ops.cpp:421-428
//   logsumexp_row_nodeops  reduction.cpp:54-66
//   vjp_LogSumExpRow       autodiff_vjp_ops.cpp:430-440
//   jvp_LogSumExpRow       autodiff_jvp_ops.cpp:421-434
// The reference evaluates each of these as a chain of tensor-library kernels
// that materialise every intermediate (max, shifted row, exponentials, sums,
// quotients).  Here every op is one kernel: each input row is read from HBM
// once into registers, the row reductions run on the held values (DPP within
// a wave, LDS across waves), and each output row is written once.
//
// Structure.  An op is a small policy (the structs under "ops") written
// against a row context that offers sum / sum2 / max reductions over the row
// and a store of an element-wise function of it.  Two contexts implement that
// interface: Resident (the row held in registers by TPR lanes, NV 16-byte
// slots per lane, G rows per workgroup -- the launch shapes and plan of the
// RMSNorm forward) and Looped (one 256-lane workgroup per row, element-wise
// accesses that re-read the row from cache; any alignment, any width).  The
// softmax forward and backward and the log-sum-exp backward also have a team
// kernel (rowops_team.hpp) for rows too wide for one workgroup's registers:
// a row over several workgroups that exchange partial sums through a caller
// workspace (the *_ws entry points), so each input row is read once.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "agk_rowops.h"
#include "rowcommon.hpp"

namespace agk {
// The team kernels' wait limit (agk_set_exchange_wait_limit, rmsnorm.hip).
int team_wait_polls();

namespace rowops {

// Pointers and scalars of one call.  Each op names the fields it reads.
struct RowArgs {
    const void* in0 = nullptr;   // row input 0, [rows, cols]
    const void* in1 = nullptr;   // row input 1, [rows, cols]
    const void* col0 = nullptr;  // column vector 0, [cols]
    const void* col1 = nullptr;  // column vector 1, [cols]
    const float* rs0 = nullptr;  // per-row fp32 input 0, [rows]
    const float* rs1 = nullptr;  // per-row fp32 input 1, [rows]
    const void* rsv = nullptr;   // per-row input of the storage type, [rows]
    void* out = nullptr;         // row output, [rows, cols]
    void* out_row = nullptr;     // per-row output of the storage type, [rows]
    float* ws0 = nullptr;        // per-row fp32 output 0, [rows]
    float* ws1 = nullptr;        // per-row fp32 output 1, [rows]
    float eps = 0.0f;
    int acc = 0;                 // out += f instead of out = f
};

// ---- reductions ----------------------------------------------------------------

struct SumR {
    static constexpr float kId = 0.0f;
    __device__ static float op(float a, float b) { return a + b; }
};
// max(a, b) as one v_max_f32.  Written as fmaxf (or any form the compiler
// recognises as a max) it costs three instructions per element here: in IEEE
// mode the compiler first quiets possible signalling NaNs in both operands.  A
// NaN in a row still reaches every result that uses the max, through
// exp(z - max).
struct MaxR {
    static constexpr float kId = -__builtin_inff();
    __device__ static float op(float a, float b) {
        float r;
        asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
        return r;
    }
};

// exp(x) = 2^(x * log2(e)) on the hardware exp2 instruction (v_exp_f32).  The
// product x*log2(e) is rounded once, so the relative error is about
// |x| * 2^-24 * ln(2) plus the instruction's 1 ulp: for the shifted logits of
// softmax and log-sum-exp (x <= 0) the large terms (x near 0) are accurate to
// ~1 ulp and the error of the small ones is far below them.  -inf gives 0.
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// Reduction over the TPR (<= 64) lanes of a row group with the pairing of
// group_sum: every pairing is symmetric, so all lanes of the group end with
// the same bits.
template <int TPR, class R>
__device__ __forceinline__ float group_reduce(float v) {
    if constexpr (TPR >= 2) v = R::op(v, dpp_mov<0xb1>(v));
    if constexpr (TPR >= 4) v = R::op(v, dpp_mov<0x4e>(v));
    if constexpr (TPR >= 8) v = R::op(v, dpp_mov<0x141>(v));
    if constexpr (TPR >= 16) v = R::op(v, dpp_mov<0x140>(v));
    if constexpr (TPR >= 32)
        v = R::op(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f)));
    if constexpr (TPR >= 64)
        v = R::op(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
    return v;
}

// LDS slots per parity for N <= 2 values per row.
template <int TPR, int G>
constexpr int red_slots() {
    return TPR > 64 ? 2 * G * (TPR / 64) : 1;
}

// Row reduction of N values for rows spread over TPR lanes, G rows per
// workgroup.  For TPR > 64 the per-wave results meet in `red` (double-buffered
// by `parity`, one barrier per reduction) and are combined in wave order.
template <int TPR, int G, int N, class R>
__device__ __forceinline__ void row_reduce(float (&v)[N],
                                           float (*red)[TPR > 64 ? 2 * G * (TPR / 64) : 1],
                                           int parity) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = group_reduce<TPR, R>(v[i]);
    if constexpr (TPR > 64) {
        constexpr int kWaves = TPR / 64;
        const int lane = threadIdx.x & 63;
        const int base = (threadIdx.x / TPR) * kWaves;
        const int wave_in_row = (threadIdx.x % TPR) >> 6;
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < N; ++i) red[parity][(base + wave_in_row) * N + i] = v[i];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < N; ++i) {
            float s = red[parity][base * N + i];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) s = R::op(s, red[parity][(base + w) * N + i]);
            v[i] = s;
        }
    }
}

// ---- row contexts --------------------------------------------------------------
// Interface used by the ops (every lane of the workgroup calls the reductions;
// store and the put_* calls act only for rows that exist):
//   ncols, inv_cols                  cols and 1 / cols as floats
//   sum(f), max(f)                   reduce f(a, b) over the row
//   sum2(f, s0, s1)                  f(a, b, o) fills o[2]; both summed
//   sum_keep(f)                      sum of f(a, b) over the row, keeping the
//                                    values where the row is held in registers
//   max_sumexp<KEEP>(m, s)           m = max over the row of a, s = sum of
//                                    fast_exp(a - m) (KEEP: kept as sum_keep
//                                    keeps them; without KEEP the resident
//                                    context folds the shift into the
//                                    exponent); one online pass in LoopedVec
//   store_kept(out, acc, f, g)       out[col] (+)= g(f(a, b)), f's values as
//                                    kept by the last sum_keep (recomputed by
//                                    the looped context)
//   store(out, acc, c0, d0, c1, d1, f)
//                                    out[col] (+)= f(a, b, u, v), u = c0[col]
//                                    (d0 when c0 is null), v likewise
//   row_f32(p), row_val(p)           p[row] (fp32 / storage type)
//   put_f32(p, v), put_val(p, v)     p[row] = v (fp32 / storage type)
// a and b are the elements of in0 and in1 (b = 0 for one-input ops).

template <class S, int TPR, int NV, int G, int NIN>
struct Resident {
    using T = typename S::T;
    static constexpr int W = S::kVec;
    static constexpr int kSlots = red_slots<TPR, G>();
    // 16 slots per lane (rows of 8193-16384 slots, one row per 1024-lane
    // workgroup): the packed row fills 64 registers, so nothing derived from
    // it is kept across a row reduction -- the exponentials are recomputed
    // when stored, and the slots are made opaque after each reduction so the
    // compiler re-unpacks them instead of holding 128 unpacked values.
    static constexpr bool kBig = NV >= 16;

    float (*red)[kSlots];
    int parity = 0;
    int t;
    int64_t row;
    bool active;
    int cols;
    float ncols, inv_cols;
    u32x4 a[NV], b[NV];
    float kept[kBig ? 1 : NV][W];

    __device__ Resident(const RowArgs& p, int64_t rows, int cols_, float (*red_)[kSlots])
        : red(red_), cols(cols_) {
        t = threadIdx.x % TPR;
        row = static_cast<int64_t>(blockIdx.x) * G + threadIdx.x / TPR;
        active = row < rows;
        ncols = static_cast<float>(cols);
        inv_cols = 1.0f / ncols;
        const int64_t off = (active ? row : 0) * static_cast<int64_t>(cols);
        const T* x = static_cast<const T*>(p.in0) + off;
        const T* y = NIN == 2 ? static_cast<const T*>(p.in1) + off : nullptr;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            const bool ok = active && col < cols;
            a[k] = ok ? load16_stream<S>(x + col) : u32x4{0u, 0u, 0u, 0u};
            if constexpr (NIN == 2)
                b[k] = ok ? load16_stream<S>(y + col) : u32x4{0u, 0u, 0u, 0u};
        }
    }

    template <class R, int N, class F>
    __device__ __forceinline__ void reduce(float (&res)[N], F f) {
        float part[N][W];
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int e = 0; e < W; ++e) part[i][e] = R::kId;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if ((t + k * TPR) * W < cols) {
                float fa[W], fb[W];
                S::unpack(a[k], fa);
                if constexpr (NIN == 2) S::unpack(b[k], fb);
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    float o[N];
                    f(fa[e], NIN == 2 ? fb[e] : 0.0f, o);
#pragma unroll
                    for (int i = 0; i < N; ++i) part[i][e] = R::op(part[i][e], o[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            float s = part[i][0];
#pragma unroll
            for (int e = 1; e < W; ++e) s = R::op(s, part[i][e]);
            res[i] = s;
        }
        row_reduce<TPR, G, N, R>(res, red, parity);
        parity ^= 1;
        refresh();
    }

    __device__ __forceinline__ void refresh() {
        if constexpr (kBig) {
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                if constexpr (NIN == 2) opaque(a[k], b[k]);
                else asm volatile("" : "+v"(a[k]));
            }
        }
    }

    template <class F>
    __device__ __forceinline__ float sum(F f) {
        float r[1];
        reduce<SumR>(r, [&](float x, float y, float (&o)[1]) { o[0] = f(x, y); });
        return r[0];
    }
    template <class F>
    __device__ __forceinline__ float max(F f) {
        float r[1];
        reduce<MaxR>(r, [&](float x, float y, float (&o)[1]) { o[0] = f(x, y); });
        return r[0];
    }
    template <class F>
    __device__ __forceinline__ void sum2(F f, float& s0, float& s1) {
        float r[2];
        reduce<SumR>(r, f);
        s0 = r[0];
        s1 = r[1];
    }

    // Without KEEP (log-sum-exp forward: only the sum is used) the shift is
    // folded into the exponent, exp2(fma(a, log2(e), -m * log2(e))): one
    // instruction fewer per element than fast_exp(a - m).  The rounding of
    // m * log2(e) scales every term by the same factor 2^d (|d| <= |m| 2^-24
    // log2(e)), i.e. moves log(s) + m by at most |m| 2^-24, the size of one
    // rounding of m.  Special values give what fast_exp(a - m) gives (-inf
    // terms 0, NaN through).
    template <bool KEEP>
    __device__ __forceinline__ void max_sumexp(float& m, float& s) {
        m = max([](float z, float) { return z; });
        const float mm = m;
        auto e = [=](float z, float) { return fast_exp(z - mm); };
        if constexpr (KEEP && !kBig) {
            s = sum_keep(e);
        } else if constexpr (KEEP) {
            s = sum(e);
        } else {
            constexpr float kLog2e = 1.4426950408889634f;
            const float nml = -mm * kLog2e;
            s = sum([=](float z, float) { return __builtin_amdgcn_exp2f(fmaf(z, kLog2e, nml)); });
        }
    }

    template <class F>
    __device__ __forceinline__ float sum_keep(F f) {
        float part[W];
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if ((t + k * TPR) * W < cols) {
                float fa[W], fb[W];
                S::unpack(a[k], fa);
                if constexpr (NIN == 2) S::unpack(b[k], fb);
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    kept[k][e] = f(fa[e], NIN == 2 ? fb[e] : 0.0f);
                    part[e] += kept[k][e];
                }
            }
        }
        float r[1] = {part[0]};
#pragma unroll
        for (int e = 1; e < W; ++e) r[0] += part[e];
        row_reduce<TPR, G, 1, SumR>(r, red, parity);
        parity ^= 1;
        return r[0];
    }

    template <class F, class Gf>
    __device__ __forceinline__ void store_kept(void* out, int acc, F f, Gf g) const {
        if (!active) return;
        T* o = static_cast<T*>(out) + row * static_cast<int64_t>(cols);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            if (col < cols) {
                float r[W];
                if constexpr (kBig) {  // recomputed: the same function of the same value
                    float fa[W], fb[W];
                    S::unpack(a[k], fa);
                    if constexpr (NIN == 2) S::unpack(b[k], fb);
#pragma unroll
                    for (int e = 0; e < W; ++e) r[e] = g(f(fa[e], NIN == 2 ? fb[e] : 0.0f));
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) r[e] = g(kept[k][e]);
                }
                if (acc) {
                    float old[W];
                    S::unpack(load16_stream<S>(o + col), old);
#pragma unroll
                    for (int e = 0; e < W; ++e) r[e] = acc_add(old[e], r[e]);
                }
                store16_stream<S>(o + col, S::pack(r));
            }
        }
    }

    template <class F>
    __device__ __forceinline__ void store(void* out, int acc, const void* c0, float d0,
                                          const void* c1, float d1, F f) const {
        if (!active) return;
        T* o = static_cast<T*>(out) + row * static_cast<int64_t>(cols);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * TPR) * W;
            if (col < cols) {
                float fa[W], fb[W], fu[W], fv[W], r[W];
                S::unpack(a[k], fa);
                if constexpr (NIN == 2) S::unpack(b[k], fb);
                if (c0) {
                    S::unpack(load16<S>(static_cast<const T*>(c0) + col), fu);
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) fu[e] = d0;
                }
                if (c1) {
                    S::unpack(load16<S>(static_cast<const T*>(c1) + col), fv);
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) fv[e] = d1;
                }
#pragma unroll
                for (int e = 0; e < W; ++e) r[e] = f(fa[e], NIN == 2 ? fb[e] : 0.0f, fu[e], fv[e]);
                if (acc) {
                    float old[W];
                    S::unpack(load16_stream<S>(o + col), old);
#pragma unroll
                    for (int e = 0; e < W; ++e) r[e] = acc_add(old[e], r[e]);
                }
                store16_stream<S>(o + col, S::pack(r));
            }
        }
    }

    __device__ float row_f32(const float* p) const { return active ? p[row] : 0.0f; }
    __device__ float row_val(const void* p) const {
        return active ? S::get(static_cast<const T*>(p) + row) : 0.0f;
    }
    __device__ void put_f32(float* p, float v) const {
        if (active && t == 0) p[row] = v;
    }
    __device__ void put_val(void* p, float v) const {
        if (active && t == 0) S::put(static_cast<T*>(p) + row, v);
    }
};

template <class S, int NIN>
struct Looped {
    using T = typename S::T;
    static constexpr int kSlots = red_slots<kBlock, 1>();

    float (*red)[kSlots];
    int parity = 0;
    int64_t row;
    int cols;
    float ncols, inv_cols;
    const T* x;
    const T* y;

    __device__ Looped(const RowArgs& p, int64_t row_, int cols_, float (*red_)[kSlots])
        : red(red_), row(row_), cols(cols_) {
        ncols = static_cast<float>(cols);
        inv_cols = 1.0f / ncols;
        const int64_t off = row * static_cast<int64_t>(cols);
        x = static_cast<const T*>(p.in0) + off;
        y = NIN == 2 ? static_cast<const T*>(p.in1) + off : nullptr;
    }

    template <class R, int N, class F>
    __device__ __forceinline__ void reduce(float (&res)[N], F f) {
#pragma unroll
        for (int i = 0; i < N; ++i) res[i] = R::kId;
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            float o[N];
            f(S::get(x + c), NIN == 2 ? S::get(y + c) : 0.0f, o);
#pragma unroll
            for (int i = 0; i < N; ++i) res[i] = R::op(res[i], o[i]);
        }
        row_reduce<kBlock, 1, N, R>(res, red, parity);
        parity ^= 1;
    }

    template <class F>
    __device__ __forceinline__ float sum(F f) {
        float r[1];
        reduce<SumR>(r, [&](float a, float b, float (&o)[1]) { o[0] = f(a, b); });
        return r[0];
    }
    template <class F>
    __device__ __forceinline__ float max(F f) {
        float r[1];
        reduce<MaxR>(r, [&](float a, float b, float (&o)[1]) { o[0] = f(a, b); });
        return r[0];
    }
    template <class F>
    __device__ __forceinline__ void sum2(F f, float& s0, float& s1) {
        float r[2];
        reduce<SumR>(r, f);
        s0 = r[0];
        s1 = r[1];
    }

    template <bool KEEP>
    __device__ __forceinline__ void max_sumexp(float& m, float& s) {
        m = max([](float z, float) { return z; });
        const float mm = m;
        auto e = [=](float z, float) { return fast_exp(z - mm); };
        if constexpr (KEEP)
            s = sum_keep(e);
        else
            s = sum(e);
    }

    template <class F>
    __device__ __forceinline__ float sum_keep(F f) {
        return sum(f);
    }

    template <class F, class Gf>
    __device__ __forceinline__ void store_kept(void* out, int acc, F f, Gf g) const {
        T* o = static_cast<T*>(out) + row * static_cast<int64_t>(cols);
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            float r = g(f(S::get(x + c), NIN == 2 ? S::get(y + c) : 0.0f));
            if (acc) r = acc_add(S::get(o + c), r);
            S::put(o + c, r);
        }
    }

    template <class F>
    __device__ __forceinline__ void store(void* out, int acc, const void* c0, float d0,
                                          const void* c1, float d1, F f) const {
        T* o = static_cast<T*>(out) + row * static_cast<int64_t>(cols);
        const T* u = static_cast<const T*>(c0);
        const T* v = static_cast<const T*>(c1);
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            float r = f(S::get(x + c), NIN == 2 ? S::get(y + c) : 0.0f, u ? S::get(u + c) : d0,
                        v ? S::get(v + c) : d1);
            if (acc) r = acc_add(S::get(o + c), r);
            S::put(o + c, r);
        }
    }

    __device__ float row_f32(const float* p) const { return p[row]; }
    __device__ float row_val(const void* p) const {
        return S::get(static_cast<const T*>(p) + row);
    }
    __device__ void put_f32(float* p, float v) const {
        if (threadIdx.x == 0) p[row] = v;
    }
    __device__ void put_val(void* p, float v) const {
        if (threadIdx.x == 0) S::put(static_cast<T*>(p) + row, v);
    }
};

// One 1024-lane workgroup per row, each pass streaming the row in 16-byte
// slots, four slots per lane in flight, through buffer resources (a slot past
// the row's body reads zeros and is skipped).  Each pass re-reads the row:
// with 1024-lane workgroups only a few hundred rows are in flight, so the
// re-reads mostly hit the Infinity Cache.  The per-lane order is slot by slot,
// element by element, then the row tree, fixed by cols and the row's offset.
//   ALIGNED: rows of whole 16-byte slots, every pointer 16-byte aligned (rows
//     too wide for the resident shapes);
//   otherwise: rows that start anywhere (cols not a multiple of the slot
//     width, or 16-byte misaligned tensors), every row tensor at the same
//     offset from a 16-byte boundary.  A row is a head of up to W-1 elements
//     before its first boundary, a body of 16-byte slots and a tail of up to
//     W-1 elements; lane t adds head element t and tail element t (scalar
//     accesses) besides its body slots.  Column vectors, whose offset from a
//     boundary then differs from row to row, are read element by element.
constexpr int kVecLanes = 1024;
constexpr int kVecBatch = 4;
// Narrower misaligned rows keep row_looped: a 1024-lane workgroup over a few
// thousand columns leaves most lanes idle (4097 bf16 columns: level forward,
// 15 % slower backward).
constexpr int kVecMinCols = 8192;

template <class S, int NIN, bool ALIGNED>
struct LoopedVec {
    using T = typename S::T;
    static constexpr int W = S::kVec;
    static constexpr int kSlots = red_slots<kVecLanes, 1>();

    float (*red)[kSlots];
    int parity = 0;
    int64_t row;
    int cols, nslot, head, tail0, ntail;
    float ncols, inv_cols;
    const T* x;
    const T* y;
    uint32_t body_bytes;

    __device__ LoopedVec(const RowArgs& p, int64_t row_, int cols_, float (*red_)[kSlots])
        : red(red_), row(row_), cols(cols_) {
        ncols = static_cast<float>(cols);
        inv_cols = 1.0f / ncols;
        const int64_t off = row * static_cast<int64_t>(cols);
        x = static_cast<const T*>(p.in0) + off;
        y = NIN == 2 ? static_cast<const T*>(p.in1) + off : nullptr;
        if constexpr (ALIGNED) {
            head = 0;
        } else {
            const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x) & 15u);
            head = mis ? static_cast<int>((16u - mis) / sizeof(T)) : 0;
            if (head > cols) head = cols;
        }
        nslot = (cols - head) / W;
        tail0 = head + nslot * W;
        ntail = cols - tail0;
        body_bytes = static_cast<uint32_t>(nslot) * 16u;
    }

    // f over the head and tail elements this lane owns (lane t: element t of
    // each), then over its body slots.
    template <class G>
    __device__ __forceinline__ void edges(G g) const {
        if constexpr (!ALIGNED) {
            const int t = threadIdx.x;
            if (t < head) g(t);
            if (t < ntail) g(tail0 + t);
        }
    }
    __device__ __forceinline__ float xa(int c) const { return S::get(x + c); }
    __device__ __forceinline__ float yb(int c) const { return NIN == 2 ? S::get(y + c) : 0.0f; }

    template <class R, int N, class F>
    __device__ __forceinline__ void reduce(float (&res)[N], F f) {
#pragma unroll
        for (int i = 0; i < N; ++i) res[i] = R::kId;
        edges([&](int c) {
            float o[N];
            f(xa(c), yb(c), o);
#pragma unroll
            for (int i = 0; i < N; ++i) res[i] = R::op(res[i], o[i]);
        });
        const rsrc_t rx = make_rsrc(x + head, body_bytes);
        const rsrc_t ry = make_rsrc(NIN == 2 ? y + head : x, NIN == 2 ? body_bytes : 0u);
        for (int base = threadIdx.x; base < nslot; base += kVecLanes * kVecBatch) {
            u32x4 va[kVecBatch], vb[kVecBatch];
#pragma unroll
            for (int k = 0; k < kVecBatch; ++k) {
                const uint32_t o = static_cast<uint32_t>(base + k * kVecLanes) * 16u;
                va[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
                if constexpr (NIN == 2) vb[k] = __builtin_amdgcn_raw_buffer_load_b128(ry, o, 0, 0);
            }
#pragma unroll
            for (int k = 0; k < kVecBatch; ++k) {
                if (base + k * kVecLanes >= nslot) break;
                float fa[W], fb[W];
                S::unpack(va[k], fa);
                if constexpr (NIN == 2) {
                    S::unpack(vb[k], fb);
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) fb[e] = 0.0f;
                }
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    float o[N];
                    f(fa[e], fb[e], o);
#pragma unroll
                    for (int i = 0; i < N; ++i) res[i] = R::op(res[i], o[i]);
                }
            }
        }
        row_reduce<kVecLanes, 1, N, R>(res, red, parity);
        parity ^= 1;
    }

    template <class F>
    __device__ __forceinline__ float sum(F f) {
        float r[1];
        reduce<SumR>(r, [&](float a, float b, float (&o)[1]) { o[0] = f(a, b); });
        return r[0];
    }
    template <class F>
    __device__ __forceinline__ float max(F f) {
        float r[1];
        reduce<MaxR>(r, [&](float a, float b, float (&o)[1]) { o[0] = f(a, b); });
        return r[0];
    }
    template <class F>
    __device__ __forceinline__ void sum2(F f, float& s0, float& s1) {
        float r[2];
        reduce<SumR>(r, f);
        s0 = r[0];
        s1 = r[1];
    }

    // One pass: per lane, each slot (or edge element) updates the running
    // maximum mn = max(m, its maximum) and s = s * exp(m - mn) + the sum of
    // its exp(a - mn) (an update that leaves mn at -inf changes nothing); then
    // M = the row maximum of m and s = the row sum of s * exp(m - M), both over
    // the row tree.  A row that is -inf throughout gives s = NaN, as the
    // two-pass rule does (its exp(-inf - -inf) terms are NaN), so such a row
    // comes out NaN on every path.
    template <bool KEEP>
    __device__ __forceinline__ void max_sumexp(float& m_out, float& s_out) {
        float m = -__builtin_inff(), s = 0.0f;
        edges([&](int c) {
            const float v = xa(c);
            const float mn = MaxR::op(m, v);
            if (mn != -__builtin_inff()) {
                s = s * fast_exp(m - mn) + fast_exp(v - mn);
                m = mn;
            }
        });
        const rsrc_t rx = make_rsrc(x + head, body_bytes);
        for (int base = threadIdx.x; base < nslot; base += kVecLanes * kVecBatch) {
            u32x4 va[kVecBatch];
#pragma unroll
            for (int k = 0; k < kVecBatch; ++k)
                va[k] = __builtin_amdgcn_raw_buffer_load_b128(
                    rx, static_cast<uint32_t>(base + k * kVecLanes) * 16u, 0, 0);
#pragma unroll
            for (int k = 0; k < kVecBatch; ++k) {
                if (base + k * kVecLanes >= nslot) break;
                float f[W];
                S::unpack(va[k], f);
                float sm = f[0];
#pragma unroll
                for (int e = 1; e < W; ++e) sm = MaxR::op(sm, f[e]);
                const float mn = MaxR::op(m, sm);
                if (mn != -__builtin_inff()) {
                    float t = 0.0f;
#pragma unroll
                    for (int e = 0; e < W; ++e) t += fast_exp(f[e] - mn);
                    s = s * fast_exp(m - mn) + t;
                    m = mn;
                }
            }
        }
        float r[1] = {m};
        row_reduce<kVecLanes, 1, 1, MaxR>(r, red, parity);
        parity ^= 1;
        const float M = r[0];
        float q[1] = {M == -__builtin_inff() ? 0.0f : s * fast_exp(m - M)};
        row_reduce<kVecLanes, 1, 1, SumR>(q, red, parity);
        parity ^= 1;
        m_out = M;
        s_out = M == -__builtin_inff() ? __builtin_nanf("") : q[0];
    }

    template <class F>
    __device__ __forceinline__ float sum_keep(F f) {
        return sum(f);
    }

    // out (+)= h(a, b, u, v) per element, u and v from the column vectors c0,
    // c1 (d0, d1 when null).
    template <class H>
    __device__ __forceinline__ void store_each(void* out, int acc, const void* c0, float d0,
                                               const void* c1, float d1, H h) const {
        T* o = static_cast<T*>(out) + row * static_cast<int64_t>(cols);
        const T* u = static_cast<const T*>(c0);
        const T* v = static_cast<const T*>(c1);
        edges([&](int c) {
            float r = h(xa(c), yb(c), u ? S::get(u + c) : d0, v ? S::get(v + c) : d1);
            if (acc) r = acc_add(S::get(o + c), r);
            S::put(o + c, r);
        });
        const rsrc_t rx = make_rsrc(x + head, body_bytes);
        const rsrc_t ry = make_rsrc(NIN == 2 ? y + head : x, NIN == 2 ? body_bytes : 0u);
        const rsrc_t ro = make_rsrc(o + head, body_bytes);
        const rsrc_t ru = make_rsrc(c0 ? u + head : x, (ALIGNED && c0) ? body_bytes : 0u);
        const rsrc_t rv = make_rsrc(c1 ? v + head : x, (ALIGNED && c1) ? body_bytes : 0u);
        for (int base = threadIdx.x; base < nslot; base += kVecLanes * kVecBatch) {
            u32x4 va[kVecBatch], vb[kVecBatch], vu[kVecBatch], vv[kVecBatch], vo[kVecBatch];
#pragma unroll
            for (int k = 0; k < kVecBatch; ++k) {
                const uint32_t off = static_cast<uint32_t>(base + k * kVecLanes) * 16u;
                va[k] = bload16_stream(rx, off);
                if constexpr (NIN == 2) vb[k] = bload16_stream(ry, off);
                if constexpr (ALIGNED) {
                    if (c0) vu[k] = __builtin_amdgcn_raw_buffer_load_b128(ru, off, 0, 0);
                    if (c1) vv[k] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
                }
                if (acc) vo[k] = bload16_stream(ro, off);
            }
#pragma unroll
            for (int k = 0; k < kVecBatch; ++k) {
                const int slot = base + k * kVecLanes;
                const uint32_t off = static_cast<uint32_t>(slot) * 16u;
                float fa[W], fb[W], fu[W], fv[W], r[W];
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    fu[e] = d0;
                    fv[e] = d1;
                }
                S::unpack(va[k], fa);
                if constexpr (NIN == 2) S::unpack(vb[k], fb);
                if constexpr (ALIGNED) {
                    if (c0) S::unpack(vu[k], fu);
                    if (c1) S::unpack(vv[k], fv);
                } else if (slot < nslot) {  // column values element by element
                    const int c = head + slot * W;
#pragma unroll
                    for (int e = 0; e < W; ++e) {
                        fu[e] = u ? S::get(u + c + e) : d0;
                        fv[e] = v ? S::get(v + c + e) : d1;
                    }
                }
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const float uu = ALIGNED ? (c0 ? fu[e] : d0) : fu[e];
                    const float vvv = ALIGNED ? (c1 ? fv[e] : d1) : fv[e];
                    r[e] = h(fa[e], NIN == 2 ? fb[e] : 0.0f, uu, vvv);
                }
                if (acc) {
                    float old[W];
                    S::unpack(vo[k], old);
#pragma unroll
                    for (int e = 0; e < W; ++e) r[e] = acc_add(old[e], r[e]);
                }
                bstore16_stream(ro, off, S::pack(r));  // past the body: dropped
            }
        }
    }

    template <class F, class Gf>
    __device__ __forceinline__ void store_kept(void* out, int acc, F f, Gf g) const {
        store_each(out, acc, nullptr, 0.0f, nullptr, 0.0f,
                   [&](float a, float b, float, float) { return g(f(a, b)); });
    }

    template <class F>
    __device__ __forceinline__ void store(void* out, int acc, const void* c0, float d0,
                                          const void* c1, float d1, F f) const {
        store_each(out, acc, c0, d0, c1, d1, f);
    }

    __device__ float row_f32(const float* p) const { return p[row]; }
    __device__ float row_val(const void* p) const {
        return S::get(static_cast<const T*>(p) + row);
    }
    __device__ void put_f32(float* p, float v) const {
        if (threadIdx.x == 0) p[row] = v;
    }
    __device__ void put_val(void* p, float v) const {
        if (threadIdx.x == 0) S::put(static_cast<T*>(p) + row, v);
    }
};

// ---- ops -------------------------------------------------------------------------

// Forward-mode product of the RMSNorm layer (in0 = x, in1 = tx, col0 = gamma,
// col1 = tgamma, rs0 = inv_rms, out = ty):
//   ty = gamma * (r * (tx - x * s)) + tgamma * (x * r),  s = r^2 * sum(tx*x) / cols
struct RmsJvp {
    static constexpr int kIn = 2;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        const float r = c.row_f32(p.rs0);
        const float dot = c.sum([](float x, float t) { return t * x; });
        const float s = (r * r * dot) * c.inv_cols;
        const bool has_tg = p.col1 != nullptr;
        c.store(p.out, 0, p.col0, 1.0f, p.col1, 0.0f,
                [=](float x, float t, float g, float tg) {
                    const float o = g * (r * (t - x * s));
                    return has_tg ? o + tg * (x * r) : o;
                });
    }
};

// LayerNorm forward (in0 = x, out = y, ws0 = mean, ws1 = rstd):
//   mean = sum(x)/cols, var = sum((x - mean)^2)/cols, rstd = 1/sqrt(var + eps),
//   y = (x - mean) * rstd
struct LnFwd {
    static constexpr int kIn = 1;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        const float mean = c.sum([](float x, float) { return x; }) / c.ncols;
        const float var = c.sum([=](float x, float) {
            const float d = x - mean;
            return d * d;
        }) / c.ncols;
        const float rstd = 1.0f / sqrtf(var + p.eps);
        c.put_f32(p.ws0, mean);
        c.put_f32(p.ws1, rstd);
        c.store(p.out, 0, nullptr, 0.0f, nullptr, 0.0f,
                [=](float x, float, float, float) { return (x - mean) * rstd; });
    }
};

// LayerNorm backward (in0 = x, in1 = dy, rs0 = mean, rs1 = rstd, out = dx):
//   xhat = (x - mean) * rstd,  dx (+)= rstd * (dy - sum(dy)/cols - xhat * sum(dy*xhat)/cols)
struct LnBwd {
    static constexpr int kIn = 2;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        const float mean = c.row_f32(p.rs0);
        const float rstd = c.row_f32(p.rs1);
        float sg = 0.0f, sgx = 0.0f;
        c.sum2(
            [=](float x, float g, float (&o)[2]) {
                o[0] = g;
                o[1] = g * ((x - mean) * rstd);
            },
            sg, sgx);
        const float mg = sg * c.inv_cols;
        const float mgx = sgx * c.inv_cols;
        c.store(p.out, p.acc, nullptr, 0.0f, nullptr, 0.0f,
                [=](float x, float g, float, float) {
                    return rstd * (g - mg - ((x - mean) * rstd) * mgx);
                });
    }
};

// Row softmax (in0 = z, out = y): y = e * (1 / sum(e)), e = exp(z - m), m = max(z);
// each exponential is computed once and kept for the store.
struct SmFwd {
    static constexpr int kIn = 1;
    static constexpr bool kResident16 = true;  // rows of 8193-16384 slots stay resident
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        float m, s;
        c.template max_sumexp<true>(m, s);
        auto e = [=](float z, float) { return fast_exp(z - m); };
        const float inv = 1.0f / s;
        c.store_kept(p.out, 0, e, [=](float v) { return v * inv; });
    }
};

// Row softmax backward from the output (in0 = y, in1 = dy, out = dz):
//   dz (+)= y * (dy - sum(y * dy))
struct SmBwd {
    static constexpr int kIn = 2;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        const float dot = c.sum([](float y, float g) { return y * g; });
        c.store(p.out, p.acc, nullptr, 0.0f, nullptr, 0.0f,
                [=](float y, float g, float, float) { return y * (g - dot); });
    }
};

// Row log-sum-exp (in0 = z, out_row = y): y = log(sum(exp(z - m))) + m.
struct LseFwd {
    static constexpr int kIn = 1;
    // bf16 rows of 8 slots per lane (32769-65536 columns) stream faster through
    // the 16-byte looped kernel's one online pass (GPT-2-sized vocabularies:
    // 52-61 % of HBM peak resident, 78 % streamed)
    static constexpr bool kStreamWideBf16 = true;
    // bf16 rows that the plan gives 2 slots per lane on 128-1024 lanes
    // (2048-16384 columns) take 4 slots per lane on half the lanes: the row's
    // two reductions, its log and its set-up are then spread over 32 elements
    // per lane instead of 16, and this read-only op is bound by instructions
    // per byte, not by HBM, at 2 slots (MI355X, 1 GiB of bf16 logits, graph
    // replays: 2048-16384 columns 70-79 % of HBM peak at 2 slots, 87-88.5 % at
    // 4; fp32 rows at 4 slots measured slower and keep the plan)
    static constexpr bool kFourSlotsBf16 = true;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        float m, s;
        c.template max_sumexp<false>(m, s);
        const float y = logf(s) + m;
        c.put_val(p.out_row, y);
        if (p.ws0 != nullptr) c.put_f32(p.ws0, y);  // the fp32 value, for the backward
    }
};

// Row log-sum-exp backward (in0 = z, rsv = dy, out = dz):
//   dz (+)= dy * (e * (1 / sum(e))),  e = exp(z - m), computed once
struct LseBwd {
    static constexpr int kIn = 1;
    static constexpr bool kResident16 = true;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        float m, s;
        c.template max_sumexp<true>(m, s);
        auto e = [=](float z, float) { return fast_exp(z - m); };
        const float inv = 1.0f / s;
        const float g = c.row_val(p.rsv);
        c.store_kept(p.out, p.acc, e, [=](float v) { return g * (v * inv); });
    }
};

// Row log-sum-exp forward-mode product (in0 = z, in1 = tz, out_row = ty):
//   ty = sum(exp(z - m) * tz) / sum(exp(z - m))
struct LseJvp {
    static constexpr int kIn = 2;
    template <class C>
    __device__ static void run(C& c, const RowArgs& p) {
        const float m = c.max([](float z, float) { return z; });
        float s = 0.0f, d = 0.0f;
        c.sum2(
            [=](float z, float t, float (&o)[2]) {
                const float e = fast_exp(z - m);
                o[0] = e;
                o[1] = e * t;
            },
            s, d);
        c.put_val(p.out_row, d / s);
    }
};

// ---- kernels and launch ------------------------------------------------------------

template <class S, int TPR, int NV, int G, class Op>
__global__ __launch_bounds__(TPR * G) void row_resident(const RowArgs p, int64_t rows, int cols) {
    using Ctx = Resident<S, TPR, NV, G, Op::kIn>;
    __shared__ float red[2][Ctx::kSlots];
    Ctx c(p, rows, cols, red);
    Op::run(c, p);
}

template <class S, class Op, bool ALIGNED>
__global__ __launch_bounds__(kVecLanes) void row_looped_vec(const RowArgs p, int64_t rows,
                                                           int cols) {
    using Ctx = LoopedVec<S, Op::kIn, ALIGNED>;
    __shared__ float red[2][Ctx::kSlots];
    const int64_t row = blockIdx.x;
    if (row >= rows) return;  // workgroup-uniform
    Ctx c(p, row, cols, red);
    Op::run(c, p);
}

template <class S, class Op>
__global__ __launch_bounds__(kBlock) void row_looped(const RowArgs p, int64_t rows, int cols) {
    using Ctx = Looped<S, Op::kIn>;
    __shared__ float red[2][Ctx::kSlots];
    const int64_t row = blockIdx.x;
    if (row >= rows) return;  // workgroup-uniform
    Ctx c(p, row, cols, red);
    Op::run(c, p);
}

inline bool aligned_or_null(const void* p) { return p == nullptr || aligned16(p); }

// Op::kStreamWideBf16 when the op declares it, else false.
template <class Op, class = void>
struct StreamWideBf16 : std::false_type {};
template <class Op>
struct StreamWideBf16<Op, std::void_t<decltype(Op::kStreamWideBf16)>>
    : std::integral_constant<bool, Op::kStreamWideBf16> {};
template <class Op>
constexpr bool stream_wide_bf16() { return StreamWideBf16<Op>::value; }

// Op::kFourSlotsBf16 when the op declares it, else false.
template <class Op, class = void>
struct FourSlotsBf16 : std::false_type {};
template <class Op>
struct FourSlotsBf16<Op, std::void_t<decltype(Op::kFourSlotsBf16)>>
    : std::integral_constant<bool, Op::kFourSlotsBf16> {};
template <class Op>
constexpr bool four_slots_bf16() { return FourSlotsBf16<Op>::value; }

// Op::kResident16 when the op declares it, else false: rows of 8193-16384
// 16-byte slots (65537-131072 bf16 or 32769-65536 fp32 columns) take a
// 1024-lane workgroup of 16 slots per lane, the row read once, instead of the
// looped kernels' two reads.  Only ops that read one row tensor and write
// one: two packed inputs would not fit beside the arithmetic.  Measured on
// MI355X at bf16 [8192, 128256]: softmax forward 846 against 878 us, log-sum-
// exp backward 863 against 878 us; the row fills a CU's registers, so a CU
// holds one row at a time (512 lanes x 32 slots: the same), which is what
// keeps both near 60 % of HBM peak rather than the two-pass bytes.
template <class Op, class = void>
struct Resident16 : std::false_type {};
template <class Op>
struct Resident16<Op, std::void_t<decltype(Op::kResident16)>>
    : std::integral_constant<bool, Op::kResident16> {};

// Every row tensor (in0, in1, out) element-aligned and at in0's offset from a
// 16-byte boundary, so that each row's head, body and tail line up in all of
// them.  Column vectors and per-row vectors may sit anywhere.
template <class T>
inline bool same_offset(const RowArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.in0);
    auto ok = [&](const void* q) {
        if (q == nullptr) return true;
        const uintptr_t b = reinterpret_cast<uintptr_t>(q);
        return (b % sizeof(T)) == 0 && ((b - a) & 15u) == 0;
    };
    return (a % sizeof(T)) == 0 && ok(p.in1) && ok(p.out);
}

// ---- rows over several workgroups (teams) -------------------------------------------

#include "rowops_team.hpp"

// When the *_ws entry points take the team kernel (agk_set_rowops_team):
// 0 never, 1 for the shapes it serves better than the one-workgroup-per-row
// kernels (the default), 2 whenever the row fits it (tests and measurement).
std::atomic<int> g_team_mode{1};

// Least parts per row for which mode 1 takes the team kernel.  Measured on
// MI355X (graph-replayed, 8192 rows, us, one-workgroup-per-row kernel against
// the team kernel):
//  - rows on a 16-byte boundary, held in registers by one workgroup up to 8192
//    slots: the softmax forward and the log-sum-exp backward gain from 3
//    parts (bf16 40000 columns 254-262 against 243-245, 48000 299-309
//    against 274-276, 65536 397-407 against 358-364; fp32 24000 level,
//    32768 362-367 against 352-353) and lose at 2 (bf16 32000 174-178
//    against 184-187); the softmax backward gains from 4 (bf16 65536 566
//    against 532, fp32 32768 538 against 521) and is level or slower at 3
//    (bf16 40000 329 against 342, 48000 403 against 401);
//  - rows off a 16-byte boundary: the backward from 2 parts (at 50257
//    columns the 16-byte looped kernel reads y and dy twice: bf16 540
//    against 438, fp32 1140 against 855); the forward and the log-sum-exp
//    backward read one tensor, which the looped kernel's second pass finds
//    in the caches, from 4 parts (bf16 50257: 313-316 against 305-306 with
//    three workgroups per CU).
template <class Op>
constexpr int team_min_parts(bool aligned) {
    if (std::is_same<Op, SmBwd>::value) return aligned ? 4 : 2;
    return aligned ? 3 : 4;
}

// Runs Op over the rows on the team kernel when the mode, the workspace and
// the rows' layout allow it; *taken tells the caller.
template <class Op, class S>
int maybe_team(const RowArgs& p, void* ws, size_t ws_bytes, int64_t rows, int cols,
               hipStream_t st, bool* taken) {
    *taken = false;
    const int mode = g_team_mode.load(std::memory_order_relaxed);
    if (ws == nullptr || mode == 0) return AGK_OK;
    bool aligned = false;
    if (!team_fits<S, Op>(p, rows, cols, 1, &aligned)) return AGK_OK;
    const TeamShape sh =
        team_shape(rows, cols, S::kVec, team_nvl<Op>(std::is_same<S, BF16>::value, aligned),
                   team_grid<Op>());
    if (mode == 1 && sh.parts < team_min_parts<Op>(aligned)) return AGK_OK;
    if (ws_bytes < team_words_bytes(rows, sh, TeamVals<Op>::value)) return AGK_OK;
    *taken = true;
    return launch_team<Op, S>(p, ws, rows, cols, aligned, st);
}

int team_wait_limit() { return agk::team_wait_polls(); }

template <class Op, class S>
int launch(const RowArgs& p, int64_t rows, int cols, hipStream_t st) {
    const bool vec = (cols % S::kVec) == 0 && aligned16(p.in0) && aligned_or_null(p.in1) &&
                     aligned_or_null(p.out) && aligned_or_null(p.col0) &&
                     aligned_or_null(p.col1);
    Plan pl;
    if (vec) pl = fwd_plan(cols / S::kVec, rows);
    if (stream_wide_bf16<Op>() && std::is_same<S, BF16>::value && pl.nv == 8) pl = Plan{};
    if (four_slots_bf16<Op>() && std::is_same<S, BF16>::value && pl.nv == 2 && pl.tpr >= 128) {
        const Plan q{pl.tpr / 2, 4, pl.tpr >= 512 ? 1 : 512 / pl.tpr};
        if (has_shape(kFwdShapes, q)) pl = q;
    }
    if constexpr (Resident16<Op>::value) {
        const int64_t nslot = cols / S::kVec;
        if (vec && pl.tpr == 0 && nslot > 8192 && nslot <= 16384) {
            if (rows > 0x7fffffffLL) return AGK_EINVAL;
            hipLaunchKernelGGL((row_resident<S, 1024, 16, 1, Op>), dim3(static_cast<unsigned>(rows)),
                               dim3(1024), 0, st, p, rows, cols);
            return check_launch();
        }
    }
    if (pl.tpr == 0) {
        if (rows > 0x7fffffffLL) return AGK_EINVAL;
        // rows short enough for 32-bit buffer offsets: whole 16-byte slots and
        // aligned pointers, or (from kVecMinCols columns) every row tensor at
        // the same offset from a 16-byte boundary
        const bool fits = static_cast<uint64_t>(cols) * sizeof(typename S::T) < 0x80000000ull;
        if (vec && fits)
            hipLaunchKernelGGL((row_looped_vec<S, Op, true>), dim3(static_cast<unsigned>(rows)),
                               dim3(kVecLanes), 0, st, p, rows, cols);
        else if (fits && cols >= kVecMinCols && same_offset<typename S::T>(p))
            hipLaunchKernelGGL((row_looped_vec<S, Op, false>), dim3(static_cast<unsigned>(rows)),
                               dim3(kVecLanes), 0, st, p, rows, cols);
        else
            hipLaunchKernelGGL((row_looped<S, Op>), dim3(static_cast<unsigned>(rows)),
                               dim3(kBlock), 0, st, p, rows, cols);
        return check_launch();
    }
    const int64_t grid = (rows + pl.g - 1) / pl.g;
    if (grid > 0x7fffffffLL) return AGK_EINVAL;
#define AGK_X(a, b, c)                                                                          \
    if (pl.tpr == a && pl.nv == b && pl.g == c) {                                               \
        hipLaunchKernelGGL((row_resident<S, a, b, c, Op>), dim3(static_cast<unsigned>(grid)),    \
                           dim3(a * c), 0, st, p, rows, cols);                                  \
        return check_launch();                                                                  \
    }
    AGK_FWD_SHAPES(AGK_X)
#undef AGK_X
    return AGK_EINVAL;
}

template <class Op>
int run(const RowArgs& p, int64_t rows, int64_t cols, int dtype, agk_stream_t stream) {
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int c = static_cast<int>(cols);
    return dtype == AGK_F32 ? launch<Op, F32>(p, rows, c, st) : launch<Op, BF16>(p, rows, c, st);
}

// ---- log-sum-exp backward from the forward's fp32 value ---------------------------
// dz (+)= dy[row] * exp(z - lse[row]): softmax(z) = exp(z - lse(z)), so with the
// forward's fp32 lse the backward is one streaming pass (read z, write dz)
// instead of two passes over a row held on chip.  Workgroups of 256 lanes
// take kLseChunkSlots 16-byte slots of one row (4 per lane).  A row is a head
// of elements up to its first 16-byte boundary, a body of slots and a tail
// (z and dz at the same offset from a boundary: SAME_OFF); the body goes
// through buffer resources sized to it, so slots past the row's end are
// dropped by the hardware.  Tensors at different offsets take the element-
// wise form.
constexpr int kLseLanes = 256;
constexpr int kLseChunkSlots = kLseLanes * 4;

template <class S, bool SAME_OFF, bool ACC>
__global__ __launch_bounds__(kLseLanes) void lse_bwd_from_value(
    const typename S::T* __restrict__ z, const float* __restrict__ lse,
    const typename S::T* __restrict__ dy, typename S::T* __restrict__ dz, int cols,
    int64_t nchunk) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    const int64_t row = static_cast<int64_t>(blockIdx.x) / nchunk;
    const int chunk = static_cast<int>(static_cast<int64_t>(blockIdx.x) - row * nchunk);
    const float L = lse[row];
    const float g = S::get(dy + row);
    const int64_t off = row * static_cast<int64_t>(cols);
    const T* zr = z + off;
    T* dr = dz + off;
    const int t = threadIdx.x;
    auto one = [&](int c) {
        float v = g * fast_exp(S::get(zr + c) - L);
        if constexpr (ACC) v = acc_add(S::get(dr + c), v);
        S::put(dr + c, v);
    };
    if constexpr (!SAME_OFF) {
        const int c0 = chunk * kLseChunkSlots * W;
        const int c1 = c0 + kLseChunkSlots * W < cols ? c0 + kLseChunkSlots * W : cols;
        for (int c = c0 + t; c < c1; c += kLseLanes) one(c);
        return;
    } else {
        const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(zr) & 15u);
        int head = mis ? static_cast<int>((16u - mis) / sizeof(T)) : 0;
        if (head > cols) head = cols;
        const int nslot = (cols - head) / W;
        const int tail0 = head + nslot * W;
        if (chunk == 0 && t < head) one(t);
        if (chunk == nchunk - 1 && t < cols - tail0) one(tail0 + t);
        const uint32_t body = static_cast<uint32_t>(nslot) * 16u;
        const rsrc_t rz = make_rsrc(zr + head, body);
        const rsrc_t ro = make_rsrc(dr + head, body);
        u32x4 v[4], o[4];
        uint32_t at[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            at[k] = static_cast<uint32_t>(chunk * kLseChunkSlots + k * kLseLanes + t) * 16u;
            v[k] = bload16_stream(rz, at[k]);
            if constexpr (ACC) o[k] = bload16_stream(ro, at[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float f[W];
            S::unpack(v[k], f);
#pragma unroll
            for (int e = 0; e < W; ++e) f[e] = g * fast_exp(f[e] - L);
            if constexpr (ACC) {
                float old[W];
                S::unpack(o[k], old);
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = acc_add(old[e], f[e]);
            }
            bstore16_stream(ro, at[k], S::pack(f));
        }
    }
}

template <class S>
int launch_lse_bwd_from_value(const void* z, const float* lse, const void* dy, void* dz,
                              int64_t rows, int cols, int acc, hipStream_t st) {
    using T = typename S::T;
    const int64_t per = static_cast<int64_t>(kLseChunkSlots) * S::kVec;
    // a head takes at most one slot's worth of columns from the body
    const int64_t nchunk = (cols + per - 1) / per;
    if (rows > 0x7fffffffLL / nchunk) return AGK_EINVAL;
    const dim3 grid(static_cast<unsigned>(rows * nchunk)), block(kLseLanes);
    const bool same = ((reinterpret_cast<uintptr_t>(z) - reinterpret_cast<uintptr_t>(dz)) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(z) % sizeof(T)) == 0 &&
                      (reinterpret_cast<uintptr_t>(dz) % sizeof(T)) == 0;
    const T* zp = static_cast<const T*>(z);
    const T* gp = static_cast<const T*>(dy);
    T* op = static_cast<T*>(dz);
#define AGK_LSE(SAME, ACC_)                                                                    \
    hipLaunchKernelGGL((lse_bwd_from_value<S, SAME, ACC_>), grid, block, 0, st, zp, lse, gp, op, \
                       cols, nchunk)
    if (same) {
        if (acc) AGK_LSE(true, true);
        else AGK_LSE(true, false);
    } else {
        if (acc) AGK_LSE(false, true);
        else AGK_LSE(false, false);
    }
#undef AGK_LSE
    return check_launch();
}

// Checks shared by every entry point; sets *done when there is nothing to do.
inline int precheck(int64_t rows, int64_t cols, int dtype, bool* done) {
    *done = false;
    if (int rc = check_sizes(rows, cols)) return rc;
    if (!valid_dtype(dtype)) return AGK_EDTYPE;
    if (rows == 0 || cols == 0) *done = true;
    return AGK_OK;
}

inline bool valid_accumulate(int accumulate) { return (accumulate & ~AGK_ACCUM_DX) == 0; }

}  // namespace rowops
}  // namespace agk

// ---- C ABI ------------------------------------------------------------------------

extern "C" {

int agk_rmsnorm_jvp(const void* x, const void* gamma, const float* inv_rms, const void* tx,
                    const void* tgamma, void* ty, int64_t rows, int64_t cols, int dtype,
                    agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (tgamma && !gamma) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!x || !inv_rms || !tx || !ty) return AGK_EINVAL;
    RowArgs p;
    p.in0 = x;
    p.in1 = tx;
    p.col0 = gamma;
    p.col1 = tgamma;
    p.rs0 = inv_rms;
    p.out = ty;
    return run<RmsJvp>(p, rows, cols, dtype, stream);
}

int agk_layernorm_fwd(const void* x, void* y, float* mean, float* rstd, int64_t rows,
                      int64_t cols, float eps, int dtype, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (done) return AGK_OK;
    if (!x || !y || !mean || !rstd) return AGK_EINVAL;
    RowArgs p;
    p.in0 = x;
    p.out = y;
    p.ws0 = mean;
    p.ws1 = rstd;
    p.eps = eps;
    return run<LnFwd>(p, rows, cols, dtype, stream);
}

int agk_layernorm_bwd(const void* x, const float* mean, const float* rstd, const void* dy,
                      void* dx, int64_t rows, int64_t cols, int dtype, int accumulate,
                      agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (!valid_accumulate(accumulate)) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!x || !mean || !rstd || !dy || !dx) return AGK_EINVAL;
    RowArgs p;
    p.in0 = x;
    p.in1 = dy;
    p.rs0 = mean;
    p.rs1 = rstd;
    p.out = dx;
    p.acc = accumulate & AGK_ACCUM_DX;
    return run<LnBwd>(p, rows, cols, dtype, stream);
}

int agk_softmax_fwd(const void* z, void* y, int64_t rows, int64_t cols, int dtype,
                    agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (done) return AGK_OK;
    if (!z || !y) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.out = y;
    return run<SmFwd>(p, rows, cols, dtype, stream);
}

int agk_softmax_bwd(const void* y, const void* dy, void* dz, int64_t rows, int64_t cols,
                    int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (!valid_accumulate(accumulate)) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!y || !dy || !dz) return AGK_EINVAL;
    RowArgs p;
    p.in0 = y;
    p.in1 = dy;
    p.out = dz;
    p.acc = accumulate & AGK_ACCUM_DX;
    return run<SmBwd>(p, rows, cols, dtype, stream);
}

int agk_logsumexp_fwd(const void* z, void* y, int64_t rows, int64_t cols, int dtype,
                      agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (rows > 0 && cols == 0) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!z || !y) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.out_row = y;
    return run<LseFwd>(p, rows, cols, dtype, stream);
}

int agk_logsumexp_bwd(const void* z, const void* dy, void* dz, int64_t rows, int64_t cols,
                      int dtype, int accumulate, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (!valid_accumulate(accumulate)) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!z || !dy || !dz) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.rsv = dy;
    p.out = dz;
    p.acc = accumulate & AGK_ACCUM_DX;
    return run<LseBwd>(p, rows, cols, dtype, stream);
}

int agk_logsumexp_fwd_keep(const void* z, void* y, float* lse, int64_t rows, int64_t cols,
                           int dtype, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (rows > 0 && cols == 0) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!z || !y || !lse) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.out_row = y;
    p.ws0 = lse;
    return run<LseFwd>(p, rows, cols, dtype, stream);
}

int agk_logsumexp_bwd_from_value(const void* z, const float* lse, const void* dy, void* dz,
                                 int64_t rows, int64_t cols, int dtype, int accumulate,
                                 agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (!valid_accumulate(accumulate)) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!z || !lse || !dy || !dz) return AGK_EINVAL;
    agk::clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int c = static_cast<int>(cols);
    const int acc = accumulate & AGK_ACCUM_DX;
    return dtype == AGK_F32
               ? launch_lse_bwd_from_value<agk::F32>(z, lse, dy, dz, rows, c, acc, st)
               : launch_lse_bwd_from_value<agk::BF16>(z, lse, dy, dz, rows, c, acc, st);
}

size_t agk_rowops_workspace_bytes(int64_t rows, int64_t cols) {
    if (agk::check_sizes(rows, cols) != AGK_OK || rows == 0 || cols == 0) return 0;
    return agk::rowops::team_ws_bytes(rows, cols);
}

int agk_rowops_team_plan(int op, int64_t rows, int64_t cols, int dtype, int aligned,
                         int32_t* plan) {
    using namespace agk::rowops;
    if (!plan) return AGK_EINVAL;
    plan[0] = plan[1] = plan[2] = 0;
    if (op < 0 || op > 2) return AGK_EINVAL;
    if (int rc = agk::check_sizes(rows, cols)) return rc;
    if (!agk::valid_dtype(dtype)) return AGK_EDTYPE;
    if (rows == 0 || cols == 0) return AGK_OK;
    const int W = dtype == AGK_F32 ? 4 : 8;
    const size_t esz = dtype == AGK_F32 ? 4u : 2u;
    if (rows > 0x7fffffffLL || static_cast<uint64_t>(cols) * esz >= 0x80000000ull) return AGK_OK;
    const bool al = aligned != 0 && cols % W == 0;
    const TeamShape sh = team_shape(rows, cols, W, team_nvl_of(op, dtype == AGK_BF16, al),
                                    op == 1 ? team_grid<SmBwd>() : team_grid<SmFwd>());
    const int mode = g_team_mode.load(std::memory_order_relaxed);
    if (sh.parts == 0 || mode == 0 || sh.teams * sh.parts > 0x7fffffffLL) return AGK_OK;
    const int least = op == 1 ? team_min_parts<SmBwd>(al) : team_min_parts<SmFwd>(al);
    if (mode == 1 && sh.parts < least) return AGK_OK;
    plan[0] = sh.parts;
    plan[1] = sh.ps;
    plan[2] = static_cast<int32_t>(sh.teams);
    return AGK_OK;
}

int agk_set_rowops_team(int mode) {
    const int prev = agk::rowops::g_team_mode.load(std::memory_order_relaxed);
    if (mode >= 0 && mode <= 2) agk::rowops::g_team_mode.store(mode, std::memory_order_relaxed);
    return prev;
}

}  // extern "C"

namespace agk {
namespace rowops {

// The *_ws entry points: the team kernel where maybe_team takes it, else the
// kernels of the workspace-free entry point.
template <class Op>
int run_ws(const RowArgs& p, void* ws, size_t ws_bytes, int64_t rows, int64_t cols, int dtype,
           agk_stream_t stream) {
    if (ws != nullptr) {
        if ((reinterpret_cast<uintptr_t>(ws) & 7u) != 0) return AGK_EINVAL;
        if (ws_bytes < team_ws_bytes(rows, cols)) return AGK_EWORKSPACE;
    }
    clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int c = static_cast<int>(cols);
    bool taken = false;
    const int rc = dtype == AGK_F32 ? maybe_team<Op, F32>(p, ws, ws_bytes, rows, c, st, &taken)
                                    : maybe_team<Op, BF16>(p, ws, ws_bytes, rows, c, st, &taken);
    if (rc != AGK_OK || taken) return rc;
    return dtype == AGK_F32 ? launch<Op, F32>(p, rows, c, st) : launch<Op, BF16>(p, rows, c, st);
}

}  // namespace rowops
}  // namespace agk

extern "C" {

int agk_softmax_fwd_ws(const void* z, void* y, void* workspace, size_t workspace_bytes,
                       int64_t rows, int64_t cols, int dtype, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (done) return AGK_OK;
    if (!z || !y) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.out = y;
    return run_ws<SmFwd>(p, workspace, workspace_bytes, rows, cols, dtype, stream);
}

int agk_softmax_bwd_ws(const void* y, const void* dy, void* dz, void* workspace,
                       size_t workspace_bytes, int64_t rows, int64_t cols, int dtype,
                       int accumulate, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (!valid_accumulate(accumulate)) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!y || !dy || !dz) return AGK_EINVAL;
    RowArgs p;
    p.in0 = y;
    p.in1 = dy;
    p.out = dz;
    p.acc = accumulate & AGK_ACCUM_DX;
    return run_ws<SmBwd>(p, workspace, workspace_bytes, rows, cols, dtype, stream);
}

int agk_logsumexp_bwd_ws(const void* z, const void* dy, void* dz, void* workspace,
                         size_t workspace_bytes, int64_t rows, int64_t cols, int dtype,
                         int accumulate, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (!valid_accumulate(accumulate)) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!z || !dy || !dz) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.rsv = dy;
    p.out = dz;
    p.acc = accumulate & AGK_ACCUM_DX;
    return run_ws<LseBwd>(p, workspace, workspace_bytes, rows, cols, dtype, stream);
}

int agk_logsumexp_jvp(const void* z, const void* tz, void* ty, int64_t rows, int64_t cols,
                      int dtype, agk_stream_t stream) {
    using namespace agk::rowops;
    bool done;
    if (int rc = precheck(rows, cols, dtype, &done)) return rc;
    if (rows > 0 && cols == 0) return AGK_EINVAL;
    if (done) return AGK_OK;
    if (!z || !tz || !ty) return AGK_EINVAL;
    RowArgs p;
    p.in0 = z;
    p.in1 = tz;
    p.out_row = ty;
    return run<LseJvp>(p, rows, cols, dtype, stream);
}

}  // extern "C"
