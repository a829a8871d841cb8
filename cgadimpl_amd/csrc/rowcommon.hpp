// rowcommon.hpp -- the pieces every row kernel of libagk_rmsnorm shares:
// storage types (fp32, bf16 with round-to-nearest-even), 16-byte streaming
// accesses, lane-group and row reductions (DPP / swizzle / LDS), the
// resident launch shapes and their plan, and the status helpers of the C ABI.
//
// A "resident" kernel gives each row of `cols` elements to a group of TPR
// lanes; each lane holds NV 16-byte slots of the row in registers (columns
// (t + k*TPR)*W .. +W for slot k), and a workgroup of TPR*G lanes holds G rows.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <type_traits>

#include "agk_rmsnorm.h"

namespace agk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;          // threads per workgroup of the looped kernels
constexpr int kTargetBlocks = 1024;  // looped backward: row blocks (partial rows)
constexpr int kMinRowsPerBlockLarge = 4;     // once rows >= kLargeRows / 8
constexpr int64_t kLargeRows = 16384;        // forward plan switch: more rows than
                                             // this take fewer slots per lane

// ---- storage types --------------------------------------------------------

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even, in hardware (gfx950 v_cvt_pk_bf16_f32;
// a NaN stays a NaN, quieted): one instruction per two values.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

struct F32 {
    using T = float;
    static constexpr int kVec = 4;  // elements per 16-byte slot
    __device__ static float get(const T* p) { return *p; }
    __device__ static void put(T* p, float v) { *p = v; }
    // v as storage holds it, kept out of any fused multiply-add
    __device__ static float stored(float v) {
        asm("" : "+v"(v));
        return v;
    }
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
    __device__ static float stored(float v) {
        v = __uint_as_float(f32_to_bf16_bits(v) << 16);
        asm("" : "+v"(v));
        return v;
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
            v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
        return v;
    }
};

// `old + v` for gradient accumulation (`grad += g`): g is rounded on its own
// first, then the sum.  The empty asm keeps the compiler from fusing the
// multiply that produced v into this add, which would round only once.
__device__ __forceinline__ float acc_add(float old, float v) {
    asm volatile("" : "+v"(v));
    return old + v;
}

// Makes v opaque to the optimiser at this point, so values derived from it
// earlier are recomputed afterwards rather than held in registers.
__device__ __forceinline__ void opaque(u32x4& a, u32x4& b) {
    asm volatile("" : "+v"(a), "+v"(b));
}

// 16-byte accesses.  load16 is for data that is reused (gamma); the
// stream variants set the non-temporal bit, for row data that each kernel
// touches exactly once, so it does not displace reused lines in L2 and the
// Infinity Cache (measured on MI355X with the RMSNorm backward at
// [65536, 4096] fp32: non-temporal loads and stores 521-525 us; plain stores
// 586-589 us, plain loads 577 us, write-through stores (sc1) 533-538 us).
template <class S>
__device__ __forceinline__ u32x4 load16(const typename S::T* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
template <class S>
__device__ __forceinline__ u32x4 load16_stream(const typename S::T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
template <class S>
__device__ __forceinline__ void store16_stream(typename S::T* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---- buffer resources ---------------------------------------------------------
// A raw buffer resource (stride 0, no swizzle) over `bytes` bytes at `base`.
// The hardware range-checks every access against `bytes`: a load at or past
// the end returns zero and a store there is dropped, without touching memory.
// Kernels use this to make tails and inactive rows branch-free: the same
// instructions run on every path, so the compiler's s_waitcnt placement can
// count exactly which loads are still in flight.  Base and size live in
// scalar registers, so they must be wave-uniform.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;      // gfx9 family: 32-bit data format, raw
constexpr int kCachePolicyNT = 2;           // non-temporal
constexpr uint32_t kOffOut = 0x80000000u;   // an offset past any buffer this code makes

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), kRsrcWord3);
}
__device__ __forceinline__ u32x4 bload16_stream(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCachePolicyNT);
}
__device__ __forceinline__ void bstore16_stream(rsrc_t r, uint32_t off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCachePolicyNT);
}
__device__ __forceinline__ float bload_f32(rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// ---- reductions -------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Sum over the TPR (<= 64) lanes of a row group; every lane of the group ends
// with the same value.  Each step adds the partner lane of a fixed pairing:
// DPP quad permutes for lanes 1 and 2 apart, DPP row mirrors for the halves of
// 8- and 16-lane rows (fused into v_add_f32_dpp), a ds_swizzle swap for the
// 16-lane halves of 32 and two lane reads for the wave halves -- no LDS round
// trips except the one swizzle.  Pairings are symmetric, so partners compute
// a + b and b + a, which are the same bits.  Every lane of the wave must be
// active (all callers reduce with the whole workgroup).
template <int TPR>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (TPR >= 2) v += dpp_mov<0xb1>(v);   // quad_perm [1,0,3,2]
    if constexpr (TPR >= 4) v += dpp_mov<0x4e>(v);   // quad_perm [2,3,0,1]
    if constexpr (TPR >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror
    if constexpr (TPR >= 16) v += dpp_mov<0x140>(v); // row_mirror
    if constexpr (TPR >= 32)                         // swap 16-lane halves of 32
        v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
    if constexpr (TPR >= 64)
        v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    return v;
}

// Row sum for a row spread over TPR lanes; the workgroup holds G such rows.
// For TPR > 64 the per-wave sums go through `red` (double-buffered by
// `parity`, so one barrier per row is enough: a wave can only overwrite a
// slot after every wave has passed the barrier that follows its last read)
// and are added in wave order.
template <int TPR, int G>
__device__ __forceinline__ float row_sum(float v, float (*red)[TPR > 64 ? G * (TPR / 64) : 1],
                                         int parity) {
    v = group_sum<TPR>(v);
    if constexpr (TPR > 64) {
        constexpr int kWaves = TPR / 64;
        const int lane = threadIdx.x & 63;
        const int wave_in_row = (threadIdx.x % TPR) >> 6;
        const int row_slot = threadIdx.x / TPR;
        if (lane == 0) red[parity][row_slot * kWaves + wave_in_row] = v;
        __syncthreads();
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += red[parity][row_slot * kWaves + w];
        v = s;
    }
    return v;
}

// ---- launch plans -------------------------------------------------------------

// A resident launch shape: TPR lanes per row, NV 16-byte slots per lane, G
// rows in flight per workgroup (workgroup = TPR * G lanes).
struct Plan {
    int tpr = 0;  // 0 = looped kernel
    int nv = 0;
    int g = 0;
};

// Instantiated shapes.  Each compiles without register spills for both
// storage types (hipcc -Rpass-analysis=kernel-resource-usage); wider rows
// take the looped kernels.
#define AGK_FWD_SHAPES(X)                                                                  \
    X(1, 1, 512) X(1, 2, 512) X(2, 2, 256) X(4, 2, 128) X(8, 2, 64) X(16, 2, 32) X(32, 2, 16) \
    X(64, 2, 4) X(64, 4, 4) X(128, 2, 2) X(128, 4, 2) X(256, 2, 1) X(256, 4, 1)            \
    X(512, 2, 1) X(512, 4, 1) X(1024, 2, 1) X(1024, 4, 1) X(1024, 8, 1)

struct Shape3 { int tpr, nv, g; };
constexpr Shape3 kFwdShapes[] = {
#define AGK_X(a, b, c) {a, b, c},
    AGK_FWD_SHAPES(AGK_X)
#undef AGK_X
};

template <size_t N>
inline bool has_shape(const Shape3 (&shapes)[N], const Plan& p) {
    for (const Shape3& s : shapes)
        if (s.tpr == p.tpr && s.nv == p.nv && s.g == p.g) return true;
    return false;
}

inline int pow2_at_least(int64_t v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Resident shapes, chosen from the row width in 16-byte slots (nslot) and the
// row count (measured on MI355X with a sweep of every instantiated shape):
//  - rows of at most 64 slots: two slots per lane (one for a one-slot row),
//    TPR = nslot / 2 rounded up to a power of two (at most 32 lanes, so a row
//    never spans waves and needs no barrier), and 512-lane workgroups of
//    512 / TPR rows.  Swept at 1 GiB over fp32 widths 64-512 and bf16 widths
//    128-1024 against 1- and 4-slot shapes and 256-lane workgroups: within
//    1 % of the best shape at every width, up to 3 % ahead of one slot per
//    lane (bf16 rows of 128-512 columns);
//  - wider rows: NV slots per lane, TPR = nslot / NV rounded up.  With many
//    rows NV = 2 (more lanes in flight per row); with fewer rows NV = 4, so
//    the grid still has enough workgroups.  NV doubles when a row would need
//    more than 1024 lanes.
// Returns tpr = 0 (looped kernel) when no instantiated shape holds the row.
template <size_t N>
inline Plan pick_plan(const Shape3 (&shapes)[N], int64_t nslot, int nv0, int small_threads,
                      int max_nv) {
    Plan p;
    if (nslot <= 64) {
        p.nv = nslot >= 2 ? 2 : 1;
        p.tpr = pow2_at_least((nslot + p.nv - 1) / p.nv);
        p.g = small_threads / p.tpr;
    } else {
        int nv = nv0;
        int64_t tpr = pow2_at_least((nslot + nv - 1) / nv);
        while (tpr > 1024 && nv < max_nv) {
            nv <<= 1;
            tpr = pow2_at_least((nslot + nv - 1) / nv);
        }
        if (tpr > 1024) return Plan{};
        if (tpr < 64) {
            tpr = 64;
            nv = pow2_at_least((nslot + 63) / 64);
        }
        p.tpr = static_cast<int>(tpr);
        p.nv = nv;
        p.g = tpr >= 256 ? 1 : static_cast<int>(256 / tpr);
    }
    if (has_shape(shapes, p)) return p;
    for (const Shape3& s : shapes)  // same (TPR, NV), another G
        if (s.tpr == p.tpr && s.nv == p.nv) return Plan{s.tpr, s.nv, s.g};
    return Plan{};
}

inline Plan fwd_plan(int64_t nslot, int64_t rows) {
    return pick_plan(kFwdShapes, nslot, rows > kLargeRows ? 2 : 4, 512, 8);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The HIP error behind the calling thread's last AGK_EHIP (hipSuccess if none).
inline thread_local hipError_t t_last_hip_error = hipSuccess;

inline int status_from_hip(hipError_t e) {
    if (e == hipSuccess) return AGK_OK;
    t_last_hip_error = e;
    return AGK_EHIP;
}

inline int check_launch() { return status_from_hip(hipGetLastError()); }

// Discards an error another component left pending on this thread (HIP keeps
// the last error until someone reads it), so that check_launch() reports only
// failures of this library's own launches.
inline void clear_pending_error() { (void)hipGetLastError(); }

// Validates sizes common to every entry point.  Returns AGK_OK, or an error.
inline int check_sizes(int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return AGK_EINVAL;
    if (cols > 0x7fffffffLL) return AGK_EINVAL;
    if (cols > 0 && rows > INT64_MAX / cols) return AGK_EINVAL;
    return AGK_OK;
}

inline bool valid_dtype(int dt) { return dt == AGK_F32 || dt == AGK_BF16; }

}  // namespace agk
