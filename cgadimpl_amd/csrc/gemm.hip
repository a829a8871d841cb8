// gemm.hip -- bf16 GEMM on CDNA4 (gfx950) MFMA with fp32 accumulation, for the
// RMSNorm + linear layer (configuration c5): the forward y = h * W and the VJP
// dh = dy * W^T, dW = h^T * dy of the reference's matmul
// (cgadimpl/src/ops/linalg.cpp:12-20, cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:258-263).
//
//   C[m, n] (+)= rowscale[m] * sum_k (A[m, k] * kscale[k]) * B[k, n]
//
// The two optional scales carry the RMSNorm into the GEMM without
// materialising h = diag(r) * x * diag(gamma):
//   y  = h * W        = diag(r) * (x * diag(gamma)) * W    kscale = gamma, rowscale = r
//   dW = h^T * dy     = diag(gamma) * (x^T * diag(r)) * dy  kscale = r,     rowscale = gamma
// (kscale multiplies the A operand as it is staged, rounding to bf16 as a
// stored h would be; rowscale multiplies the fp32 accumulator.)
//
// Two kernels share the tile shape.  When K is a multiple of 64 and there is
// no k-scale, the product runs on the direct-to-LDS kernel further below,
// which stages whole 128-byte lines of either operand layout through two
// 64-deep LDS stages without registers; otherwise the register-staged kernel
// described here runs.
//
// Kernel shape.  A workgroup of 512 lanes (8 waves, 2 along M x 4 along N)
// computes a 256 x 256 tile of C; each wave owns 128 x 64 of it as 4 x 2
// v_mfma_f32_32x32x16_bf16 accumulators (128 fp32 registers per lane).  K is
// walked in steps of 64: the next step's A and B tiles are loaded from HBM /
// L2 into registers while the current step's tiles are multiplied out of LDS,
// then written to the other half of a double-buffered LDS (one barrier per
// step).  LDS rows are k-contiguous (each MFMA operand is 8 consecutive k of
// one row or column, one 16-byte LDS read).  An operand stored with k
// contiguous in memory ([rows][K])
// is copied in 16-byte chunks; an operand stored with k strided ([K][rows])
// is read 4 k-rows x 8 values per lane and transposed in registers
// (v_perm_b32) into 8-byte LDS writes.
//
// LDS rows are 128 bytes, unpadded, with XOR-swizzled 16-byte chunks (lds_off:
// no bank conflicts, measured with SQ_LDS_BANK_CONFLICT), and the
// global loads are issued unconditionally at clamped in-range addresses (out
// of range values are zeroed afterwards), so the compiler can keep the next
// step's loads in flight across the MFMA block.
//
// MFMA lane layout (checked on MI355X): A operand lane l holds row l % 32,
// k = (l / 32) * 8 .. +7; B operand lane l holds column l % 32, the same k;
// accumulator element e of lane l is C[8 * (e / 4) + 4 * (l / 32) + e % 4][l % 32].

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <atomic>

#include "agk_rmsnorm.h"

namespace agk_gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kThreads = 512;
constexpr int kWavesN = 4;
constexpr int WM = 128, WN = 64;            // per-wave tile
constexpr int TM = WM / 32, TN = WN / 32;   // MFMA tiles per wave
constexpr int kStride = BK;                 // bf16 per LDS row (128 bytes)
constexpr int kStageElems = (BM + BN) * kStride;

// LDS position of k-chunk c (8 bf16 = 16 bytes) of row `row`: chunks are
// XOR-swizzled by the row's low bits, so the 8 lanes of a 16-byte fragment
// read (8 consecutive rows, one chunk) and the 8-byte writes of the
// transposing stager (rows 8 apart) land on different banks.
__device__ __forceinline__ int lds_off(int row, int c) {
    return row * kStride + ((c ^ (row & 7) ^ ((row >> 3) & 7)) << 3);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32: NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
// lo16(a) | lo16(b) << 16 and hi16(a) | hi16(b) << 16 (v_perm_b32)
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// ---- operand staging --------------------------------------------------------
// An operand tile is R = 256 rows (of A: m, of B: n) by BK = 64 k.
//
// k-contiguous source ([rows][ld], k along the row): chunk c = tid + j*512,
// row = c / 8, 8-element k-chunk c % 8 (every chunk of a thread has the same
// k-chunk, tid % 8).
// k-strided source ([K][ld], rows along the row): lane owns 8 rows
// (8 * (tid % 32) ..) at 4 consecutive k (4 * (tid / 32) ..).
template <bool KCONTIG>
struct Stage {
    u32x4 v[4];
};

template <bool KCONTIG, bool SCALE>
__device__ __forceinline__ void load_tile(Stage<KCONTIG>& s, const uint16_t* __restrict__ src,
                                          int64_t ld, int row0, int rows, int k0, int K,
                                          const float* __restrict__ kscale) {
    const int tid = threadIdx.x;
    if constexpr (KCONTIG) {
        const int kc = (tid & 7) * 8;
        const int k = k0 + kc;
        float ks[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // past K: chunks are zero
        if constexpr (SCALE) {
            if (k < K) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(kscale + k);
                const f32x4 b = *reinterpret_cast<const f32x4*>(kscale + k + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ks[e] = a[e];
                    ks[e + 4] = b[e];
                }
            }
        }
        const int kcl = k < K ? k : K - 8;  // in-range address; zeroed below
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = (tid >> 3) + j * (kThreads / 8);
            const int grow = row0 + row;
            const int gcl = grow < rows ? grow : rows - 1;
            u32x4 v = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(gcl) * ld + kcl);
            if (!(grow < rows && k < K)) v = u32x4{0u, 0u, 0u, 0u};
            if constexpr (SCALE) {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    v[w] = pack_bf16(bf16_lo(v[w]) * ks[2 * w], bf16_hi(v[w]) * ks[2 * w + 1]);
            }
            s.v[j] = v;
        }
    } else {
        const int r = (tid & 31) * 8;
        const int kq = (tid >> 5) * 4;
        const int grow = row0 + r;
        const int gcl = grow < rows ? grow : rows - 8;  // in-range address; zeroed below
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = k0 + kq + j;
            const int kcl = k < K ? k : K - 1;
            u32x4 v = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(kcl) * ld + gcl);
            if (!(grow < rows && k < K)) v = u32x4{0u, 0u, 0u, 0u};
            if constexpr (SCALE) {
                const float ks = k < K ? kscale[k] : 0.0f;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    v[w] = pack_bf16(bf16_lo(v[w]) * ks, bf16_hi(v[w]) * ks);
            }
            s.v[j] = v;
        }
    }
}

template <bool KCONTIG>
__device__ __forceinline__ void store_tile(const Stage<KCONTIG>& s, uint16_t* lds) {
    const int tid = threadIdx.x;
    if constexpr (KCONTIG) {
        const int c = tid & 7;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = (tid >> 3) + j * (kThreads / 8);
            *reinterpret_cast<u32x4*>(lds + lds_off(row, c)) = s.v[j];
        }
    } else {
        // s.v[j] holds k = kq + j for rows r .. r+7 (two rows per word);
        // row r + e receives its 4 k values as one 8-byte write.
        const int r = (tid & 31) * 8;
        const int kq = (tid >> 5) * 4;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const u32x2 even = {lo_pair(s.v[0][w], s.v[1][w]), lo_pair(s.v[2][w], s.v[3][w])};
            const u32x2 odd = {hi_pair(s.v[0][w], s.v[1][w]), hi_pair(s.v[2][w], s.v[3][w])};
            *reinterpret_cast<u32x2*>(lds + lds_off(r + 2 * w, kq >> 3) + (kq & 7)) = even;
            *reinterpret_cast<u32x2*>(lds + lds_off(r + 2 * w + 1, kq >> 3) + (kq & 7)) = odd;
        }
    }
}

__device__ __forceinline__ bf16x8 lds_frag(const uint16_t* lds, int row, int k) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + lds_off(row, k >> 3)));
}

// ---- tile order ----------------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup L runs on
// XCD L % 8), each XCD with its own L2.  The tile order below gives each XCD
// a contiguous chunk of a grouped ordering (group_m m-tiles x all n-tiles,
// column by column), so the ~32 workgroups resident on one XCD at a time
// cover about group_m x 32 / group_m tiles and share their A row-panels and B
// column-panels in that XCD's L2, instead of every neighbouring tile landing
// on a different XCD.  group_m = 4 unless a measured order is known for the
// shape (tuned_group_m).
constexpr int kXcds = 8;
constexpr int kGroupM = 4;

__device__ __forceinline__ void tile_of(int L, int tiles_m, int tiles_n, int group_m, int& tm,
                                        int& tn) {
    const int T = tiles_m * tiles_n;
    const int x = L % kXcds, s = L / kXcds;
    const int q = T / kXcds, r = T % kXcds;  // XCDs below r get q + 1 tiles
    const int g = x < r ? x * (q + 1) + s : r * (q + 1) + (x - r) * q + s;
    const int per_group = group_m * tiles_n;
    const int group = g / per_group;
    const int gm0 = group * group_m;
    const int gsize = tiles_m - gm0 < group_m ? tiles_m - gm0 : group_m;
    const int in = g - group * per_group;
    tm = gm0 + in % gsize;
    tn = in / gsize;
}

// The product rounded to bf16, plus a bf16 bias term (then rounded again when
// stored): `matmul(X, W^T) + b` with its two roundings, as a bf16 product and
// a bf16 sum give them.
__device__ __forceinline__ float with_bias(float v, uint16_t b) {
    v = __uint_as_float(f32_to_bf16_bits(v) << 16);
    return v + __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// ---- the kernel ---------------------------------------------------------------

template <bool A_KCONTIG, bool B_KCONTIG, bool KSCALE, bool OUT_F32>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B, int64_t ldb,
    void* __restrict__ C, int64_t ldc, int M, int N, int K, const float* __restrict__ kscale,
    const float* __restrict__ rowscale, const uint16_t* __restrict__ colbias, int accumulate,
    int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStageElems];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / kWavesN;
    const int wn = wave % kWavesN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, kGroupM, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    Stage<A_KCONTIG> sa;
    Stage<B_KCONTIG> sb;
    const int nk = (K + BK - 1) / BK;
    load_tile<A_KCONTIG, KSCALE>(sa, A, lda, m0, M, 0, K, kscale);
    load_tile<B_KCONTIG, false>(sb, B, ldb, n0, N, 0, K, nullptr);
    store_tile<A_KCONTIG>(sa, lds);
    store_tile<B_KCONTIG>(sb, lds + BM * kStride);
    __syncthreads();

    const int frow = lane & 31;
    const int fk = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const uint16_t* cur = lds + (kt & 1) * kStageElems;
        const bool more = kt + 1 < nk;
        if (more) {
            load_tile<A_KCONTIG, KSCALE>(sa, A, lda, m0, M, (kt + 1) * BK, K, kscale);
            load_tile<B_KCONTIG, false>(sb, B, ldb, n0, N, (kt + 1) * BK, K, nullptr);
        }
        // fragments of k-substep ks + 16 are read while ks is multiplied
        bf16x8 af[2][TM], bf[2][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[0][i] = lds_frag(cur, wm * WM + i * 32 + frow, fk);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[0][j] = lds_frag(cur + BM * kStride, wn * WN + j * 32 + frow, fk);
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            const int c = s & 1;
            if (s + 1 < BK / 16) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[c ^ 1][i] = lds_frag(cur, wm * WM + i * 32 + frow, (s + 1) * 16 + fk);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bf[c ^ 1][j] = lds_frag(cur + BM * kStride, wn * WN + j * 32 + frow,
                                            (s + 1) * 16 + fk);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[c][i], bf[c][j],
                                                                        acc[i][j], 0, 0, 0);
        }
        if (more) {
            uint16_t* nxt = lds + ((kt + 1) & 1) * kStageElems;
            store_tile<A_KCONTIG>(sa, nxt);
            store_tile<B_KCONTIG>(sb, nxt + BM * kStride);
        }
        __syncthreads();
    }

    // epilogue: element e of acc[i][j] is C[row][col] below
    const int col_l = lane & 31;
    const int row_l = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm * WM + i * 32 + 8 * (e >> 2) + row_l + (e & 3);
            if (row >= M) continue;
            const float rs = rowscale ? rowscale[row] : 1.0f;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + wn * WN + j * 32 + col_l;
                if (col >= N) continue;
                float v = acc[i][j][e] * rs;
                // accumulation rounds the product first (no fused multiply-add)
                asm volatile("" : "+v"(v));
                if constexpr (OUT_F32) {
                    float* p = static_cast<float*>(C) + static_cast<int64_t>(row) * ldc + col;
                    *p = accumulate ? *p + v : v;
                } else {
                    uint16_t* p = static_cast<uint16_t*>(C) + static_cast<int64_t>(row) * ldc + col;
                    if (accumulate) v = __uint_as_float(static_cast<uint32_t>(*p) << 16) + v;
                    if (colbias) v = with_bias(v, colbias[col]);
                    *p = static_cast<uint16_t>(f32_to_bf16_bits(v));
                }
            }
        }
    }
}

// ---- direct-to-LDS kernel: both operands k-contiguous, K a multiple of 64 ----
// Staging without registers: buffer_load_dwordx4 ... lds writes lane l's 16
// bytes to LDS at (wave-uniform base) + 16 * l, so one wave instruction fills
// a contiguous kilobyte of LDS; each lane fetches the global chunk that belongs
// at its position of the swizzled layout.  Rows past M or N are fetched from
// the last valid row (never stored).  The epilogue store_c writes the wave's
// 128 x 64 block of C.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// GENERAL: rowscale, a column bias (bf16 output only) and accumulate
// honoured; CHECK: rows past M and columns past N skipped.  store_c picks the
// variant once per call (uniform values), so the common plain, interior store
// has no per-element branches.
template <bool OUT_F32, bool GENERAL, bool CHECK>
__device__ __forceinline__ void store_c_impl(const f32x16 (&acc)[TM][TN], void* __restrict__ C,
                                             int64_t ldc, int M, int N, int m0, int n0, int wm,
                                             int wn, int lane, const float* __restrict__ rowscale,
                                             const uint16_t* __restrict__ colbias,
                                             int accumulate) {
    const int col_l = lane & 31;
    const int row_l = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm * WM + i * 32 + 8 * (e >> 2) + row_l + (e & 3);
            if (CHECK && row >= M) continue;
            float rs = 1.0f;
            if constexpr (GENERAL) rs = rowscale ? rowscale[row] : 1.0f;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + wn * WN + j * 32 + col_l;
                if (CHECK && col >= N) continue;
                float v = acc[i][j][e];
                if constexpr (GENERAL) {
                    v *= rs;
                    // accumulation rounds the product first (no fused multiply-add)
                    asm volatile("" : "+v"(v));
                }
                if constexpr (OUT_F32) {
                    float* p = static_cast<float*>(C) + static_cast<int64_t>(row) * ldc + col;
                    if constexpr (GENERAL) {
                        *p = accumulate ? *p + v : v;
                    } else {
                        // Plain fp32 stores are whole 128-byte lines per 32 lanes:
                        // non-temporal, so a round's C tiles (64 MB) do not evict
                        // the operand panels from L2 and stream out as they come.
                        // Measured on dW at c5 (4096 x 11008 x 8192, one box, three
                        // alternations): 557-561 -> 528-529 us.  bf16 outputs keep
                        // ordinary stores: no gain there, and the RMSNorm backward
                        // reads dh from the caches right after its product.
                        __builtin_nontemporal_store(v, p);
                    }
                } else {
                    uint16_t* p = static_cast<uint16_t*>(C) + static_cast<int64_t>(row) * ldc + col;
                    if constexpr (GENERAL) {
                        if (accumulate) v = __uint_as_float(static_cast<uint32_t>(*p) << 16) + v;
                        if (colbias) v = with_bias(v, colbias[col]);
                    }
                    *p = static_cast<uint16_t>(f32_to_bf16_bits(v));
                }
            }
        }
    }
}

// bn: the columns the calling tile covers from n0 (BN, or BN / 2 for a half tile).
template <bool OUT_F32>
__device__ __forceinline__ void store_c(const f32x16 (&acc)[TM][TN], void* __restrict__ C,
                                        int64_t ldc, int M, int N, int m0, int n0, int wm, int wn,
                                        int lane, const float* __restrict__ rowscale,
                                        const uint16_t* __restrict__ colbias, int accumulate,
                                        int bn = BN) {
    if (rowscale != nullptr || colbias != nullptr || accumulate) {
        store_c_impl<OUT_F32, true, true>(acc, C, ldc, M, N, m0, n0, wm, wn, lane, rowscale,
                                          colbias, accumulate);
    } else if (m0 + BM <= M && n0 + bn <= N) {
        store_c_impl<OUT_F32, false, false>(acc, C, ldc, M, N, m0, n0, wm, wn, lane, nullptr,
                                            nullptr, 0);
    } else {
        store_c_impl<OUT_F32, false, true>(acc, C, ldc, M, N, m0, n0, wm, wn, lane, nullptr,
                                           nullptr, 0);
    }
}

// ---- direct-to-LDS kernel -----------------------------------------------------
// The same 256 x 256 tile, over 4 waves of 128 x 128 (2 x 2; 4 x 4 MFMA tiles
// per wave, whose 256 accumulator registers live in AGPRs).  K is walked in
// 64-deep tiles through two LDS stages of 64 KiB (32 KiB per operand), filled by
// `buffer_load_dwordx4 ... lds`, so staging takes no registers.  Each operand is
// staged in the layout it has in memory:
// - k-contiguous ([rows][K]): 256 LDS rows of 64 k (128 bytes, 8 XOR-swizzled
//   16-byte chunks: lds_off above); a fragment is one 16-byte read.
// - k-strided (TR; [K][cols], the columns contiguous): 64 LDS rows of one k
//   each, 256 columns (512 bytes, 32 chunks whose 64-byte groups are XOR-
//   swizzled by k % 4: tr_off); a fragment is two ds_read_b64_tr_b16.  Within
//   each 16 lanes that instruction hands lane 4a + b, for e = 0..3, the element
//   at offset b from the address of lane 4e + a (checked on MI355X), so lane s
//   pointing at k0 + s / 4, column c0 + 4 (s % 4) gives lane j the four k
//   k0 .. k0 + 3 of column c0 + j: the MFMA operand layout.  No transposed copy
//   of the operand is made.
// Either way one load instruction moves 1 KiB of whole 128-byte lines, and the
// LDS destination of load j of wave w is the same kilobyte.
//
// Why this shape (measured on MI355X, c5 products):
// - Whole 128-byte rows per load: 32-deep tiles (64 bytes per row) asked L2 for
//   each line twice, half at a time, and the L1's queue of pending misses, not
//   HBM, set the pace (twice hipBLASLt's L2 request count for the same bytes,
//   TCP_TCC_READ_REQ).
// - One wave per SIMD with a 128 x 128 block reads a third fewer LDS bytes per
//   MFMA than two waves of 128 x 64, and its stream of 64 MFMAs per tile has
//   the loads and fragment reads interleaved between them; it was 4-6 % faster
//   than eight waves of 128 x 64 with the same stages.
//
// Schedule of tile t (after the barrier that makes tile t visible and frees the
// other stage): the 16 loads of tile t + 1 go into the other stage, one per
// two MFMAs of the first two substeps; the fragments run one 16-deep substep
// ahead of the MFMAs, so the substep that straddles the barrier (the last of
// tile t - 1) multiplies while tile t's first fragments are read.  At the end
// of the tile each wave waits for its own loads and reads, then the barrier.
constexpr int kDirectThreads = 256;
constexpr int kTrRow = 256;               // bf16 per LDS row of a k-strided operand

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_t;

// Element offset of column col (a multiple of 4) of k-row k in a k-strided stage.
__device__ __forceinline__ int tr_off(int k, int col) {
    return k * kTrRow + ((((col >> 3) ^ ((k & 3) << 2))) << 3) + (col & 7);
}

struct DirectStage {
    __amdgpu_buffer_rsrc_t ra, rb;  // the tile's A and B (base and size in SGPRs)
    uint32_t oa[8], ob[8];          // byte offset of each lane's chunk, per load
    int step_a, step_b;             // bytes from one 64-deep k-tile to the next
};

// Load j of a wave (j = 0..7) fills kilobyte wave * 8 + j of one operand's half
// of `stage`; tile t's data starts t * step bytes into the operand.
__device__ __forceinline__ void direct_issue_a(const DirectStage& d, uint16_t* stage, int t,
                                               int wave) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(d.ra, (lds_ptr_t)(stage + (wave * 8 + j) * 512),
                                                 16, d.oa[j], t * d.step_a, 0, 0);
}
__device__ __forceinline__ void direct_issue_b(const DirectStage& d, uint16_t* stage, int t,
                                               int wave) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            d.rb, (lds_ptr_t)(stage + BM * BK + (wave * 8 + j) * 512), 16, d.ob[j], t * d.step_b,
            0, 0);
}

// Per-lane byte offsets of one operand's loads.  rows: valid rows (k-contiguous)
// or columns (k-strided) of the tile; ld: leading dimension in elements.
template <bool TR>
__device__ __forceinline__ void direct_offsets(uint32_t (&o)[8], int wave, int lane, int rows,
                                               int64_t ld) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if constexpr (!TR) {
            const int row = wave * 64 + j * 8 + (lane >> 3);
            const int c = (lane & 7) ^ (row & 7) ^ ((row >> 3) & 7);  // chunk of slot lane % 8
            const int r = row < rows ? row : rows - 1;  // rows past M or N: the last valid row
            o[j] = (static_cast<uint32_t>(r) * static_cast<uint32_t>(ld) + c * 8) * 2;
        } else {
            const int k = wave * 16 + j * 2 + (lane >> 5);
            const int c = (lane & 31) ^ ((k & 3) << 2);  // chunk of slot lane % 32
            const int col = c * 8 < rows ? c * 8 : rows - 8;  // columns past M or N: the last 8
            o[j] = (static_cast<uint32_t>(k) * static_cast<uint32_t>(ld) + col) * 2;
        }
    }
}

// The fragments of one 16-deep substep s (0..3) of a wave: 4 of A (128 rows),
// NB of B (32 NB columns: 4 for the 256 x 256 tile, 2 for the 256 x 128 half
// tiles of a last round).
template <int NB>
struct Frags {
    bf16x8 a[TM], b[NB];
};

// MFMA operand lane l (row or column l % 32, k 8 (l / 32) .. + 7) of block
// column base c0, substep s, from a k-strided stage: two transposing reads of
// four k each.
__device__ __forceinline__ bf16x8 tr_frag(const uint16_t* lds, int c0, int s, int lane) {
    const int g = lane >> 4, sl = lane & 15;
    const int k = s * 16 + (g >> 1) * 8 + (sl >> 2);
    const int col = c0 + (g & 1) * 16 + 4 * (sl & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(lds + tr_off(k, col)));
    const s16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(lds + tr_off(k + 4, col)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// bc: the wave's first B column within the stage.
template <bool A_TR, bool B_TR, int NB>
__device__ __forceinline__ void read_frags(Frags<NB>& f, const uint16_t* stage, int s, int wm,
                                           int bc, int frow, int fk, int lane) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        if constexpr (A_TR) f.a[i] = tr_frag(stage, wm * WM + i * 32, s, lane);
        else f.a[i] = lds_frag(stage, wm * WM + i * 32 + frow, s * 16 + fk);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        if constexpr (B_TR) f.b[j] = tr_frag(stage + BM * BK, bc + j * 32, s, lane);
        else f.b[j] = lds_frag(stage + BM * kStride, bc + j * 32 + frow, s * 16 + fk);
    }
}

template <int NB>
__device__ __forceinline__ void mfma_sub(const Frags<NB>& f, f32x16 (&acc)[TM][NB]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Scheduling groups: one load, one fragment read, two MFMAs (AGK_LRM); one
// fragment read, two MFMAs (AGK_RM).  Eight of them cover a substep's 16 MFMAs.
#define AGK_LRM                                         \
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#define AGK_RM                                          \
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#define AGK_X8(g) g g g g g g g g

// Tile t of nk.  FIRST (tile 0) has no straddling substep; every step loads
// tile t + 1 (the last tile again at the end, into the stage nothing reads
// again).  Entering, f1 holds substep 3 of tile t - 1.  NB = 4: the 256 x 256
// tile, whose substeps interleave one load, one fragment read and two MFMAs;
// NB = 2 (half tiles): the same loads and reads around half the MFMAs, left to
// the compiler's schedule.
#define AGK_SUBSTEP_LRM    \
    if constexpr (NB == 4) { \
        AGK_X8(AGK_LRM)    \
    }
#define AGK_SUBSTEP_RM     \
    if constexpr (NB == 4) { \
        AGK_X8(AGK_RM)     \
    }
template <bool FIRST, bool A_TR, bool B_TR, int NB>
__device__ __forceinline__ void direct_step(const DirectStage& d, const uint16_t* cur,
                                            uint16_t* other, int t, int nk,
                                            f32x16 (&acc)[TM][NB], Frags<NB>& f0, Frags<NB>& f1,
                                            int wm, int bc, int frow, int fk, int lane,
                                            int wave) {
    const int tn = t + 1 < nk ? t + 1 : nk - 1;
    direct_issue_a(d, other, tn, wave);
    read_frags<A_TR, B_TR>(f0, cur, 0, wm, bc, frow, fk, lane);
    if constexpr (!FIRST) {
        mfma_sub(f1, acc);
        AGK_SUBSTEP_LRM
    }
    __builtin_amdgcn_sched_barrier(0);
    direct_issue_b(d, other, tn, wave);
    read_frags<A_TR, B_TR>(f1, cur, 1, wm, bc, frow, fk, lane);
    mfma_sub(f0, acc);
    AGK_SUBSTEP_LRM
    __builtin_amdgcn_sched_barrier(0);
    read_frags<A_TR, B_TR>(f0, cur, 2, wm, bc, frow, fk, lane);
    mfma_sub(f1, acc);
    AGK_SUBSTEP_RM
    __builtin_amdgcn_sched_barrier(0);
    read_frags<A_TR, B_TR>(f1, cur, 3, wm, bc, frow, fk, lane);
    mfma_sub(f0, acc);
    AGK_SUBSTEP_RM
    __builtin_amdgcn_sched_barrier(0);
    // This wave's loads of tile t + 1 have landed and its reads of tile t are
    // done; after the barrier every wave's are.  A bare barrier:
    // __syncthreads()'s fence adds nothing here (vmcnt and lgkmcnt are zero).
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// One tile's k loop and store.  NB = 4: the 256 x 256 tile at (m0, n0), wave
// (wm, wn) owning its 128 x 128 block; NB = 2: the 256 x 128 half of that tile
// starting at column n0 + half_off, wave (wm, wn) owning a 128 x 64 block.
// Both stage the tile's full 256 B columns (the same loads).
template <bool OUT_F32, bool A_TR, bool B_TR, int NB>
__device__ __forceinline__ void direct_tile(const DirectStage& d, uint16_t* st0, uint16_t* st1,
                                            void* __restrict__ C, int64_t ldc, int M, int N,
                                            int K, int m0, int n0, int half_off, int wm, int wn,
                                            int lane, int wave,
                                            const float* __restrict__ rowscale,
                                            const uint16_t* __restrict__ colbias,
                                            int accumulate) {
    f32x16 acc[TM][NB];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int nk = K / BK;  // >= 1: K is a positive multiple of 64
    const int frow = lane & 31;
    const int fk = (lane >> 5) * 8;  // MFMA operand lanes 32..63 hold k 8..15
    const int bc = half_off + wn * (NB * 32);  // the wave's first B column in the stage
    direct_issue_a(d, st0, 0, wave);
    direct_issue_b(d, st0, 0, wave);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    Frags<NB> f0, f1;
    direct_step<true, A_TR, B_TR>(d, st0, st1, 0, nk, acc, f0, f1, wm, bc, frow, fk, lane, wave);
    int t = 1;
    for (; t + 1 < nk; t += 2) {
        direct_step<false, A_TR, B_TR>(d, st1, st0, t, nk, acc, f0, f1, wm, bc, frow, fk, lane,
                                       wave);
        direct_step<false, A_TR, B_TR>(d, st0, st1, t + 1, nk, acc, f0, f1, wm, bc, frow, fk,
                                       lane, wave);
    }
    if (t < nk)
        direct_step<false, A_TR, B_TR>(d, st1, st0, t, nk, acc, f0, f1, wm, bc, frow, fk, lane,
                                       wave);
    mfma_sub(f1, acc);  // substep 3 of the last tile

    if constexpr (NB == 4) {
        // the wave's 128 x 128 block leaves as two 128 x 64 halves (store_c's layout)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x16 part[TM][TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) part[i][j] = acc[i][h * TN + j];
            store_c<OUT_F32>(part, C, ldc, M, N, m0, n0, wm, 2 * wn + h, lane, rowscale, colbias,
                             accumulate);
        }
    } else {
        store_c<OUT_F32>(acc, C, ldc, M, N, m0, n0 + half_off, wm, wn, lane, rowscale, colbias,
                         accumulate, BN / 2);
    }
}

// A_TR: A stored [K][lda] (its m contiguous); B_TR: B stored [K][ldb] (its n
// contiguous).  Otherwise the operand is [rows][ld] with k contiguous.
// Workgroups below full_tiles compute whole 256 x 256 tiles (tile_of's order);
// the ones after them split each remaining tile into two 256 x 128 halves
// (workgroup full_tiles + 2 h + q: half q of tile full_tiles + h), so that a
// last round of few tiles runs on twice as many CUs for half as long.  Every
// output element is summed in the same k order either way (bit-identical).
template <bool OUT_F32, bool A_TR, bool B_TR>
__global__ __launch_bounds__(kDirectThreads) void gemm_nt_direct_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B, int64_t ldb,
    void* __restrict__ C, int64_t ldc, int M, int N, int K, const float* __restrict__ rowscale,
    const uint16_t* __restrict__ colbias, int accumulate, int tiles_m, int tiles_n, int group_m,
    int full_tiles) {
    __shared__ __attribute__((aligned(16))) uint16_t st0[kStageElems];
    __shared__ __attribute__((aligned(16))) uint16_t st1[kStageElems];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform, so kept in scalar registers (LDS destinations of the loads)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int L = static_cast<int>(blockIdx.x);
    const bool halves = L >= full_tiles;
    const int tile = halves ? full_tiles + ((L - full_tiles) >> 1) : L;
    int tm, tn;
    tile_of(tile, tiles_m, tiles_n, group_m, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;

    const int rows_a = M - m0 < BM ? M - m0 : BM;
    const int rows_b = N - n0 < BN ? N - n0 : BN;
    DirectStage d;
    // the resources span the bytes the tile's loads can address (their k
    // position is the scalar offset, always inside the operand)
    d.ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(A_TR ? A + m0 : A + static_cast<int64_t>(m0) * lda),
        static_cast<short>(0),
        static_cast<int>(A_TR ? ((K - 1) * lda + rows_a) * 2 : ((rows_a - 1) * lda + K) * 2),
        0x00020000);
    d.rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(B_TR ? B + n0 : B + static_cast<int64_t>(n0) * ldb),
        static_cast<short>(0),
        static_cast<int>(B_TR ? ((K - 1) * ldb + rows_b) * 2 : ((rows_b - 1) * ldb + K) * 2),
        0x00020000);
    d.step_a = A_TR ? static_cast<int>(BK * lda * 2) : BK * 2;
    d.step_b = B_TR ? static_cast<int>(BK * ldb * 2) : BK * 2;
    direct_offsets<A_TR>(d.oa, wave, lane, rows_a, lda);
    direct_offsets<B_TR>(d.ob, wave, lane, rows_b, ldb);

    if (!halves)
        direct_tile<OUT_F32, A_TR, B_TR, 4>(d, st0, st1, C, ldc, M, N, K, m0, n0, 0, wm, wn, lane,
                                            wave, rowscale, colbias, accumulate);
    else
        direct_tile<OUT_F32, A_TR, B_TR, 2>(d, st0, st1, C, ldc, M, N, K, m0, n0,
                                            ((L - full_tiles) & 1) * (BN / 2), wm, wn, lane,
                                            wave, rowscale, colbias, accumulate);
}

// C for an empty reduction (K == 0): zeros, or the bf16 column bias in every
// row; rows of ldc, n columns of 4- or 2-byte elements (a kernel, not a memset
// node, so that the call can be captured).
__global__ __launch_bounds__(256) void zero_c_kernel(void* __restrict__ C, int64_t ldc, int n,
                                                     int elem_bytes,
                                                     const uint16_t* __restrict__ colbias) {
    char* p = static_cast<char*>(C) + static_cast<int64_t>(blockIdx.x) * ldc * elem_bytes;
    if (colbias) {  // bf16 output
        uint16_t* q = reinterpret_cast<uint16_t*>(p);
        for (int64_t i = threadIdx.x; i < n; i += 256) q[i] = colbias[i];
        return;
    }
    for (int64_t i = threadIdx.x; i < static_cast<int64_t>(n) * elem_bytes; i += 256) p[i] = 0;
}

// ---- transpose ----------------------------------------------------------------
// dst[c][r] = src[r][c] for a rows x cols bf16 matrix (rows, cols multiples of
// 8).  A 256-lane workgroup moves a 128 x 128 tile: each lane reads an 8 x 8
// block as 8 coalesced 16-byte row pieces, transposes it in registers
// (v_perm_b32) and writes its 8 columns as 16-byte pieces into an LDS tile
// laid out [dst row][src row] (rows padded by 16 bytes); after a barrier the
// tile leaves as coalesced 16-byte pieces of dst rows.  HBM-bound: one read and
// one write of the matrix.
constexpr int kTrTile = 128;
constexpr int kTrStride = kTrTile + 8;

__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ src,
                                                             int64_t ld_src,
                                                             uint16_t* __restrict__ dst,
                                                             int64_t ld_dst, int rows, int cols,
                                                             int tiles_c) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kTrTile * kTrStride];
    const int t = threadIdx.x;
    const int r0 = (blockIdx.x / tiles_c) * kTrTile;
    const int c0 = (blockIdx.x % tiles_c) * kTrTile;
    const int bc = t & 15, br = t >> 4;  // this lane's 8 x 8 block
    const int gr = r0 + br * 8, gc = c0 + bc * 8;
    if (gr < rows && gc < cols) {
        u32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(gr + i) * ld_src + gc));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const u32x4 even = {lo_pair(v[0][w], v[1][w]), lo_pair(v[2][w], v[3][w]),
                                lo_pair(v[4][w], v[5][w]), lo_pair(v[6][w], v[7][w])};
            const u32x4 odd = {hi_pair(v[0][w], v[1][w]), hi_pair(v[2][w], v[3][w]),
                               hi_pair(v[4][w], v[5][w]), hi_pair(v[6][w], v[7][w])};
            *reinterpret_cast<u32x4*>(tile + (bc * 8 + 2 * w) * kTrStride + br * 8) = even;
            *reinterpret_cast<u32x4*>(tile + (bc * 8 + 2 * w + 1) * kTrStride + br * 8) = odd;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int lr = (t >> 4) + 16 * j;  // dst row within the tile
        const int ch = t & 15;             // 16-byte piece of it
        const int dr = c0 + lr, dc = r0 + ch * 8;
        if (dr < cols && dc < rows)
            __builtin_nontemporal_store(
                *reinterpret_cast<const u32x4*>(tile + lr * kTrStride + ch * 8),
                reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(dr) * ld_dst + dc));
    }
}

inline int launch_transpose(const void* src, int64_t ld_src, void* dst, int64_t ld_dst, int rows,
                            int cols, hipStream_t st) {
    const int tr = (rows + kTrTile - 1) / kTrTile, tc = (cols + kTrTile - 1) / kTrTile;
    hipLaunchKernelGGL(transpose_bf16_kernel, dim3(tr * tc), dim3(256), 0, st,
                       static_cast<const uint16_t*>(src), ld_src, static_cast<uint16_t*>(dst),
                       ld_dst, rows, cols, tc);
    return hipGetLastError() == hipSuccess ? AGK_OK : AGK_EHIP;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (looked up once per device; 256 on
// MI355X), for the direct kernel's last-round split.
inline int device_cus() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cached[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
        v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
    return v;
}

// How many tiles the direct kernel computes whole: all of them, unless the
// last round (tiles beyond a multiple of the CU count) would fill at most half
// of the CUs; those tiles then run as two 256 x 128 halves each.
inline int direct_full_tiles(int tiles, int cus) {
    const int rem = tiles % cus;
    return (rem != 0 && 2 * rem <= cus) ? tiles - rem : tiles;
}

template <bool AK, bool BK_, bool KS, bool F32>
int launch(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int M,
           int N, int K, const float* kscale, const float* rowscale, const uint16_t* colbias,
           int accumulate, hipStream_t st) {
    const int tiles_m = (M + BM - 1) / BM;
    const int tiles_n = (N + BN - 1) / BN;
    hipLaunchKernelGGL((gemm_bf16_kernel<AK, BK_, KS, F32>), dim3(tiles_m * tiles_n),
                       dim3(kThreads), 0, st, static_cast<const uint16_t*>(A), lda,
                       static_cast<const uint16_t*>(B), ldb, C, ldc, M, N, K, kscale, rowscale,
                       colbias, accumulate, tiles_m, tiles_n);
    return hipGetLastError() == hipSuccess ? AGK_OK : AGK_EHIP;
}

// Dispatch over (A k-contiguous, B k-contiguous, k-scale, fp32 output).
template <bool AK, bool BK_, bool KS>
int dispatch_out(int c_dtype, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
                 int64_t ldc, int M, int N, int K, const float* ks, const float* rs,
                 const uint16_t* cb, int acc, hipStream_t st) {
    return c_dtype == AGK_F32 ? launch<AK, BK_, KS, true>(A, lda, B, ldb, C, ldc, M, N, K, ks, rs,
                                                          cb, acc, st)
                              : launch<AK, BK_, KS, false>(A, lda, B, ldb, C, ldc, M, N, K, ks,
                                                           rs, cb, acc, st);
}
template <bool AK, bool BK_>
int dispatch_ks(bool has_ks, int c_dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
                void* C, int64_t ldc, int M, int N, int K, const float* ks, const float* rs,
                const uint16_t* cb, int acc, hipStream_t st) {
    return has_ks ? dispatch_out<AK, BK_, true>(c_dtype, A, lda, B, ldb, C, ldc, M, N, K, ks, rs,
                                                cb, acc, st)
                  : dispatch_out<AK, BK_, false>(c_dtype, A, lda, B, ldb, C, ldc, M, N, K, ks, rs,
                                                 cb, acc, st);
}

}  // namespace agk_gemm

namespace agk_gemm {

// Tile orders measured on MI355X for the products of the RMSNorm + linear
// layer at its headline size (M = 8192 rows, K = 4096, N = 11008), with
// random bf16 operands; every other shape takes kGroupM.  The best group size
// depends on the shape in ways no simple rule captured (the same y layout
// with K = 8192 is fastest at 4, with 16384 rows at 2), so only shapes that
// were measured are listed.  Microseconds per product, group size 2 / 4 / 8:
//   y  = h W     (32 x 43 tiles, 64 k-steps, A k-contiguous, B k-strided):
//                 531-537 / 551-561 / 549-558
//   dh = dy W^T  (32 x 16 tiles, 172 k-steps, both k-contiguous):
//                 565-570 / 506-516 / 493-499
// (dW = h^T dy, 16 x 43 tiles, measured 524-550 at every group size: 4.)
// The order changes only which workgroup computes which tile: results are
// bit-identical.
struct TunedOrder {
    int tiles_m, tiles_n, nk;
    bool a_tr, b_tr;
    int group_m;
};
constexpr TunedOrder kTunedOrders[] = {
    {32, 43, 64, false, true, 2},     // y
    {32, 16, 172, false, false, 8},   // dh
};

inline int tuned_group_m(int tiles_m, int tiles_n, int nk, bool a_tr, bool b_tr) {
    for (const TunedOrder& t : kTunedOrders)
        if (t.tiles_m == tiles_m && t.tiles_n == tiles_n && t.nk == nk && t.a_tr == a_tr &&
            t.b_tr == b_tr)
            return t.group_m;
    return kGroupM;
}

// Whether a call takes the direct-to-LDS kernel.  A k-scale keeps the call on
// the register-staged kernel: the direct kernel's loads go from memory to LDS
// without passing registers, so the scale would have to be applied to every A
// fragment after its LDS read (unpack, multiply, round, repack: about 20 VALU
// operations per fragment).  Measured on MI355X for y (8192 x 11008 x 4096,
// A k-contiguous, the scale staged in LDS), that variant was bit-identical to
// the staged kernel's but ran 759-819 us against 551 us without the scale,
// while all it saves the RMSNorm + linear layer is writing and reading h
// (about 15 us).
inline bool direct_eligible(int64_t K, const float* kscale) {
    return kscale == nullptr && K % BK == 0;
}

// No layout needs a workspace: the direct kernel stages either layout of each
// operand itself.  (The workspace arguments stay in the ABI for callers that
// pass one.)
inline size_t workspace_for(int64_t, int64_t, int64_t, int, int, const float*) { return 0; }

}  // namespace agk_gemm

extern "C" size_t agk_gemm_bf16_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_trans,
                                                int b_trans) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return agk_gemm::workspace_for(M, N, K, a_trans, b_trans, nullptr);
}

extern "C" int agk_transpose_bf16(const void* src, int64_t ld_src, void* dst, int64_t ld_dst,
                                  int64_t rows, int64_t cols, agk_stream_t stream) {
    using namespace agk_gemm;
    if (rows < 0 || cols < 0 || rows > 0x7fffffffLL || cols > 0x7fffffffLL) return AGK_EINVAL;
    if (rows == 0 || cols == 0) return AGK_OK;
    if (!src || !dst || rows % 8 || cols % 8 || ld_src % 8 || ld_dst % 8) return AGK_EINVAL;
    if (ld_src < cols || ld_dst < rows || !aligned16(src) || !aligned16(dst)) return AGK_EINVAL;
    (void)hipGetLastError();
    return launch_transpose(src, ld_src, dst, ld_dst, static_cast<int>(rows),
                            static_cast<int>(cols), reinterpret_cast<hipStream_t>(stream));
}

namespace agk_gemm {

// agk_gemm_bf16 with an optional bf16 column bias (bf16 output, no rowscale,
// no accumulation: the caller has checked).
int gemm_impl(const void* A, int64_t lda, int a_trans, const void* B, int64_t ldb, int b_trans,
              void* C, int64_t ldc, int c_dtype, int64_t M, int64_t N, int64_t K,
              const float* kscale, const float* rowscale, const uint16_t* colbias, int accumulate,
              agk_stream_t stream) {
    if (M < 0 || N < 0 || K < 0 || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
        return AGK_EINVAL;
    if (c_dtype != AGK_F32 && c_dtype != AGK_BF16) return AGK_EDTYPE;
    if (M == 0 || N == 0) return AGK_OK;
    if (!C || ldc < N) return AGK_EINVAL;
    if (K == 0) {  // empty reduction (A and B may be null): C = 0 (+ bias), or C as it was
        if (accumulate) return AGK_OK;
        (void)hipGetLastError();
        hipLaunchKernelGGL(zero_c_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(stream), C, ldc,
                           static_cast<int>(N), c_dtype == AGK_F32 ? 4 : 2, colbias);
        return hipGetLastError() == hipSuccess ? AGK_OK : AGK_EHIP;
    }
    if (!A || !B) return AGK_EINVAL;
    // 16-byte vector accesses along the contiguous dimension of each operand
    if ((M | N | K) % 8 != 0) return AGK_EINVAL;
    if (lda % 8 || ldb % 8 || ldc < N) return AGK_EINVAL;
    if (lda < (a_trans ? M : K) || ldb < (b_trans ? K : N)) return AGK_EINVAL;
    if (!aligned16(A) || !aligned16(B)) return AGK_EINVAL;
    if (kscale && !aligned16(kscale)) return AGK_EINVAL;
    (void)hipGetLastError();  // report only this call's launch failures
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const int acc = accumulate != 0;

    // The direct-to-LDS kernel reads either layout of each operand; the
    // buffer resources span a tile's rows (or k-rows) in 31-bit byte offsets.
    auto fits = [&](int64_t ld, bool tr) {
        return (tr ? (K - 1) * ld + BM : (BM - 1) * ld + K) * 2 <= 0x7fffffffLL;
    };
    const bool a_tr = a_trans != 0, b_tr = b_trans == 0;
    if (direct_eligible(K, kscale) && fits(lda, a_tr) && fits(ldb, b_tr)) {
        const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
        const int gm = tuned_group_m(tiles_m, tiles_n, k / BK, a_tr, b_tr);
        const int tiles = tiles_m * tiles_n;
        const int full = direct_full_tiles(tiles, device_cus());
        const dim3 grid(full + 2 * (tiles - full)), block(kDirectThreads);
        const uint16_t* a16 = static_cast<const uint16_t*>(A);
        const uint16_t* b16 = static_cast<const uint16_t*>(B);
#define AGK_DIRECT(F32, ATR, BTR)                                                              \
    hipLaunchKernelGGL((gemm_nt_direct_kernel<F32, ATR, BTR>), grid, block, 0, st, a16, lda, b16, \
                       ldb, C, ldc, m, n, k, rowscale, colbias, acc, tiles_m, tiles_n, gm, full)
        const bool f32 = c_dtype == AGK_F32;
        if (f32) {
            if (a_tr && b_tr) AGK_DIRECT(true, true, true);
            else if (a_tr) AGK_DIRECT(true, true, false);
            else if (b_tr) AGK_DIRECT(true, false, true);
            else AGK_DIRECT(true, false, false);
        } else {
            if (a_tr && b_tr) AGK_DIRECT(false, true, true);
            else if (a_tr) AGK_DIRECT(false, true, false);
            else if (b_tr) AGK_DIRECT(false, false, true);
            else AGK_DIRECT(false, false, false);
        }
#undef AGK_DIRECT
        return hipGetLastError() == hipSuccess ? AGK_OK : AGK_EHIP;
    }
    // Leading dimensions too large for the direct kernel's offsets, K not a
    // multiple of 64, or a k-scale: the register-staged kernel.
    const bool ak = !a_trans, bk = b_trans != 0, ks = kscale != nullptr;
    const uint16_t* cb = colbias;
    if (ak && bk) return dispatch_ks<true, true>(ks, c_dtype, A, lda, B, ldb, C, ldc, m, n, k, kscale, rowscale, cb, acc, st);
    if (ak && !bk) return dispatch_ks<true, false>(ks, c_dtype, A, lda, B, ldb, C, ldc, m, n, k, kscale, rowscale, cb, acc, st);
    if (!ak && bk) return dispatch_ks<false, true>(ks, c_dtype, A, lda, B, ldb, C, ldc, m, n, k, kscale, rowscale, cb, acc, st);
    return dispatch_ks<false, false>(ks, c_dtype, A, lda, B, ldb, C, ldc, m, n, k, kscale, rowscale, cb, acc, st);
}

}  // namespace agk_gemm

extern "C" int agk_gemm_bf16(const void* A, int64_t lda, int a_trans, const void* B, int64_t ldb,
                             int b_trans, void* C, int64_t ldc, int c_dtype, int64_t M, int64_t N,
                             int64_t K, const float* kscale, const float* rowscale,
                             int accumulate, void* workspace, size_t workspace_bytes,
                             agk_stream_t stream) {
    (void)workspace;  // every layout is staged as it lies
    (void)workspace_bytes;
    return agk_gemm::gemm_impl(A, lda, a_trans, B, ldb, b_trans, C, ldc, c_dtype, M, N, K, kscale,
                               rowscale, nullptr, accumulate, stream);
}

extern "C" int agk_linear_bf16(const void* X, int64_t ldx, const void* W, int64_t ldw,
                               const void* bias, void* Y, int64_t ldy, int64_t M, int64_t N,
                               int64_t K, agk_stream_t stream) {
    if (bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) return AGK_EINVAL;
    // Y [M][N] = X [M][K] * (W [N][K])^T: A k-contiguous, B stored as B^T
    return agk_gemm::gemm_impl(X, ldx, 0, W, ldw, 1, Y, ldy, AGK_BF16, M, N, K, nullptr, nullptr,
                               static_cast<const uint16_t*>(bias), 0, stream);
}
