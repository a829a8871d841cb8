// gemm_f32.hip -- fp32 GEMM for the graph layer's matmul on float32 tensors
// (cgadimpl/src/ops/linalg.cpp:12-20 and its VJP's products,
// cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:258-263), on CDNA4's fp32
// matrix instruction v_mfma_f32_32x32x2_f32.  Not on the RMSNorm layer's
// measured path (its products are bf16, gemm.hip): a general kernel for any
// sizes, leading dimensions, layouts and alignment.
//
//   C[M][ldc] (+)= op(A) op(B)
//
// Shape.  A workgroup of 256 lanes (4 waves, 2 x 2) computes a TILE x TILE
// tile of C; each wave owns (TILE / 2)^2 of it as 32 x 32 MFMA accumulators
// (TILE 128: 2 x 2 of them, 64 AGPRs).  Products with fewer 128-tiles than
// the GPU has CUs take TILE 64 (four times the workgroups).
// K is walked in steps of 16 through two LDS stages (40 KiB per workgroup, so
// four workgroups share a CU and hide each other's load latency): the next
// step's 8 + 8 values per lane are loaded into registers while the current
// step is multiplied, then written to the other stage (one barrier per step).
//
// Operands.  Each operand is staged as a logical [rows][K] matrix (A: M rows,
// B: N rows) into LDS laid out [k][row], whatever its memory layout:
//  - k contiguous in memory (A as [M][K], B given as B^T [N][K]): lane t loads
//    k (t % 4) * 4 .. + 3 of rows t / 4 + 64 i as one 16-byte access when the
//    rows are 16-byte aligned, else k = t % 16 of rows t / 16 + 16 i (16
//    neighbouring lanes read 64 contiguous bytes either way);
//  - rows contiguous (A given as A^T [K][M], B as [K][N]): lane t loads row
//    t % 128 of k = t / 128 + 2 i, 128 neighbouring lanes 512 bytes.
// Elements outside the matrix are staged as zeros, so edge tiles need no
// other special case.  LDS k-rows are kStride = 160 floats apart: k and k + 1
// start 32 banks apart, so an MFMA operand read (lanes 0-31 at k, 32-63 at
// k + 1, 32 consecutive rows each) touches every bank once.
//
// MFMA lane layout (the 32 x 32 block instructions' layout, as in gemm.hip):
// A operand lane l holds row l % 32, k = l / 32; B operand lane l holds
// column l % 32, the same k; accumulator element e of lane l is
// C[8 * (e / 4) + 4 * (l / 32) + e % 4][l % 32].
//
// Determinism: every output element is summed in the same k order in every
// call (no split-K, no atomics), so results are bit-identical run to run.
// Rounding: fp32 products and sums in the matrix core; the bound is that of
// fp32 summation, |C - exact| <= (K + 1) 2^-24 (|A| |B|).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "agk_rmsnorm.h"
#include "rowcommon.hpp"

namespace agk_sgemm {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 16;
constexpr int kThreads = 256;
constexpr int kStride = 160;              // floats per LDS k-row (at most 128 used)
constexpr int kStage = BK * kStride;      // floats per operand per stage

// One operand's values for one k-step: element (row r0 + row, k0 + k) of the
// logical [rows][K] matrix, at p[row * ld + k] (KC) or p[k * ld + row] (!KC);
// TILE * BK / 256 values per lane.
// KC with VEC (16-byte aligned rows, ld a multiple of 4): lane t loads the
// four k (t % 4) * 4 .. + 3 of rows t / 4 + 64 i as one 16-byte access (a
// group of four k past K element by element).
template <int TILE, bool KC, bool VEC>
__device__ __forceinline__ void load_step(float (&v)[TILE * BK / kThreads],
                                          const float* __restrict__ p, int64_t ld, int r0,
                                          int rows, int k0, int K) {
    const int t = threadIdx.x;
    if constexpr (KC && VEC) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < TILE * BK / kThreads / 4; ++i) {
            const int row = t / 4 + (kThreads / 4) * i;
            const int gr = r0 + row, gk = k0 + (t % 4) * 4;
            f32x4 q = {0.0f, 0.0f, 0.0f, 0.0f};
            if (gr < rows) {
                const float* a = p + static_cast<int64_t>(gr) * ld + gk;
                if (gk + 3 < K) {
                    q = *reinterpret_cast<const f32x4*>(a);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) q[e] = gk + e < K ? a[e] : 0.0f;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] = q[e];
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TILE * BK / kThreads; ++i) {
        const int row = KC ? t / BK + (kThreads / BK) * i : t % TILE;
        const int k = KC ? t % BK : t / TILE + (kThreads / TILE) * i;
        const int gr = r0 + row, gk = k0 + k;
        v[i] = (gr < rows && gk < K)
                   ? (KC ? p[static_cast<int64_t>(gr) * ld + gk] : p[static_cast<int64_t>(gk) * ld + gr])
                   : 0.0f;
    }
}

template <int TILE, bool KC, bool VEC>
__device__ __forceinline__ void store_step(const float (&v)[TILE * BK / kThreads], float* lds) {
    const int t = threadIdx.x;
    if constexpr (KC && VEC) {
#pragma unroll
        for (int i = 0; i < TILE * BK / kThreads / 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                lds[((t % 4) * 4 + e) * kStride + t / 4 + (kThreads / 4) * i] = v[4 * i + e];
        return;
    }
#pragma unroll
    for (int i = 0; i < TILE * BK / kThreads; ++i) {
        const int row = KC ? t / BK + (kThreads / BK) * i : t % TILE;
        const int k = KC ? t % BK : t / TILE + (kThreads / TILE) * i;
        lds[k * kStride + row] = v[i];
    }
}

// A_KC: A is [M][lda] (k contiguous), else A^T [K][lda]; B_KC: B is given as
// B^T [N][ldb] (k contiguous), else B [K][ldb].
template <int TILE, bool A_KC, bool B_KC, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    float* __restrict__ C, int64_t ldc, int M, int N, int K, int accumulate, int tiles_n) {
    __shared__ float lds[2][2 * kStage];  // [stage][A k-rows, then B k-rows]

    constexpr int NT = TILE / 64;  // 32 x 32 MFMA blocks per wave along each dimension
    constexpr int WT = TILE / 2;   // the wave's block of C is WT x WT
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = (static_cast<int>(blockIdx.x) / tiles_n) * TILE;
    const int n0 = (static_cast<int>(blockIdx.x) % tiles_n) * TILE;

    f32x16 acc[NT][NT];
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    float va[TILE * BK / kThreads], vb[TILE * BK / kThreads];
    const int nk = (K + BK - 1) / BK;
    load_step<TILE, A_KC, VEC>(va, A, lda, m0, M, 0, K);
    load_step<TILE, B_KC, VEC>(vb, B, ldb, n0, N, 0, K);
    store_step<TILE, A_KC, VEC>(va, lds[0]);
    store_step<TILE, B_KC, VEC>(vb, lds[0] + kStage);
    __syncthreads();

    const int fr = lane & 31;  // operand row / column within a 32-block
    const int fk = lane >> 5;  // operand k within a 2-deep MFMA step
    for (int kt = 0; kt < nk; ++kt) {
        const float* as = lds[kt & 1];
        const float* bs = as + kStage;
        const bool more = kt + 1 < nk;
        if (more) {
            load_step<TILE, A_KC, VEC>(va, A, lda, m0, M, (kt + 1) * BK, K);
            load_step<TILE, B_KC, VEC>(vb, B, ldb, n0, N, (kt + 1) * BK, K);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float a[NT], b[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) a[i] = as[(kk + fk) * kStride + wm * WT + i * 32 + fr];
#pragma unroll
            for (int j = 0; j < NT; ++j) b[j] = bs[(kk + fk) * kStride + wn * WT + j * 32 + fr];
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            float* nxt = lds[(kt + 1) & 1];
            store_step<TILE, A_KC, VEC>(va, nxt);
            store_step<TILE, B_KC, VEC>(vb, nxt + kStage);
        }
        __syncthreads();
    }

    const int col_l = lane & 31;
    const int row_l = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < NT; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm * WT + i * 32 + 8 * (e >> 2) + row_l + (e & 3);
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int col = n0 + wn * WT + j * 32 + col_l;
                if (col >= N) continue;
                float* p = C + static_cast<int64_t>(row) * ldc + col;
                const float v = acc[i][j][e];
                *p = accumulate ? agk::acc_add(*p, v) : v;
            }
        }
    }
}

// C = 0 over M rows of N columns (ldc apart): the empty sum (K == 0).  A
// kernel, not a memset, so that the call can be captured.
__global__ __launch_bounds__(256) void zero_rows_kernel(float* __restrict__ C, int64_t ldc,
                                                        int N) {
    float* r = C + static_cast<int64_t>(blockIdx.x) * ldc;
    for (int c = threadIdx.x; c < N; c += 256) r[c] = 0.0f;
}

}  // namespace agk_sgemm

extern "C" int agk_gemm_f32(const float* A, int64_t lda, int a_trans, const float* B, int64_t ldb,
                            int b_trans, float* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                            int accumulate, agk_stream_t stream) {
    using namespace agk_sgemm;
    constexpr int64_t kMax = 0x7fffffffLL;
    if (M < 0 || N < 0 || K < 0 || M > kMax || N > kMax || K > kMax) return AGK_EINVAL;
    if (M == 0 || N == 0) return AGK_OK;
    if (!C || ldc < N) return AGK_EINVAL;
    if (K > 0) {
        if (!A || !B) return AGK_EINVAL;
        if (lda < (a_trans ? M : K) || ldb < (b_trans ? K : N)) return AGK_EINVAL;
    }
    agk::clear_pending_error();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    if (K == 0) {  // the empty sum: zeros, or C as it was
        if (accumulate) return AGK_OK;
        hipLaunchKernelGGL(zero_rows_kernel, dim3(static_cast<unsigned>(m)), dim3(256), 0, st, C,
                           ldc, n);
        return agk::check_launch();
    }
    // 128 x 128 tiles, or 64 x 64 when the 128-tiles would not fill the CUs
    int cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    const bool small = ((M + 127) / 128) * ((N + 127) / 128) < cus;
    const int tile = small ? 64 : 128;
    const int64_t tiles_m = (M + tile - 1) / tile, tiles_n = (N + tile - 1) / tile;
    if (tiles_m * tiles_n > kMax) return AGK_EINVAL;
    const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n)), block(kThreads);
    const int acc = accumulate != 0;
    const int tn = static_cast<int>(tiles_n);
    // A k-contiguous unless given transposed; B k-contiguous only when given as B^T
    const bool a_kc = a_trans == 0, b_kc = b_trans != 0;
    // 16-byte loads of the k-contiguous operands when their rows allow it
    auto vec_ok = [](const float* p, int64_t ld) {
        return (reinterpret_cast<uintptr_t>(p) & 15u) == 0 && ld % 4 == 0;
    };
    const bool vec = (!a_kc || vec_ok(A, lda)) && (!b_kc || vec_ok(B, ldb));
#define AGK_F32(T, AK, BKC)                                                                   \
    do {                                                                                      \
        if (vec)                                                                              \
            hipLaunchKernelGGL((gemm_f32_kernel<T, AK, BKC, true>), grid, block, 0, st, A, lda, \
                               B, ldb, C, ldc, m, n, k, acc, tn);                             \
        else                                                                                  \
            hipLaunchKernelGGL((gemm_f32_kernel<T, AK, BKC, false>), grid, block, 0, st, A,     \
                               lda, B, ldb, C, ldc, m, n, k, acc, tn);                        \
    } while (0)
#define AGK_F32_LAYOUTS(T)                  \
    if (a_kc && b_kc) AGK_F32(T, true, true);   \
    else if (a_kc) AGK_F32(T, true, false);     \
    else if (b_kc) AGK_F32(T, false, true);     \
    else AGK_F32(T, false, false);
    if (small) {
        AGK_F32_LAYOUTS(64)
    } else {
        AGK_F32_LAYOUTS(128)
    }
#undef AGK_F32_LAYOUTS
#undef AGK_F32
    return agk::check_launch();
}
