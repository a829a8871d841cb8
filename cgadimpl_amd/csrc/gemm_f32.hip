// gemm_f32.hip -- fp32 GEMM for the graph layer's matmul on float32 tensors
// (cgadimpl/src/ops/linalg.cpp:12-20 and its VJP,
// cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:258-263).  A plain library GEMM:
// it runs rocBLAS's sgemm (no fused work, not on the RMSNorm layer's path; the
// layer's products are bf16 on the hand-written MFMA kernel in gemm.hip).
// Host code only.
//
// Determinism: every handle has atomics disallowed, so rocBLAS picks kernels
// without atomic split-K reductions and a call gives the same bits every run.
// Handles: one per device, created on first use with that device current and
// kept for the life of the process (never destroyed, so no teardown ordering
// against the HIP runtime); a mutex serialises the enqueue of calls, which
// return as soon as the work is queued on the caller's stream.

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <stdint.h>

#include <mutex>

#include "agk_rmsnorm.h"
#include "rowcommon.hpp"

namespace {

constexpr int kMaxDevices = 64;

struct Handles {
    std::mutex mu;
    rocblas_handle h[kMaxDevices] = {};
};

Handles& handles() {
    static Handles* p = new Handles;  // intentionally leaked: outlives every caller
    return *p;
}

int status_of(rocblas_status s) {
    switch (s) {
        case rocblas_status_success: return AGK_OK;
        case rocblas_status_invalid_size:
        case rocblas_status_invalid_pointer:
        case rocblas_status_invalid_value: return AGK_EINVAL;
        default: return AGK_EHIP;
    }
}

}  // namespace

extern "C" int agk_gemm_f32(const float* A, int64_t lda, int a_trans, const float* B, int64_t ldb,
                            int b_trans, float* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                            int accumulate, agk_stream_t stream) {
    constexpr int64_t kMax = 0x7fffffffLL;  // rocblas_int
    if (M < 0 || N < 0 || K < 0 || M > kMax || N > kMax || K > kMax) return AGK_EINVAL;
    if (M == 0 || N == 0) return AGK_OK;
    if (!C || ldc < N || ldc > kMax) return AGK_EINVAL;
    if (K > 0) {
        if (!A || !B) return AGK_EINVAL;
        if (lda < (a_trans ? M : K) || ldb < (b_trans ? K : N) || lda > kMax || ldb > kMax)
            return AGK_EINVAL;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return AGK_EHIP;
    Handles& hs = handles();
    std::lock_guard<std::mutex> lock(hs.mu);
    rocblas_handle& h = hs.h[dev];
    if (!h) {
        if (rocblas_create_handle(&h) != rocblas_status_success) {
            h = nullptr;
            return AGK_EHIP;
        }
        if (rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed) != rocblas_status_success)
            return AGK_EHIP;
    }
    if (rocblas_set_stream(h, reinterpret_cast<hipStream_t>(stream)) != rocblas_status_success)
        return AGK_EHIP;
    // Row-major C = op(A) op(B) is column-major C^T = op(B)^T op(A)^T: the
    // row-major arrays, read as column-major, are the transposes already.
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    // K == 0: an empty sum; sgemm scales C by beta (zeros, or C unchanged)
    // without reading the operands, which may be null: C stands in for them,
    // with the smallest leading dimensions sgemm accepts for their layouts
    auto at_least_1 = [](int64_t v) { return v > 1 ? v : int64_t{1}; };
    const float* a = K > 0 ? A : C;
    const float* b = K > 0 ? B : C;
    const rocblas_int ld_a =
        static_cast<rocblas_int>(K > 0 ? lda : at_least_1(a_trans ? M : K));
    const rocblas_int ld_b =
        static_cast<rocblas_int>(K > 0 ? ldb : at_least_1(b_trans ? K : N));
    return status_of(rocblas_sgemm(h, b_trans ? rocblas_operation_transpose : rocblas_operation_none,
                                   a_trans ? rocblas_operation_transpose : rocblas_operation_none,
                                   static_cast<rocblas_int>(N), static_cast<rocblas_int>(M),
                                   static_cast<rocblas_int>(K), &alpha, b, ld_b, a, ld_a, &beta,
                                   C, static_cast<rocblas_int>(ldc)));
}
