/*
 * agk_rmsnorm.h -- C ABI of the MI355X (gfx950) RMSNorm layer kernels.
 *
 * This is the drop-in boundary for cgadimpl's RMSNorm layer path,
 *     y = x * rsqrt(mean(x^2, last axis) + eps) * gamma
 * and its vector-Jacobian product (dx, dgamma).  The C++ autodiff layer
 * (ag::rms, ag::mul, ag::rms_norm, vjp_RMSNorm, vjp_Mul, vjp_RMSNormAffine)
 * calls these entry points; nothing C++ or torch-specific crosses the ABI.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are device pointers (hipMalloc'd or equivalent).
 *   - Tensors are row-major and contiguous: [rows, cols] with the normalised
 *     axis last, so a [B, T, D] activation is rows = B*T, cols = D.
 *   - agk_dtype names the storage type of x, y, dy, dx and gamma.  Arithmetic
 *     is fp32 in every case; inv_rms and dgamma are always fp32.
 *   - Work is enqueued on `stream` (0 = the null stream) and returns without
 *     synchronising.  Entry points hold no global state: concurrent calls on
 *     different streams are safe as long as their buffers do not overlap.
 *   - Results are deterministic: the same inputs on the same device give the
 *     same bits, dgamma included (fixed-order reductions, no float atomics).
 *   - Return value is an agk_status; nothing here calls exit() or throws.
 *   - rows == 0 or cols == 0 is a valid empty call (a no-op, except that a
 *     non-accumulating backward zero-fills dgamma[cols]).
 *   - Pointers need no particular alignment.  16-byte aligned pointers with
 *     cols a multiple of the vector width take the 128-bit path; anything
 *     else takes the scalar path of the same kernels.
 *
 * The historic kernel plugin that this ABI follows (raw pointers, element
 * counts and a stream, caller-allocated gradient buffers) is exercised at
 * cgadimpl/Tests/test_kernels_gpu.cpp:50,90,120-121 and loaded at :143.
 */
#ifndef AGK_RMSNORM_H
#define AGK_RMSNORM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same layout as HIP's hipStream_t, so a hipStream_t converts directly. */
typedef struct ihipStream_t* agk_stream_t;

typedef enum {
    AGK_OK = 0,
    AGK_EINVAL = 1,     /* null pointer, negative size, size overflow        */
    AGK_EDTYPE = 2,     /* unsupported storage dtype                         */
    AGK_EWORKSPACE = 3, /* workspace missing or smaller than required        */
    AGK_EHIP = 4        /* a HIP runtime call or kernel launch failed        */
} agk_status;

typedef enum {
    AGK_F32 = 0,
    AGK_BF16 = 1
} agk_dtype;

/* `accumulate` argument of the backward entry points: a bit per output.
 * A set bit adds into that output (the reference's Node::accumulate_grad,
 * grad += g, cgadimpl/src/core/graph.cpp:44-47); a clear bit overwrites it,
 * which is what a fresh, zero-filled reference gradient would end up holding
 * without the caller having to zero-fill it first.  Other bits are invalid.  */
typedef enum {
    AGK_ACCUM_NONE = 0,
    AGK_ACCUM_DX = 1,      /* dx (or da) += ...          */
    AGK_ACCUM_DGAMMA = 2,  /* dgamma (or db) += ...      */
    AGK_ACCUM_ALL = 3
} agk_accumulate;

/* Forward of the RMSNorm layer.
 * Replaces the eager forward of `ag::rms(x) * gamma`:
 *   rms_nodeops   cgadimpl/src/ops/normalization.cpp:23-35
 *                 (x*x, reduce_mean over the last axis, +eps, sqrt, 1/., x*r)
 *   mul_nodeops   cgadimpl/src/ops/arithmetic.cpp:31-39  (broadcast * gamma)
 * gamma == NULL means no scale (ag::rms alone).  inv_rms[rows] receives
 * r = 1/sqrt(mean(x^2)+eps) per row, which the backward reads (the reference
 * keeps the same tensor on the node's tape, normalization.cpp:29).           */
int agk_rmsnorm_fwd(const void* x, const void* gamma, void* y, float* inv_rms,
                    int64_t rows, int64_t cols, float eps, int dtype,
                    agk_stream_t stream);

/* Bytes of workspace agk_rmsnorm_bwd needs for these sizes: fp32 dgamma
 * partials, one row of cols floats per row block, where a row block is
 *   rpb = ceil(rows / 1024) rows, at least 4 once rows >= 2048,
 * so nblk = ceil(rows / rpb) and the size is nblk * cols * 4 bytes.  Depends
 * only on rows and cols, never on the device, so the dgamma summation order
 * is the same everywhere.                                                    */
size_t agk_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols);

/* Backward (VJP) of the RMSNorm layer.
 * Replaces, for the graph `ag::rms(x) * gamma` seeded with dy:
 *   vjp_Mul              cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:54-59
 *   reduce_for_broadcast autodiff_vjp_ops.cpp:15-35  (dgamma = sum over rows)
 *   vjp_RMSNorm          autodiff_vjp_ops.cpp:368-377
 *   Node::accumulate_grad cgadimpl/src/core/graph.cpp:44-47 (grad += g)
 * computing
 *   g = dy*gamma, dot = sum_j g*x, dx = r*(g - x*r*r*dot/cols),
 *   dgamma = sum_rows dy*x*r.
 * gamma == NULL means no scale.  dx == NULL skips dx (only dgamma wanted);
 * dgamma == NULL skips the dgamma reduction; both NULL is a no-op.
 * accumulate is a set of agk_accumulate bits (AGK_ACCUM_DX, AGK_ACCUM_DGAMMA).
 * workspace must hold at least agk_rmsnorm_bwd_workspace_bytes(rows, cols)
 * bytes when dgamma != NULL.                                                 */
int agk_rmsnorm_bwd(const void* x, const void* gamma, const float* inv_rms,
                    const void* dy, void* dx, float* dgamma, void* workspace,
                    size_t workspace_bytes, int64_t rows, int64_t cols,
                    int dtype, int accumulate, agk_stream_t stream);

/* Broadcast multiply y[i, j] = a[i, j] * b[j]: mul_nodeops with b of shape
 * [1, cols] or [cols] (cgadimpl/src/ops/arithmetic.cpp:31-39).  Used when the
 * layer is written unfused, as `ag::rms(x) * gamma`.                         */
int agk_mul_rowbcast_fwd(const void* a, const void* b, void* y, int64_t rows,
                         int64_t cols, int dtype, agk_stream_t stream);

/* Workspace for agk_mul_rowbcast_bwd (same rule as the RMSNorm backward). */
size_t agk_mul_rowbcast_bwd_workspace_bytes(int64_t rows, int64_t cols);

/* vjp_Mul for that broadcast (autodiff_vjp_ops.cpp:54-59 with
 * reduce_for_broadcast, :15-35):  da (+)= gy*b,  db (+)= sum_rows gy*a.
 * da or db may be NULL to skip that gradient.  db is fp32.  accumulate:
 * AGK_ACCUM_DX adds into da, AGK_ACCUM_DGAMMA adds into db.                 */
int agk_mul_rowbcast_bwd(const void* gy, const void* a, const void* b,
                         void* da, float* db, void* workspace,
                         size_t workspace_bytes, int64_t rows, int64_t cols,
                         int dtype, int accumulate, agk_stream_t stream);

/* Diagnostic, with no counterpart in the reference: the launch shape the
 * library picks for a forward (backward = 0) or backward (backward != 0)
 * call of these sizes with 16-byte aligned pointers.  plan[5] receives
 *   {lanes per row, 16-byte slots per lane, rows per workgroup,
 *    rows per dgamma block (backward), dgamma blocks (backward)};
 * lanes per row == 0 means the looped kernel (rows that are not a whole
 * number of 16-byte slots, or too wide to keep in registers).  Used by the
 * tests to run every reachable shape.                                        */
int agk_rmsnorm_launch_plan(int64_t rows, int64_t cols, int dtype, int backward,
                            int32_t* plan);

/* Human-readable name of a status code (static storage). */
const char* agk_status_str(int status);

/* The HIP runtime's description of the error behind the calling thread's
 * most recent AGK_EHIP (static storage; "no HIP error" if there was none).
 * The reference prints the CUDA error string before exiting
 * (cgadimpl/src/runtime/cuda_graphs.cpp:12-19); here the caller decides.   */
const char* agk_last_error(void);

/* Library version string, "agk_rmsnorm <major>.<minor> gfx950". */
const char* agk_version(void);

#ifdef __cplusplus
}
#endif

#endif /* AGK_RMSNORM_H */
