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

/* Narrowest row (in elements, either dtype) that can take the split paths:
 * rows too wide for the register-resident kernels, 16-byte aligned, are cut
 * into 4096-column segments and 2048-column chunks, each its own workgroup,
 * so that a few long rows still spread over the whole GPU.                  */
#define AGK_WIDE_MIN_COLS 16385

/* Forward of the RMSNorm layer.
 * Replaces the eager forward of `ag::rms(x) * gamma`:
 *   rms_nodeops   cgadimpl/src/ops/normalization.cpp:23-35
 *                 (x*x, reduce_mean over the last axis, +eps, sqrt, 1/., x*r)
 *   mul_nodeops   cgadimpl/src/ops/arithmetic.cpp:31-39  (broadcast * gamma)
 * gamma == NULL means no scale (ag::rms alone).  inv_rms[rows] receives
 * r = 1/sqrt(mean(x^2)+eps) per row, which the backward reads (the reference
 * keeps the same tensor on the node's tape, normalization.cpp:29).
 * y may be x itself (in place).  Rows too wide for the resident kernels
 * use y's first bytes of each row for partial sums until the last of the
 * call's kernels overwrites them; an in-place call takes the
 * one-workgroup-per-row kernel instead.                                      */
int agk_rmsnorm_fwd(const void* x, const void* gamma, void* y, float* inv_rms,
                    int64_t rows, int64_t cols, float eps, int dtype,
                    agk_stream_t stream);

/* agk_rmsnorm_fwd with a workspace: the same results (y and inv_rms bit-
 * identical to agk_rmsnorm_fwd's on the same inputs), computed with one HBM
 * read of x for rows of AGK_WIDE_MIN_COLS to 1048576 columns, at least 4 of
 * them, that the split path would take (16-byte aligned, y apart from x):
 * each row is held by several workgroups that exchange their partial sums of
 * squares through the workspace (agk_rmsnorm_fwd reads such rows twice).
 * Same reference as agk_rmsnorm_fwd (rms_nodeops, normalization.cpp:23-35;
 * mul_nodeops, arithmetic.cpp:31-39).  workspace == NULL is agk_rmsnorm_fwd;
 * otherwise it must be 8-byte aligned (AGK_EINVAL) and hold at least
 * agk_rmsnorm_fwd_workspace_bytes(rows, cols) bytes (AGK_EWORKSPACE):
 * rows * ceil(cols / 4096) * 8 bytes for those sizes, 0 for others.  The
 * workspace is scratch (its contents on entry do not matter), and calls that
 * share one must not overlap in time.  No reference counterpart for the
 * workspace itself: the reference's forward allocates its intermediates.    */
size_t agk_rmsnorm_fwd_workspace_bytes(int64_t rows, int64_t cols);

int agk_rmsnorm_fwd_ws(const void* x, const void* gamma, void* y, float* inv_rms,
                       void* workspace, size_t workspace_bytes, int64_t rows,
                       int64_t cols, float eps, int dtype, agk_stream_t stream);

/* Bytes of workspace agk_rmsnorm_bwd needs for these sizes: fp32 dgamma
 * partials, one row of cols floats per workgroup.  The size is nblk * cols * 4
 * bytes with nblk = ceil(rows / rpb), rpb = ceil(rows / 1024) rows (at least
 * 4 once rows >= 2048): the count the looped kernel (unaligned or too-wide
 * rows) uses, never fewer than the 256 rows the register-resident kernel
 * uses from 256 rows up.  Below 256 rows the register-resident path sums
 * dgamma down the columns in the same launch and uses no partial rows (the
 * size is still returned, for the looped kernel).  From AGK_WIDE_MIN_COLS
 * columns on it is at least what the split backward uses: about 16 MiB of
 * dgamma partial rows (nrb = ceil(rows / ceil(rows / min(rows,
 * ceil(2048 / ceil(cols / 2048))))) rows of cols floats), rows *
 * ceil(cols / 4096) segment partials and rows coefficients, each region
 * rounded up to 256 bytes.  Depends only on rows and cols, never on the
 * device or the dtype, so the dgamma summation order is the same everywhere. */
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
 * bytes when dgamma != NULL.  With dgamma == NULL it may be NULL; rows of at
 * least AGK_WIDE_MIN_COLS columns then take the one-workgroup-per-row-block
 * kernel, and take the split path only when a 16-byte aligned workspace is
 * given that holds the split path's row statistics (rows * ceil(cols / 4096)
 * segment partials and rows coefficients, fp32, each region rounded up to
 * 256 bytes; agk_rmsnorm_bwd_workspace_bytes(rows, cols) always does).      */
int agk_rmsnorm_bwd(const void* x, const void* gamma, const float* inv_rms,
                    const void* dy, void* dx, float* dgamma, void* workspace,
                    size_t workspace_bytes, int64_t rows, int64_t cols,
                    int dtype, int accumulate, agk_stream_t stream);

/* The backward above without a workspace: no counterpart in the reference.
 * For callers that cannot allocate device memory around the call (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and accumulate bits as agk_rmsnorm_bwd; the dgamma
 * partial rows go to a scratch array the library holds in each device's
 * memory (AGK_NOALLOC_SCRATCH_BYTES per device, for the life of the process)
 * instead of a caller workspace, and the call allocates nothing.  Sizes whose
 * partial rows exceed the array (more than 256 * cols * 4 bytes on the
 * register-resident path; the split path's partial rows, segment sums and
 * coefficients for aligned rows of AGK_WIDE_MIN_COLS columns and more, about
 * 16 MiB + rows * ceil(cols / 4096) * 4 bytes; the looped path's row blocks
 * otherwise) return AGK_EWORKSPACE.  With dgamma == NULL only the split
 * path's row statistics must fit, and the split path is taken: dx equals
 * agk_rmsnorm_bwd's given a workspace of agk_rmsnorm_bwd_workspace_bytes
 * (what the reference-shaped callers pass).  Every call on a device shares that
 * device's array: calls that overlap in time on one device race, so callers
 * serialise them (one stream per device, or their own ordering).           */
#define AGK_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int agk_rmsnorm_bwd_noalloc(const void* x, const void* gamma, const float* inv_rms,
                            const void* dy, void* dx, float* dgamma, int64_t rows,
                            int64_t cols, int dtype, int accumulate, agk_stream_t stream);

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

/* Element-wise multiply under numpy broadcasting, for every shape pair the
 * row-vector kernels above do not cover: mul_nodeops's `a->value * b->value`
 * (cgadimpl/src/ops/arithmetic.cpp:31-39) with the tensor library's
 * broadcasting.  Shapes (row-major, contiguous, at most 8 axes each) align at
 * the trailing axis; each aligned axis pair must be equal or contain a 1.
 * agk_mul_bcast_shape writes the output shape (out_shape may be NULL to get
 * only out_ndim); AGK_EINVAL for incompatible shapes.
 * agk_mul_bcast_fwd: y (+)= a * b in dtype (accumulate != 0 adds into y, the
 * product rounded to storage first).  An empty output is a no-op.          */
int agk_mul_bcast_shape(const int64_t* a_shape, int a_ndim, const int64_t* b_shape,
                        int b_ndim, int64_t* out_shape, int* out_ndim);
int agk_mul_bcast_fwd(const void* a, const int64_t* a_shape, int a_ndim,
                      const void* b, const int64_t* b_shape, int b_ndim, void* y,
                      int dtype, int accumulate, agk_stream_t stream);

/* vjp_Mul with reduce_for_broadcast for those shapes
 * (cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:54-59, :15-35):
 *   da (+)= sum over a's broadcast axes of gy * b,  db (+)= ... of gy * a.
 * gy has the output's shape.  The gradient of an operand whose aligned shape
 * is the output's is the element-wise product in dtype; the gradient of a
 * broadcast operand is an fp32 array of the operand's shape, summed from
 * exact products in fp64 in a fixed order (bit-identical run to run).
 * da or db NULL skips that gradient.  accumulate: AGK_ACCUM_DX adds into da,
 * AGK_ACCUM_DGAMMA adds into db.  An empty output gives zero gradients (or
 * leaves them when accumulating).                                          */
int agk_mul_bcast_bwd(const void* gy, const void* a, const int64_t* a_shape, int a_ndim,
                      const void* b, const int64_t* b_shape, int b_ndim, void* da,
                      void* db, int dtype, int accumulate, agk_stream_t stream);

/* dst[0 .. n) = value, stored in dtype (bf16: rounded to nearest even):
 * OwnTensor::Tensor::full, which the reference's scalar literal
 * Value(float) uses (cgadimpl/src/core/graph.cpp:91-105).  A kernel, not a
 * memset, so that it can be captured into a HIP graph (the value travels as
 * a kernel argument).  n == 0 is a no-op.                                  */
int agk_fill(void* dst, int64_t n, float value, int dtype, agk_stream_t stream);

/* fp32 GEMM for the graph layer's matmul on float32 tensors
 * (cgadimpl/src/ops/linalg.cpp:12-20; VJP autodiff_vjp_ops.cpp:258-263):
 *   C[M][ldc] (+)= op(A) op(B), all fp32, row-major,
 *   A: a_trans == 0 -> [M][lda], else [K][lda];  B: b_trans == 0 -> [K][ldb],
 *   else [N][ldb].  Hand-written on the fp32 matrix instruction
 *   (v_mfma_f32_32x32x2_f32), 128 x 128 tiles, no split-K and no atomics:
 *   bit-identical run to run.  Not on the RMSNorm layer's bf16 path.  M == 0
 *   or N == 0 is a no-op; K == 0 writes zeros (or leaves C when
 *   accumulating).  No alignment or multiple-of-8 requirements; a kernel
 *   launch only, so it may be captured into a HIP graph.                     */
int agk_gemm_f32(const float* A, int64_t lda, int a_trans, const float* B, int64_t ldb,
                 int b_trans, float* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                 int accumulate, agk_stream_t stream);

/* Column sums out[j] (+)= sum_i x[i, j] of a rows x cols matrix, in fp32 and
 * in a fixed order (the same two-stage partial-row reduction as dgamma; no
 * float atomics, bit-identical run to run): OwnTensor::reduce_sum(gy, {0})
 * in vjp_Linear (cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:272-279), the
 * bias gradient.  accumulate: 0 overwrites out, 1 adds into it.  workspace:
 * agk_sum_rows_workspace_bytes(rows, cols) bytes.                          */
size_t agk_sum_rows_workspace_bytes(int64_t rows, int64_t cols);
int agk_sum_rows(const void* x, float* out, void* workspace, size_t workspace_bytes,
                 int64_t rows, int64_t cols, int dtype, int accumulate,
                 agk_stream_t stream);

/* Both VJPs of the unfused layer y = ag::rms(x) * gamma in one pass over the
 * rows: vjp_Mul with reduce_for_broadcast (autodiff_vjp_ops.cpp:54-59,
 * :15-35) followed by vjp_RMSNorm (autodiff_vjp_ops.cpp:368-377) on the
 * gradient it produced.  With h = rms(x) = x * inv_rms (inv_rms from
 * agk_rmsnorm_fwd with gamma == NULL):
 *   dr = gy * gamma                 (overwritten: the gradient of h)
 *   dx (+)= RMSNorm VJP of dr       (NULL to skip)
 *   dgamma (+)= sum_rows gy * h     (fp32, NULL to skip)
 * Every output is bit-identical to agk_mul_rowbcast_bwd(gy, h, gamma, dr,
 * dgamma) followed by agk_rmsnorm_bwd(x, NULL, inv_rms, dr, dx) on the same
 * inputs (same rounding of dr and h to storage, same summation orders), with
 * x and dy read once instead of h, gy and dr twice; for rows of at least
 * AGK_WIDE_MIN_COLS columns, when this call and that agk_rmsnorm_bwd call
 * both have a workspace (both take the split path) or neither has.
 * accumulate: AGK_ACCUM_DX adds into dx, AGK_ACCUM_DGAMMA into dgamma;
 * workspace as for agk_rmsnorm_bwd (required when dgamma != NULL).          */
int agk_rms_mul_bwd(const void* x, const void* gamma, const float* inv_rms,
                    const void* gy, void* dr, void* dx, float* dgamma,
                    void* workspace, size_t workspace_bytes, int64_t rows,
                    int64_t cols, int dtype, int accumulate, agk_stream_t stream);

/* bf16 GEMM on MFMA with fp32 accumulation, for the RMSNorm + linear layer:
 *   C[m, n] (+)= rowscale[m] * sum_k (A[m, k] * kscale[k]) * B[k, n]
 * Replaces the tensor-library matmul behind the reference's matmul node and
 * its VJP (cgadimpl/src/ops/linalg.cpp:12-20: Y = A B;
 * cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:258-263: dA += gy B^T,
 * dB += A^T gy).
 *   A: a_trans == 0 -> stored [M][lda] (row m, k contiguous);
 *      a_trans != 0 -> stored [K][lda] (A^T, m contiguous).
 *   B: b_trans == 0 -> stored [K][ldb] (n contiguous);
 *      b_trans != 0 -> stored [N][ldb] (B^T, k contiguous).
 *   C: [M][ldc], c_dtype AGK_F32 or AGK_BF16 (round to nearest even);
 *      accumulate != 0 adds into C.
 *   kscale (nullable, fp32 [K]): multiplies A's column k as A is staged, the
 *      product rounded to bf16 (h = x * gamma without materialising h);
 *   rowscale (nullable, fp32 [M]): multiplies row m of the fp32 result.
 *   workspace (nullable, unused): every layout is staged as it lies (k-strided
 *      operands read with transposing LDS reads when kscale == NULL and
 *      K % 64 == 0; otherwise transposed in registers while staged), so
 *      agk_gemm_bf16_workspace_bytes is 0; the argument stays for callers.
 * A, B, kscale 16-byte aligned; M, N, K, lda, ldb multiples of 8;
 * the result is deterministic (fixed accumulation order).
 * M == 0 or N == 0 is a no-op; K == 0 (an empty sum, A and B may be NULL)
 * writes zeros to C, or leaves C as it is when accumulating.                */
int agk_gemm_bf16(const void* A, int64_t lda, int a_trans, const void* B, int64_t ldb,
                  int b_trans, void* C, int64_t ldc, int c_dtype, int64_t M, int64_t N,
                  int64_t K, const float* kscale, const float* rowscale, int accumulate,
                  void* workspace, size_t workspace_bytes, agk_stream_t stream);

/* The linear layer's forward, Y = X W^T + bias, bf16 in and out with fp32
 * accumulation: linear_nodeops (cgadimpl/src/ops/linalg.cpp:21-33,
 * `matmul(X, W.t()) + b`).  X [M][ldx] (k contiguous), W [N][ldw] (the
 * reference's (out, in) layout), bias bf16 [N] or NULL, Y [M][ldy].  Each
 * element is the product rounded to bf16, plus the bias, rounded again: the
 * two roundings of the reference's bf16 matmul and bf16 add.  The bias is
 * added in the GEMM's store, with no extra pass over Y.  Sizes and alignment
 * as agk_gemm_bf16 (M, N, K, ldx, ldw multiples of 8; X, W 16-byte aligned);
 * K == 0 writes the bias (or zeros) to every row.                          */
int agk_linear_bf16(const void* X, int64_t ldx, const void* W, int64_t ldw,
                    const void* bias, void* Y, int64_t ldy, int64_t M, int64_t N,
                    int64_t K, agk_stream_t stream);

/* Bytes of workspace agk_gemm_bf16 uses: 0 for every shape and layout (kept so
 * that callers sizing a workspace from it need no change). */
size_t agk_gemm_bf16_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_trans, int b_trans);

/* dst[c][r] = src[r][c] for a bf16 matrix of rows x cols (multiples of 8),
 * 16-byte aligned, leading dimensions multiples of 8.  No reference
 * counterpart: the reference's OwnTensor `.t()` feeding matmul
 * (autodiff_vjp_ops.cpp:261-262) is a view; here operands are laid out for
 * the matrix cores explicitly.                                               */
int agk_transpose_bf16(const void* src, int64_t ld_src, void* dst, int64_t ld_dst,
                       int64_t rows, int64_t cols, agk_stream_t stream);

/* Testing knob, with no counterpart in the reference: how many times a
 * workgroup of a team kernel (the wide backward, agk_rmsnorm_fwd_ws) polls
 * for the other workgroups' partial sums of a row before it recomputes a
 * missing one from the inputs itself (the same bits; default 4096).  polls >= 0 sets it
 * for the process; a negative value only reads it.  Returns the previous
 * value.  0 makes every wait end at its first look, so the tests can run the
 * recompute path; the results do not change.                                */
int agk_set_exchange_wait_limit(int polls);

/* Testing and measurement knob, with no counterpart in the reference:
 * enabled = 0 keeps the wide RMSNorm backward off the team kernel (rows then
 * take the split path: row statistics, then dx and dgamma tiles, reading x
 * and dy twice), 1 restores the default; a negative value only reads it.
 * Process-wide; returns the previous value (1 or 0).                         */
int agk_set_team_backward(int enabled);

/* Testing and measurement knob, with no counterpart in the reference:
 * enabled = 0 keeps agk_rmsnorm_fwd_ws off the team kernel (wide rows then
 * take agk_rmsnorm_fwd's split path), 1 restores the default; a negative
 * value only reads it.  Process-wide; returns the previous value (1 or 0).  */
int agk_set_team_forward(int enabled);

/* Diagnostic, with no counterpart in the reference: the launch shape the
 * library picks for a forward (backward = 0), backward (backward = 1) or
 * forward given a workspace (agk_rmsnorm_fwd_ws; backward = 2) call of
 * these sizes with 16-byte aligned pointers (other values: AGK_EINVAL).
 * plan[5] receives
 *   {lanes per row, 16-byte slots per lane, rows per workgroup,
 *    rows per dgamma partial row (backward; ceil(rows / partial rows)),
 *    dgamma partial rows (backward)};
 * rows per workgroup == 0 (backward, or forward given a workspace) is a team
 * kernel: a row held by lanes per row / 256 workgroups of 256 lanes that
 * exchange their partial sums (backward: 8192 bf16 columns each, and 4096
 * or 8192 fp32 -- 8192 where 4096-column parts would number 32 or more, or
 * where a team of 8192-column parts gets 16 rows or more, given rows enough
 * for 512 / parts teams; forward: 16384 bf16, and 8192 or 16384 fp32 --
 * 16384 where 8192-column parts would number 16 or more, or where a team of
 * them would get at most 4 rows, given rows enough for 512 / parts teams), the teams taking the rows in turn
 * (plan[3] = rows per team, plan[4] = teams);
 * lanes per row == 0 means a path that does not keep rows in registers:
 * the split path when slots per lane > 0 (then plan[1] = 4096-column
 * segments per row, plan[2] = 2048-column chunks per row, and for the
 * backward plan[3] = rows per tile, plan[4] = dgamma partial rows, 0 when
 * the tiles write dgamma directly), else the looped kernel (rows that are
 * not a whole number of 16-byte slots, or too wide for registers and not
 * split).  A resident backward of at most 255 rows reports 0 partial rows:
 * it runs row and column workgroups in one launch and writes dgamma
 * directly.  Used by the tests to run every reachable shape.                 */
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
