/*
 * agk_rowops.h -- C ABI of the row kernels that share the RMSNorm layer's
 * row-reduce skeleton: the forward-mode product (JVP) of RMSNorm, LayerNorm,
 * row softmax and row log-sum-exp, with their vector-Jacobian products.
 *
 * Implemented by the same library as agk_rmsnorm.h (libagk_rmsnorm.so), with
 * the same conventions: device pointers; row-major contiguous [rows, cols]
 * with the reduced axis last; `dtype` is the storage type (AGK_F32 or
 * AGK_BF16) of every [rows, cols] tensor and of the per-row values that have
 * the storage type (noted below), arithmetic is fp32; per-row statistics are
 * fp32; work is enqueued on `stream` without synchronising; no global state;
 * deterministic results; an agk_status is returned.
 *
 * `accumulate` (backward entry points): AGK_ACCUM_NONE overwrites the output,
 * AGK_ACCUM_DX adds into it (Node::accumulate_grad, grad += g,
 * cgadimpl/src/core/graph.cpp:44-47); other bits are AGK_EINVAL.
 *
 * rows == 0 or cols == 0 is a no-op returning AGK_OK, except for
 * agk_logsumexp_fwd / agk_logsumexp_jvp with rows > 0 and cols == 0, which
 * return AGK_EINVAL (the log-sum-exp of an empty row is not defined there).
 *
 * Any alignment and any cols are accepted: 16-byte aligned tensors with cols
 * a multiple of the vector width (4 fp32 / 8 bf16) take the register-resident
 * kernels (one HBM read per input element, one write per output element);
 * anything else takes a looped kernel that re-reads the row from cache.
 */
#ifndef AGK_ROWOPS_H
#define AGK_ROWOPS_H

#include "agk_rmsnorm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Forward-mode derivative of the RMSNorm layer y = x * r * gamma with
 * r = 1/sqrt(mean(x^2) + eps) (r is the inv_rms saved by agk_rmsnorm_fwd):
 *     ty = gamma * r * (tx - x * r^2 * sum(tx * x) / cols) + tgamma * x * r
 * i.e. t*r - y*r*sum(t*y)/cols for the unscaled node, plus the gamma terms.
 * Replaces jvp_RMSNorm, cgadimpl/src/autodiff/autodiff_jvp_ops.cpp:366-379,
 * with that rule corrected: the reference divides by tape[0], which holds
 * 1/rms (normalization.cpp:26-29), so it returns t/r - ... instead of t*r - ...
 * gamma == NULL: no scale (ag::rms); tgamma == NULL: gamma has no tangent.
 * tgamma without gamma is AGK_EINVAL.  ty may not alias x or tx.             */
int agk_rmsnorm_jvp(const void* x, const void* gamma, const float* inv_rms,
                    const void* tx, const void* tgamma, void* ty,
                    int64_t rows, int64_t cols, int dtype, agk_stream_t stream);

/* LayerNorm without affine parameters, y = (x - mean) / sqrt(var + eps),
 * mean and (biased) var over the last axis.  Replaces laynor_nodeops,
 * cgadimpl/src/ops/normalization.cpp:10-22 (which fixes eps = 1e-5).
 * Saves mean[rows] and rstd[rows] = 1/sqrt(var + eps) in fp32 for the
 * backward (the reference's tape holds var and mean, :15-16).  The variance
 * is computed from the register-held row as mean((x - mean)^2), like the
 * reference's x_minus_mean pass, not as E[x^2] - mean^2.                     */
int agk_layernorm_fwd(const void* x, void* y, float* mean, float* rstd,
                      int64_t rows, int64_t cols, float eps, int dtype,
                      agk_stream_t stream);

/* VJP of LayerNorm, replacing vjp_LayerNorm,
 * cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:351-365:
 *     xhat = (x - mean) * rstd
 *     dx (+)= rstd * (dy - sum(dy)/cols - xhat * sum(dy * xhat)/cols)
 * which is the reference's d_xhat + d_var*(x-mean)*2/D + d_mean/D with its
 * sum(x - mean) term (zero up to rounding) dropped.  The Jacobian is
 * symmetric, so the same call with dy = a tangent gives the JVP.             */
int agk_layernorm_bwd(const void* x, const float* mean, const float* rstd,
                      const void* dy, void* dx, int64_t rows, int64_t cols,
                      int dtype, int accumulate, agk_stream_t stream);

/* Row softmax, y = exp(z - max(z)) / sum(exp(z - max(z))) over the last
 * axis.  Replaces softmax_row_nodeops, cgadimpl/src/ops/reduction.cpp:42-53. */
int agk_softmax_fwd(const void* z, void* y, int64_t rows, int64_t cols,
                    int dtype, agk_stream_t stream);

/* VJP of the row softmax from its output, dz (+)= y * (dy - sum(y * dy)),
 * replacing vjp_SoftmaxRow, autodiff_vjp_ops.cpp:421-428.  The Jacobian is
 * symmetric: with dy = a tangent of z this is jvp_SoftmaxRow
 * (autodiff_jvp_ops.cpp:411-420).                                            */
int agk_softmax_bwd(const void* y, const void* dy, void* dz, int64_t rows,
                    int64_t cols, int dtype, int accumulate, agk_stream_t stream);

/* Row log-sum-exp, y[row] = log(sum(exp(z - m))) + m with m = max(z) over
 * the last axis.  y has `rows` elements of the storage type (the reference's
 * [.., 1] output).  Replaces logsumexp_row_nodeops, reduction.cpp:54-66.     */
int agk_logsumexp_fwd(const void* z, void* y, int64_t rows, int64_t cols,
                      int dtype, agk_stream_t stream);

/* VJP of the row log-sum-exp: dz (+)= dy[row] * softmax(z), softmax
 * recomputed from z (max, then sum of exponentials) as the reference does,
 * vjp_LogSumExpRow, autodiff_vjp_ops.cpp:430-440.  dy has `rows` elements of
 * the storage type.                                                          */
int agk_logsumexp_bwd(const void* z, const void* dy, void* dz, int64_t rows,
                      int64_t cols, int dtype, int accumulate,
                      agk_stream_t stream);

/* agk_logsumexp_fwd that also writes lse[row], the same value in fp32 (the
 * storage-type y of bf16 rows is too coarse for the backward below), for the
 * graph layer's tape.                                                        */
int agk_logsumexp_fwd_keep(const void* z, void* y, float* lse, int64_t rows,
                           int64_t cols, int dtype, agk_stream_t stream);

/* VJP of the row log-sum-exp from the forward's fp32 value:
 *     dz (+)= dy[row] * exp(z - lse[row])
 * softmax(z) = exp(z - logsumexp(z)), so this is the reference's
 * vjp_LogSumExpRow (autodiff_vjp_ops.cpp:430-440) without recomputing the
 * row maximum and sum: one read of z and one write of dz, any row width at
 * the streaming rate.  The result equals agk_logsumexp_bwd's to fp32
 * rounding (the exponent carries lse's rounding, |lse| * 2^-24 relative).
 * dy has `rows` elements of the storage type, lse `rows` fp32 values.      */
int agk_logsumexp_bwd_from_value(const void* z, const float* lse, const void* dy,
                                 void* dz, int64_t rows, int64_t cols, int dtype,
                                 int accumulate, agk_stream_t stream);

/* JVP of the row log-sum-exp: ty[row] = sum(softmax(z) * tz) over the row,
 * jvp_LogSumExpRow, autodiff_jvp_ops.cpp:421-434.  ty has `rows` elements of
 * the storage type.                                                          */
int agk_logsumexp_jvp(const void* z, const void* tz, void* ty, int64_t rows,
                      int64_t cols, int dtype, agk_stream_t stream);

/* ---- the same ops with a workspace: rows over several workgroups ----------
 * agk_softmax_fwd_ws, agk_softmax_bwd_ws and agk_logsumexp_bwd_ws compute
 * what agk_softmax_fwd, agk_softmax_bwd and agk_logsumexp_bwd compute (the
 * same references: softmax_row_nodeops, reduction.cpp:42-53; vjp_SoftmaxRow,
 * autodiff_vjp_ops.cpp:421-428; vjp_LogSumExpRow, :430-440).  Given a
 * workspace, wide rows are spread over a team of parts = ceil(slots / 2048)
 * workgroups (slots = the row's 16-byte slots) that exchange their partial
 * row sums through the workspace, so each input row is read from HBM once
 * (the workspace-free calls re-read rows too wide for one workgroup's
 * registers): rows on a 16-byte boundary from 3 parts (the softmax
 * backward from 4), rows that do not start on one (every row tensor at the
 * same offset from one) from 4 parts (the softmax backward from 2).
 * Results are within fp32
 * rounding of the workspace-free calls' (the row sums are added in another
 * order, and the forward and the log-sum-exp backward scale each range's
 * exp(z - range max) by exp(range max - row max)) and bit-identical run to
 * run.  workspace == NULL takes the workspace-free kernels;
 * otherwise it must be 8-byte aligned and hold at least
 * agk_rowops_workspace_bytes(rows, cols) bytes (AGK_EINVAL / AGK_EWORKSPACE
 * if not): rows * parts * 16 bytes, parts = ceil(ceil(cols / W) / 2048) for
 * W = 4 (fp32), or for W = 8 (bf16) where fp32 rows would need more than 64
 * parts; 0 where that is below 2 or above 64 (rows that one workgroup holds,
 * or too wide for the team kernel).  The workspace is scratch: its contents
 * on entry do not matter, and calls that share one must not overlap in time. */
size_t agk_rowops_workspace_bytes(int64_t rows, int64_t cols);

int agk_softmax_fwd_ws(const void* z, void* y, void* workspace,
                       size_t workspace_bytes, int64_t rows, int64_t cols,
                       int dtype, agk_stream_t stream);

int agk_softmax_bwd_ws(const void* y, const void* dy, void* dz, void* workspace,
                       size_t workspace_bytes, int64_t rows, int64_t cols,
                       int dtype, int accumulate, agk_stream_t stream);

int agk_logsumexp_bwd_ws(const void* z, const void* dy, void* dz, void* workspace,
                         size_t workspace_bytes, int64_t rows, int64_t cols,
                         int dtype, int accumulate, agk_stream_t stream);

/* Testing and measurement knob, with no counterpart in the reference: when
 * the *_ws calls above take the team kernel.  0: never; 1 (default): for the
 * rows described above; 2: for every row it can hold (up to 64 workgroups of
 * 2048 16-byte slots).  A value outside 0..2 only reads the setting.
 * Process-wide; returns the previous value.  Their wait on other workgroups
 * is agk_set_exchange_wait_limit's (agk_rmsnorm.h).                          */
int agk_set_rowops_team(int mode);

/* Testing knob, with no counterpart in the reference: the team launch that
 * op (0 agk_softmax_fwd_ws, 1 agk_softmax_bwd_ws, 2 agk_logsumexp_bwd_ws)
 * takes for these sizes under the current mode, given a workspace, with
 * every row tensor 16-byte aligned (aligned != 0; cols a multiple of the
 * vector width) or all at one other offset from a boundary (aligned == 0).
 * plan[0] = workgroups per row (0: the workspace-free kernels run instead),
 * plan[1] = 16-byte slots per workgroup, plan[2] = rows in flight (teams).  */
int agk_rowops_team_plan(int op, int64_t rows, int64_t cols, int dtype,
                         int aligned, int32_t* plan);

#ifdef __cplusplus
}
#endif

#endif /* AGK_ROWOPS_H */
