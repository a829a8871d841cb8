// ops.hpp -- forward operations of the RMSNorm layer path and its neighbours.
//
// The reference writes the layer as two graph ops, `ag::rms(x) * gamma`
// (cgadimpl/include/ad/ops/ops.hpp:81,124; forward in
// cgadimpl/src/ops/normalization.cpp:23-35 and arithmetic.cpp:31-39).  Both
// are here with the same names and meaning, running on the HIP kernels behind
// include/agk_rmsnorm.h, plus the fused layer rms_norm(x, gamma, eps), one node
// whose forward and backward are one kernel call each.  matmul, laynor,
// softmax_row and logsumexp_row (ops.hpp:62,78,96-97) run on the GEMM and the
// row kernels of include/agk_rowops.h.
#pragma once

#include <memory>

#include "ag/graph.hpp"

namespace ag {

// x * (mean(x^2, last axis) + 1e-5)^(-1/2).  eps is 1e-5 as in the reference
// (normalization.cpp:26).  Tape: {inv_rms [rows] fp32, y}.
Value rms(const Value& x);

// The fused RMSNorm layer: x * rsqrt(mean(x^2) + eps) * gamma, gamma of shape
// [D] or [1, D] for x of shape [..., D].  Tape: {inv_rms [rows] fp32}.  The
// gradient of gamma is fp32 whatever gamma's storage type.
Value rms_norm(const Value& x, const Value& gamma, float eps = 1e-5f);

// Element-wise product under numpy broadcasting (cgadimpl/src/ops/arithmetic.cpp:31-39):
// equal shapes and a row vector ([D] or [1, D]) over the other's leading axes
// take the row kernels, every other broadcast (e.g. [B, T, D] * [B, 1, D], a
// 0-d or [1] scalar) the general broadcast kernels.  The output has the
// broadcast shape.  The gradient of a broadcast operand is fp32, summed over
// its broadcast axes; an operand that covers the output gets its gradient in
// its own dtype.  Shapes that do not broadcast, or operands of different
// dtypes, throw std::runtime_error.
Value mul(const Value& a, const Value& b);
inline Value operator*(const Value& a, const Value& b) { return mul(a, b); }

// a [..., K] times b [K, N] -> [..., N] (cgadimpl/src/ops/linalg.cpp:12-20).
// bf16 operands run on the MFMA GEMM; a's gradient is bf16, b's is fp32 (a
// weight accumulates in fp32).  fp32 operands run on the fp32 GEMM, with fp32
// gradients.  Operands of different dtypes throw std::runtime_error.
Value matmul(const Value& a, const Value& b);

// x [..., K] times w [N, K] transposed, plus b [N] or [1, N] -> [..., N], all
// bf16, on the MFMA GEMM with the bias added in its store
// (cgadimpl/src/ops/linalg.cpp:21-33, `matmul(x, w.t()) + b`, with its two
// bf16 roundings).  x's gradient is bf16; w's and b's are fp32.  Forward mode
// uses the rule tx w^T + x tw^T + tb (the reference's jvp_Linear,
// autodiff_jvp_ops.cpp:256-265, multiplies by w where w^T belongs).
Value linear(const Value& x, const Value& w, const Value& b);

// (x - mean) / sqrt(var + 1e-5) over the last axis (normalization.cpp:10-22;
// eps fixed as there).  Tape: {mean, rstd}, fp32 [..., 1].
Value laynor(const Value& x);

// Row softmax over the last axis (cgadimpl/src/ops/reduction.cpp:42-53).
Value softmax_row(const Value& z);

// Row log-sum-exp over the last axis, [..., D] -> [..., 1] (reduction.cpp:54-66).
Value logsumexp_row(const Value& z);

namespace detail {
std::shared_ptr<Node> rms_nodeops(const std::shared_ptr<Node>& x);
std::shared_ptr<Node> rms_norm_nodeops(const std::shared_ptr<Node>& x,
                                       const std::shared_ptr<Node>& gamma, float eps);
std::shared_ptr<Node> mul_nodeops(const std::shared_ptr<Node>& a,
                                  const std::shared_ptr<Node>& b);
std::shared_ptr<Node> matmul_nodeops(const std::shared_ptr<Node>& a,
                                     const std::shared_ptr<Node>& b);
std::shared_ptr<Node> linear_nodeops(const std::shared_ptr<Node>& x,
                                     const std::shared_ptr<Node>& w,
                                     const std::shared_ptr<Node>& b);
std::shared_ptr<Node> laynor_nodeops(const std::shared_ptr<Node>& x);
std::shared_ptr<Node> softmax_row_nodeops(const std::shared_ptr<Node>& z);
std::shared_ptr<Node> logsumexp_row_nodeops(const std::shared_ptr<Node>& z);
}  // namespace detail

}  // namespace ag
