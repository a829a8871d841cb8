// ops.cpp -- forward ops, VJP and JVP rules of the RMSNorm layer path and its
// neighbours, on the HIP kernels behind include/agk_rmsnorm.h and
// include/agk_rowops.h.
//
// Reference behaviour (paths relative to the reference tree):
//   rms_nodeops      cgadimpl/src/ops/normalization.cpp:23-35
//   mul_nodeops      cgadimpl/src/ops/arithmetic.cpp:31-39
//   matmul_nodeops   cgadimpl/src/ops/linalg.cpp:12-20
//   linear_nodeops   cgadimpl/src/ops/linalg.cpp:21-33
//   laynor_nodeops   normalization.cpp:10-22
//   softmax_row_nodeops, logsumexp_row_nodeops  cgadimpl/src/ops/reduction.cpp:42-66
//   vjp_RMSNorm      cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:368-377
//   vjp_Mul          autodiff_vjp_ops.cpp:54-59, with reduce_for_broadcast :15-35
//   vjp_MatMul       autodiff_vjp_ops.cpp:258-263
//   vjp_Linear       autodiff_vjp_ops.cpp:272-279
//   vjp_LayerNorm    autodiff_vjp_ops.cpp:351-365
//   vjp_SoftmaxRow, vjp_LogSumExpRow  autodiff_vjp_ops.cpp:421-440
//   jvp_* rules      cgadimpl/src/autodiff/autodiff_jvp_ops.cpp (Mul :24-31,
//                    MatMul :245-249, RMSNorm :366-379 corrected, SoftmaxRow
//                    :411-420, LogSumExpRow :421-434; LayerNorm, which the
//                    reference leaves unimplemented (:360-362), uses its
//                    symmetric Jacobian: the VJP kernel applied to the tangent)
//   accumulate_grad  cgadimpl/src/core/graph.cpp:44-47
// Each forward records the same node structure as the reference (inputs,
// tape, child_grad_count, the node-created hook); each VJP adds its
// contribution into the inputs' gradients under their mutexes, with the
// addition done by the kernel (see Node::grad_for_write).
#include <algorithm>
#include <mutex>

#include "ag/autodiff.hpp"
#include "ag/ops.hpp"
#include "agk_rowops.h"
#include "check.hpp"

namespace ag {

using internal::agk_check;
using internal::fail;

namespace {

int agk_dtype_of(Dtype d) { return d == Dtype::Float32 ? AGK_F32 : AGK_BF16; }

agk_stream_t stream_arg() { return reinterpret_cast<agk_stream_t>(current_stream()); }

// [cols], [1, cols], [1, 1, cols], ...: a row vector broadcast over leading axes.
bool is_row_vector(const Tensor& t, int64_t cols) {
    if (t.dim() < 1 || t.shape().back() != cols) return false;
    for (int64_t i = 0; i + 1 < t.dim(); ++i)
        if (t.shape()[i] != 1) return false;
    return true;
}

// The output shape of a * b under the tensor library's broadcasting (numpy
// rules: shapes aligned at the trailing axis, extents equal or 1).
std::vector<int64_t> mul_out_shape(const Tensor& a, const Tensor& b, const char* op) {
    int64_t out[8];
    int nd = 0;
    const std::vector<int64_t>& as = a.shape();
    const std::vector<int64_t>& bs = b.shape();
    if (agk_mul_bcast_shape(as.data(), static_cast<int>(as.size()), bs.data(),
                            static_cast<int>(bs.size()), out, &nd) != AGK_OK) {
        auto str = [](const std::vector<int64_t>& s) {
            std::string r = "[";
            for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
            return r + "]";
        };
        fail(std::string(op) + ": shapes " + str(as) + " and " + str(bs) +
             " do not broadcast (or have more than 8 axes)");
    }
    return std::vector<int64_t>(out, out + nd);
}

// Which kernels a product takes: equal shapes and a row vector broadcast over
// the other operand's rows have their own; every other broadcast the general
// ones (agk_mul_bcast_*).
enum class MulForm { Equal, RowB, RowA, General };

MulForm mul_form(const Tensor& av, const Tensor& bv, const std::vector<int64_t>& out) {
    if (av.shape() == bv.shape()) return MulForm::Equal;
    int64_t n = 1;
    for (int64_t e : out) n *= e;
    if (av.dim() >= 1 && is_row_vector(bv, av.cols()) && n == av.numel()) return MulForm::RowB;
    if (bv.dim() >= 1 && is_row_vector(av, bv.cols()) && n == bv.numel()) return MulForm::RowA;
    return MulForm::General;
}

// Whether an operand covers the whole output (its gradient then keeps its dtype).
bool covers_output(const Tensor& t, const std::vector<int64_t>& out) {
    if (t.dim() > static_cast<int64_t>(out.size())) return false;
    const size_t pad = out.size() - static_cast<size_t>(t.dim());
    for (size_t i = 0; i < out.size(); ++i) {
        const int64_t e = i < pad ? 1 : t.shape()[i - pad];
        if (e != out[i]) return false;
    }
    return true;
}

std::vector<int64_t> row_stat_shape(const Tensor& x) {
    std::vector<int64_t> s = x.shape();
    if (s.empty()) s.push_back(1);
    s.back() = 1;  // the reference keeps r as [..., 1] (reduce_mean keepdim)
    return s;
}

void link_inputs(const std::shared_ptr<Node>& n, std::vector<std::shared_ptr<Node>> ins) {
    for (auto& p : ins)
        if (p) p->child_grad_count++;
    n->inputs = std::move(ins);
    debug::on_node_created(n);
}

void require_value(const std::shared_ptr<Node>& n, const char* op) {
    if (!n || !n->value.defined()) fail(std::string(op) + ": undefined input");
}

void check_upstream(const Node* n, const Tensor& gy, const char* op) {
    if (!gy.defined() || gy.shape() != n->value.shape() || gy.dtype() != n->value.dtype())
        fail(std::string(op) + ": upstream gradient does not match the node's value");
}

// Locks the gradient mutexes of up to two (possibly identical) nodes.
struct GradLocks {
    std::unique_lock<std::mutex> l[3];
    GradLocks(Node* x, Node* y, Node* z = nullptr) {
        Node* u[3];
        int n = 0;
        for (Node* p : {x, y, z})
            if (p && std::find(u, u + n, p) == u + n) u[n++] = p;
        for (int i = 0; i < n; ++i)
            l[i] = std::unique_lock<std::mutex>(u[i]->grad_mutex, std::defer_lock);
        if (n == 1)
            l[0].lock();
        else if (n == 2)
            std::lock(l[0], l[1]);
        else if (n == 3)
            std::lock(l[0], l[1], l[2]);
    }
};

// C = op(A) op(B) on the MFMA GEMM, with the workspace that lets it run its
// k-contiguous kernel (from the pool, or the capture arena).
void gemm(const void* A, int64_t lda, bool at, const void* B, int64_t ldb, bool bt, void* C,
          int64_t ldc, Dtype cdt, int64_t M, int64_t N, int64_t K, bool acc, const char* what) {
    const size_t wsb = agk_gemm_bf16_workspace_bytes(M, N, K, at, bt);
    std::unique_ptr<Storage> ws;
    if (wsb) ws = std::make_unique<Storage>(wsb, current_stream());
    agk_check(agk_gemm_bf16(A, lda, at, B, ldb, bt, C, ldc, agk_dtype_of(cdt), M, N, K, nullptr,
                            nullptr, acc ? 1 : 0, ws ? ws->data() : nullptr, wsb, stream_arg()),
              what);
}

// The same product on fp32 operands (the fp32 MFMA kernel behind agk_gemm_f32).
void gemm_f32(const void* A, int64_t lda, bool at, const void* B, int64_t ldb, bool bt, void* C,
              int64_t ldc, int64_t M, int64_t N, int64_t K, bool acc, const char* what) {
    agk_check(agk_gemm_f32(static_cast<const float*>(A), lda, at, static_cast<const float*>(B),
                           ldb, bt, static_cast<float*>(C), ldc, M, N, K, acc ? 1 : 0,
                           stream_arg()),
              what);
}

// C (+)= op(A) op(B) in the operands' dtype family: bf16 operands on the MFMA
// kernel (C in cdt), fp32 operands through gemm_f32 (C fp32).
void product(bool f32, const void* A, int64_t lda, bool at, const void* B, int64_t ldb, bool bt,
             void* C, int64_t ldc, Dtype cdt, int64_t M, int64_t N, int64_t K, bool acc,
             const char* what) {
    if (f32)
        gemm_f32(A, lda, at, B, ldb, bt, C, ldc, M, N, K, acc, what);
    else
        gemm(A, lda, at, B, ldb, bt, C, ldc, cdt, M, N, K, acc, what);
}

// The rows of a matmul operand [..., K]: the product of its leading axes.
// (Tensor::rows() divides numel by the last axis and so reports 0 rows for
// K == 0, where the product still has rows: zeros.)
int64_t lead_rows(const Tensor& t) {
    int64_t r = 1;
    for (int64_t i = 0; i + 1 < t.dim(); ++i) r *= t.shape()[i];
    return r;
}

// A tangent of `like`'s shape and dtype that is all zeros.
Tensor zero_tangent(const Tensor& like) { return Tensor::zeros(like.shape(), like.dtype()); }

}  // namespace

namespace detail {

// The exchange workspace of the RMSNorm forward's team kernel (rows wider
// than one workgroup holds: x read once), from the pool on the current
// stream; null when the shape needs none.
static std::unique_ptr<Storage> rms_fwd_workspace(const Tensor& t, size_t* bytes) {
    *bytes = agk_rmsnorm_fwd_workspace_bytes(t.rows(), t.cols());
    return *bytes ? std::make_unique<Storage>(*bytes, current_stream()) : nullptr;
}

std::shared_ptr<Node> rms_nodeops(const std::shared_ptr<Node>& x) {
    require_value(x, "rms");
    const Tensor& xv = x->value;
    if (xv.dim() < 1) fail("rms: input needs at least one axis");
    constexpr float kEps = 1e-5f;  // fixed, as cgadimpl/src/ops/normalization.cpp:26
    Tensor y = Tensor::empty(xv.shape(), xv.dtype());
    auto inv = std::make_shared<Tensor>(Tensor::empty(row_stat_shape(xv), Dtype::Float32));
    size_t ws_bytes = 0;
    const std::unique_ptr<Storage> ws = rms_fwd_workspace(xv, &ws_bytes);
    agk_check(agk_rmsnorm_fwd_ws(xv.data(), nullptr, y.data(), static_cast<float*>(inv->data()),
                                 ws ? ws->data() : nullptr, ws_bytes, xv.rows(), xv.cols(), kEps,
                                 agk_dtype_of(xv.dtype()), stream_arg()),
              "rms");
    auto n = std::make_shared<Node>(y, Op::RMSNorm, x->requires_grad(), "rmsnorm");
    n->eps = kEps;
    n->tape.push_back(inv);
    n->tape.push_back(std::make_shared<Tensor>(y));
    link_inputs(n, {x});
    return n;
}

std::shared_ptr<Node> rms_norm_nodeops(const std::shared_ptr<Node>& x,
                                       const std::shared_ptr<Node>& gamma, float eps) {
    require_value(x, "rms_norm");
    require_value(gamma, "rms_norm");
    if (x == gamma) fail("rms_norm: x and gamma must be different nodes");
    const Tensor& xv = x->value;
    const Tensor& gv = gamma->value;
    if (xv.dim() < 1) fail("rms_norm: input needs at least one axis");
    if (!is_row_vector(gv, xv.cols()))
        fail("rms_norm: gamma must have shape [D] or [1, D] with D = x.shape[-1]");
    if (gv.dtype() != xv.dtype()) fail("rms_norm: gamma and x must have the same dtype");
    Tensor y = Tensor::empty(xv.shape(), xv.dtype());
    auto inv = std::make_shared<Tensor>(Tensor::empty(row_stat_shape(xv), Dtype::Float32));
    size_t ws_bytes = 0;
    const std::unique_ptr<Storage> ws = rms_fwd_workspace(xv, &ws_bytes);
    agk_check(agk_rmsnorm_fwd_ws(xv.data(), gv.data(), y.data(), static_cast<float*>(inv->data()),
                                 ws ? ws->data() : nullptr, ws_bytes, xv.rows(), xv.cols(), eps,
                                 agk_dtype_of(xv.dtype()), stream_arg()),
              "rms_norm");
    auto n = std::make_shared<Node>(y, Op::RMSNormAffine,
                                    x->requires_grad() || gamma->requires_grad(), "rms_norm");
    n->eps = eps;
    n->tape.push_back(inv);
    link_inputs(n, {x, gamma});
    return n;
}

// A scalar literal (Value(float)) next to an operand of another dtype: the
// same literal in that dtype (a new leaf; the caller's literal is unchanged).
std::shared_ptr<Node> literal_like(const std::shared_ptr<Node>& lit, const Tensor& other) {
    if (!lit->is_scalar_literal || lit->value.dtype() == other.dtype()) return lit;
    auto n = std::make_shared<Node>(Tensor::full({1}, lit->literal_value, other.dtype()),
                                    Op::Leaf, false, "scalar_literal");
    n->is_scalar_literal = true;
    n->literal_value = lit->literal_value;
    return n;
}

std::shared_ptr<Node> mul_nodeops(const std::shared_ptr<Node>& a_in,
                                  const std::shared_ptr<Node>& b_in) {
    require_value(a_in, "mul");
    require_value(b_in, "mul");
    const std::shared_ptr<Node> a = literal_like(a_in, b_in->value);
    const std::shared_ptr<Node> b = literal_like(b_in, a->value);
    const Tensor& av = a->value;
    const Tensor& bv = b->value;
    if (av.dtype() != bv.dtype()) fail("mul: operands must have the same dtype");
    const int dt = agk_dtype_of(av.dtype());
    const std::vector<int64_t> out = mul_out_shape(av, bv, "mul");
    Tensor y = Tensor::empty(out, av.dtype());
    switch (mul_form(av, bv, out)) {
        case MulForm::Equal:
            agk_check(agk_mul_rowbcast_fwd(av.data(), bv.data(), y.data(), 1, av.numel(), dt,
                                           stream_arg()),
                      "mul");
            break;
        case MulForm::RowB:
            agk_check(agk_mul_rowbcast_fwd(av.data(), bv.data(), y.data(), av.rows(), av.cols(),
                                           dt, stream_arg()),
                      "mul");
            break;
        case MulForm::RowA:
            agk_check(agk_mul_rowbcast_fwd(bv.data(), av.data(), y.data(), bv.rows(), bv.cols(),
                                           dt, stream_arg()),
                      "mul");
            break;
        case MulForm::General:
            agk_check(agk_mul_bcast_fwd(av.data(), av.shape().data(),
                                        static_cast<int>(av.dim()), bv.data(), bv.shape().data(),
                                        static_cast<int>(bv.dim()), y.data(), dt, 0,
                                        stream_arg()),
                      "mul");
            break;
    }
    auto n = std::make_shared<Node>(y, Op::Mul, a->requires_grad() || b->requires_grad(), "*");
    link_inputs(n, {a, b});
    return n;
}

std::shared_ptr<Node> matmul_nodeops(const std::shared_ptr<Node>& a,
                                     const std::shared_ptr<Node>& b) {
    require_value(a, "matmul");
    require_value(b, "matmul");
    const Tensor& av = a->value;
    const Tensor& bv = b->value;
    const bool f32 = av.dtype() == Dtype::Float32 && bv.dtype() == Dtype::Float32;
    if (!f32 && (av.dtype() != Dtype::BFloat16 || bv.dtype() != Dtype::BFloat16))
        fail("matmul: operands must both be bfloat16 (the bf16 matrix-core kernel) or both "
             "float32 (a library sgemm)");
    if (bv.dim() != 2 || av.dim() < 1 || av.cols() != bv.shape()[0])
        fail("matmul: expects a [..., K] and b [K, N]");
    const int64_t M = lead_rows(av), K = av.cols(), N = bv.shape()[1];
    if (!f32 && (M % 8 || N % 8 || K % 8))
        fail("matmul: bfloat16 operands need M, N and K multiples of 8");
    std::vector<int64_t> ys = av.shape();
    ys.back() = N;
    Tensor y = Tensor::empty(ys, av.dtype());
    if (M && N)  // K == 0: the GEMM's empty sum writes zeros
        product(f32, av.data(), K, false, bv.data(), N, false, y.data(), N, av.dtype(), M, N, K,
                false, "matmul");
    auto n = std::make_shared<Node>(y, Op::MatMul, a->requires_grad() || b->requires_grad(),
                                    "matmul");
    link_inputs(n, {a, b});
    return n;
}

std::shared_ptr<Node> linear_nodeops(const std::shared_ptr<Node>& x,
                                     const std::shared_ptr<Node>& w,
                                     const std::shared_ptr<Node>& b) {
    require_value(x, "linear");
    require_value(w, "linear");
    require_value(b, "linear");
    const Tensor& xv = x->value;
    const Tensor& wv = w->value;
    const Tensor& bv = b->value;
    if (xv.dtype() != Dtype::BFloat16 || wv.dtype() != Dtype::BFloat16 ||
        bv.dtype() != Dtype::BFloat16)
        fail("linear: x, w and b must be bfloat16 (the product runs on the bf16 matrix cores)");
    if (wv.dim() != 2 || xv.dim() < 1 || xv.cols() != wv.shape()[1])
        fail("linear: expects x [..., K] and w [N, K]");
    const int64_t M = lead_rows(xv), K = xv.cols(), N = wv.shape()[0];
    if (!is_row_vector(bv, N)) fail("linear: b must have shape [N] or [1, N]");
    if (M % 8 || N % 8 || K % 8) fail("linear: the batch, N and K must be multiples of 8");
    std::vector<int64_t> ys = xv.shape();
    ys.back() = N;
    Tensor y = Tensor::empty(ys, Dtype::BFloat16);
    agk_check(agk_linear_bf16(xv.data(), K, wv.data(), K, bv.data(), y.data(), N, M, N, K,
                              stream_arg()),
              "linear");
    auto n = std::make_shared<Node>(
        y, Op::Linear, x->requires_grad() || w->requires_grad() || b->requires_grad(), "linear");
    link_inputs(n, {x, w, b});
    return n;
}

std::shared_ptr<Node> laynor_nodeops(const std::shared_ptr<Node>& x) {
    require_value(x, "laynor");
    const Tensor& xv = x->value;
    if (xv.dim() < 1) fail("laynor: input needs at least one axis");
    constexpr float kEps = 1e-5f;  // fixed, as cgadimpl/src/ops/normalization.cpp:14
    Tensor y = Tensor::empty(xv.shape(), xv.dtype());
    auto mean = std::make_shared<Tensor>(Tensor::empty(row_stat_shape(xv), Dtype::Float32));
    auto rstd = std::make_shared<Tensor>(Tensor::empty(row_stat_shape(xv), Dtype::Float32));
    agk_check(agk_layernorm_fwd(xv.data(), y.data(), static_cast<float*>(mean->data()),
                                static_cast<float*>(rstd->data()), xv.rows(), xv.cols(), kEps,
                                agk_dtype_of(xv.dtype()), stream_arg()),
              "laynor");
    auto n = std::make_shared<Node>(y, Op::LayerNorm, x->requires_grad(), "layernor");
    n->eps = kEps;
    n->tape.push_back(mean);
    n->tape.push_back(rstd);
    link_inputs(n, {x});
    return n;
}

// The exchange workspace of the row ops' team kernel (rows too wide for one
// workgroup), from the pool on the current stream; null when the shape needs
// none.
static std::unique_ptr<Storage> rowops_workspace(const Tensor& t, size_t* bytes) {
    *bytes = agk_rowops_workspace_bytes(t.rows(), t.cols());
    return *bytes ? std::make_unique<Storage>(*bytes, current_stream()) : nullptr;
}

std::shared_ptr<Node> softmax_row_nodeops(const std::shared_ptr<Node>& z) {
    require_value(z, "softmax_row");
    const Tensor& zv = z->value;
    if (zv.dim() < 1) fail("softmax_row: input needs at least one axis");
    Tensor y = Tensor::empty(zv.shape(), zv.dtype());
    size_t ws_bytes = 0;
    const std::unique_ptr<Storage> ws = rowops_workspace(zv, &ws_bytes);
    agk_check(agk_softmax_fwd_ws(zv.data(), y.data(), ws ? ws->data() : nullptr, ws_bytes,
                                 zv.rows(), zv.cols(), agk_dtype_of(zv.dtype()), stream_arg()),
              "softmax_row");
    auto n = std::make_shared<Node>(y, Op::SoftmaxRow, z->requires_grad(), "softmax_row");
    link_inputs(n, {z});
    return n;
}

std::shared_ptr<Node> logsumexp_row_nodeops(const std::shared_ptr<Node>& z) {
    require_value(z, "logsumexp_row");
    const Tensor& zv = z->value;
    if (zv.dim() < 1 || zv.cols() == 0) fail("logsumexp_row: needs a non-empty last axis");
    Tensor y = Tensor::empty(row_stat_shape(zv), zv.dtype());
    // Tape: the same values in fp32 (a bf16 y is too coarse for exp(z - y)).
    auto lse = std::make_shared<Tensor>(Tensor::empty(row_stat_shape(zv), Dtype::Float32));
    agk_check(agk_logsumexp_fwd_keep(zv.data(), y.data(), static_cast<float*>(lse->data()),
                                     zv.rows(), zv.cols(), agk_dtype_of(zv.dtype()),
                                     stream_arg()),
              "logsumexp_row");
    auto n = std::make_shared<Node>(y, Op::LogSumExpRow, z->requires_grad(), "logsumexp_row");
    n->tape.push_back(lse);
    link_inputs(n, {z});
    return n;
}

// ---- VJP rules --------------------------------------------------------------

void vjp_Leaf(Node*, const Tensor&) {}

// X.grad += r * (gy - x * r^2 * sum(gy * x) / D)   (autodiff_vjp_ops.cpp:368-377)
void vjp_RMSNorm(Node* n, const Tensor& gy) {
    Node* X = n->inputs[0].get();
    if (!X->requires_grad()) return;
    check_upstream(n, gy, "vjp_RMSNorm");
    const Tensor& x = X->value;
    const Tensor& inv = *n->tape[0];
    GradLocks lock(X, nullptr);
    bool acc = false;
    Tensor& dx = X->grad_for_write(x.dtype(), &acc);
    // no dgamma, so no workspace is required; wide rows take the split path
    // with one
    std::unique_ptr<Storage> ws;
    size_t ws_bytes = 0;
    if (x.cols() >= AGK_WIDE_MIN_COLS) {
        ws_bytes = agk_rmsnorm_bwd_workspace_bytes(x.rows(), x.cols());
        ws = std::make_unique<Storage>(ws_bytes, current_stream());
    }
    agk_check(agk_rmsnorm_bwd(x.data(), nullptr, static_cast<const float*>(inv.data()), gy.data(),
                              dx.data(), nullptr, ws ? ws->data() : nullptr, ws_bytes, x.rows(),
                              x.cols(), agk_dtype_of(x.dtype()),
                              acc ? AGK_ACCUM_DX : AGK_ACCUM_NONE, stream_arg()),
              "vjp_RMSNorm");
}

// The fused layer: dx as vjp_RMSNorm with g = gy * gamma, and
// dgamma += sum over rows of gy * x * r (vjp_Mul + reduce_for_broadcast).
void vjp_RMSNormAffine(Node* n, const Tensor& gy) {
    Node* X = n->inputs[0].get();
    Node* G = n->inputs[1].get();
    const bool want_dx = X->requires_grad();
    const bool want_dg = G->requires_grad();
    if (!want_dx && !want_dg) return;
    check_upstream(n, gy, "vjp_RMSNormAffine");
    const Tensor& x = X->value;
    const Tensor& inv = *n->tape[0];
    GradLocks lock(X, G);
    int acc = AGK_ACCUM_NONE;
    void* dx = nullptr;
    float* dg = nullptr;
    if (want_dx) {
        bool a = false;
        dx = X->grad_for_write(x.dtype(), &a).data();
        if (a) acc |= AGK_ACCUM_DX;
    }
    std::unique_ptr<Storage> ws;
    size_t ws_bytes = 0;
    if (want_dg) {
        bool a = false;
        dg = static_cast<float*>(G->grad_for_write(Dtype::Float32, &a).data());
        if (a) acc |= AGK_ACCUM_DGAMMA;
        ws_bytes = agk_rmsnorm_bwd_workspace_bytes(x.rows(), x.cols());
        ws = std::make_unique<Storage>(ws_bytes, current_stream());
    }
    agk_check(agk_rmsnorm_bwd(x.data(), G->value.data(), static_cast<const float*>(inv.data()),
                              gy.data(), dx, dg, ws ? ws->data() : nullptr, ws_bytes, x.rows(),
                              x.cols(), agk_dtype_of(x.dtype()), acc, stream_arg()),
              "vjp_RMSNormAffine");
    // ws returns to the pool on the same stream, after the kernels that use it
}

// The unfused layer y = rms(x) * gamma, from vjp_Mul with F = rms(x) (the full
// operand) and Rw = gamma (the broadcast row).  During backward, when this Mul
// is the last consumer of F still due and F has no gradient yet, F's gradient
// is final once this VJP has written it, so F's own VJP (vjp_RMSNorm) can run
// here in the same pass over the rows: agk_rms_mul_bwd reads x and gy once
// and writes F.grad = gy*gamma, X.grad (+)= and Rw.grad (+)= exactly the
// values the two VJPs write one after the other.  backward then skips F's
// VJP.  Returns false (nothing done) when the pattern does not apply.
static bool vjp_mul_of_rms(Node* F, Node* Rw, const Tensor& gy, bool want_row) {
    if (!internal::in_backward() || F->op != Op::RMSNorm || F->inputs.size() != 1 ||
        F->tape.empty() || F->vjp_done || F->child_grad_count.load() != 1)
        return false;
    Node* X = F->inputs[0].get();
    if (!X || X == Rw || X == F || !X->requires_grad()) return false;
    GradLocks lock(F, Rw, X);
    if (F->grad.defined() && !F->grad_is_materialized_zero) return false;  // not the only one
    const Tensor& x = X->value;
    const Tensor& row = Rw->value;
    const Tensor& inv = *F->tape[0];
    bool a = false;
    void* dr = F->grad_for_write(F->value.dtype(), &a).data();  // overwritten (a is false)
    int acc = AGK_ACCUM_NONE;
    void* dx = X->grad_for_write(x.dtype(), &a).data();
    if (a) acc |= AGK_ACCUM_DX;
    float* drow = nullptr;
    std::unique_ptr<Storage> ws;
    size_t ws_bytes = 0;
    if (want_row) {
        drow = static_cast<float*>(Rw->grad_for_write(Dtype::Float32, &a).data());
        if (a) acc |= AGK_ACCUM_DGAMMA;
    }
    // a workspace for the row gradient, and for wide rows (the split path,
    // as vjp_RMSNorm takes it)
    if (want_row || x.cols() >= AGK_WIDE_MIN_COLS) {
        ws_bytes = agk_rmsnorm_bwd_workspace_bytes(x.rows(), x.cols());
        ws = std::make_unique<Storage>(ws_bytes, current_stream());
    }
    agk_check(agk_rms_mul_bwd(x.data(), row.data(), static_cast<const float*>(inv.data()),
                              gy.data(), dr, dx, drow, ws ? ws->data() : nullptr, ws_bytes,
                              x.rows(), x.cols(), agk_dtype_of(x.dtype()), acc, stream_arg()),
              "vjp_Mul (rms(x) * gamma)");
    F->vjp_done = true;
    debug::count_fused_rms_mul_vjp();
    return true;
}

// A.grad += gy * B,  B.grad += reduce_for_broadcast(gy * A)   (autodiff_vjp_ops.cpp:54-59)
void vjp_Mul(Node* n, const Tensor& gy) {
    Node* A = n->inputs[0].get();
    Node* B = n->inputs[1].get();
    const bool want_a = A->requires_grad();
    const bool want_b = B->requires_grad();
    if (!want_a && !want_b) return;
    check_upstream(n, gy, "vjp_Mul");
    const Tensor& av = A->value;
    const Tensor& bv = B->value;
    const int dt = agk_dtype_of(av.dtype());
    const std::vector<int64_t>& out = n->value.shape();
    const MulForm form = mul_form(av, bv, out);
    if (form == MulForm::General) {
        // any other broadcast: each gradient summed over its operand's
        // broadcast axes (fp32), or the element-wise product (dtype) for an
        // operand that covers the output
        GradLocks lock(A, B);
        int acc = AGK_ACCUM_NONE;
        void* da = nullptr;
        void* db = nullptr;
        if (want_a) {
            bool a = false;
            da = A->grad_for_write(covers_output(av, out) ? av.dtype() : Dtype::Float32, &a).data();
            if (a) acc |= AGK_ACCUM_DX;
        }
        if (want_b) {
            bool a = false;
            db = B->grad_for_write(covers_output(bv, out) ? bv.dtype() : Dtype::Float32, &a).data();
            if (a) acc |= AGK_ACCUM_DGAMMA;
        }
        agk_check(agk_mul_bcast_bwd(gy.data(), av.data(), av.shape().data(),
                                    static_cast<int>(av.dim()), bv.data(), bv.shape().data(),
                                    static_cast<int>(bv.dim()), da, db, dt, acc, stream_arg()),
                  "vjp_Mul");
        return;
    }
    if (form == MulForm::Equal) {
        GradLocks lock(A, B);
        // equal shapes: dA = gy * B and dB = gy * A, both element-wise, each in
        // its operand's dtype (one launch per gradient; A == B adds twice)
        const int64_t cnt = av.numel();
        if (want_a) {
            bool a = false;
            void* da = A->grad_for_write(av.dtype(), &a).data();
            agk_check(agk_mul_rowbcast_bwd(gy.data(), nullptr, bv.data(), da, nullptr, nullptr, 0,
                                           1, cnt, dt, a ? AGK_ACCUM_DX : AGK_ACCUM_NONE,
                                           stream_arg()),
                      "vjp_Mul");
        }
        if (want_b) {
            bool a = false;
            void* db = B->grad_for_write(bv.dtype(), &a).data();
            agk_check(agk_mul_rowbcast_bwd(gy.data(), nullptr, av.data(), db, nullptr, nullptr, 0,
                                           1, cnt, dt, a ? AGK_ACCUM_DX : AGK_ACCUM_NONE,
                                           stream_arg()),
                      "vjp_Mul");
        }
        return;
    }
    // row-vector broadcast: `full` is [..., D], `row` is [D] / [1, D]
    const bool b_is_row = form == MulForm::RowB;
    Node* F = b_is_row ? A : B;
    Node* Rw = b_is_row ? B : A;
    const Tensor& full = F->value;
    const Tensor& row = Rw->value;
    const bool want_full = F->requires_grad();
    const bool want_row = Rw->requires_grad();
    if (want_full && vjp_mul_of_rms(F, Rw, gy, want_row)) return;
    GradLocks lock(F, Rw);
    int acc = AGK_ACCUM_NONE;
    void* dfull = nullptr;
    float* drow = nullptr;
    if (want_full) {
        bool a = false;
        dfull = F->grad_for_write(full.dtype(), &a).data();
        if (a) acc |= AGK_ACCUM_DX;
    }
    std::unique_ptr<Storage> ws;
    size_t ws_bytes = 0;
    if (want_row) {
        bool a = false;
        drow = static_cast<float*>(Rw->grad_for_write(Dtype::Float32, &a).data());
        if (a) acc |= AGK_ACCUM_DGAMMA;
        ws_bytes = agk_mul_rowbcast_bwd_workspace_bytes(full.rows(), full.cols());
        ws = std::make_unique<Storage>(ws_bytes, current_stream());
    }
    agk_check(agk_mul_rowbcast_bwd(gy.data(), full.data(), row.data(), dfull, drow,
                                   ws ? ws->data() : nullptr, ws_bytes, full.rows(), full.cols(),
                                   dt, acc, stream_arg()),
              "vjp_Mul");
}

// A.grad += gy B^T (bf16), B.grad += A^T gy (fp32)   (autodiff_vjp_ops.cpp:258-263)
void vjp_MatMul(Node* n, const Tensor& gy) {
    Node* A = n->inputs[0].get();
    Node* B = n->inputs[1].get();
    const bool want_a = A->requires_grad();
    const bool want_b = B->requires_grad();
    if (!want_a && !want_b) return;
    check_upstream(n, gy, "vjp_MatMul");
    const Tensor& av = A->value;
    const Tensor& bv = B->value;
    const int64_t M = lead_rows(av), K = av.cols(), N = bv.shape()[1];
    // bf16: dA in bf16, dB in fp32; fp32 operands: both fp32
    const bool f32 = av.dtype() == Dtype::Float32;
    const Dtype da_dt = f32 ? Dtype::Float32 : Dtype::BFloat16;
    GradLocks lock(A, B);
    // dB first: dA is what the producer of A's VJP reads next, so it is the
    // product left in the caches.  The two products are independent.
    if (want_b) {
        bool acc = false;
        Tensor& db = B->grad_for_write(Dtype::Float32, &acc);
        if (K && N)  // M == 0: an empty sum over the batch
            product(f32, av.data(), K, true, gy.data(), N, false, db.data(), N, Dtype::Float32, K,
                    N, M, acc, "vjp_MatMul dB");
    }
    if (want_a) {
        bool acc = false;
        Tensor& da = A->grad_for_write(da_dt, &acc);
        if (M && K)  // N == 0: an empty sum (zeros, or da unchanged when accumulating)
            product(f32, gy.data(), N, false, bv.data(), N, true, da.data(), K, da_dt, M, K, N,
                    acc, "vjp_MatMul dA");
    }
}

// X.grad += gy W (bf16), W.grad += gy^T X (fp32), b.grad += sum over rows of gy
// (fp32, agk_sum_rows)   (autodiff_vjp_ops.cpp:272-279)
void vjp_Linear(Node* n, const Tensor& gy) {
    Node* X = n->inputs[0].get();
    Node* Wn = n->inputs[1].get();
    Node* Bn = n->inputs[2].get();
    const bool want_x = X->requires_grad();
    const bool want_w = Wn->requires_grad();
    const bool want_b = Bn->requires_grad();
    if (!want_x && !want_w && !want_b) return;
    check_upstream(n, gy, "vjp_Linear");
    const Tensor& xv = X->value;
    const Tensor& wv = Wn->value;
    const int64_t M = lead_rows(xv), K = xv.cols(), N = wv.shape()[0];
    GradLocks lock(X, Wn, Bn);
    if (want_w) {  // [N, K] = gy^T [N, M] . X [M, K]
        bool acc = false;
        Tensor& dw = Wn->grad_for_write(Dtype::Float32, &acc);
        if (N && K)
            gemm(gy.data(), N, true, xv.data(), K, false, dw.data(), K, Dtype::Float32, N, K, M,
                 acc, "vjp_Linear dW");
    }
    if (want_b) {
        bool acc = false;
        Tensor& db = Bn->grad_for_write(Dtype::Float32, &acc);
        const size_t wsb = agk_sum_rows_workspace_bytes(M, N);
        std::unique_ptr<Storage> ws;
        if (wsb) ws = std::make_unique<Storage>(wsb, current_stream());
        agk_check(agk_sum_rows(gy.data(), static_cast<float*>(db.data()),
                               ws ? ws->data() : nullptr, wsb, M, N, AGK_BF16, acc ? 1 : 0,
                               stream_arg()),
                  "vjp_Linear db");
    }
    // dX last, as in vjp_MatMul: the producer of X's VJP reads it next.
    if (want_x) {  // [M, K] = gy [M, N] . W [N, K]
        bool acc = false;
        Tensor& dx = X->grad_for_write(Dtype::BFloat16, &acc);
        if (M && K)
            gemm(gy.data(), N, false, wv.data(), K, false, dx.data(), K, Dtype::BFloat16, M, K,
                 N, acc, "vjp_Linear dX");
    }
}

// X.grad += rstd * (gy - mean(gy) - xhat * mean(gy * xhat))   (autodiff_vjp_ops.cpp:351-365)
void vjp_LayerNorm(Node* n, const Tensor& gy) {
    Node* X = n->inputs[0].get();
    if (!X->requires_grad()) return;
    check_upstream(n, gy, "vjp_LayerNorm");
    const Tensor& x = X->value;
    GradLocks lock(X, nullptr);
    bool acc = false;
    Tensor& dx = X->grad_for_write(x.dtype(), &acc);
    agk_check(agk_layernorm_bwd(x.data(), static_cast<const float*>(n->tape[0]->data()),
                                static_cast<const float*>(n->tape[1]->data()), gy.data(),
                                dx.data(), x.rows(), x.cols(), agk_dtype_of(x.dtype()),
                                acc ? AGK_ACCUM_DX : AGK_ACCUM_NONE, stream_arg()),
              "vjp_LayerNorm");
}

// Z.grad += y * (gy - sum(y * gy))   (autodiff_vjp_ops.cpp:421-428)
void vjp_SoftmaxRow(Node* n, const Tensor& gy) {
    Node* Z = n->inputs[0].get();
    if (!Z->requires_grad()) return;
    check_upstream(n, gy, "vjp_SoftmaxRow");
    const Tensor& y = n->value;
    GradLocks lock(Z, nullptr);
    bool acc = false;
    Tensor& dz = Z->grad_for_write(y.dtype(), &acc);
    size_t ws_bytes = 0;
    const std::unique_ptr<Storage> ws = rowops_workspace(y, &ws_bytes);
    agk_check(agk_softmax_bwd_ws(y.data(), gy.data(), dz.data(), ws ? ws->data() : nullptr,
                                 ws_bytes, y.rows(), y.cols(), agk_dtype_of(y.dtype()),
                                 acc ? AGK_ACCUM_DX : AGK_ACCUM_NONE, stream_arg()),
              "vjp_SoftmaxRow");
}

// Z.grad += gy * softmax(z)   (autodiff_vjp_ops.cpp:430-440)
void vjp_LogSumExpRow(Node* n, const Tensor& gy) {
    Node* Z = n->inputs[0].get();
    if (!Z->requires_grad()) return;
    check_upstream(n, gy, "vjp_LogSumExpRow");
    const Tensor& z = Z->value;
    GradLocks lock(Z, nullptr);
    bool acc = false;
    Tensor& dz = Z->grad_for_write(z.dtype(), &acc);
    // softmax(z) = exp(z - lse): one pass over z with the forward's fp32 value
    // (the reference recomputes the row maximum and sum, the same quantity)
    const Tensor& lse = *n->tape.at(0);
    agk_check(agk_logsumexp_bwd_from_value(z.data(), static_cast<const float*>(lse.data()),
                                           gy.data(), dz.data(), z.rows(), z.cols(),
                                           agk_dtype_of(z.dtype()),
                                           acc ? AGK_ACCUM_DX : AGK_ACCUM_NONE, stream_arg()),
              "vjp_LogSumExpRow");
}

// ---- JVP rules ------------------------------------------------------------------
// Each returns the tangent of n, or an undefined Tensor when every input
// tangent is zero.  `tan(p)` is the tangent of input p (undefined: zero).

using TangentOf = std::function<const Tensor&(Node*)>;

namespace {
void check_tangent(const Tensor& t, const Tensor& like, const char* op) {
    if (t.defined() && (t.shape() != like.shape() || t.dtype() != like.dtype()))
        fail(std::string(op) + ": a tangent must have its node's shape and dtype");
}
}  // namespace

Tensor jvp_Leaf(Node*, const TangentOf&) { return Tensor(); }  // seeds are set by jvp()

// tA * B + A * tB   (autodiff_jvp_ops.cpp:24-31)
Tensor jvp_Mul(Node* n, const TangentOf& tan) {
    Node* A = n->inputs[0].get();
    Node* B = n->inputs[1].get();
    const Tensor& ta = tan(A);
    const Tensor& tb = tan(B);
    if (!ta.defined() && !tb.defined()) return Tensor();
    check_tangent(ta, A->value, "jvp_Mul");
    check_tangent(tb, B->value, "jvp_Mul");
    const Tensor& av = A->value;
    const Tensor& bv = B->value;
    Tensor out = Tensor::empty(n->value.shape(), n->value.dtype());
    const int dt = agk_dtype_of(av.dtype());
    const MulForm form = mul_form(av, bv, n->value.shape());
    if (form == MulForm::General) {  // out = tA * B + A * tB, each broadcast
        bool first = true;
        auto add = [&](const Tensor& x, const Tensor& y) {
            agk_check(agk_mul_bcast_fwd(x.data(), x.shape().data(), static_cast<int>(x.dim()),
                                        y.data(), y.shape().data(), static_cast<int>(y.dim()),
                                        out.data(), dt, first ? 0 : 1, stream_arg()),
                      "jvp_Mul");
            first = false;
        };
        if (ta.defined()) add(ta, bv);
        if (tb.defined()) add(av, tb);
        return out;
    }
    // full [..., D] times row [D]: out (+)= t_full * row and full * t_row, each
    // through the broadcast multiply's da path (equal shapes: one row of numel)
    const bool equal = form == MulForm::Equal;
    const bool b_is_row = form == MulForm::RowB;
    const Tensor& full = equal || b_is_row ? av : bv;
    const int64_t rows = equal ? 1 : full.rows();
    const int64_t cols = equal ? full.numel() : full.cols();
    bool first = true;
    auto add_product = [&](const Tensor& f, const Tensor& r) {  // out (+)= f * r
        agk_check(agk_mul_rowbcast_bwd(f.data(), nullptr, r.data(), out.data(), nullptr, nullptr,
                                       0, rows, cols, dt, first ? AGK_ACCUM_NONE : AGK_ACCUM_DX,
                                       stream_arg()),
                  "jvp_Mul");
        first = false;
    };
    if (equal) {
        if (ta.defined()) add_product(ta, bv);
        if (tb.defined()) add_product(tb, av);
    } else {
        Node* F = b_is_row ? A : B;
        Node* Rw = b_is_row ? B : A;
        const Tensor& tf = tan(F);
        const Tensor& tr = tan(Rw);
        if (tf.defined()) add_product(tf, Rw->value);
        if (tr.defined()) add_product(F->value, tr);
    }
    return out;
}

// tA B + A tB   (autodiff_jvp_ops.cpp:245-249)
Tensor jvp_MatMul(Node* n, const TangentOf& tan) {
    Node* A = n->inputs[0].get();
    Node* B = n->inputs[1].get();
    const Tensor& ta = tan(A);
    const Tensor& tb = tan(B);
    if (!ta.defined() && !tb.defined()) return Tensor();
    check_tangent(ta, A->value, "jvp_MatMul");
    check_tangent(tb, B->value, "jvp_MatMul");
    const Tensor& av = A->value;
    const Tensor& bv = B->value;
    const int64_t M = lead_rows(av), K = av.cols(), N = bv.shape()[1];
    const bool f32 = av.dtype() == Dtype::Float32;
    Tensor out = Tensor::empty(n->value.shape(), n->value.dtype());
    if (M == 0 || N == 0) return out;
    bool acc = false;
    if (ta.defined()) {
        product(f32, ta.data(), K, false, bv.data(), N, false, out.data(), N, out.dtype(), M, N,
                K, false, "jvp_MatMul");
        acc = true;
    }
    if (tb.defined())
        product(f32, av.data(), K, false, tb.data(), N, false, out.data(), N, out.dtype(), M, N,
                K, acc, "jvp_MatMul");
    return out;
}

// t*r - y*r*sum(t*y)/D   (autodiff_jvp_ops.cpp:366-379, corrected)
Tensor jvp_RMSNorm(Node* n, const TangentOf& tan) {
    Node* X = n->inputs[0].get();
    const Tensor& tx = tan(X);
    if (!tx.defined()) return Tensor();
    check_tangent(tx, X->value, "jvp_RMSNorm");
    const Tensor& x = X->value;
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    agk_check(agk_rmsnorm_jvp(x.data(), nullptr, static_cast<const float*>(n->tape[0]->data()),
                              tx.data(), nullptr, out.data(), x.rows(), x.cols(),
                              agk_dtype_of(x.dtype()), stream_arg()),
              "jvp_RMSNorm");
    return out;
}

// gamma * (t*r - y*r*sum(t*y)/D) + tgamma * x * r  (the rule above, then jvp_Mul)
Tensor jvp_RMSNormAffine(Node* n, const TangentOf& tan) {
    Node* X = n->inputs[0].get();
    Node* G = n->inputs[1].get();
    const Tensor& tx = tan(X);
    const Tensor& tg = tan(G);
    if (!tx.defined() && !tg.defined()) return Tensor();
    check_tangent(tx, X->value, "jvp_RMSNormAffine");
    check_tangent(tg, G->value, "jvp_RMSNormAffine");
    const Tensor& x = X->value;
    const Tensor txz = tx.defined() ? tx : zero_tangent(x);
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    agk_check(agk_rmsnorm_jvp(x.data(), G->value.data(),
                              static_cast<const float*>(n->tape[0]->data()), txz.data(),
                              tg.defined() ? tg.data() : nullptr, out.data(), x.rows(), x.cols(),
                              agk_dtype_of(x.dtype()), stream_arg()),
              "jvp_RMSNormAffine");
    return out;
}

// The LayerNorm Jacobian is symmetric: its VJP kernel applied to the tangent.
// tx W^T + X tW^T + tb: the corrected rule (the reference's jvp_Linear,
// autodiff_jvp_ops.cpp:256-265, multiplies by W and tW untransposed).  The
// first product carries tb in its store; the second adds into it.
Tensor jvp_Linear(Node* n, const TangentOf& tan) {
    Node* X = n->inputs[0].get();
    Node* Wn = n->inputs[1].get();
    Node* Bn = n->inputs[2].get();
    const Tensor& tx = tan(X);
    const Tensor& tw = tan(Wn);
    const Tensor& tb = tan(Bn);
    if (!tx.defined() && !tw.defined() && !tb.defined()) return Tensor();
    check_tangent(tx, X->value, "jvp_Linear");
    check_tangent(tw, Wn->value, "jvp_Linear");
    check_tangent(tb, Bn->value, "jvp_Linear");
    const Tensor& xv = X->value;
    const Tensor& wv = Wn->value;
    const int64_t M = lead_rows(xv), K = xv.cols(), N = wv.shape()[0];
    Tensor out = Tensor::empty(n->value.shape(), Dtype::BFloat16);
    if (M == 0 || N == 0) return out;
    const void* bias = tb.defined() ? tb.data() : nullptr;
    if (tx.defined() || !tw.defined()) {  // tx W^T + tb (K = 0 when only tb: the bias rows)
        const bool use_x = tx.defined();
        agk_check(agk_linear_bf16(use_x ? tx.data() : nullptr, K, wv.data(), K, bias, out.data(),
                                  N, M, N, use_x ? K : 0, stream_arg()),
                  "jvp_Linear");
        if (tw.defined())
            gemm(xv.data(), K, false, tw.data(), K, true, out.data(), N, Dtype::BFloat16, M, N, K,
                 true, "jvp_Linear");
    } else {  // X tW^T + tb
        agk_check(agk_linear_bf16(xv.data(), K, tw.data(), K, bias, out.data(), N, M, N, K,
                                  stream_arg()),
                  "jvp_Linear");
    }
    return out;
}

Tensor jvp_LayerNorm(Node* n, const TangentOf& tan) {
    Node* X = n->inputs[0].get();
    const Tensor& tx = tan(X);
    if (!tx.defined()) return Tensor();
    check_tangent(tx, X->value, "jvp_LayerNorm");
    const Tensor& x = X->value;
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    agk_check(agk_layernorm_bwd(x.data(), static_cast<const float*>(n->tape[0]->data()),
                                static_cast<const float*>(n->tape[1]->data()), tx.data(),
                                out.data(), x.rows(), x.cols(), agk_dtype_of(x.dtype()),
                                AGK_ACCUM_NONE, stream_arg()),
              "jvp_LayerNorm");
    return out;
}

// y * (t - sum(y * t))   (autodiff_jvp_ops.cpp:411-420)
Tensor jvp_SoftmaxRow(Node* n, const TangentOf& tan) {
    Node* Z = n->inputs[0].get();
    const Tensor& tz = tan(Z);
    if (!tz.defined()) return Tensor();
    check_tangent(tz, Z->value, "jvp_SoftmaxRow");
    const Tensor& y = n->value;
    Tensor out = Tensor::empty(y.shape(), y.dtype());
    size_t ws_bytes = 0;
    const std::unique_ptr<Storage> ws = rowops_workspace(y, &ws_bytes);
    agk_check(agk_softmax_bwd_ws(y.data(), tz.data(), out.data(), ws ? ws->data() : nullptr,
                                 ws_bytes, y.rows(), y.cols(), agk_dtype_of(y.dtype()),
                                 AGK_ACCUM_NONE, stream_arg()),
              "jvp_SoftmaxRow");
    return out;
}

// sum(softmax(z) * t)   (autodiff_jvp_ops.cpp:421-434)
Tensor jvp_LogSumExpRow(Node* n, const TangentOf& tan) {
    Node* Z = n->inputs[0].get();
    const Tensor& tz = tan(Z);
    if (!tz.defined()) return Tensor();
    check_tangent(tz, Z->value, "jvp_LogSumExpRow");
    const Tensor& z = Z->value;
    Tensor out = Tensor::empty(n->value.shape(), z.dtype());
    agk_check(agk_logsumexp_jvp(z.data(), tz.data(), out.data(), z.rows(), z.cols(),
                                agk_dtype_of(z.dtype()), stream_arg()),
              "jvp_LogSumExpRow");
    return out;
}

}  // namespace detail

Value rms(const Value& x) { return Value(detail::rms_nodeops(x.node)); }

Value rms_norm(const Value& x, const Value& gamma, float eps) {
    return Value(detail::rms_norm_nodeops(x.node, gamma.node, eps));
}

Value mul(const Value& a, const Value& b) { return Value(detail::mul_nodeops(a.node, b.node)); }

Value matmul(const Value& a, const Value& b) {
    return Value(detail::matmul_nodeops(a.node, b.node));
}

Value linear(const Value& x, const Value& w, const Value& b) {
    return Value(detail::linear_nodeops(x.node, w.node, b.node));
}

Value laynor(const Value& x) { return Value(detail::laynor_nodeops(x.node)); }

Value softmax_row(const Value& z) { return Value(detail::softmax_row_nodeops(z.node)); }

Value logsumexp_row(const Value& z) { return Value(detail::logsumexp_row_nodeops(z.node)); }

}  // namespace ag
