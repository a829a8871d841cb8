// ops.cpp -- forward ops and VJP rules of the RMSNorm layer path, on the HIP
// kernels behind include/agk_rmsnorm.h.
//
// Reference behaviour (paths relative to the reference tree):
//   rms_nodeops      cgadimpl/src/ops/normalization.cpp:23-35
//   mul_nodeops      cgadimpl/src/ops/arithmetic.cpp:31-39
//   vjp_RMSNorm      cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:368-377
//   vjp_Mul          autodiff_vjp_ops.cpp:54-59, with reduce_for_broadcast :15-35
//   accumulate_grad  cgadimpl/src/core/graph.cpp:44-47
// Each forward records the same node structure as the reference (inputs,
// tape, child_grad_count, the node-created hook); each VJP adds its
// contribution into the inputs' gradients under their mutexes, with the
// addition done by the kernel (see Node::grad_for_write).
#include <mutex>

#include "ag/autodiff.hpp"
#include "ag/ops.hpp"
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
    std::unique_lock<std::mutex> a, b;
    GradLocks(Node* x, Node* y) {
        if (x == y || !y) {
            a = std::unique_lock<std::mutex>(x->grad_mutex);
        } else {
            a = std::unique_lock<std::mutex>(x->grad_mutex, std::defer_lock);
            b = std::unique_lock<std::mutex>(y->grad_mutex, std::defer_lock);
            std::lock(a, b);
        }
    }
};

}  // namespace

namespace detail {

std::shared_ptr<Node> rms_nodeops(const std::shared_ptr<Node>& x) {
    require_value(x, "rms");
    const Tensor& xv = x->value;
    if (xv.dim() < 1) fail("rms: input needs at least one axis");
    constexpr float kEps = 1e-5f;  // fixed, as cgadimpl/src/ops/normalization.cpp:26
    Tensor y = Tensor::empty(xv.shape(), xv.dtype());
    auto inv = std::make_shared<Tensor>(Tensor::empty(row_stat_shape(xv), Dtype::Float32));
    agk_check(agk_rmsnorm_fwd(xv.data(), nullptr, y.data(), static_cast<float*>(inv->data()),
                              xv.rows(), xv.cols(), kEps, agk_dtype_of(xv.dtype()), stream_arg()),
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
    agk_check(agk_rmsnorm_fwd(xv.data(), gv.data(), y.data(), static_cast<float*>(inv->data()),
                              xv.rows(), xv.cols(), eps, agk_dtype_of(xv.dtype()), stream_arg()),
              "rms_norm");
    auto n = std::make_shared<Node>(y, Op::RMSNormAffine,
                                    x->requires_grad() || gamma->requires_grad(), "rms_norm");
    n->eps = eps;
    n->tape.push_back(inv);
    link_inputs(n, {x, gamma});
    return n;
}

std::shared_ptr<Node> mul_nodeops(const std::shared_ptr<Node>& a,
                                  const std::shared_ptr<Node>& b) {
    require_value(a, "mul");
    require_value(b, "mul");
    const Tensor& av = a->value;
    const Tensor& bv = b->value;
    if (av.dtype() != bv.dtype()) fail("mul: operands must have the same dtype");
    const int dt = agk_dtype_of(av.dtype());
    Tensor y;
    if (av.shape() == bv.shape()) {
        y = Tensor::empty(av.shape(), av.dtype());
        agk_check(agk_mul_rowbcast_fwd(av.data(), bv.data(), y.data(), 1, av.numel(), dt,
                                       stream_arg()),
                  "mul");
    } else if (av.dim() >= 1 && is_row_vector(bv, av.cols())) {
        y = Tensor::empty(av.shape(), av.dtype());
        agk_check(agk_mul_rowbcast_fwd(av.data(), bv.data(), y.data(), av.rows(), av.cols(), dt,
                                       stream_arg()),
                  "mul");
    } else if (bv.dim() >= 1 && is_row_vector(av, bv.cols())) {
        y = Tensor::empty(bv.shape(), bv.dtype());
        agk_check(agk_mul_rowbcast_fwd(bv.data(), av.data(), y.data(), bv.rows(), bv.cols(), dt,
                                       stream_arg()),
                  "mul");
    } else {
        fail("mul: only equal shapes or a row vector broadcast over the leading axes are "
             "supported");
    }
    auto n = std::make_shared<Node>(y, Op::Mul, a->requires_grad() || b->requires_grad(), "*");
    link_inputs(n, {a, b});
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
    agk_check(agk_rmsnorm_bwd(x.data(), nullptr, static_cast<const float*>(inv.data()), gy.data(),
                              dx.data(), nullptr, nullptr, 0, x.rows(), x.cols(),
                              agk_dtype_of(x.dtype()), acc ? AGK_ACCUM_DX : AGK_ACCUM_NONE,
                              stream_arg()),
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
    GradLocks lock(A, B);
    if (av.shape() == bv.shape()) {
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
    const bool b_is_row = is_row_vector(bv, av.cols()) && av.dim() >= 1;
    Node* F = b_is_row ? A : B;
    Node* Rw = b_is_row ? B : A;
    const Tensor& full = F->value;
    const Tensor& row = Rw->value;
    const bool want_full = F->requires_grad();
    const bool want_row = Rw->requires_grad();
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

}  // namespace detail

Value rms(const Value& x) { return Value(detail::rms_nodeops(x.node)); }

Value rms_norm(const Value& x, const Value& gamma, float eps) {
    return Value(detail::rms_norm_nodeops(x.node, gamma.node, eps));
}

Value mul(const Value& a, const Value& b) { return Value(detail::mul_nodeops(a.node, b.node)); }

}  // namespace ag
