// nn.cpp -- the RMSNorm layer module.
#include "ag/nn.hpp"

#include "ag/ops.hpp"

namespace ag::nn {

void Module::zero_grad() {
    for (Value& p : parameters()) {
        p.node->grad = Tensor();
        p.node->grad_is_materialized_zero = false;
        p.node->grad_is_borrowed = false;
    }
}

RMSNorm::RMSNorm(int64_t dim, float eps_, Dtype dt) : eps(eps_) {
    Tensor g = Tensor::ones({dim}, dt);
    g.set_requires_grad(true);
    gamma = make_tensor(g, "rmsnorm.gamma");
}

Value RMSNorm::operator()(const Value& x) const { return rms_norm(x, gamma, eps); }

}  // namespace ag::nn
