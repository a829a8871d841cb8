// autodiff.hpp -- reverse-mode driver and the VJP table.
//
// Same entry points and semantics as cgadimpl/include/ad/autodiff/autodiff.hpp
// and cgadimpl/include/ad/detail/autodiff_ops.hpp:18-25:
//   backward() assigns the seed to the root's gradient (ones when no seed is
//   given) and runs each node's VJP in reverse topological order, either on
//   the calling thread or, with enable_parallel, on worker threads that take
//   a node once every consumer of it has run (dependency counters);
//   gradients accumulate across backward() calls until zero_grad().
// All VJP kernels are enqueued on the stream that is current on the thread
// that calls backward(), worker threads included, so they run in dependency
// order on the device.
#pragma once

#include "ag/graph.hpp"

namespace ag {

void zero_grad(const Value& root);
void backward(const Value& root, const Tensor* grad_seed = nullptr, bool enable_parallel = false);

// VJP of one node: reads n->inputs, n->tape and the upstream gradient gy and
// adds its contribution into the gradients of the inputs that require grad.
using VjpFn = void (*)(Node* n, const Tensor& gy);
VjpFn vjp_lookup(Op op);

namespace detail {
#define AG_OP(name, arity, str) void vjp_##name(Node* n, const Tensor& gy);
#include "ag/ops.def"
#undef AG_OP
}  // namespace detail

}  // namespace ag
