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

#include <functional>
#include <unordered_map>

#include "ag/graph.hpp"

namespace ag {

void zero_grad(const Value& root);
void backward(const Value& root, const Tensor* grad_seed = nullptr, bool enable_parallel = false);

// VJP of one node: reads n->inputs, n->tape and the upstream gradient gy and
// adds its contribution into the gradients of the inputs that require grad.
using VjpFn = void (*)(Node* n, const Tensor& gy);
VjpFn vjp_lookup(Op op);

// Forward mode (cgadimpl/include/ad/autodiff/autodiff.hpp:15,
// cgadimpl/src/core/autodiff.cpp:221-250): the tangent of root for the given
// tangents of some nodes (normally leaves), each of its node's shape and
// dtype.  Nodes without a seed, whose inputs carry no tangent, have a zero
// tangent; the result is zeros if nothing reaches the root.  Kernels run on
// the current stream.  Differs from the reference where it is wrong: a seeded
// leaf keeps its seed (the reference's jvp_Leaf replaces it with an empty
// tensor, autodiff_jvp_ops.cpp:189-192), and the RMSNorm rule is the
// corrected one (autodiff_jvp_ops.cpp:366-379 divides by 1/rms).
Tensor jvp(const Value& root, const std::unordered_map<Node*, Tensor>& seed);

// JVP of one node: the tangent of n from the tangents of its inputs
// (tangent_of returns an undefined Tensor for a zero tangent); an undefined
// result is a zero tangent.
using JvpFn = Tensor (*)(Node* n, const std::function<const Tensor&(Node*)>& tangent_of);
JvpFn jvp_lookup(Op op);

namespace detail {
#define AG_OP(name, arity, str)                          \
    void vjp_##name(Node* n, const Tensor& gy);           \
    Tensor jvp_##name(Node* n, const std::function<const Tensor&(Node*)>& tangent_of);
#include "ag/ops.def"
#undef AG_OP
}  // namespace detail

}  // namespace ag
