// graph.hpp -- Value / Node, the eager dynamic graph of the autodiff layer.
//
// Mirrors cgadimpl/include/ad/core/graph.hpp:18-93 for the fields the RMSNorm
// layer path uses: a Node holds its value, its gradient, its inputs (owning),
// a tape of saved tensors, the op, a dependency counter and a mutex for
// gradient accumulation, post-accumulation hooks and the stream it was
// created on; a Value is a shared handle to a Node.
//
// One deliberate difference: the reference's Node constructor zero-fills a
// gradient of the value's shape for every node that requires grad
// (cgadimpl/src/core/graph.cpp:28-37) and each VJP then runs grad += g
// (graph.cpp:44-47).  Here a gradient stays undefined until the first VJP
// writes it; grad_for_write() tells that VJP whether to overwrite (first
// contribution) or add (later ones), and the kernel does the addition in the
// same pass, so neither the zero-fill nor the separate += pass is needed.
// Reading a gradient that never arrived through Value::grad() yields zeros,
// as in the reference.
#pragma once

#include <atomic>
#include <functional>
#include <memory>
#include <mutex>
#include <vector>

#include "ag/tensor.hpp"

namespace ag {

enum class Op : uint8_t {
#define AG_OP(name, arity, str) name,
#include "ag/ops.def"
#undef AG_OP
    Count
};

inline constexpr size_t OpCount = static_cast<size_t>(Op::Count);

const char* op_name(Op op);
int op_arity(Op op);

struct Node;
using HookFn = std::function<void(Node*)>;

struct Value {
    std::shared_ptr<Node> node;

    Value() = default;
    explicit Value(std::shared_ptr<Node> n) : node(std::move(n)) {}
    // A scalar literal (cgadimpl/include/ad/core/graph.hpp:22,
    // cgadimpl/src/core/graph.cpp:91-105): a leaf holding a one-element [1]
    // float32 tensor, named "scalar_literal", that requires no gradient.  Not
    // explicit, as in the reference, so `rms(x) * 0.5f` and `0.5f * rms(x)`
    // convert the float.  Used with a bfloat16 operand, mul takes the literal
    // in bfloat16 (rounded to nearest even).
    Value(float v);

    const std::vector<int64_t>& shape() const;
    Tensor& val();
    const Tensor& val() const;
    // The accumulated gradient; zeros of the value's shape if none arrived.
    Tensor& grad();
    void register_hook(HookFn hook);
};

struct Node : std::enable_shared_from_this<Node> {
    Tensor value;
    Tensor grad;  // undefined until the first gradient contribution
    // grad holds zeros that Value::grad() created for a reader (the next
    // contribution overwrites it, possibly with another dtype)
    bool grad_is_materialized_zero = false;
    // grad shares the caller's seed tensor (backward's grad_seed); it is copied
    // before any contribution is added into it
    bool grad_is_borrowed = false;

    std::vector<std::shared_ptr<Node>> inputs;
    std::vector<std::shared_ptr<Tensor>> tape;

    const char* debug_name = "";
    Op op = Op::Leaf;
    bool is_leaf = false;
    float eps = 0.0f;  // RMSNorm / RMSNormAffine: the eps of the forward pass
    // Value(float): the literal's value, so an op can take it in another dtype
    bool is_scalar_literal = false;
    float literal_value = 0.0f;

    std::atomic<int> child_grad_count{0};
    std::mutex grad_mutex;
    // Set during backward by a consumer's VJP that ran this node's VJP too
    // (vjp_Mul on rms(x) * gamma); backward then skips this node's VJP once.
    bool vjp_done = false;

    std::vector<HookFn> post_acc_grad_hooks;
    void register_hook(HookFn hook) { post_acc_grad_hooks.push_back(std::move(hook)); }

    struct ExecutionContext {
        hipStream_t stream = nullptr;
        int device = 0;
    };
    ExecutionContext creation_context;

    bool requires_grad_flag_ = false;
    bool requires_grad() const { return requires_grad_flag_; }
    const std::vector<int64_t>& shape() const { return value.shape(); }

    Node(const Tensor& v, Op op_, bool req_grad, const char* name = "");

    // For a VJP about to write this node's gradient, with grad_mutex held:
    // returns the gradient buffer (allocated with dtype `dt` on the current
    // stream if none has arrived yet) and sets *accumulate to whether the
    // kernel must add into it (true) or may overwrite it (false).
    Tensor& grad_for_write(Dtype dt, bool* accumulate);
};

// A leaf node holding `v` (requires_grad taken from the tensor, as in
// cgadimpl/include/ad/core/graph.hpp:82-84).
inline Value make_tensor(const Tensor& v, const char* name = "") {
    return Value(std::make_shared<Node>(v, Op::Leaf, v.requires_grad(), name));
}

// Every node reachable from root, inputs before the nodes that use them
// (cgadimpl/src/core/graph.cpp:77-88).
std::vector<Node*> topo_from(Node* root);

namespace debug {
// Called by every forward op with the node it created (the reference's
// debug::on_node_created, cgadimpl/src/tools/debug.cpp:96-109); no-op unless
// a hook is installed.
using NodeCreatedHook = void (*)(const std::shared_ptr<Node>&);
void set_on_node_created(NodeCreatedHook hook);
void on_node_created(const std::shared_ptr<Node>& n);
// How many times backward has run the two VJPs of rms(x) * gamma as one pass
// (vjp_Mul with agk_rms_mul_bwd) in this process; no reference counterpart.
uint64_t fused_rms_mul_vjps();
void count_fused_rms_mul_vjp();
}  // namespace debug

}  // namespace ag
