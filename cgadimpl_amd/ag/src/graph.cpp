// graph.cpp -- nodes, values, topological order, the node-created hook.
#include "ag/graph.hpp"

#include <unordered_set>

#include "check.hpp"

namespace ag {

using internal::fail;

const char* op_name(Op op) {
    switch (op) {
#define AG_OP(name, arity, str) \
    case Op::name:              \
        return str;
#include "ag/ops.def"
#undef AG_OP
        default:
            return "?";
    }
}

int op_arity(Op op) {
    switch (op) {
#define AG_OP(name, arity, str) \
    case Op::name:              \
        return arity;
#include "ag/ops.def"
#undef AG_OP
        default:
            return -1;
    }
}

Node::Node(const Tensor& v, Op op_, bool req_grad, const char* name)
    : value(v), debug_name(name), op(op_), is_leaf(op_ == Op::Leaf), requires_grad_flag_(req_grad) {
    creation_context.stream = current_stream();
    (void)hipGetDevice(&creation_context.device);
}

Tensor& Node::grad_for_write(Dtype dt, bool* accumulate) {
    if (!grad.defined() || grad_is_materialized_zero) {
        grad = Tensor::empty(value.shape(), dt);
        grad_is_materialized_zero = false;
        grad_is_borrowed = false;
        *accumulate = false;
        return grad;
    }
    if (grad.dtype() != dt)
        fail(std::string("gradient of node '") + debug_name + "' is " + dtype_name(grad.dtype()) +
             ", a contribution of " + dtype_name(dt) + " cannot be added to it");
    if (grad_is_borrowed) {  // the caller's seed tensor: copy before adding into it
        Tensor own = Tensor::empty(grad.shape(), grad.dtype());
        own.copy_from(grad);
        grad = own;
        grad_is_borrowed = false;
    }
    *accumulate = true;
    return grad;
}

Value::Value(float v)
    : node(std::make_shared<Node>(Tensor::full({1}, v, Dtype::Float32), Op::Leaf, false,
                                  "scalar_literal")) {
    node->is_scalar_literal = true;
    node->literal_value = v;
}

const std::vector<int64_t>& Value::shape() const { return node->value.shape(); }
Tensor& Value::val() { return node->value; }
const Tensor& Value::val() const { return node->value; }

Tensor& Value::grad() {
    if (!node->grad.defined()) {
        node->grad = Tensor::zeros(node->value.shape(), node->value.dtype());
        node->grad_is_materialized_zero = true;
    }
    return node->grad;
}

void Value::register_hook(HookFn hook) {
    if (node) node->register_hook(std::move(hook));
}

std::vector<Node*> topo_from(Node* root) {
    std::vector<Node*> order;
    if (!root) return order;
    std::unordered_set<Node*> seen;
    // iterative depth-first search; a node is emitted after all its inputs
    std::vector<std::pair<Node*, size_t>> stack;
    stack.emplace_back(root, 0);
    seen.insert(root);
    while (!stack.empty()) {
        auto& [n, next] = stack.back();
        if (next < n->inputs.size()) {
            Node* p = n->inputs[next++].get();
            if (p && seen.insert(p).second) stack.emplace_back(p, 0);
        } else {
            order.push_back(n);
            stack.pop_back();
        }
    }
    return order;
}

namespace debug {
namespace {
NodeCreatedHook g_hook = nullptr;
std::atomic<uint64_t> g_fused_rms_mul{0};
}
void set_on_node_created(NodeCreatedHook hook) { g_hook = hook; }
uint64_t fused_rms_mul_vjps() { return g_fused_rms_mul.load(); }
void count_fused_rms_mul_vjp() { g_fused_rms_mul.fetch_add(1); }
void on_node_created(const std::shared_ptr<Node>& n) {
    if (g_hook) g_hook(n);
}
}  // namespace debug

}  // namespace ag
