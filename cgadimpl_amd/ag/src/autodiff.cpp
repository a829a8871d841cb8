// autodiff.cpp -- backward(), zero_grad(), jvp() and the VJP / JVP tables.
//
// Follows cgadimpl/src/core/autodiff.cpp:27-170: topological order from the
// root, dependency counters, the root's gradient assigned from the seed
// (ones without one), then every node's VJP in reverse order, sequentially or
// on worker threads (a node becomes ready when all its consumers have run).
// Differences, both deliberate:
//   - every VJP launches on the stream that is current where backward() was
//     called (worker threads take it over), where the reference's workers
//     fall back to the null stream; one stream keeps the device order equal
//     to the dependency order the host enforces;
//   - a node whose gradient never arrived (no consumer contributed) has a
//     zero upstream gradient, so its VJP is skipped instead of run on zeros.
#include <algorithm>
#include <condition_variable>
#include <deque>
#include <exception>
#include <thread>

#include "ag/autodiff.hpp"
#include "check.hpp"

namespace ag {

using internal::fail;

VjpFn vjp_lookup(Op op) {
    switch (op) {
#define AG_OP(name, arity, str) \
    case Op::name:              \
        return &detail::vjp_##name;
#include "ag/ops.def"
#undef AG_OP
        default:
            return nullptr;
    }
}

JvpFn jvp_lookup(Op op) {
    switch (op) {
#define AG_OP(name, arity, str) \
    case Op::name:              \
        return &detail::jvp_##name;
#include "ag/ops.def"
#undef AG_OP
        default:
            return nullptr;
    }
}

Tensor jvp(const Value& root, const std::unordered_map<Node*, Tensor>& seed) {
    if (!root.node) fail("jvp: empty root");
    const std::vector<Node*> order = topo_from(root.node.get());
    std::unordered_map<Node*, Tensor> tangent;
    tangent.reserve(order.size());
    const Tensor none;
    auto tangent_of = [&](Node* p) -> const Tensor& {
        auto it = tangent.find(p);
        return it == tangent.end() ? none : it->second;
    };
    for (Node* n : order) {
        Tensor t;
        if (n->op == Op::Leaf) {
            auto it = seed.find(n);
            if (it != seed.end()) {
                const Tensor& s = it->second;
                if (s.defined() && (s.shape() != n->value.shape() || s.dtype() != n->value.dtype()))
                    fail("jvp: a seed must have its node's shape and dtype");
                t = s;
            }
        } else if (JvpFn fn = jvp_lookup(n->op)) {
            t = fn(n, tangent_of);
        }
        if (t.defined()) tangent[n] = t;
    }
    const Tensor& out = tangent_of(root.node.get());
    if (out.defined()) return out;
    return Tensor::zeros(root.node->value.shape(), root.node->value.dtype());
}

void zero_grad(const Value& root) {
    for (Node* n : topo_from(root.node.get()))
        if (n->requires_grad()) {
            n->grad = Tensor();  // reads as zeros; the next contribution overwrites
            n->grad_is_materialized_zero = false;
            n->grad_is_borrowed = false;
        }
}

namespace {

thread_local bool t_in_backward = false;

struct InBackward {
    InBackward() { t_in_backward = true; }
    ~InBackward() { t_in_backward = false; }
};

void run_node(Node* n) {
    if (n->vjp_done) {  // a consumer's VJP already ran this one
        n->vjp_done = false;
    } else if (n->grad.defined()) {
        VjpFn fn = vjp_lookup(n->op);
        if (fn) fn(n, n->grad);
    }
    for (auto& hook : n->post_acc_grad_hooks) hook(n);
}

// Sets every node's child_grad_count to the number of its consumers in
// `order` that will run a VJP (reference: autodiff.cpp:37-49); returns how
// many nodes will run.
size_t count_consumers(const std::vector<Node*>& order) {
    for (Node* n : order) {
        n->child_grad_count = 0;
        n->vjp_done = false;
    }
    size_t pending = 0;
    for (Node* n : order) {
        if (!n->requires_grad()) continue;
        ++pending;
        for (auto& p : n->inputs)
            if (p && p->requires_grad()) p->child_grad_count++;
    }
    return pending;
}

void backward_parallel(const std::vector<Node*>& order, Node* root, hipStream_t stream) {
    const size_t pending = count_consumers(order);

    std::mutex mu;
    std::condition_variable cv;
    std::deque<Node*> ready{root};
    size_t done = 0;
    std::exception_ptr error;

    auto worker = [&]() {
        StreamGuard guard(stream);
        InBackward in_backward;
        for (;;) {
            Node* n = nullptr;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return !ready.empty() || done == pending || error; });
                if (done == pending || error) return;
                n = ready.front();
                ready.pop_front();
            }
            try {
                run_node(n);
            } catch (...) {
                std::lock_guard<std::mutex> lk(mu);
                if (!error) error = std::current_exception();
                cv.notify_all();
                return;
            }
            std::lock_guard<std::mutex> lk(mu);
            for (auto& p : n->inputs)
                if (p && p->requires_grad() && p->child_grad_count.fetch_sub(1) == 1)
                    ready.push_back(p.get());
            ++done;
            cv.notify_all();
        }
    };

    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t nthreads = std::min<size_t>({static_cast<size_t>(hw), pending, 64});
    std::vector<std::thread> threads;
    threads.reserve(nthreads);
    for (size_t i = 0; i < nthreads; ++i) threads.emplace_back(worker);
    for (auto& t : threads) t.join();
    if (error) std::rethrow_exception(error);
    if (done != pending) fail("backward: dependency counting left nodes unprocessed");
}

}  // namespace

void backward(const Value& root, const Tensor* grad_seed, bool enable_parallel) {
    if (!root.node) fail("backward: empty root");
    Node* r = root.node.get();
    if (!r->requires_grad()) return;  // no input of the graph requires grad
    const std::vector<Node*> order = topo_from(r);

    // seed: assignment, not accumulation (reference autodiff.cpp:53-55)
    if (grad_seed) {
        if (grad_seed->shape() != r->value.shape() || grad_seed->dtype() != r->value.dtype())
            fail("backward: the seed must have the root's shape and dtype");
        r->grad = *grad_seed;
        r->grad_is_borrowed = true;
    } else {
        r->grad = Tensor::ones(r->value.shape(), r->value.dtype());
        r->grad_is_borrowed = false;
    }
    r->grad_is_materialized_zero = false;

    if (!enable_parallel) {
        count_consumers(order);
        InBackward in_backward;
        for (auto it = order.rbegin(); it != order.rend(); ++it) {
            Node* n = *it;
            if (!n->requires_grad()) continue;
            run_node(n);
            for (auto& p : n->inputs)
                if (p && p->requires_grad()) p->child_grad_count--;
        }
        return;
    }
    backward_parallel(order, r, current_stream());
}

namespace internal {
bool in_backward() { return t_in_backward; }
}  // namespace internal

}  // namespace ag
