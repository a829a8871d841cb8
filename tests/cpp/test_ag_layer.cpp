// test_ag_layer.cpp -- the ag:: graph layer (Value, rms, rms_norm, mul,
// matmul, laynor, softmax_row, logsumexp_row, backward, jvp, GraphRunner) on
// the GPU.
//
//   test_ag_layer selftest [name ...]
//                              checks below (all, or the named groups); prints
//                              PASS/FAIL per check and exits with the number
//                              of failures
//   test_ag_layer dump <dir>   reads <dir>/meta.txt ("rows cols dtype eps",
//                              dtype 0 = f32, 1 = bf16) and x.bin, gamma.bin,
//                              dy.bin; writes the outputs of the fused layer
//                              (rms_norm, sequential and parallel backward) and
//                              of the unfused graph rms(x) * gamma, for the
//                              Python tests to compare against the CPU oracle
//
// The checks follow the reference's own tests: the numerical-gradient check
// of rms on a [4,10] input (cgadimpl/Tests/test_core_ops_gpu.cpp:38-84,
// 262-267), gradient accumulation across backward calls and zero_grad
// (Tests/test_phase1_advanced.cpp:32-64), sequential against parallel
// backward (Tests/dependency_counter_correctness/test_dependency_correctness.cpp),
// and broadcast-multiply gradients (test_core_ops_gpu.cpp:198-205).  Forward
// mode is checked against central differences of host fp64 restatements of
// each op, matmul against a host fp64 product, and hipGraph capture by
// replaying a captured forward + backward on changed inputs, with eager work
// in between, against eager runs (bitwise: the kernels are deterministic).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "ag/ag.hpp"
#include "agk_rmsnorm.h"

using namespace ag;

namespace {

int g_failures = 0;

void report(const char* name, bool ok, const std::string& detail = "") {
    std::printf("[%s] %s%s%s\n", ok ? "PASS" : "FAIL", name, detail.empty() ? "" : ": ",
                detail.c_str());
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

std::vector<float> normal(size_t n, uint64_t seed, double sd = 1.0) {
    std::mt19937_64 eng(seed);
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = 1.0 - static_cast<double>(eng() >> 11) * 0x1.0p-53;
        const double u2 = static_cast<double>(eng() >> 11) * 0x1.0p-53;
        const double rad = std::sqrt(-2.0 * std::log(u1));
        v[i] = static_cast<float>(sd * rad * std::cos(6.283185307179586 * u2));
        if (i + 1 < n) v[i + 1] = static_cast<float>(sd * rad * std::sin(6.283185307179586 * u2));
    }
    return v;
}

std::vector<float> uniform(size_t n, uint64_t seed, double lo, double hi) {
    std::mt19937_64 eng(seed);
    std::vector<float> v(n);
    for (auto& f : v) f = static_cast<float>(lo + (hi - lo) * (eng() >> 11) * 0x1.0p-53);
    return v;
}

Value leaf(const std::vector<float>& v, const std::vector<int64_t>& shape, const char* name,
           bool req = true) {
    Tensor t = Tensor::from_host_f32(v, shape);
    t.set_requires_grad(req);
    return make_tensor(t, name);
}

double max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    double m = 0.0;
    for (size_t i = 0; i < a.size(); ++i) m = std::max(m, std::fabs(double(a[i]) - double(b[i])));
    return m;
}

double max_abs(const std::vector<float>& a) {
    double m = 0.0;
    for (float f : a) m = std::max(m, std::fabs(double(f)));
    return m;
}

// sum(f()) in fp64 from the forward output
double loss_of(const std::function<Value()>& f) {
    std::vector<float> y = f().val().to_host_f32();
    double s = 0.0;
    for (float v : y) s += v;
    return s;
}

// Central differences of sum(f()) with respect to the leaf p (the reference's
// numerical_gradient, with the loss accumulated in fp64 on the host).
std::vector<float> numerical_gradient(Value& p, const std::function<Value()>& f, float h) {
    std::vector<float> orig = p.val().to_host_f32();
    std::vector<float> grad(orig.size());
    const std::vector<int64_t> shape = p.val().shape();
    for (size_t i = 0; i < orig.size(); ++i) {
        std::vector<float> v = orig;
        v[i] = orig[i] + h;
        const float up = v[i];
        p.val() = Tensor::from_host_f32(v, shape);
        const double lp = loss_of(f);
        v[i] = orig[i] - h;
        const float dn = v[i];
        p.val() = Tensor::from_host_f32(v, shape);
        const double lm = loss_of(f);
        grad[i] = static_cast<float>((lp - lm) / (double(up) - double(dn)));
    }
    p.val() = Tensor::from_host_f32(orig, shape);
    return grad;
}

void check_grad(const char* name, Value& p, const std::function<Value()>& f, float h = 1e-3f,
                double tol = 1e-3) {
    std::vector<float> analytic = p.grad().to_host_f32();
    std::vector<float> num = numerical_gradient(p, f, h);
    const double e = max_abs_diff(analytic, num);
    report(name, e <= tol, "max |analytic - numerical| = " + std::to_string(e));
}

// ---- checks ------------------------------------------------------------------

void test_reference_pattern() {
    // run_test("RMSNorm"): a = randn[4,10]; backward(sum(rms(a))); check_grad
    Value a = leaf(normal(40, 1), {4, 10}, "a");
    auto f = [&]() { return rms(a); };
    backward(f());  // seed = ones, i.e. the gradient of sum(rms(a))
    check_grad("rms [4,10] numerical gradient (reference pattern)", a, f);
}

void test_fused_layer_gradients() {
    Value x = leaf(normal(36, 2), {3, 12}, "x");
    Value g = leaf(uniform(12, 3, 0.5, 1.5), {12}, "gamma");
    std::vector<float> dyv = normal(36, 4);
    Tensor dy = Tensor::from_host_f32(dyv, {3, 12});
    // loss = sum(dy * y): check with a seed of dy against sum(y * dy)
    auto f = [&]() { return rms_norm(x, g, 1e-5f) * make_tensor(dy); };
    backward(rms_norm(x, g, 1e-5f), &dy);
    check_grad("rms_norm dx numerical gradient", x, f);
    check_grad("rms_norm dgamma numerical gradient", g, f);
}

void fused_matches_unfused_case(int64_t R, int64_t D);

void test_fused_matches_unfused() {
    fused_matches_unfused_case(64, 256);
    fused_matches_unfused_case(3, 40000);  // split paths for wide rows
    fused_matches_unfused_case(260, 20480);  // one-pass backward for wide rows
}

void fused_matches_unfused_case(int64_t R, int64_t D) {
    std::vector<float> xv = normal(R * D, 5), gv = uniform(D, 6, 0.5, 1.5), dyv = normal(R * D, 7);
    Tensor dy = Tensor::from_host_f32(dyv, {R, D});
    Value x1 = leaf(xv, {R, D}, "x1"), g1 = leaf(gv, {1, D}, "g1");
    Value y1 = rms_norm(x1, g1, 1e-5f);
    backward(y1, &dy);
    Value x2 = leaf(xv, {R, D}, "x2"), g2 = leaf(gv, {1, D}, "g2");
    Value y2 = rms(x2) * g2;
    backward(y2, &dy);
    const double ey = max_abs_diff(y1.val().to_host_f32(), y2.val().to_host_f32()) /
                      max_abs(y2.val().to_host_f32());
    const double ex = max_abs_diff(x1.grad().to_host_f32(), x2.grad().to_host_f32()) /
                      max_abs(x2.grad().to_host_f32());
    const double eg = max_abs_diff(g1.grad().to_host_f32(), g2.grad().to_host_f32()) /
                      max_abs(g2.grad().to_host_f32());
    const std::string shape = " [" + std::to_string(R) + "," + std::to_string(D) + "]";
    report(("rms_norm(x, g) == rms(x) * g" + shape).c_str(), ey <= 1e-5 && ex <= 1e-5 && eg <= 1e-5,
           "y " + std::to_string(ey) + " dx " + std::to_string(ex) + " dgamma " +
               std::to_string(eg));
    // gamma * rms(x): the broadcast operand first
    Value x3 = leaf(xv, {R, D}, "x3"), g3 = leaf(gv, {D}, "g3");
    Value y3 = g3 * rms(x3);
    backward(y3, &dy);
    report(("gamma * rms(x) == rms(x) * gamma" + shape).c_str(),
           y3.val().to_host_f32() == y2.val().to_host_f32() &&
               x3.grad().to_host_f32() == x2.grad().to_host_f32() &&
               g3.grad().to_host_f32() == g2.grad().to_host_f32());
}

std::vector<uint16_t> to_bf16_bits(const std::vector<float>& v) {
    std::vector<uint16_t> b(v.size());
    for (size_t i = 0; i < v.size(); ++i) {
        uint32_t u;
        std::memcpy(&u, &v[i], 4);
        u += 0x7fffu + ((u >> 16) & 1u);
        b[i] = static_cast<uint16_t>(u >> 16);
    }
    return b;
}

Tensor device(const std::vector<float>& v, const std::vector<int64_t>& shape, Dtype dt) {
    if (dt == Dtype::Float32) return Tensor::from_host_f32(v, shape);
    const std::vector<uint16_t> b = to_bf16_bits(v);
    return Tensor::from_host(b.data(), shape, dt);
}

std::vector<char> bytes_of(const Tensor& t) {
    std::vector<char> b(t.nbytes());
    if (!b.empty()) t.copy_to_host(b.data());
    return b;
}

// backward of rms(x) * gamma runs both VJPs in one pass (agk_rms_mul_bwd,
// from vjp_Mul); every gradient it leaves (x, gamma and rms(x) itself) must be
// bit-identical to the two separate kernels, agk_mul_rowbcast_bwd and then
// agk_rmsnorm_bwd, on the same tensors.
void composition_case(const char* name, int64_t R, int64_t D, Dtype dt, bool parallel,
                      bool gamma_first, bool gamma_2d) {
    const int dtc = dt == Dtype::Float32 ? AGK_F32 : AGK_BF16;
    Tensor xt = device(normal(R * D, 40 + D, 2.0), {R, D}, dt);
    Tensor gt = device(uniform(D, 41 + D, 0.5, 1.5), gamma_2d ? std::vector<int64_t>{1, D}
                                                               : std::vector<int64_t>{D}, dt);
    Tensor dy = device(normal(R * D, 42 + D), {R, D}, dt);
    xt.set_requires_grad(true);
    gt.set_requires_grad(true);
    Value x = make_tensor(xt, "x"), g = make_tensor(gt, "gamma");
    Value h = rms(x);
    Value y = gamma_first ? g * h : h * g;
    const uint64_t fused_before = debug::fused_rms_mul_vjps();
    backward(y, &dy, parallel);
    const bool fused = debug::fused_rms_mul_vjps() == fused_before + 1;

    agk_stream_t st = reinterpret_cast<agk_stream_t>(current_stream());
    const Tensor& inv = *h.node->tape[0];
    Tensor dr = Tensor::empty({R, D}, dt), dx = Tensor::empty({R, D}, dt);
    Tensor dg = Tensor::empty({D}, Dtype::Float32);
    const size_t wsb = agk_rmsnorm_bwd_workspace_bytes(R, D);
    Tensor ws = Tensor::empty({static_cast<int64_t>(wsb / 4) + 1}, Dtype::Float32);
    const int rc1 = agk_mul_rowbcast_bwd(dy.data(), h.val().data(), g.val().data(), dr.data(),
                                         static_cast<float*>(dg.data()), ws.data(), wsb, R, D,
                                         dtc, 0, st);
    // as vjp_RMSNorm calls it: a workspace for rows of AGK_WIDE_MIN_COLS or more
    const bool wide = D >= AGK_WIDE_MIN_COLS;
    const int rc2 = agk_rmsnorm_bwd(x.val().data(), nullptr, static_cast<const float*>(inv.data()),
                                    dr.data(), dx.data(), nullptr, wide ? ws.data() : nullptr,
                                    wide ? wsb : 0, R, D, dtc, 0, st);
    const bool same = rc1 == AGK_OK && rc2 == AGK_OK && bytes_of(h.grad()) == bytes_of(dr) &&
                      bytes_of(x.grad()) == bytes_of(dx) && bytes_of(g.grad()) == bytes_of(dg);
    report(name, fused && same,
           std::string(fused ? "one pass" : "NOT fused") + (same ? ", bit-identical" : ", DIFFER"));
}

void test_composition_backward() {
    composition_case("rms(x) * gamma backward, one pass == two VJPs (f32 [64,256])", 64, 256,
                     Dtype::Float32, false, false, false);
    composition_case("... parallel backward, gamma * rms(x), gamma [1, D]", 64, 256,
                     Dtype::Float32, true, true, true);
    composition_case("... f32 [300,4096] (several rows per workgroup)", 300, 4096,
                     Dtype::Float32, false, false, false);
    composition_case("... bf16 [96,1024]", 96, 1024, Dtype::BFloat16, false, false, false);
    composition_case("... bf16 [40,8192]", 40, 8192, Dtype::BFloat16, true, false, false);
    composition_case("... f32 [33,250] (looped kernel: rows not a multiple of 16 bytes)", 33, 250,
                     Dtype::Float32, false, false, false);
    composition_case("... bf16 [17,100] (looped kernel)", 17, 100, Dtype::BFloat16, true, false,
                     false);
    composition_case("... f32 [3,40000] (split path for wide rows)", 3, 40000, Dtype::Float32,
                     false, false, false);
    composition_case("... bf16 [300,24576] (one-pass kernel for wide rows)", 300, 24576,
                     Dtype::BFloat16, true, false, false);

    // rms(x) with a second consumer: the one-pass rule must not fire (its
    // gradient is not final when the Mul runs); checked numerically.
    Value x = leaf(normal(24, 43), {4, 6}, "x");
    Value g = leaf(uniform(6, 44, 0.5, 1.5), {6}, "g");
    Tensor dy = Tensor::from_host_f32(normal(24, 45), {4, 6});
    auto f = [&]() {
        Value h = rms(x);
        return ((h * g) * h) * make_tensor(dy);
    };
    const uint64_t before = debug::fused_rms_mul_vjps();
    {
        Value h = rms(x);
        backward((h * g) * h, &dy);
    }
    report("rms(x) used twice: not fused", debug::fused_rms_mul_vjps() == before);
    check_grad("rms(x) used twice: dx numerical gradient", x, f);
    check_grad("rms(x) used twice: dgamma numerical gradient", g, f);

    // Accumulation.  A new graph over the same leaves: the one-pass kernel adds
    // into x's and gamma's gradients (its accumulating variant).
    Value x2 = leaf(normal(64 * 128, 46), {64, 128}, "x2");
    Value g2 = leaf(uniform(128, 47, 0.5, 1.5), {128}, "g2");
    Tensor dy2 = Tensor::from_host_f32(normal(64 * 128, 48), {64, 128});
    Value y2 = rms(x2) * g2;
    backward(y2, &dy2);
    const std::vector<float> dx1 = x2.grad().to_host_f32(), dg1 = g2.grad().to_host_f32();
    const uint64_t f0 = debug::fused_rms_mul_vjps();
    backward(rms(x2) * g2, &dy2);
    const bool fused_again = debug::fused_rms_mul_vjps() == f0 + 1;
    std::vector<float> dxa = x2.grad().to_host_f32(), dga = g2.grad().to_host_f32();
    bool doubled = true;
    for (size_t i = 0; i < dx1.size(); ++i) doubled &= dxa[i] == dx1[i] + dx1[i];
    for (size_t i = 0; i < dg1.size(); ++i) doubled &= dga[i] == dg1[i] + dg1[i];
    report("rms(x) * gamma, a second graph: one pass adds into x and gamma",
           fused_again && doubled);
    // A second backward over the same graph: rms(x)'s gradient from the first
    // is still there, so the Mul's is not its only contribution and the rule
    // stands aside; as in the reference, rms(x)'s VJP then propagates the
    // accumulated 2*dr, so x.grad gains 2*dx1 (exact: scaling by 2) and
    // gamma.grad gains dg1.
    zero_grad(y2);
    backward(y2, &dy2);
    const uint64_t f1 = debug::fused_rms_mul_vjps();
    backward(y2, &dy2);
    const bool stood_aside = debug::fused_rms_mul_vjps() == f1;
    dxa = x2.grad().to_host_f32();
    dga = g2.grad().to_host_f32();
    bool tripled = true;
    for (size_t i = 0; i < dx1.size(); ++i) tripled &= dxa[i] == dx1[i] + 2.0f * dx1[i];
    for (size_t i = 0; i < dg1.size(); ++i) tripled &= dga[i] == dg1[i] + dg1[i];
    report("rms(x) * gamma, the same graph again: rms(x).grad accumulates (reference semantics)",
           stood_aside && tripled);
}

void test_accumulation_and_zero_grad() {
    const int64_t R = 16, D = 64;
    Value x = leaf(normal(R * D, 8), {R, D}, "x");
    Value g = leaf(uniform(D, 9, 0.5, 1.5), {D}, "g");
    Tensor dy = Tensor::from_host_f32(normal(R * D, 10), {R, D});
    Value y = rms_norm(x, g, 1e-5f);
    backward(y, &dy);
    std::vector<float> dx1 = x.grad().to_host_f32(), dg1 = g.grad().to_host_f32();
    backward(y, &dy);  // accumulates (reference Test 21)
    std::vector<float> dx2 = x.grad().to_host_f32(), dg2 = g.grad().to_host_f32();
    bool doubled = true;
    for (size_t i = 0; i < dx1.size(); ++i) doubled &= dx2[i] == dx1[i] + dx1[i];
    for (size_t i = 0; i < dg1.size(); ++i) doubled &= dg2[i] == dg1[i] + dg1[i];
    report("gradients accumulate across backward calls", doubled);
    zero_grad(y);  // reference Test 22
    bool zero = max_abs(x.grad().to_host_f32()) == 0.0 && max_abs(g.grad().to_host_f32()) == 0.0;
    report("zero_grad clears gradients", zero);
    backward(y, &dy);
    report("backward after zero_grad equals the first backward",
           x.grad().to_host_f32() == dx1 && g.grad().to_host_f32() == dg1);
}

void test_parallel_matches_sequential() {
    const int64_t R = 48, D = 512;
    std::vector<float> xv = normal(R * D, 11), dyv = normal(R * D, 12);
    std::vector<float> g1v = uniform(D, 13, 0.5, 1.5), g2v = uniform(D, 14, 0.5, 1.5),
                       g3v = uniform(D, 15, 0.5, 1.5);
    Tensor dy = Tensor::from_host_f32(dyv, {R, D});
    auto run = [&](bool parallel, std::vector<std::vector<float>>& grads) {
        Value x = leaf(xv, {R, D}, "x");
        Value g1 = leaf(g1v, {D}, "g1"), g2 = leaf(g2v, {D}, "g2"), g3 = leaf(g3v, {1, D}, "g3");
        Value h1 = rms_norm(x, g1, 1e-5f);
        Value h2 = rms_norm(h1, g2, 1e-5f);
        Value h3 = rms(h2) * g3;
        Value y = h3 * h1;  // diamond: h1 has two consumers
        backward(y, &dy, parallel);
        grads = {x.grad().to_host_f32(), g1.grad().to_host_f32(), g2.grad().to_host_f32(),
                 g3.grad().to_host_f32()};
    };
    std::vector<std::vector<float>> seq, par;
    run(false, seq);
    run(true, par);
    report("parallel backward == sequential backward (diamond graph, bitwise)", seq == par);
}

void test_weight_tying() {
    Value x = leaf(normal(24, 16), {4, 6}, "x");
    Value g = leaf(uniform(6, 17, 0.5, 1.5), {6}, "g");
    Tensor dy = Tensor::from_host_f32(normal(24, 18), {4, 6});
    auto f = [&]() { return rms_norm(rms_norm(x, g, 1e-2f), g, 1e-2f) * make_tensor(dy); };
    backward(rms_norm(rms_norm(x, g, 1e-2f), g, 1e-2f), &dy);
    check_grad("tied gamma (two layers): dgamma numerical gradient", g, f);
    check_grad("tied gamma (two layers): dx numerical gradient", x, f);
}

void test_module() {
    nn::RMSNorm layer(128, 1e-6f);
    Value x = leaf(normal(8 * 128, 19), {8, 128}, "x");
    Value y = layer(x);
    backward(y);
    std::vector<float> dg = layer.gamma.grad().to_host_f32();
    // gamma = 1 and dy = 1: dgamma = column sums of y
    std::vector<float> yv = y.val().to_host_f32();
    double e = 0.0;
    for (int j = 0; j < 128; ++j) {
        double s = 0.0;
        for (int i = 0; i < 8; ++i) s += yv[i * 128 + j];
        e = std::max(e, std::fabs(s - dg[j]));
    }
    report("nn::RMSNorm: dgamma = column sums of y for a ones seed", e <= 1e-5,
           std::to_string(e));
    layer.zero_grad();
    report("nn::RMSNorm::zero_grad", max_abs(layer.gamma.grad().to_host_f32()) == 0.0);
}

void test_errors() {
    Value x = leaf(normal(32, 20), {4, 8}, "x");
    Value bad = leaf(uniform(7, 21, 0.5, 1.5), {7}, "bad");
    bool threw = false;
    try {
        rms_norm(x, bad);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("rms_norm with a gamma of the wrong width throws", threw);
    threw = false;
    try {
        mul(x, leaf(normal(12, 22), {4, 3}, "y"));
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("mul with shapes that do not broadcast throws", threw);
    threw = false;
    try {
        Tensor seed = Tensor::ones({2, 8});
        backward(rms(x), &seed);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("backward with a seed of the wrong shape throws", threw);
}

// mul under general broadcasting: gradients against numerical gradients (the
// reference pattern) and the tangent against tA * B + A * tB on the host.
void test_broadcast_mul() {
    struct Case {
        std::vector<int64_t> sa, sb, out;
    };
    const Case cases[] = {{{2, 3, 4}, {2, 1, 4}, {2, 3, 4}},
                          {{3, 1}, {1, 5}, {3, 5}},
                          {{2, 3, 4}, {3, 1}, {2, 3, 4}},
                          {{1}, {2, 3}, {2, 3}}};
    uint64_t seed = 80;
    for (const Case& c : cases) {
        auto numel = [](const std::vector<int64_t>& s) {
            int64_t n = 1;
            for (int64_t e : s) n *= e;
            return static_cast<size_t>(n);
        };
        const std::string tag = "[" + std::to_string(c.sa.size()) + "-d]*[" +
                                std::to_string(c.sb.size()) + "-d] -> " +
                                std::to_string(numel(c.out)) + " elements";
        Value a = leaf(normal(numel(c.sa), seed++), c.sa, "a");
        Value b = leaf(normal(numel(c.sb), seed++), c.sb, "b");
        Value w = leaf(normal(numel(c.out), seed++), c.out, "w", false);
        auto f = [&]() { return (a * b) * w; };
        report(("broadcast mul output shape " + tag).c_str(), (a * b).val().shape() == c.out);
        backward(f());
        check_grad(("broadcast mul da == numerical gradient " + tag).c_str(), a, f);
        check_grad(("broadcast mul db == numerical gradient " + tag).c_str(), b, f);
        // forward mode: tA * B + A * tB, on the host by explicit broadcasting
        Tensor ta = Tensor::from_host_f32(normal(numel(c.sa), seed++), c.sa);
        Tensor tb = Tensor::from_host_f32(normal(numel(c.sb), seed++), c.sb);
        Value a2 = leaf(a.val().to_host_f32(), c.sa, "a2"), b2 = leaf(b.val().to_host_f32(), c.sb, "b2");
        std::vector<float> ty = jvp(a2 * b2, {{a2.node.get(), ta}, {b2.node.get(), tb}}).to_host_f32();
        const std::vector<float> av = a.val().to_host_f32(), bv = b.val().to_host_f32(),
                                 tav = ta.to_host_f32(), tbv = tb.to_host_f32();
        const size_t nd = c.out.size();
        auto src = [&](const std::vector<int64_t>& s, const std::vector<int64_t>& idx) {
            size_t off = 0;
            const size_t pad = nd - s.size();
            for (size_t i = pad; i < nd; ++i)
                off = off * s[i - pad] + (s[i - pad] == 1 ? 0 : idx[i]);
            return off;
        };
        double err = 0.0;
        std::vector<int64_t> idx(nd, 0);
        for (size_t o = 0; o < ty.size(); ++o) {
            size_t r = o;
            for (size_t i = nd; i-- > 0;) {
                idx[i] = static_cast<int64_t>(r % c.out[i]);
                r /= c.out[i];
            }
            const size_t ia = src(c.sa, idx), ib = src(c.sb, idx);
            const double t1 = double(tav[ia]) * bv[ib], t2 = double(av[ia]) * tbv[ib];
            // relative to the terms' size: the two may cancel
            err = std::max(err, std::fabs(ty[o] - (t1 + t2)) / (std::fabs(t1) + std::fabs(t2) + 1e-6));
        }
        report(("broadcast mul jvp == tA * B + A * tB " + tag).c_str(), err <= 1e-6,
               std::to_string(err));
    }
}

// matmul on float32 operands (the library sgemm path): gradients against
// numerical gradients, values against a host fp64 product, the tangent
// against tA B + A tB, with sizes that are not multiples of 8.
void test_matmul_f32() {
    const int64_t M = 5, K = 7, N = 3;
    Value a = leaf(normal(M * K, 90), {M, K}, "a");
    Value b = leaf(normal(K * N, 91), {K, N}, "b");
    Value w = leaf(normal(M * N, 92), {M, N}, "w", false);
    auto f = [&]() { return matmul(a, b) * w; };
    const std::vector<float> y = matmul(a, b).val().to_host_f32();
    const std::vector<float> av = a.val().to_host_f32(), bv = b.val().to_host_f32();
    double err = 0.0;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double s = 0.0, mag = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                s += double(av[i * K + k]) * bv[k * N + j];
                mag += std::fabs(double(av[i * K + k]) * bv[k * N + j]);
            }
            err = std::max(err, std::fabs(y[i * N + j] - s) / (mag + 1e-30));
        }
    report("matmul f32 [5,7] x [7,3] == host fp64 product", err <= 1e-6, std::to_string(err));
    report("matmul f32: output is float32",
           matmul(a, b).val().dtype() == Dtype::Float32 &&
               matmul(a, b).val().shape() == std::vector<int64_t>{M, N});
    backward(f());
    report("matmul f32: da and db are float32",
           a.grad().dtype() == Dtype::Float32 && b.grad().dtype() == Dtype::Float32);
    check_grad("matmul f32 da == numerical gradient", a, f);
    check_grad("matmul f32 db == numerical gradient", b, f);
    Tensor ta = Tensor::from_host_f32(normal(M * K, 93), {M, K});
    Tensor tb = Tensor::from_host_f32(normal(K * N, 94), {K, N});
    Value a2 = leaf(av, {M, K}, "a2"), b2 = leaf(bv, {K, N}, "b2");
    const std::vector<float> ty =
        jvp(matmul(a2, b2), {{a2.node.get(), ta}, {b2.node.get(), tb}}).to_host_f32();
    const std::vector<float> tav = ta.to_host_f32(), tbv = tb.to_host_f32();
    double ej = 0.0;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double s = 0.0, mag = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const double t1 = double(tav[i * K + k]) * bv[k * N + j];
                const double t2 = double(av[i * K + k]) * tbv[k * N + j];
                s += t1 + t2;
                mag += std::fabs(t1) + std::fabs(t2);
            }
            ej = std::max(ej, std::fabs(ty[i * N + j] - s) / (mag + 1e-30));
        }
    report("matmul f32 jvp == tA B + A tB", ej <= 1e-6, std::to_string(ej));
    bool threw = false;
    try {
        const std::vector<uint16_t> hb(static_cast<size_t>(M * K), 0x3f80);  // ones
        Value h = make_tensor(Tensor::from_host(hb.data(), {M, K}, Dtype::BFloat16), "h");
        matmul(h, b);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("matmul of bf16 by f32 throws", threw);
}

void test_empty_batch() {
    Value x = make_tensor(Tensor::empty({0, 16}).set_requires_grad(true), "x");
    Value g = leaf(uniform(16, 23, 0.5, 1.5), {16}, "g");
    Value y = rms_norm(x, g);
    backward(y);
    report("empty batch: dgamma is zero", max_abs(g.grad().to_host_f32()) == 0.0 &&
                                              y.val().numel() == 0);
}

void test_bf16_layer() {
    const int64_t R = 32, D = 1024;
    std::vector<float> xv = normal(R * D, 24, 2.0), gv = uniform(D, 25, 0.5, 1.5);
    auto to_bf16 = [](const std::vector<float>& v) {
        std::vector<uint16_t> b(v.size());
        for (size_t i = 0; i < v.size(); ++i) {
            uint32_t u;
            std::memcpy(&u, &v[i], 4);
            u += 0x7fffu + ((u >> 16) & 1u);
            b[i] = static_cast<uint16_t>(u >> 16);
        }
        return b;
    };
    std::vector<uint16_t> xb = to_bf16(xv), gb = to_bf16(gv);
    Tensor xt = Tensor::from_host(xb.data(), {R, D}, Dtype::BFloat16);
    Tensor gt = Tensor::from_host(gb.data(), {D}, Dtype::BFloat16);
    xt.set_requires_grad(true);
    gt.set_requires_grad(true);
    Value x1 = make_tensor(xt, "x"), g1 = make_tensor(gt, "g");
    Value y1 = rms_norm(x1, g1, 1e-5f);
    backward(y1);
    Tensor xt2 = Tensor::from_host(xb.data(), {R, D}, Dtype::BFloat16);
    Tensor gt2 = Tensor::from_host(gb.data(), {D}, Dtype::BFloat16);
    xt2.set_requires_grad(true);
    gt2.set_requires_grad(true);
    Value x2 = make_tensor(xt2, "x2"), g2 = make_tensor(gt2, "g2");
    Value y2 = rms(x2) * g2;
    backward(y2);
    const double ey = max_abs_diff(y1.val().to_host_f32(), y2.val().to_host_f32()) /
                      max_abs(y2.val().to_host_f32());
    const double eg = max_abs_diff(g1.grad().to_host_f32(), g2.grad().to_host_f32()) /
                      max_abs(g2.grad().to_host_f32());
    report("bf16: rms_norm == rms * gamma (1e-2), dgamma is fp32",
           ey <= 1e-2 && eg <= 1e-2 && g1.grad().dtype() == Dtype::Float32,
           "y " + std::to_string(ey) + " dgamma " + std::to_string(eg));
}

void test_seed_not_modified() {
    const int64_t R = 8, D = 32;
    Value x = leaf(normal(R * D, 26), {R, D}, "x");
    Tensor seed = Tensor::from_host_f32(normal(R * D, 27), {R, D});
    std::vector<float> seed_before = seed.to_host_f32();
    backward(x, &seed);  // the root is the leaf: its gradient is the seed
    Value g = leaf(uniform(D, 28, 0.5, 1.5), {D}, "g");
    backward(rms_norm(x, g), &seed);  // adds into x's gradient
    report("a seed shared as a root gradient is copied before accumulation",
           seed.to_host_f32() == seed_before);
}

void test_user_stream() {
    const int64_t R = 64, D = 1024;
    std::vector<float> xv = normal(R * D, 29), gv = uniform(D, 30, 0.5, 1.5);
    std::vector<float> ref_dx, ref_dg;
    {
        Value x = leaf(xv, {R, D}, "x"), g = leaf(gv, {D}, "g");
        backward(rms_norm(x, g));
        ref_dx = x.grad().to_host_f32();
        ref_dg = g.grad().to_host_f32();
    }
    hipStream_t s;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        report("user stream", false, "hipStreamCreate failed");
        return;
    }
    {
        StreamGuard guard(s);
        Value x = leaf(xv, {R, D}, "x"), g = leaf(gv, {D}, "g");
        backward(rms_norm(x, g), nullptr, true);
        report("layer on a user stream (parallel backward) == null stream",
               x.grad().to_host_f32() == ref_dx && g.grad().to_host_f32() == ref_dg);
    }
    (void)hipStreamSynchronize(s);
    release_stream_cache(s);  // before the handle dies (a new stream may reuse it)
    (void)hipStreamDestroy(s);
}


// ---- matmul, the row ops beside RMSNorm, forward mode, graph capture ----------

float bf16_round(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    std::memcpy(&f, &u, 4);
    return f;
}

Value bf16_leaf(const std::vector<float>& v, const std::vector<int64_t>& shape, const char* name,
                bool req = true) {
    std::vector<uint16_t> b = to_bf16_bits(v);
    Tensor t = Tensor::from_host(b.data(), shape, Dtype::BFloat16);
    t.set_requires_grad(req);
    return make_tensor(t, name);
}

// A broadcast operand's gradient is fp32 (summed over the broadcast axes),
// while an operand that covers a product's output gets its gradient in its own
// dtype.  A bf16 node that receives both kinds cannot add them: backward
// throws (a documented restriction), naming the gradient that did not match.
void test_bf16_mixed_gradient_dtypes() {
    const int64_t B = 2, T = 3, D = 8;
    Value x = bf16_leaf(normal(B * T * D, 95), {B, T, D}, "x");
    Value s = bf16_leaf(normal(B * D, 96), {B, 1, D}, "s");
    bool threw = false;
    std::string what;
    try {
        Value root = (x * s) * (s * s);  // s: fp32 from the first product, bf16 from s * s
        backward(root);
    } catch (const std::runtime_error& e) {
        threw = true;
        what = e.what();
    }
    report("bf16 node with fp32 and bf16 gradient contributions: backward throws", threw &&
           (what.find("gradient") != std::string::npos), what);
    // the same graph in fp32 has one gradient dtype throughout and runs
    Value xf = leaf(normal(B * T * D, 95), {B, T, D}, "xf");
    Value sf = leaf(normal(B * D, 96), {B, 1, D}, "sf");
    bool ran = true;
    try {
        backward((xf * sf) * (sf * sf));
    } catch (const std::runtime_error& e) {
        ran = false;
        what = e.what();
    }
    report("the same graph in fp32 runs", ran && sf.grad().dtype() == Dtype::Float32, what);
}

// Scalar literals (Value(float), as cgadimpl/include/ad/core/graph.hpp:22 and
// cgadimpl/src/core/graph.cpp:91-105): `rms(x) * s` and `s * rms(x)` compile,
// give rms(x) scaled by s, and differentiate to the rms VJP of s * dy.  The
// reference products are taken on the host in the same IEEE arithmetic, so
// the comparisons are bitwise.
void test_scalar_literal() {
    const int64_t R = 37, D = 1030;
    const std::vector<float> xv = normal(R * D, 97), dyv = normal(R * D, 98);
    Tensor dy = Tensor::from_host_f32(dyv, {R, D});
    for (const float sc : {0.75f, -1.5f}) {
        Value xa = leaf(xv, {R, D}, "xa");
        Value ya = rms(xa) * sc;  // float converts to a scalar literal
        backward(ya, &dy);
        Value xb = leaf(xv, {R, D}, "xb");
        Value yb = sc * rms(xb);  // the literal first
        backward(yb, &dy);
        Value xr = leaf(xv, {R, D}, "xr");
        Value yr = rms(xr);
        std::vector<float> dys = dyv;
        for (float& v : dys) v *= sc;
        Tensor dy_scaled = Tensor::from_host_f32(dys, {R, D});
        backward(yr, &dy_scaled);
        std::vector<float> want_y = yr.val().to_host_f32();
        for (float& v : want_y) v *= sc;
        const std::vector<float> want_dx = xr.grad().to_host_f32();
        const std::string tag = " (s = " + std::to_string(sc) + ")";
        report(("rms(x) * s == s * rms(x) == rms(x) scaled, dx == rms VJP of s * dy" + tag).c_str(),
               ya.val().to_host_f32() == want_y && yb.val().to_host_f32() == want_y &&
                   xa.grad().to_host_f32() == want_dx && xb.grad().to_host_f32() == want_dx);
    }
    // a literal is a [1] fp32 leaf that takes no gradient
    Value lit(0.5f);
    report("Value(float) is a [1] float32 leaf named scalar_literal, no gradient",
           lit.shape() == std::vector<int64_t>{1} && lit.val().dtype() == Dtype::Float32 &&
               !lit.node->requires_grad() && std::string(lit.node->debug_name) == "scalar_literal" &&
               lit.val().to_host_f32() == std::vector<float>{0.5f});
    // bf16: the literal is taken in bf16 (0.75 is exact), the product rounded
    Value xh = bf16_leaf(xv, {R, D}, "xh");
    Value yh = rms(xh) * 0.75f;
    Value xh2 = bf16_leaf(xv, {R, D}, "xh2");
    std::vector<float> want = rms(xh2).val().to_host_f32();
    for (float& v : want) v = bf16_round(v * 0.75f);
    report("bf16 rms(x) * 0.75f: the literal in bf16, the product rounded",
           yh.val().dtype() == Dtype::BFloat16 && yh.val().to_host_f32() == want &&
               lit.val().dtype() == Dtype::Float32);
}

std::vector<float> rounded(const std::vector<float>& v) {
    std::vector<float> o(v.size());
    for (size_t i = 0; i < v.size(); ++i) o[i] = bf16_round(v[i]);
    return o;
}

double rel_err(const std::vector<float>& got, const std::vector<double>& ref) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < ref.size(); ++i) {
        num = std::max(num, std::fabs(double(got[i]) - ref[i]));
        den = std::max(den, std::fabs(ref[i]));
    }
    return den > 0 ? num / den : num;
}

// host fp64 restatements, row-major [R, D]
using Vec = std::vector<double>;
Vec to_d(const std::vector<float>& v) { return Vec(v.begin(), v.end()); }

Vec host_rms_layer(const Vec& x, const Vec* g, int64_t R, int64_t D, double eps) {
    Vec y(x.size());
    for (int64_t i = 0; i < R; ++i) {
        double ss = 0.0;
        for (int64_t j = 0; j < D; ++j) ss += x[i * D + j] * x[i * D + j];
        const double r = 1.0 / std::sqrt(ss / D + eps);
        for (int64_t j = 0; j < D; ++j) y[i * D + j] = x[i * D + j] * r * (g ? (*g)[j] : 1.0);
    }
    return y;
}

Vec host_laynor(const Vec& x, int64_t R, int64_t D, double eps = 1e-5) {
    Vec y(x.size());
    for (int64_t i = 0; i < R; ++i) {
        double m = 0.0, v = 0.0;
        for (int64_t j = 0; j < D; ++j) m += x[i * D + j];
        m /= D;
        for (int64_t j = 0; j < D; ++j) v += (x[i * D + j] - m) * (x[i * D + j] - m);
        v /= D;
        for (int64_t j = 0; j < D; ++j) y[i * D + j] = (x[i * D + j] - m) / std::sqrt(v + eps);
    }
    return y;
}

Vec host_softmax(const Vec& z, int64_t R, int64_t D) {
    Vec y(z.size());
    for (int64_t i = 0; i < R; ++i) {
        double m = -INFINITY, s = 0.0;
        for (int64_t j = 0; j < D; ++j) m = std::max(m, z[i * D + j]);
        for (int64_t j = 0; j < D; ++j) s += std::exp(z[i * D + j] - m);
        for (int64_t j = 0; j < D; ++j) y[i * D + j] = std::exp(z[i * D + j] - m) / s;
    }
    return y;
}

Vec host_lse(const Vec& z, int64_t R, int64_t D) {
    Vec y(R);
    for (int64_t i = 0; i < R; ++i) {
        double m = -INFINITY, s = 0.0;
        for (int64_t j = 0; j < D; ++j) m = std::max(m, z[i * D + j]);
        for (int64_t j = 0; j < D; ++j) s += std::exp(z[i * D + j] - m);
        y[i] = std::log(s) + m;
    }
    return y;
}

Vec axpy(const Vec& x, const Vec& t, double h) {
    Vec o(x.size());
    for (size_t i = 0; i < x.size(); ++i) o[i] = x[i] + h * t[i];
    return o;
}

Vec central(const std::function<Vec(double)>& f, double h = 1e-4) {
    Vec p = f(h), m = f(-h), o(p.size());
    for (size_t i = 0; i < p.size(); ++i) o[i] = (p[i] - m[i]) / (2 * h);
    return o;
}

// softmax_row on rows too wide for one workgroup (the row ops' team kernel,
// whose exchange workspace the graph layer takes from its pool): forward and
// VJP against a host double-precision softmax, aligned rows and rows that
// start off a 16-byte boundary (50257 columns).
void test_wide_softmax() {
    for (int64_t D : {int64_t{40000}, int64_t{50257}}) {
        const int64_t R = 3;
        Vec zd = to_d(normal(R * D, 70 + D));
        for (double& v : zd) v *= 4.0;
        std::vector<float> zf(zd.begin(), zd.end());
        zd.assign(zf.begin(), zf.end());  // the values the device holds
        Value z = leaf(zf, {R, D}, "z");
        std::vector<float> gf = normal(R * D, 71 + D);
        Tensor gy = Tensor::from_host_f32(gf, {R, D});
        Value y = softmax_row(z);
        backward(y, &gy);
        const Vec ys = host_softmax(zd, R, D);
        Vec dz(ys.size());
        for (int64_t i = 0; i < R; ++i) {
            double dot = 0.0;
            for (int64_t j = 0; j < D; ++j) dot += ys[i * D + j] * gf[i * D + j];
            for (int64_t j = 0; j < D; ++j) dz[i * D + j] = ys[i * D + j] * (gf[i * D + j] - dot);
        }
        const double ey = rel_err(y.val().to_host_f32(), ys);
        const double ed = rel_err(z.grad().to_host_f32(), dz);
        const std::string tag = "softmax_row [3," + std::to_string(D) + "] (team kernel)";
        report((tag + " forward == host").c_str(), ey <= 1e-5, std::to_string(ey));
        report((tag + " VJP == host").c_str(), ed <= 1e-5, std::to_string(ed));
    }
}

// rms_norm and rms on rows too wide for one workgroup: the forward's team
// kernel (x read once, its exchange workspace from the graph layer's pool)
// and the backward's, against host double precision.
void test_wide_rms() {
    for (int64_t D : {int64_t{40000}, int64_t{70000}}) {
        const int64_t R = 5;
        const double eps = 1e-5;
        std::vector<float> xf = normal(R * D, 80 + D), gf = uniform(D, 81 + D, 0.5, 1.5),
                           dyf = normal(R * D, 82 + D);
        const Vec xd = to_d(xf), gd = to_d(gf);
        Value x = leaf(xf, {R, D}, "x"), g = leaf(gf, {D}, "g");
        Tensor dy = Tensor::from_host_f32(dyf, {R, D});
        Value y = rms_norm(x, g, 1e-5f);
        backward(y, &dy);
        Value x2 = leaf(xf, {R, D}, "x2");
        Value h = rms(x2);
        const Vec ys = host_rms_layer(xd, &gd, R, D, eps), hs = host_rms_layer(xd, nullptr, R, D, eps);
        Vec dx(R * D), dg(D, 0.0);
        for (int64_t i = 0; i < R; ++i) {
            double ss = 0.0, dot = 0.0;
            for (int64_t j = 0; j < D; ++j) ss += xd[i * D + j] * xd[i * D + j];
            const double r = 1.0 / std::sqrt(ss / D + eps);
            for (int64_t j = 0; j < D; ++j) dot += dyf[i * D + j] * gd[j] * xd[i * D + j];
            for (int64_t j = 0; j < D; ++j) {
                dx[i * D + j] = r * (dyf[i * D + j] * gd[j] - xd[i * D + j] * r * r * dot / D);
                dg[j] += dyf[i * D + j] * xd[i * D + j] * r;
            }
        }
        const std::string tag = "rms_norm [5," + std::to_string(D) + "] (team kernels)";
        const double ey = rel_err(y.val().to_host_f32(), ys), eh = rel_err(h.val().to_host_f32(), hs);
        const double ex = rel_err(x.grad().to_host_f32(), dx), eg = rel_err(g.grad().to_host_f32(), dg);
        report((tag + " forward == host").c_str(), ey <= 1e-5, std::to_string(ey));
        report(("rms [5," + std::to_string(D) + "] forward == host").c_str(), eh <= 1e-5,
               std::to_string(eh));
        report((tag + " dx == host").c_str(), ex <= 1e-5, std::to_string(ex));
        report((tag + " dgamma == host").c_str(), eg <= 1e-5, std::to_string(eg));
    }
}

void test_row_ops_gradients() {
    // the reference pattern: [4,10] input, numerical gradient of sum(f(a))
    Value a = leaf(normal(40, 60), {4, 10}, "a");
    auto fl = [&]() { return laynor(a); };
    Tensor dy = Tensor::from_host_f32(normal(40, 61), {4, 10});
    Value w = leaf(dy.to_host_f32(), {4, 10}, "w", false);
    auto fw = [&]() { return laynor(a) * w; };
    backward(fl(), &dy);
    check_grad("laynor [4,10] numerical gradient", a, fw);
    zero_grad(fl());
    auto fs = [&]() { return softmax_row(a) * w; };
    backward(softmax_row(a), &dy);
    check_grad("softmax_row [4,10] numerical gradient", a, fs);
    zero_grad(fs());
    auto fz = [&]() { return logsumexp_row(a); };
    backward(fz());
    check_grad("logsumexp_row [4,10] numerical gradient", a, fz);
    report("logsumexp_row output shape [4,1]",
           fz().val().shape() == std::vector<int64_t>{4, 1});
}

void test_jvp() {
    const int64_t R = 5, D = 24;
    const double eps = 1e-5;
    std::vector<float> xv = normal(R * D, 70), gv = uniform(D, 71, 0.5, 1.5),
                       txv = normal(R * D, 72), tgv = normal(D, 73);
    const Vec xd = to_d(xv), gd = to_d(gv), txd = to_d(txv), tgd = to_d(tgv);
    Tensor tx = Tensor::from_host_f32(txv, {R, D}), tg = Tensor::from_host_f32(tgv, {D});

    Value x = leaf(xv, {R, D}, "x"), g = leaf(gv, {D}, "g");
    Tensor ty = jvp(rms_norm(x, g, 1e-5f), {{x.node.get(), tx}, {g.node.get(), tg}});
    Vec fd = central([&](double h) {
        Vec gh = axpy(gd, tgd, h);
        return host_rms_layer(axpy(xd, txd, h), &gh, R, D, eps);
    });
    const double e1 = rel_err(ty.to_host_f32(), fd);
    report("jvp rms_norm(x, g) along (tx, tg) == central differences", e1 <= 1e-4,
           std::to_string(e1));

    Value x2 = leaf(xv, {R, D}, "x2"), g2 = leaf(gv, {1, D}, "g2");
    Tensor tg2 = Tensor::from_host_f32(tgv, {1, D});
    Tensor ty2 = jvp(rms(x2) * g2, {{x2.node.get(), tx}, {g2.node.get(), tg2}});
    const double e2 = rel_err(ty2.to_host_f32(), to_d(ty.to_host_f32()));
    report("jvp rms(x) * g == jvp rms_norm(x, g)", e2 <= 1e-5, std::to_string(e2));

    Value x3 = leaf(xv, {R, D}, "x3");
    const double e3 = rel_err(jvp(rms(x3), {{x3.node.get(), tx}}).to_host_f32(),
                              central([&](double h) {
                                  return host_rms_layer(axpy(xd, txd, h), nullptr, R, D, eps);
                              }));
    report("jvp rms(x) (the corrected rule) == central differences", e3 <= 1e-4,
           std::to_string(e3));

    Value x4 = leaf(xv, {R, D}, "x4");
    const double e4 = rel_err(jvp(laynor(x4), {{x4.node.get(), tx}}).to_host_f32(),
                              central([&](double h) { return host_laynor(axpy(xd, txd, h), R, D); }));
    report("jvp laynor == central differences", e4 <= 1e-4, std::to_string(e4));

    Value x5 = leaf(xv, {R, D}, "x5");
    const double e5 = rel_err(jvp(softmax_row(x5), {{x5.node.get(), tx}}).to_host_f32(),
                              central([&](double h) { return host_softmax(axpy(xd, txd, h), R, D); }));
    report("jvp softmax_row == central differences", e5 <= 1e-4, std::to_string(e5));

    Value x6 = leaf(xv, {R, D}, "x6");
    const double e6 = rel_err(jvp(logsumexp_row(x6), {{x6.node.get(), tx}}).to_host_f32(),
                              central([&](double h) { return host_lse(axpy(xd, txd, h), R, D); }));
    report("jvp logsumexp_row == central differences", e6 <= 1e-4, std::to_string(e6));

    // a composition: softmax_row(laynor(rms_norm(x, g))) along tx only
    Value x7 = leaf(xv, {R, D}, "x7"), g7 = leaf(gv, {D}, "g7");
    Tensor ty7 = jvp(softmax_row(laynor(rms_norm(x7, g7, 1e-5f))), {{x7.node.get(), tx}});
    const double e7 = rel_err(ty7.to_host_f32(), central([&](double h) {
        return host_softmax(host_laynor(host_rms_layer(axpy(xd, txd, h), &gd, R, D, eps), R, D),
                            R, D);
    }));
    report("jvp of softmax_row(laynor(rms_norm(x, g))) == central differences", e7 <= 1e-4,
           std::to_string(e7));

    // a seed that does not reach the root gives a zero tangent
    Value x8 = leaf(xv, {R, D}, "x8"), other = leaf(xv, {R, D}, "other");
    report("jvp without a seed on the path is zero",
           max_abs(jvp(rms(x8), {{other.node.get(), tx}}).to_host_f32()) == 0.0);
}

void test_matmul_layer() {
    const int64_t M = 64, K = 128, N = 96;
    const double eps = 1e-5;
    std::vector<float> xv = rounded(normal(M * K, 80)), gv = rounded(uniform(K, 81, 0.5, 1.5)),
                       wv = rounded(normal(K * N, 82, 0.05)), dyv = rounded(normal(M * N, 83));
    std::vector<uint16_t> dyb = to_bf16_bits(dyv);
    Tensor dy = Tensor::from_host(dyb.data(), {M, N}, Dtype::BFloat16);
    auto run = [&](bool parallel, std::vector<std::vector<float>>& out) {
        Value x = bf16_leaf(xv, {M, K}, "x"), g = bf16_leaf(gv, {K}, "g"),
              W = bf16_leaf(wv, {K, N}, "W");
        Value y = matmul(rms_norm(x, g, 1e-5f), W);
        backward(y, &dy, parallel);
        out = {y.val().to_host_f32(), x.grad().to_host_f32(), g.grad().to_host_f32(),
               W.grad().to_host_f32()};
        report("matmul: dx bf16, dgamma and dW fp32",
               x.grad().dtype() == Dtype::BFloat16 && g.grad().dtype() == Dtype::Float32 &&
                   W.grad().dtype() == Dtype::Float32);
    };
    std::vector<std::vector<float>> seq, par;
    run(false, seq);
    run(true, par);
    report("matmul(rms_norm(x, g), W): parallel backward == sequential (bitwise)", seq == par);
    // host fp64 reference with bf16 rounding where the graph stores bf16 (h, dh)
    Vec h(M * K), y(M * N, 0.0), dh(M * K, 0.0), dW(K * N, 0.0), dx(M * K), dg(K, 0.0);
    std::vector<double> r(M);
    for (int64_t i = 0; i < M; ++i) {
        double ss = 0.0;
        for (int64_t k = 0; k < K; ++k) ss += double(xv[i * K + k]) * xv[i * K + k];
        r[i] = 1.0 / std::sqrt(ss / K + eps);
        for (int64_t k = 0; k < K; ++k) h[i * K + k] = bf16_round(float(xv[i * K + k] * r[i] * gv[k]));
    }
    for (int64_t i = 0; i < M; ++i)
        for (int64_t k = 0; k < K; ++k)
            for (int64_t j = 0; j < N; ++j) {
                y[i * N + j] += h[i * K + k] * wv[k * N + j];
                dh[i * K + k] += double(dyv[i * N + j]) * wv[k * N + j];
                dW[k * N + j] += h[i * K + k] * dyv[i * N + j];
            }
    for (auto& v : dh) v = bf16_round(float(v));
    for (int64_t i = 0; i < M; ++i) {
        double dot = 0.0;
        for (int64_t k = 0; k < K; ++k) dot += dh[i * K + k] * gv[k] * xv[i * K + k];
        for (int64_t k = 0; k < K; ++k) {
            const double gk = dh[i * K + k] * gv[k];
            dx[i * K + k] = r[i] * (gk - xv[i * K + k] * r[i] * r[i] * dot / K);
            dg[k] += dh[i * K + k] * xv[i * K + k] * r[i];
        }
    }
    const double ey = rel_err(seq[0], y), ex = rel_err(seq[1], dx), eg = rel_err(seq[2], dg),
                 ew = rel_err(seq[3], dW);
    report("matmul(rms_norm(x, g), W) vs host fp64 (y, dx, dgamma, dW)",
           ey <= 1e-2 && ex <= 3e-2 && eg <= 1e-2 && ew <= 1e-2,
           "y " + std::to_string(ey) + " dx " + std::to_string(ex) + " dgamma " +
               std::to_string(eg) + " dW " + std::to_string(ew));
    // forward mode through the product: tangent of W only
    Value x = bf16_leaf(xv, {M, K}, "x"), W = bf16_leaf(wv, {K, N}, "W");
    std::vector<float> twv = rounded(normal(K * N, 84, 0.05));
    std::vector<uint16_t> twb = to_bf16_bits(twv);
    Tensor tw = Tensor::from_host(twb.data(), {K, N}, Dtype::BFloat16);
    Tensor ty = jvp(matmul(x, W), {{W.node.get(), tw}});
    Vec tref(M * N, 0.0);
    for (int64_t i = 0; i < M; ++i)
        for (int64_t k = 0; k < K; ++k)
            for (int64_t j = 0; j < N; ++j) tref[i * N + j] += double(xv[i * K + k]) * twv[k * N + j];
    const double et = rel_err(ty.to_host_f32(), tref);
    report("jvp matmul(x, W) along tW == x tW", et <= 1e-2, std::to_string(et));

    bool threw = false;
    try {
        matmul(bf16_leaf(normal(64, 85), {8, 8}, "bf16a"), leaf(normal(64, 86), {8, 8}, "f32b"));
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("matmul of a bf16 by an fp32 operand throws", threw);
    threw = false;
    try {
        matmul(bf16_leaf(normal(64, 87), {8, 8}, "a"), bf16_leaf(normal(128, 88), {16, 8}, "b"));
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("matmul with mismatched inner dimensions throws", threw);
}

// A captured forward + backward, replayed on changed inputs with eager work in
// between, against eager runs of the same graph.
// linear(x, w, b) = x w^T + b (the reference's Linear test shapes, x [16, 32],
// w [8, 32] (out, in), b [1, 8], and a wider one), in bf16: forward, the
// three gradients and forward mode against host fp64 with the graph's bf16
// roundings; sequential against parallel backward bitwise; errors.
void test_linear_layer() {
    for (const auto& shape :
         {std::tuple<int64_t, int64_t, int64_t>{16, 32, 8}, {96, 136, 200}}) {
        const int64_t M = std::get<0>(shape), K = std::get<1>(shape), N = std::get<2>(shape);
        const std::string tag = "[" + std::to_string(M) + "," + std::to_string(K) + "] x [" +
                                std::to_string(N) + "," + std::to_string(K) + "]^T";
        std::vector<float> xv = rounded(normal(M * K, 90 + K)), wv = rounded(normal(N * K, 91 + K, 0.2)),
                           bv = rounded(normal(N, 92 + K)), dyv = rounded(normal(M * N, 93 + K));
        std::vector<uint16_t> dyb = to_bf16_bits(dyv);
        Tensor dy = Tensor::from_host(dyb.data(), {M, N}, Dtype::BFloat16);
        auto run = [&](bool parallel, std::vector<std::vector<float>>& out) {
            Value x = bf16_leaf(xv, {M, K}, "x"), w = bf16_leaf(wv, {N, K}, "w"),
                  b = bf16_leaf(bv, {1, N}, "b");
            Value y = linear(x, w, b);
            backward(y, &dy, parallel);
            out = {y.val().to_host_f32(), x.grad().to_host_f32(), w.grad().to_host_f32(),
                   b.grad().to_host_f32()};
            report(("linear " + tag + ": dx bf16, dw and db fp32").c_str(),
                   x.grad().dtype() == Dtype::BFloat16 && w.grad().dtype() == Dtype::Float32 &&
                       b.grad().dtype() == Dtype::Float32 && b.grad().shape() == b.val().shape());
        };
        std::vector<std::vector<float>> seq, par;
        run(false, seq);
        run(true, par);
        report(("linear " + tag + ": parallel backward == sequential (bitwise)").c_str(),
               seq == par);
        Vec y(M * N, 0.0), dx(M * K, 0.0), dw(N * K, 0.0), db(N, 0.0);
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = 0; j < N; ++j) {
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) {
                    acc += double(xv[i * K + k]) * wv[j * K + k];
                    dx[i * K + k] += double(dyv[i * N + j]) * wv[j * K + k];
                    dw[j * K + k] += double(dyv[i * N + j]) * xv[i * K + k];
                }
                // the product rounded to bf16, then the bf16 sum with b
                y[i * N + j] = bf16_round(bf16_round(float(acc)) + bv[j]);
                db[j] += dyv[i * N + j];
            }
        const double ey = rel_err(seq[0], y), ex = rel_err(seq[1], dx), ew = rel_err(seq[2], dw),
                     eb = rel_err(seq[3], db);
        report(("linear " + tag + " vs host fp64 (y, dx, dw, db)").c_str(),
               ey <= 1e-2 && ex <= 1e-2 && ew <= 1e-5 && eb <= 1e-6,
               "y " + std::to_string(ey) + " dx " + std::to_string(ex) + " dw " +
                   std::to_string(ew) + " db " + std::to_string(eb));

        // forward mode along (tx, tw, tb), each alone and all together
        std::vector<float> txv = rounded(normal(M * K, 94 + K)), twv = rounded(normal(N * K, 95 + K, 0.2)),
                           tbv = rounded(normal(N, 96 + K));
        std::vector<uint16_t> txb = to_bf16_bits(txv), twb = to_bf16_bits(twv), tbb = to_bf16_bits(tbv);
        Tensor tx = Tensor::from_host(txb.data(), {M, K}, Dtype::BFloat16);
        Tensor tw = Tensor::from_host(twb.data(), {N, K}, Dtype::BFloat16);
        Tensor tb = Tensor::from_host(tbb.data(), {1, N}, Dtype::BFloat16);
        for (int mask = 1; mask < 8; ++mask) {
            Value x = bf16_leaf(xv, {M, K}, "x"), w = bf16_leaf(wv, {N, K}, "w"),
                  b = bf16_leaf(bv, {1, N}, "b");
            std::unordered_map<Node*, Tensor> seed;
            if (mask & 1) seed[x.node.get()] = tx;
            if (mask & 2) seed[w.node.get()] = tw;
            if (mask & 4) seed[b.node.get()] = tb;
            Tensor ty = jvp(linear(x, w, b), seed);
            Vec ref(M * N, 0.0);
            for (int64_t i = 0; i < M; ++i)
                for (int64_t j = 0; j < N; ++j) {
                    double v = (mask & 4) ? tbv[j] : 0.0;
                    for (int64_t k = 0; k < K; ++k) {
                        if (mask & 1) v += double(txv[i * K + k]) * wv[j * K + k];
                        if (mask & 2) v += double(xv[i * K + k]) * twv[j * K + k];
                    }
                    ref[i * N + j] = v;
                }
            const double et = rel_err(ty.to_host_f32(), ref);
            report(("jvp linear " + tag + " along" + ((mask & 1) ? " tx" : "") +
                    ((mask & 2) ? " tw" : "") + ((mask & 4) ? " tb" : ""))
                       .c_str(),
                   et <= 1e-2, std::to_string(et));
        }
    }
    bool threw = false;
    try {
        linear(leaf(normal(64, 97), {8, 8}, "x32"), leaf(normal(64, 98), {8, 8}, "w32"),
               leaf(normal(8, 99), {8}, "b32"));
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("linear of fp32 operands throws", threw);
    threw = false;
    try {
        linear(bf16_leaf(normal(64, 100), {8, 8}, "x"), bf16_leaf(normal(128, 101), {8, 16}, "w"),
               bf16_leaf(normal(8, 102), {8}, "b"));
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("linear with mismatched input widths throws", threw);
    threw = false;
    try {
        linear(bf16_leaf(normal(64, 103), {8, 8}, "x"), bf16_leaf(normal(64, 104), {8, 8}, "w"),
               bf16_leaf(normal(16, 105), {16}, "b"));
    } catch (const std::runtime_error&) {
        threw = true;
    }
    report("linear with a bias of the wrong width throws", threw);

    // an empty batch: y is empty, dw = 0 (the GEMM's empty reduction) and db = 0
    {
        Tensor xe = Tensor::empty({0, 32}, Dtype::BFloat16);
        xe.set_requires_grad(true);
        Value x = make_tensor(xe, "x0"), w = bf16_leaf(normal(8 * 32, 106), {8, 32}, "w0"),
              b = bf16_leaf(normal(8, 107), {8}, "b0");
        Value y = linear(x, w, b);
        Tensor seed = Tensor::empty({0, 8}, Dtype::BFloat16);
        backward(y, &seed);
        report("linear on an empty batch: dw and db are zero",
               y.val().numel() == 0 && max_abs(w.grad().to_host_f32()) == 0.0 &&
                   max_abs(b.grad().to_host_f32()) == 0.0 &&
                   w.grad().dtype() == Dtype::Float32);
    }
}

// matmul with an empty dimension: the forward gives an empty or zero result and
// the backward leaves the gradients at the GEMM's empty-sum values (zero), as
// the reference's matmul of empty tensors does.
void test_matmul_empty() {
    {  // empty batch: y [0, 16]; dB = A^T gy is an empty sum, so zero
        Tensor ae = Tensor::empty({0, 32}, Dtype::BFloat16);
        ae.set_requires_grad(true);
        Value a = make_tensor(ae, "a0"), b = bf16_leaf(normal(32 * 16, 108), {32, 16}, "b0");
        Value y = matmul(a, b);
        Tensor seed = Tensor::empty({0, 16}, Dtype::BFloat16);
        backward(y, &seed);
        report("matmul on an empty batch: dB is zero",
               y.val().numel() == 0 && max_abs(b.grad().to_host_f32()) == 0.0 &&
                   b.grad().dtype() == Dtype::Float32 && a.grad().numel() == 0);
    }
    {  // K == 0: y = 0 [8, 16]; dA and dB are empty
        Tensor ae = Tensor::empty({8, 0}, Dtype::BFloat16), be = Tensor::empty({0, 16}, Dtype::BFloat16);
        ae.set_requires_grad(true);
        be.set_requires_grad(true);
        Value a = make_tensor(ae, "a1"), b = make_tensor(be, "b1");
        Value y = matmul(a, b);
        std::vector<uint16_t> sb = to_bf16_bits(rounded(normal(8 * 16, 109)));
        Tensor seed = Tensor::from_host(sb.data(), {8, 16}, Dtype::BFloat16);
        backward(y, &seed);
        const double ymax = max_abs(y.val().to_host_f32());
        report("matmul with an empty reduction: y is zero, dA and dB are empty",
               y.val().numel() == 128 && ymax == 0.0 && a.grad().numel() == 0 &&
                   b.grad().numel() == 0,
               "y numel " + std::to_string(y.val().numel()) + " max|y| " + std::to_string(ymax) +
                   ", dA numel " + std::to_string(a.grad().numel()) + ", dB numel " +
                   std::to_string(b.grad().numel()));
    }
    {  // linear with K == 0: y = the bias in every row; db = column sums of gy
        Tensor xe = Tensor::empty({8, 0}, Dtype::BFloat16), we = Tensor::empty({16, 0}, Dtype::BFloat16);
        xe.set_requires_grad(true);
        we.set_requires_grad(true);
        const std::vector<float> bvals = rounded(normal(16, 111));
        Value x = make_tensor(xe, "x3"), w = make_tensor(we, "w3"), b = bf16_leaf(bvals, {16}, "b3");
        Value y = linear(x, w, b);
        const std::vector<float> gv = rounded(normal(8 * 16, 112));
        std::vector<uint16_t> sb = to_bf16_bits(gv);
        Tensor seed = Tensor::from_host(sb.data(), {8, 16}, Dtype::BFloat16);
        backward(y, &seed);
        const std::vector<float> yv = y.val().to_host_f32(), db = b.grad().to_host_f32();
        double ey = 0.0, eb = 0.0;
        for (int64_t j = 0; j < 16; ++j) {
            double s = 0.0;
            for (int64_t i = 0; i < 8; ++i) {
                ey = std::max(ey, std::fabs(double(yv[i * 16 + j]) - bvals[j]));
                s += gv[i * 16 + j];
            }
            eb = std::max(eb, std::fabs(db[j] - s));
        }
        report("linear with an empty reduction: y is the bias rows, db the column sums of gy",
               ey == 0.0 && eb <= 1e-5 && x.grad().numel() == 0 && w.grad().numel() == 0,
               "max |y - b| " + std::to_string(ey) + ", max |db - sum gy| " + std::to_string(eb));
    }
    {  // N == 0: y [8, 0]; dA = gy B^T is an empty sum, so zero
        Value a = bf16_leaf(normal(8 * 32, 110), {8, 32}, "a2");
        Tensor be = Tensor::empty({32, 0}, Dtype::BFloat16);
        be.set_requires_grad(true);
        Value b = make_tensor(be, "b2");
        Value y = matmul(a, b);
        Tensor seed = Tensor::empty({8, 0}, Dtype::BFloat16);
        backward(y, &seed);
        report("matmul with no output columns: dA is zero",
               y.val().numel() == 0 && max_abs(a.grad().to_host_f32()) == 0.0 &&
                   a.grad().numel() == 8 * 32);
    }
}

// The captured graph holds the unfused composition rms(.) * g2 too, whose
// backward runs as one pass (agk_rms_mul_bwd) inside the capture.
void test_graph_capture(bool parallel) {
    const int64_t R = 256, D = 1024;
    std::vector<float> gv = uniform(D, 91, 0.5, 1.5), g2v = uniform(D, 93, 0.5, 1.5);
    GraphRunner runner(size_t(64) << 20);
    StreamGuard guard(runner.get_stream());
    Tensor xt = Tensor::from_host_f32(normal(R * D, 90), {R, D});
    xt.set_requires_grad(true);
    Tensor gt = Tensor::from_host_f32(gv, {D});
    gt.set_requires_grad(true);
    Tensor dyt = Tensor::from_host_f32(normal(R * D, 92), {R, D});
    Tensor g2t = Tensor::from_host_f32(g2v, {1, D});
    g2t.set_requires_grad(true);
    Value x = make_tensor(xt, "x"), g = make_tensor(gt, "g"), g2 = make_tensor(g2t, "g2");
    const uint64_t fused_before = debug::fused_rms_mul_vjps();
    runner.begin_capture();
    Value s = softmax_row(laynor(rms(rms_norm(x, g, 1e-5f)) * g2));
    backward(s, &dyt, parallel);
    runner.end_capture();
    const bool fused_in_capture = debug::fused_rms_mul_vjps() == fused_before + 1;
    const size_t used = runner.arena_bytes_used();
    bool same = true;
    for (int rep = 0; rep < 3; ++rep) {
        std::vector<float> xv = normal(R * D, 100 + rep);
        xt.copy_from(Tensor::from_host_f32(xv, {R, D}));
        {  // eager work on the same stream between replays
            Value e = leaf(normal(R * D, 200 + rep), {R, D}, "e"), ge = leaf(gv, {D}, "ge");
            backward(rms_norm(e, ge, 1e-5f), &dyt);
        }
        if (!runner.replay()) same = false;
        (void)hipStreamSynchronize(runner.get_stream());
        Value xe = leaf(xv, {R, D}, "xe"), ge = leaf(gv, {D}, "ge"), g2e = leaf(g2v, {1, D}, "g2e");
        Value se = softmax_row(laynor(rms(rms_norm(xe, ge, 1e-5f)) * g2e));
        backward(se, &dyt, parallel);
        same = same && s.val().to_host_f32() == se.val().to_host_f32() &&
               x.grad().to_host_f32() == xe.grad().to_host_f32() &&
               g.grad().to_host_f32() == ge.grad().to_host_f32() &&
               g2.grad().to_host_f32() == g2e.grad().to_host_f32();
    }
    report(parallel ? "graph replay == eager, 3 replays on new inputs (parallel backward)"
                    : "graph replay == eager, 3 replays on new inputs",
           same && fused_in_capture,
           "arena bytes used " + std::to_string(used) +
               (fused_in_capture ? ", rms(.) * g2 backward in one pass" : ", NOT fused"));
}

void test_graph_capture_rules() {
    GraphRunner runner(size_t(1) << 20);
    StreamGuard guard(runner.get_stream());
    std::vector<float> xv = normal(64, 95);
    Value x = leaf(xv, {4, 16}, "x");
    runner.begin_capture();
    Value y = rms(x);
    bool zeros_threw = false, seedless_threw = false, huge_threw = false;
    try {
        (void)Tensor::zeros({4});
    } catch (const std::runtime_error&) {
        zeros_threw = true;
    }
    try {
        backward(y);  // a ones seed needs a fill
    } catch (const std::runtime_error&) {
        seedless_threw = true;
    }
    try {
        (void)Tensor::empty({int64_t(1) << 20});  // 4 MiB > the 1 MiB arena
    } catch (const std::runtime_error&) {
        huge_threw = true;
    }
    runner.end_capture();
    report("capture: zeros(), a seedless backward and arena overflow throw",
           zeros_threw && seedless_threw && huge_threw);
    const bool replayed = runner.replay();
    (void)hipStreamSynchronize(runner.get_stream());
    Value xe = leaf(xv, {4, 16}, "xe");
    report("capture: the ops before the failures replay",
           replayed && y.val().to_host_f32() == rms(xe).val().to_host_f32());
    GraphRunner idle;
    report("replay without a capture returns false", !idle.replay());
}

// Storage's block cache: a freed block is handed to the next fitting
// allocation on the same stream, never to another stream; release returns
// everything.
void test_block_cache() {
    release_cached_memory();
    const bool empty0 = cached_bytes() == 0;
    void* p1 = nullptr;
    {
        Tensor t = Tensor::empty({1024, 1024});
        p1 = t.data();
    }
    const bool cached = cached_bytes() >= (size_t(4) << 20);
    Tensor t2 = Tensor::empty({1000, 1024});  // fits the cached 4 MiB block
    const bool reused = t2.data() == p1 && cached_bytes() == 0;
    Tensor t3 = Tensor::empty({2048, 1024});  // larger than anything cached
    const bool fresh = t3.data() != p1;
    report("block cache: a freed block is reused on its stream, a larger request is not served",
           empty0 && cached && reused && fresh);

    hipStream_t s = nullptr;
    (void)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    void* ps = nullptr;
    {
        StreamGuard guard(s);
        Tensor ts = Tensor::empty({512, 1024});
        ps = ts.data();
    }
    Tensor tn = Tensor::empty({512, 1024});  // the null stream: must not take s's block
    const bool separate = tn.data() != ps;
    release_cached_memory();
    const bool released = cached_bytes() == 0;
    (void)hipStreamDestroy(s);
    report("block cache: blocks stay with their stream; release empties the cache",
           separate && released);

    // many distinct sizes under a small cap: the cache never holds more than
    // the cap, the oldest blocks go back to the pool first
    const size_t cap = size_t(64) << 20;
    set_cache_limit(cap);
    bool under = cache_limit() == cap;
    uint64_t state = 12345;
    size_t peak = 0;
    for (int i = 0; i < 300; ++i) {
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        const int64_t floats = 1024 + static_cast<int64_t>((state >> 33) % (4u << 20));
        { Tensor t = Tensor::empty({floats}); }
        peak = std::max(peak, cached_bytes());
        under = under && cached_bytes() <= cap;
    }
    report("block cache: 300 distinct sizes stay under a 64 MiB cap",
           under && peak > cap / 2, "peak " + std::to_string(peak));

    // a stream's blocks are dropped when the stream is retired
    hipStream_t s2 = nullptr;
    (void)hipStreamCreateWithFlags(&s2, hipStreamNonBlocking);
    const size_t before = cached_bytes();
    {
        StreamGuard guard(s2);
        Tensor ts = Tensor::empty({256, 1024});
    }
    const bool held = cached_bytes() >= before + (size_t(1) << 20);
    release_stream_cache(s2);
    const bool dropped = cached_bytes() == before;
    (void)hipStreamSynchronize(s2);
    (void)hipStreamDestroy(s2);
    set_cache_limit(kDefaultCacheLimit);
    release_cached_memory();
    report("block cache: release_stream_cache drops that stream's blocks only", held && dropped);

    // blocks of a stream destroyed without release_stream_cache: evicting them
    // (by lowering the cap, then by a free past it) names no dead stream
    bool evicted_ok = true;
    std::string why;
    try {
        for (int round = 0; round < 2; ++round) {
            hipStream_t s3 = nullptr;
            (void)hipStreamCreateWithFlags(&s3, hipStreamNonBlocking);
            {
                StreamGuard guard(s3);
                Tensor a = Tensor::empty({512, 1024});
                Tensor b = Tensor::empty({300, 1024});
            }
            (void)hipStreamSynchronize(s3);
            (void)hipStreamDestroy(s3);
            if (round == 0) {
                set_cache_limit(0);
            } else {
                set_cache_limit(size_t(1) << 20);
                { Tensor big = Tensor::empty({1024, 1024}); }  // 4 MiB freed past the cap
            }
            evicted_ok = evicted_ok && cached_bytes() <= cache_limit();
        }
    } catch (const std::exception& e) {
        evicted_ok = false;
        why = e.what();
    }
    set_cache_limit(kDefaultCacheLimit);
    release_cached_memory();
    report("block cache: blocks of a destroyed stream are evicted without error",
           evicted_ok && cached_bytes() == 0, why);
}

// Runs the named checks (all of them when `only` is empty).
// The reference's integration test (Tests/test_kitchen_sink_mlp.cpp:14-29, 111-113) trains a
// small MLP with rms() inside on the GPU and asserts that the loss goes down and stays finite.
// The same on this path's ops: linear -> laynor -> rms(.) * gamma -> linear, all bf16 on the
// device; the softmax cross-entropy and its gradient (the backward seed) are taken on the host,
// and plain gradient descent updates fp32 master weights that are written back as bf16 each
// step.  Labels come from a fixed random linear teacher, so the classes are learnable.
void test_mlp_training() {
    const int64_t B = 64, IN = 64, H = 32, OUT = 8;
    const int epochs = 30;
    const float lr = 0.5f;
    auto bits = [](const std::vector<float>& v) {
        std::vector<uint16_t> b(v.size());
        for (size_t i = 0; i < v.size(); ++i) {
            uint32_t u;
            std::memcpy(&u, &v[i], 4);
            u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
            b[i] = static_cast<uint16_t>(u >> 16);
        }
        return b;
    };
    auto param = [&](const std::vector<float>& v, std::vector<int64_t> shape, const char* name) {
        std::vector<uint16_t> b = bits(v);
        Tensor t = Tensor::from_host(b.data(), shape, Dtype::BFloat16);
        t.set_requires_grad(true);
        return make_tensor(t, name);
    };
    const std::vector<float> xv = normal(B * IN, 40), teacher = normal(IN * OUT, 41);
    std::vector<int> label(B);
    for (int64_t b = 0; b < B; ++b) {
        double best = -1e300;
        for (int64_t o = 0; o < OUT; ++o) {
            double z = 0.0;
            for (int64_t i = 0; i < IN; ++i) z += double(xv[b * IN + i]) * teacher[i * OUT + o];
            if (z > best) best = z, label[b] = static_cast<int>(o);
        }
    }
    std::vector<float> W1 = normal(H * IN, 42, 0.1), b1(H, 0.0f), gam(H, 1.0f),
                       W2 = normal(OUT * H, 43, 0.1), b2(OUT, 0.0f);
    const std::vector<uint16_t> xb = bits(xv);
    const Tensor xt = Tensor::from_host(xb.data(), {B, IN}, Dtype::BFloat16);
    std::vector<double> losses;
    bool finite = true;
    for (int ep = 0; ep < epochs; ++ep) {
        Value x = make_tensor(xt, "x");
        Value w1 = param(W1, {H, IN}, "W1"), c1 = param(b1, {H}, "b1"), g = param(gam, {H}, "g");
        Value w2 = param(W2, {OUT, H}, "W2"), c2 = param(b2, {OUT}, "b2");
        Value logits = linear(rms(laynor(linear(x, w1, c1))) * g, w2, c2);
        const std::vector<float> z = logits.val().to_host_f32();
        std::vector<float> dz(z.size());
        double loss = 0.0;
        for (int64_t b = 0; b < B; ++b) {
            double m = -1e300, se = 0.0;
            for (int64_t o = 0; o < OUT; ++o) m = std::max(m, double(z[b * OUT + o]));
            for (int64_t o = 0; o < OUT; ++o) se += std::exp(double(z[b * OUT + o]) - m);
            loss += m + std::log(se) - z[b * OUT + label[b]];
            for (int64_t o = 0; o < OUT; ++o)
                dz[b * OUT + o] = static_cast<float>(
                    (std::exp(double(z[b * OUT + o]) - m) / se - (o == label[b] ? 1.0 : 0.0)) / B);
        }
        loss /= B;
        losses.push_back(loss);
        finite = finite && std::isfinite(loss);
        const std::vector<uint16_t> sb = bits(dz);
        const Tensor seed = Tensor::from_host(sb.data(), {B, OUT}, Dtype::BFloat16);
        backward(logits, &seed);
        const std::pair<std::vector<float>*, Value*> ps[] = {
            {&W1, &w1}, {&b1, &c1}, {&gam, &g}, {&W2, &w2}, {&b2, &c2}};
        for (auto& [master, v] : ps) {
            const std::vector<float> gr = v->grad().to_host_f32();
            for (size_t i = 0; i < master->size(); ++i) {
                finite = finite && std::isfinite(gr[i]);
                (*master)[i] -= lr * gr[i];
            }
        }
    }
    char detail[160];
    std::snprintf(detail, sizeof detail, "loss %.4f -> %.4f (epoch 10: %.4f)", losses.front(),
                  losses.back(), losses[10]);
    report("MLP with rms(.) * gamma trains (linear, laynor, rms, mul, linear)",
           finite && losses[10] < losses.front() && losses.back() < 0.25 * losses.front(), detail);
}

int selftest(const std::vector<std::string>& only) {
    const std::pair<const char*, void (*)()> tests[] = {
        {"reference_pattern", test_reference_pattern},
        {"fused_layer_gradients", test_fused_layer_gradients},
        {"fused_matches_unfused", test_fused_matches_unfused},
        {"composition_backward", test_composition_backward},
        {"accumulation_and_zero_grad", test_accumulation_and_zero_grad},
        {"parallel_matches_sequential", test_parallel_matches_sequential},
        {"weight_tying", test_weight_tying},
        {"module", test_module},
        {"errors", test_errors},
        {"broadcast_mul", test_broadcast_mul},
        {"matmul_f32", test_matmul_f32},
        {"empty_batch", test_empty_batch},
        {"bf16_layer", test_bf16_layer},
        {"bf16_mixed_gradient_dtypes", test_bf16_mixed_gradient_dtypes},
        {"scalar_literal", test_scalar_literal},
        {"seed_not_modified", test_seed_not_modified},
        {"user_stream", test_user_stream},
        {"row_ops_gradients", test_row_ops_gradients},
        {"wide_softmax", test_wide_softmax},
        {"wide_rms", test_wide_rms},
        {"jvp", test_jvp},
        {"matmul_layer", test_matmul_layer},
        {"linear_layer", test_linear_layer},
        {"matmul_empty", test_matmul_empty},
        {"graph_capture", [] { test_graph_capture(false); }},
        {"graph_capture_parallel", [] { test_graph_capture(true); }},
        {"graph_capture_rules", test_graph_capture_rules},
        {"block_cache", test_block_cache},
        {"mlp_training", test_mlp_training},
    };
    for (auto& [name, fn] : tests) {
        if (!only.empty() && std::find(only.begin(), only.end(), name) == only.end()) continue;
        std::printf("-- %s\n", name);
        std::fflush(stdout);
        try {
            fn();
        } catch (const std::exception& e) {
            report(name, false, std::string("exception: ") + e.what());
        }
    }
    std::printf("%d failure(s)\n", g_failures);
    return g_failures;
}

// ---- dump mode -------------------------------------------------------------

std::vector<char> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

void write_tensor(const std::string& path, const Tensor& t) {
    std::vector<char> buf(t.nbytes());
    if (!buf.empty()) t.copy_to_host(buf.data());
    std::ofstream f(path, std::ios::binary);
    f.write(buf.data(), static_cast<std::streamsize>(buf.size()));
}

int dump(const std::string& dir) {
    std::ifstream meta(dir + "/meta.txt");
    int64_t rows = 0, cols = 0;
    int dt = 0;
    float eps = 1e-5f;
    meta >> rows >> cols >> dt >> eps;
    const Dtype dtype = dt == 0 ? Dtype::Float32 : Dtype::BFloat16;
    std::vector<char> xb = read_file(dir + "/x.bin"), gb = read_file(dir + "/gamma.bin"),
                      dyb = read_file(dir + "/dy.bin");
    auto make = [&](const std::vector<char>& b, std::vector<int64_t> shape, bool req) {
        Tensor t = Tensor::from_host(b.data(), shape, dtype);
        t.set_requires_grad(req);
        return t;
    };
    Tensor dy = make(dyb, {rows, cols}, false);
    const std::pair<const char*, bool> fused_runs[] = {{"fused", false}, {"fused_par", true}};
    for (auto& [tag, parallel] : fused_runs) {
        Value x = make_tensor(make(xb, {rows, cols}, true), "x");
        Value g = make_tensor(make(gb, {cols}, true), "gamma");
        Value y = rms_norm(x, g, eps);
        backward(y, &dy, parallel);
        write_tensor(dir + "/y_" + tag + ".bin", y.val());
        write_tensor(dir + "/inv_" + tag + ".bin", *y.node->tape[0]);
        write_tensor(dir + "/dx_" + tag + ".bin", x.grad());
        write_tensor(dir + "/dg_" + tag + ".bin", g.grad());
    }
    {
        Value x = make_tensor(make(xb, {rows, cols}, true), "x");
        Value g = make_tensor(make(gb, {1, cols}, true), "gamma");
        Value y = rms(x) * g;  // eps fixed at 1e-5 by ag::rms
        backward(y, &dy);
        write_tensor(dir + "/y_unfused.bin", y.val());
        write_tensor(dir + "/dx_unfused.bin", x.grad());
        write_tensor(dir + "/dg_unfused.bin", g.grad());
    }
    // scalar literals on both sides: rms(x) * 0.75f and -1.5f * rms(x)
    const std::pair<const char*, float> scaled_runs[] = {{"scaled_r", 0.75f},
                                                         {"scaled_l", -1.5f}};
    for (auto& [tag, sc] : scaled_runs) {
        Value x = make_tensor(make(xb, {rows, cols}, true), "x");
        Value y = std::string(tag) == "scaled_r" ? rms(x) * sc : sc * rms(x);
        backward(y, &dy);
        write_tensor(dir + "/y_" + tag + ".bin", y.val());
        write_tensor(dir + "/dx_" + tag + ".bin", x.grad());
    }
    std::printf("dumped %lld x %lld %s\n", static_cast<long long>(rows),
                static_cast<long long>(cols), dtype_name(dtype));
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc >= 2 && std::string(argv[1]) == "selftest")
            return selftest(std::vector<std::string>(argv + 2, argv + argc));
        if (argc >= 3 && std::string(argv[1]) == "dump") return dump(argv[2]);
        std::fprintf(stderr, "usage: %s selftest | dump <dir>\n", argv[0]);
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
