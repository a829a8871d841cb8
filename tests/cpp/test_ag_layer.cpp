// test_ag_layer.cpp -- the ag:: graph layer (Value, rms, rms_norm, mul,
// backward) on the GPU.
//
//   test_ag_layer selftest     checks below; prints PASS/FAIL per check and
//                              exits with the number of failures
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
// and broadcast-multiply gradients (test_core_ops_gpu.cpp:198-205).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "ag/ag.hpp"

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

void test_fused_matches_unfused() {
    const int64_t R = 64, D = 256;
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
    report("rms_norm(x, g) == rms(x) * g", ey <= 1e-5 && ex <= 1e-5 && eg <= 1e-5,
           "y " + std::to_string(ey) + " dx " + std::to_string(ex) + " dgamma " +
               std::to_string(eg));
    // gamma * rms(x): the broadcast operand first
    Value x3 = leaf(xv, {R, D}, "x3"), g3 = leaf(gv, {D}, "g3");
    Value y3 = g3 * rms(x3);
    backward(y3, &dy);
    report("gamma * rms(x) == rms(x) * gamma",
           y3.val().to_host_f32() == y2.val().to_host_f32() &&
               x3.grad().to_host_f32() == x2.grad().to_host_f32() &&
               g3.grad().to_host_f32() == g2.grad().to_host_f32());
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
    (void)hipStreamDestroy(s);
}

int selftest() {
    const std::pair<const char*, void (*)()> tests[] = {
        {"reference_pattern", test_reference_pattern},
        {"fused_layer_gradients", test_fused_layer_gradients},
        {"fused_matches_unfused", test_fused_matches_unfused},
        {"accumulation_and_zero_grad", test_accumulation_and_zero_grad},
        {"parallel_matches_sequential", test_parallel_matches_sequential},
        {"weight_tying", test_weight_tying},
        {"module", test_module},
        {"errors", test_errors},
        {"empty_batch", test_empty_batch},
        {"bf16_layer", test_bf16_layer},
        {"seed_not_modified", test_seed_not_modified},
        {"user_stream", test_user_stream},
    };
    for (auto& [name, fn] : tests) {
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
    std::printf("dumped %lld x %lld %s\n", static_cast<long long>(rows),
                static_cast<long long>(cols), dtype_name(dtype));
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc >= 2 && std::string(argv[1]) == "selftest") return selftest();
        if (argc >= 3 && std::string(argv[1]) == "dump") return dump(argv[2]);
        std::fprintf(stderr, "usage: %s selftest | dump <dir>\n", argv[0]);
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
