// rmsnorm_layer.cpp -- the RMSNorm layer benchmark through the graph layer.
//
// The reference's Benchmark/RMSNormLayer.cpp:1-5 is an empty stub; this is
// the program it would be.  Each step builds the layer on the tape exactly as
// a user of the reference's API writes it, seeds the output gradient and runs
// ag::backward:
//   fused    y = nn::RMSNorm(D, eps)(x)            one forward kernel, one
//                                                 backward call (dx, dgamma)
//   unfused  y = ag::rms(x) * gamma                the reference's composition
//                                                 (normalization.cpp:23-35 then
//                                                 arithmetic.cpp:31-39): two
//                                                 forward and two backward calls
// Inputs live on the device before timing starts; the timed region is `steps`
// steps on one stream between two device synchronisations.  Eagerly, that
// includes the graph layer's host work (node creation, topological order, the
// pool allocations of every output and gradient); captured, one step is
// recorded once with ag::GraphRunner (the reference's CudaGraphRunner) and
// each timed step is one replay of the recorded forward + backward.  One JSON
// line per graph and run mode, with algorithmic bytes per step
// 5*R*D*s + 2*D*s + 2*R*4 + D*4 (the fused layer's traffic; the unfused graph
// moves more than that).
//
// Usage: rmsnorm_layer [B T D] [steps] [warmup] [f32|bf16] [fused|unfused|both]
//                      [eager|captured|all]
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "ag/ag.hpp"

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Uniform floats in [lo, hi) from a 64-bit linear congruential generator: the
// timing does not depend on the distribution, only on the values being finite.
std::vector<float> host_uniform(size_t n, uint64_t seed, float lo, float hi) {
    std::vector<float> v(n);
    uint64_t s = seed * 0x9E3779B97F4A7C15ULL + 1;
    for (size_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        v[i] = lo + (hi - lo) * static_cast<float>(s >> 40) * (1.0f / 16777216.0f);
    }
    return v;
}

ag::Tensor device_tensor(const std::vector<float>& host, const std::vector<int64_t>& shape,
                         ag::Dtype dt) {
    ag::Tensor t = ag::Tensor::from_host_f32(host, shape);
    if (dt == ag::Dtype::Float32) return t;
    // bf16 storage: round on the host (nearest even) and upload the raw bits
    std::vector<uint16_t> bits(host.size());
    for (size_t i = 0; i < host.size(); ++i) {
        uint32_t u;
        std::memcpy(&u, &host[i], 4);
        u += 0x7fffu + ((u >> 16) & 1u);
        bits[i] = static_cast<uint16_t>(u >> 16);
    }
    return ag::Tensor::from_host(bits.data(), shape, dt);
}

}  // namespace

int main(int argc, char** argv) {
    try {
        std::vector<int64_t> shape = {32, 2048, 4096};
        int steps = 20, warmup = 5;
        std::string dtype = "f32", mode = "both", run = "all";
        if (argc >= 4) shape = {std::atoll(argv[1]), std::atoll(argv[2]), std::atoll(argv[3])};
        if (argc >= 5) steps = std::atoi(argv[4]);
        if (argc >= 6) warmup = std::atoi(argv[5]);
        if (argc >= 7) dtype = argv[6];
        if (argc >= 8) mode = argv[7];
        if (argc >= 9) run = argv[8];
        if (steps < 1 || warmup < 0 || (dtype != "f32" && dtype != "bf16") ||
            (mode != "fused" && mode != "unfused" && mode != "both") ||
            (run != "eager" && run != "captured" && run != "all"))
            throw std::runtime_error(
                "usage: rmsnorm_layer [B T D] [steps] [warmup] [f32|bf16] [fused|unfused|both] "
                "[eager|captured|all]");
        const ag::Dtype dt = dtype == "f32" ? ag::Dtype::Float32 : ag::Dtype::BFloat16;
        const int64_t D = shape[2], R = shape[0] * shape[1];
        const size_t n = static_cast<size_t>(R * D);
        const float eps = 1e-6f;

        hipStream_t stream;
        check(hipStreamCreate(&stream), "hipStreamCreate");
        ag::StreamGuard guard(stream);

        ag::Tensor x = device_tensor(host_uniform(n, 1, -2.f, 2.f), shape, dt);
        x.set_requires_grad(true);
        const ag::Tensor dy = device_tensor(host_uniform(n, 2, -1.f, 1.f), shape, dt);
        ag::nn::RMSNorm layer(D, eps, dt);
        layer.gamma.val().copy_from(device_tensor(host_uniform(D, 3, 0.5f, 1.5f), {D}, dt));

        const double s = dt == ag::Dtype::Float32 ? 4.0 : 2.0;
        const double bytes = 5.0 * R * D * s + 2.0 * D * s + 2.0 * R * 4 + D * 4.0;
        auto report = [&](const char* path, const char* how, double sec) {
            const double ms = sec * 1e3 / steps;
            const double gbs = bytes / (ms * 1e-3) / 1e9;
            std::printf(
                "{\"path\": \"graph layer, %s, %s\", \"shape\": [%lld, %lld, %lld], "
                "\"dtype\": \"%s\", \"steps\": %d, \"warmup\": %d, \"ms_per_step\": %.5f, "
                "\"gbs\": %.1f, \"pct_of_hbm_peak\": %.2f}\n",
                path, how, static_cast<long long>(shape[0]), static_cast<long long>(shape[1]),
                static_cast<long long>(shape[2]), dtype.c_str(), steps, warmup, ms, gbs,
                100.0 * gbs / 8000.0);
            std::fflush(stdout);
        };
        auto seconds_since = [](std::chrono::steady_clock::time_point t0) {
            return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        };
        for (const char* m : {"fused", "unfused"}) {
            if (mode != "both" && mode != m) continue;
            const bool fused = std::strcmp(m, "fused") == 0;
            const char* path = fused ? "nn::RMSNorm (fused)" : "ag::rms(x) * gamma (unfused)";
            auto step = [&]() {
                ag::Value xv = ag::make_tensor(x, "x");
                ag::Value y = fused ? layer(xv) : ag::rms(xv) * layer.gamma;
                ag::backward(y, &dy);
                layer.zero_grad();
            };
            for (int i = 0; i < warmup; ++i) step();
            check(hipDeviceSynchronize(), "warm-up");
            if (run != "captured") {
                const auto t0 = std::chrono::steady_clock::now();
                for (int i = 0; i < steps; ++i) step();
                check(hipDeviceSynchronize(), "timed steps");
                report(path, "eager", seconds_since(t0));
            }
            if (run != "eager") {
                // every buffer of one step (outputs, saved tensors, gradients,
                // workspaces) comes from the capture arena
                ag::GraphRunner runner(static_cast<size_t>(4.5 * R * D * s) + (size_t(64) << 20));
                runner.begin_capture();
                step();
                runner.end_capture();
                for (int i = 0; i < warmup; ++i) runner.replay();
                check(hipDeviceSynchronize(), "replay warm-up");
                const auto t0 = std::chrono::steady_clock::now();
                for (int i = 0; i < steps; ++i) runner.replay();
                check(hipDeviceSynchronize(), "timed replays");
                report(path, "captured", seconds_since(t0));
            }
        }
        check(hipStreamSynchronize(stream), "hipStreamSynchronize");
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "rmsnorm_layer: %s\n", e.what());
        return 1;
    }
}
