// nn.hpp -- the RMSNorm layer as a module.
//
// The reference has nn::Module / nn::Linear (cgadimpl/include/nn/nn.hpp:9-54)
// but no RMSNorm module, and its benchmark's RMSNormLayer is an empty stub
// (Benchmark/RMSNormLayer.cpp:1-5).  This is the layer those would define:
// a learned per-channel gain gamma (initialised to ones) applied with the
// fused rms_norm op.
#pragma once

#include <vector>

#include "ag/graph.hpp"

namespace ag::nn {

class Module {
  public:
    virtual ~Module() = default;
    virtual std::vector<Value> parameters() = 0;
    // Clears the gradients of the parameters (they read as zeros afterwards).
    void zero_grad();
};

class RMSNorm : public Module {
  public:
    explicit RMSNorm(int64_t dim, float eps = 1e-5f, Dtype dt = Dtype::Float32);
    Value operator()(const Value& x) const;
    std::vector<Value> parameters() override { return {gamma}; }

    Value gamma;
    float eps;
};

}  // namespace ag::nn
