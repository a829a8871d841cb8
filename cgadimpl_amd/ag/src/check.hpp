// check.hpp -- turning HIP and C-ABI failures into exceptions.  The reference
// throws std::runtime_error for unsupported cases
// (cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:380) and exits on CUDA errors
// (cgadimpl/src/runtime/cuda_graphs.cpp:12-19); this layer throws for both,
// with the HIP error text, and leaves the decision to the caller.
#pragma once

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

#include "agk_rmsnorm.h"

namespace ag::internal {

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

inline void agk_check(int rc, const char* what) {
    if (rc == AGK_OK) return;
    std::string msg = std::string(what) + ": " + agk_status_str(rc);
    if (rc == AGK_EHIP) msg += std::string(" (") + agk_last_error() + ")";
    throw std::runtime_error(msg);
}

[[noreturn]] inline void fail(const std::string& msg) { throw std::runtime_error(msg); }

// True on a thread while it runs ag::backward's VJPs: only there may a VJP
// also run its producer's VJP (backward knows which consumers are still due).
bool in_backward();

}  // namespace ag::internal
