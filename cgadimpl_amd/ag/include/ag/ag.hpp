// ag.hpp -- the whole graph layer (the reference's umbrella header is
// cgadimpl/include/ad/ag_all.hpp).
#pragma once

#include "ag/autodiff.hpp"
#include "ag/graph.hpp"
#include "ag/nn.hpp"
#include "ag/ops.hpp"
#include "ag/runtime.hpp"
#include "ag/tensor.hpp"
