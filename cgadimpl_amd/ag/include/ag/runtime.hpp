// runtime.hpp -- capture of graph-layer work into a HIP graph, and replay.
//
// The reference's CudaGraphRunner (cgadimpl/include/ad/runtime/cuda_graphs.hpp:
// 25-61, cgadimpl/src/runtime/cuda_graphs.cpp:34-76) with the same four calls:
// begin_capture() makes a private non-blocking stream the calling thread's
// current stream and starts capturing it, so every op and VJP the thread runs
// (and the parallel-backward workers, which take over that stream) is
// recorded instead of executed; end_capture() stops, instantiates the graph
// and restores the previous current stream; replay() launches the whole
// recorded forward + backward with one call on the runner's stream.
//
// Memory.  Buffers created during the capture (node values, saved tensors,
// gradients, workspaces) come from a capture arena of `arena_bytes` that the
// runner allocates before the capture begins, never from the stream-ordered
// pool: a replay writes the same addresses, so the tensors of the captured
// Values hold the results of the latest replay.  Values and gradients keep
// their arena alive after the runner is gone.
//
// Run the step once eagerly before capturing it, so that the kernels' code is
// loaded and pools are warm outside the capture.
//
// Rules for the captured region (violations throw std::runtime_error):
//   - no host transfers and no Tensor::zeros/ones (memset) inside it: create
//     inputs and the backward seed before begin_capture();
//   - gradients that do not exist when the capture starts are written, not
//     accumulated, by every replay (each replay is one step of zero_grad +
//     backward); gradients that exist are accumulated into at every replay.
// Inputs are updated in place between replays (Tensor::copy_from or host
// copies into the same tensors); replay() orders after work on the runner's
// stream only, so write inputs on get_stream() or synchronise first.
//
// Differences from the reference: failures throw instead of printing or
// exiting; end_capture() restores the previous stream instead of the null
// stream; capturing again replaces the previous graph.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <memory>

#include "ag/tensor.hpp"

namespace ag {

class GraphRunner {
  public:
    explicit GraphRunner(size_t arena_bytes = size_t(1) << 30);
    ~GraphRunner();
    GraphRunner(const GraphRunner&) = delete;
    GraphRunner& operator=(const GraphRunner&) = delete;

    void begin_capture();
    void end_capture();
    // Launches the captured graph on get_stream(); false if nothing was captured.
    bool replay();

    hipStream_t get_stream() const { return stream_; }
    bool is_capturing() const { return capturing_; }
    size_t arena_bytes_used() const { return arena_ ? arena_->used() : 0; }

  private:
    void destroy_graph();

    size_t arena_bytes_;
    hipStream_t stream_ = nullptr;
    hipStream_t prev_stream_ = nullptr;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
    bool capturing_ = false;
    std::shared_ptr<CaptureArena> arena_;
};

// The reference's name for it.
using CudaGraphRunner = GraphRunner;

}  // namespace ag
