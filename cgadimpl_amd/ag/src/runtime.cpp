// runtime.cpp -- GraphRunner: hipGraph capture and replay of graph-layer work.
#include "ag/runtime.hpp"

#include "check.hpp"

namespace ag {

using internal::hip_check;

GraphRunner::GraphRunner(size_t arena_bytes) : arena_bytes_(arena_bytes) {
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreateWithFlags");
}

GraphRunner::~GraphRunner() {
    if (capturing_) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        set_capture_arena(stream_, nullptr);
        set_current_stream(prev_stream_);
    }
    destroy_graph();
    if (stream_) {
        (void)hipStreamSynchronize(stream_);
        // blocks cached under this stream must not pass to a later stream
        // that happens to reuse its handle
        try {
            release_stream_cache(stream_);
        } catch (...) {
        }
        (void)hipStreamDestroy(stream_);
    }
}

void GraphRunner::destroy_graph() {
    if (exec_) (void)hipGraphExecDestroy(exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
    exec_ = nullptr;
    graph_ = nullptr;
}

void GraphRunner::begin_capture() {
    if (capturing_) return;
    destroy_graph();
    // a fresh arena per capture: tensors of an earlier capture keep theirs
    arena_ = std::make_shared<CaptureArena>(arena_bytes_);
    prev_stream_ = current_stream();
    set_current_stream(stream_);
    set_capture_arena(stream_, arena_);
    const hipError_t e = hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        set_capture_arena(stream_, nullptr);
        set_current_stream(prev_stream_);
        hip_check(e, "hipStreamBeginCapture");
    }
    capturing_ = true;
}

void GraphRunner::end_capture() {
    if (!capturing_) return;
    capturing_ = false;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(stream_, &g);
    set_capture_arena(stream_, nullptr);
    set_current_stream(prev_stream_);
    if (e != hipSuccess && g) (void)hipGraphDestroy(g);
    hip_check(e, "hipStreamEndCapture");
    graph_ = g;
    hip_check(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
}

bool GraphRunner::replay() {
    if (!exec_) return false;
    hip_check(hipGraphLaunch(exec_, stream_), "hipGraphLaunch");
    return true;
}

}  // namespace ag
