// tensor.hpp -- the device tensor the graph layer holds in its nodes.
//
// The reference keeps every value and gradient in an OwnTensor::Tensor
// (cgadimpl/include/tensor.hpp:6-15), whose library is not part of this
// build.  This is the part of that interface the RMSNorm layer path uses:
// a row-major, contiguous block of fp32 or bf16 elements on the current HIP
// device with a shape, plus host transfers for tests and callers.
//
// Memory comes from HIP's stream-ordered pool (hipMallocAsync on the calling
// thread's current stream, returned with hipFreeAsync on the same stream when
// the last reference goes), with the pool told to keep freed memory, so the
// per-call gradient and workspace buffers of a training loop are recycled
// without device-wide synchronisation.  A tensor is stream-ordered to the
// stream it was allocated on: work on another stream must be ordered against
// that stream by the caller.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <vector>

namespace ag {

enum class Dtype : uint8_t { Float32 = 0, BFloat16 = 1 };

size_t dtype_size(Dtype dt);
const char* dtype_name(Dtype dt);

// The stream GPU work of the calling thread is enqueued on (nullptr = the
// null stream).  Thread-local, like the reference's current_stream()
// (cgadimpl/include/ad/runtime/cuda_graphs.hpp:12-23).
hipStream_t current_stream();
void set_current_stream(hipStream_t stream);

// RAII: makes `stream` current for the lifetime of the guard.
class StreamGuard {
  public:
    explicit StreamGuard(hipStream_t stream) : prev_(current_stream()) {
        set_current_stream(stream);
    }
    ~StreamGuard() { set_current_stream(prev_); }
    StreamGuard(const StreamGuard&) = delete;
    StreamGuard& operator=(const StreamGuard&) = delete;

  private:
    hipStream_t prev_;
};

// Device memory for the allocations made on a stream while it is being
// captured into a HIP graph (see ag/runtime.hpp).  One hipMalloc'd block,
// handed out in 256-byte aligned pieces that are never reused: a captured
// graph replays the same addresses, so every buffer it touches must stay put
// for as long as the graph or a tensor in the block lives.  Pool memory that
// is released on the capturing stream during capture is kept here too and
// freed with the arena, since a stream-ordered free would otherwise become a
// node of the graph and run again at every replay.
class CaptureArena {
  public:
    explicit CaptureArena(size_t bytes);
    ~CaptureArena();
    CaptureArena(const CaptureArena&) = delete;
    CaptureArena& operator=(const CaptureArena&) = delete;
    void* take(size_t bytes);          // throws when the block is exhausted
    void defer_free(void* pool_ptr);   // freed when the arena is destroyed
    size_t used() const;
    size_t capacity() const { return capacity_; }

  private:
    void* base_ = nullptr;
    size_t capacity_ = 0;
    size_t used_ = 0;
    std::vector<void*> deferred_;
    mutable std::mutex mu_;
};

// Routes Storage allocations on `stream` to `arena` while it is set (nullptr
// clears it).  Used by GraphRunner around a capture.
void set_capture_arena(hipStream_t stream, std::shared_ptr<CaptureArena> arena);
// The arena set for `stream`, or nullptr.
std::shared_ptr<CaptureArena> capture_arena(hipStream_t stream);

// One device allocation: from the stream-ordered pool, or from the capture
// arena of the stream when it is being captured.  A pool block goes, when its
// Storage is destroyed, to a cache kept per stream (and device), and the next
// allocation of a fitting size on the same stream takes it: the stream orders
// the new user's work after the old user's, as the pool itself would, and no
// hipFreeAsync is called on the hot path (it blocks the calling thread on this
// runtime, which kept the host from running ahead of the GPU).  Blocks never
// move between streams.  The cache holds at most cache_limit() bytes per
// device: a block freed past the limit sends the device's oldest cached blocks
// back to HIP (one device synchronisation, then hipFree; the streams they were
// cached under are never called, so a destroyed stream's blocks are safe to
// evict).  When the pool cannot serve a request, the cache is emptied and the
// request retried once, unless a stream is being captured.
class Storage {
  public:
    Storage(size_t bytes, hipStream_t stream);
    ~Storage();
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;
    void* data() const { return ptr_; }
    size_t bytes() const { return bytes_; }
    hipStream_t stream() const { return stream_; }

  private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
    size_t block_ = 0;  // bytes of the pool block behind ptr_ (>= bytes_)
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    std::shared_ptr<CaptureArena> arena_;  // set: the memory belongs to the arena
};

// Returns every cached pool block of the current device to HIP (after a
// device synchronisation), to give the memory back.
void release_cached_memory();
// Returns the cached blocks of `stream` (current device) to HIP, after a
// device synchronisation.  Call it before destroying a stream that graph-layer
// tensors were allocated on: a later stream created with the same handle would
// otherwise take blocks whose last users it is not ordered after.
void release_stream_cache(hipStream_t stream);
// Bytes held in the cache on the current device (diagnostic).
size_t cached_bytes();
// The most bytes the cache holds per device (default kDefaultCacheLimit).
// Lowering it evicts the oldest blocks at once.
constexpr size_t kDefaultCacheLimit = size_t(4) << 30;
void set_cache_limit(size_t bytes);
size_t cache_limit();

class Tensor {
  public:
    Tensor() = default;  // undefined: no shape, no storage

    // Uninitialised / zero-filled / filled device tensors on the current stream.
    // zeros() and ones() fill with hipMemset*, so they throw while the current
    // stream is being captured into a graph (memset nodes are kept out of
    // captured graphs); empty() works there.
    static Tensor empty(const std::vector<int64_t>& shape, Dtype dt = Dtype::Float32);
    static Tensor zeros(const std::vector<int64_t>& shape, Dtype dt = Dtype::Float32);
    static Tensor ones(const std::vector<int64_t>& shape, Dtype dt = Dtype::Float32);
    // Every element `value` (stored in dt), written by a kernel (agk_fill), so
    // it may be called while the current stream is captured.
    static Tensor full(const std::vector<int64_t>& shape, float value,
                       Dtype dt = Dtype::Float32);
    // Copies `shape`-many elements of `dt` from host memory (bf16 as raw bits).
    static Tensor from_host(const void* src, const std::vector<int64_t>& shape,
                            Dtype dt = Dtype::Float32);
    static Tensor from_host_f32(const std::vector<float>& src, const std::vector<int64_t>& shape);

    // Synchronous copies to host memory (wait for the tensor's stream).
    void copy_to_host(void* dst) const;
    std::vector<float> to_host_f32() const;  // bf16 decoded to fp32
    // Device-to-device copy on the current stream (shapes must hold the same count).
    void copy_from(const Tensor& src);

    bool defined() const { return static_cast<bool>(storage_); }
    const std::vector<int64_t>& shape() const { return shape_; }
    Dtype dtype() const { return dtype_; }
    int64_t numel() const;
    int64_t dim() const { return static_cast<int64_t>(shape_.size()); }
    // Normalised axis = the last one: cols() = shape.back(), rows() = numel()/cols().
    int64_t cols() const;
    int64_t rows() const;
    size_t nbytes() const { return static_cast<size_t>(numel()) * dtype_size(dtype_); }
    void* data() const { return storage_ ? storage_->data() : nullptr; }

    // Same storage, another shape with the same element count.
    Tensor reshape(const std::vector<int64_t>& shape) const;

    // The reference's tensors carry requires_grad, which make_tensor() reads
    // (cgadimpl/include/ad/core/graph.hpp:82-84).
    bool requires_grad() const { return requires_grad_; }
    Tensor& set_requires_grad(bool on) {
        requires_grad_ = on;
        return *this;
    }

  private:
    std::vector<int64_t> shape_;
    Dtype dtype_ = Dtype::Float32;
    bool requires_grad_ = false;
    std::shared_ptr<Storage> storage_;
};

}  // namespace ag
