// tensor.cpp -- device tensors on HIP's stream-ordered memory pool.
#include "ag/tensor.hpp"

#include <cstring>
#include <mutex>
#include <numeric>

#include "check.hpp"

namespace ag {

using internal::fail;
using internal::hip_check;

namespace {

thread_local hipStream_t t_current_stream = nullptr;

// The default pool of each device keeps freed blocks for reuse (release
// threshold = unlimited) instead of handing them back to the driver at every
// synchronisation, so steady-state training steps allocate nothing new.
void retain_pool_memory() {
    static std::mutex mu;
    static bool done[256] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    if (dev < 0 || dev >= 256 || done[dev]) return;
    hipMemPool_t pool;
    hip_check(hipDeviceGetDefaultMemPool(&pool, dev), "hipDeviceGetDefaultMemPool");
    uint64_t threshold = UINT64_MAX;
    hip_check(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold),
              "hipMemPoolSetAttribute");
    done[dev] = true;
}

int64_t count(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) fail("ag::Tensor: negative dimension");
        n *= d;
    }
    return n;
}

float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

size_t dtype_size(Dtype dt) { return dt == Dtype::Float32 ? 4 : 2; }
const char* dtype_name(Dtype dt) { return dt == Dtype::Float32 ? "float32" : "bfloat16"; }

hipStream_t current_stream() { return t_current_stream; }
void set_current_stream(hipStream_t stream) { t_current_stream = stream; }

Storage::Storage(size_t bytes, hipStream_t stream) : bytes_(bytes), stream_(stream) {
    if (bytes == 0) return;
    retain_pool_memory();
    hip_check(hipMallocAsync(&ptr_, bytes, stream), "hipMallocAsync");
}

Storage::~Storage() {
    if (ptr_) (void)hipFreeAsync(ptr_, stream_);
}

Tensor Tensor::empty(const std::vector<int64_t>& shape, Dtype dt) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dt;
    t.storage_ = std::make_shared<Storage>(static_cast<size_t>(count(shape)) * dtype_size(dt),
                                           current_stream());
    return t;
}

Tensor Tensor::zeros(const std::vector<int64_t>& shape, Dtype dt) {
    Tensor t = empty(shape, dt);
    if (t.nbytes())
        hip_check(hipMemsetAsync(t.data(), 0, t.nbytes(), current_stream()), "hipMemsetAsync");
    return t;
}

Tensor Tensor::ones(const std::vector<int64_t>& shape, Dtype dt) {
    Tensor t = empty(shape, dt);
    const size_t n = static_cast<size_t>(t.numel());
    if (n == 0) return t;
    if (dt == Dtype::Float32)
        hip_check(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(t.data()), 0x3f800000u, n,
                                    current_stream()),
                  "hipMemsetD32Async");
    else
        hip_check(hipMemsetD16Async(reinterpret_cast<hipDeviceptr_t>(t.data()), 0x3f80u, n,
                                    current_stream()),
                  "hipMemsetD16Async");
    return t;
}

Tensor Tensor::from_host(const void* src, const std::vector<int64_t>& shape, Dtype dt) {
    Tensor t = empty(shape, dt);
    if (t.nbytes()) {
        hip_check(hipMemcpyAsync(t.data(), src, t.nbytes(), hipMemcpyHostToDevice,
                                 current_stream()),
                  "hipMemcpyAsync H2D");
        hip_check(hipStreamSynchronize(current_stream()), "hipStreamSynchronize");
    }
    return t;
}

Tensor Tensor::from_host_f32(const std::vector<float>& src, const std::vector<int64_t>& shape) {
    if (static_cast<int64_t>(src.size()) != count(shape))
        fail("ag::Tensor::from_host_f32: element count does not match the shape");
    return from_host(src.data(), shape, Dtype::Float32);
}

void Tensor::copy_to_host(void* dst) const {
    if (!defined()) fail("ag::Tensor::copy_to_host: undefined tensor");
    if (!nbytes()) return;
    hip_check(hipMemcpyAsync(dst, data(), nbytes(), hipMemcpyDeviceToHost, current_stream()),
              "hipMemcpyAsync D2H");
    hip_check(hipStreamSynchronize(current_stream()), "hipStreamSynchronize");
}

std::vector<float> Tensor::to_host_f32() const {
    std::vector<float> out(static_cast<size_t>(numel()));
    if (dtype_ == Dtype::Float32) {
        copy_to_host(out.data());
    } else {
        std::vector<uint16_t> bits(out.size());
        copy_to_host(bits.data());
        for (size_t i = 0; i < bits.size(); ++i) out[i] = bf16_bits_to_f32(bits[i]);
    }
    return out;
}

void Tensor::copy_from(const Tensor& src) {
    if (!defined() || !src.defined()) fail("ag::Tensor::copy_from: undefined tensor");
    if (src.numel() != numel() || src.dtype() != dtype_)
        fail("ag::Tensor::copy_from: element count or dtype differs");
    if (nbytes())
        hip_check(hipMemcpyAsync(data(), src.data(), nbytes(), hipMemcpyDeviceToDevice,
                                 current_stream()),
                  "hipMemcpyAsync D2D");
}

int64_t Tensor::numel() const { return defined() ? count(shape_) : 0; }

int64_t Tensor::cols() const { return shape_.empty() ? 1 : shape_.back(); }

int64_t Tensor::rows() const {
    const int64_t c = cols();
    return c ? numel() / c : 0;
}

Tensor Tensor::reshape(const std::vector<int64_t>& shape) const {
    if (count(shape) != numel()) fail("ag::Tensor::reshape: element count differs");
    Tensor t = *this;
    t.shape_ = shape;
    return t;
}

}  // namespace ag
