// tensor.cpp -- device tensors on HIP's stream-ordered memory pool.
#include "ag/tensor.hpp"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <iterator>
#include <list>
#include <map>
#include <mutex>
#include <numeric>
#include <string>
#include <vector>

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

// ---- capture arenas ------------------------------------------------------------

CaptureArena::CaptureArena(size_t bytes) : capacity_(bytes) {
    if (bytes) hip_check(hipMalloc(&base_, bytes), "hipMalloc (capture arena)");
}

CaptureArena::~CaptureArena() {
    for (void* p : deferred_) (void)hipFree(p);
    if (base_) (void)hipFree(base_);
}

void* CaptureArena::take(size_t bytes) {
    std::lock_guard<std::mutex> lock(mu_);
    const size_t off = (used_ + 255) & ~size_t(255);
    if (off > capacity_ || bytes > capacity_ - off)
        fail("graph capture: the capture arena (" + std::to_string(capacity_) +
             " bytes) cannot hold another " + std::to_string(bytes) +
             " bytes; construct the GraphRunner with a larger arena");
    used_ = off + bytes;
    return static_cast<char*>(base_) + off;
}

void CaptureArena::defer_free(void* pool_ptr) {
    std::lock_guard<std::mutex> lock(mu_);
    deferred_.push_back(pool_ptr);
}

size_t CaptureArena::used() const {
    std::lock_guard<std::mutex> lock(mu_);
    return used_;
}

namespace {
std::mutex g_arena_mu;
std::vector<std::pair<hipStream_t, std::shared_ptr<CaptureArena>>> g_arenas;
std::atomic<int> g_narenas{0};
}  // namespace

void set_capture_arena(hipStream_t stream, std::shared_ptr<CaptureArena> arena) {
    std::lock_guard<std::mutex> lock(g_arena_mu);
    for (auto it = g_arenas.begin(); it != g_arenas.end(); ++it)
        if (it->first == stream) {
            g_arenas.erase(it);
            break;
        }
    if (arena) g_arenas.emplace_back(stream, std::move(arena));
    g_narenas.store(static_cast<int>(g_arenas.size()));
}

std::shared_ptr<CaptureArena> capture_arena(hipStream_t stream) {
    if (g_narenas.load() == 0) return nullptr;  // no capture anywhere: the usual case
    std::lock_guard<std::mutex> lock(g_arena_mu);
    for (auto& [s, a] : g_arenas)
        if (s == stream) return a;
    return nullptr;
}

// ---- storage --------------------------------------------------------------------

namespace {

// Freed pool blocks by (device, stream), then by size.  A request takes the
// smallest cached block of at least its size and at most 5/4 of it.  The bytes
// held per device are capped (cache_limit): a block freed past the cap pushes
// out the device's oldest cached blocks.  A block's stream is used only as a
// key: the stream may have been destroyed since the block was cached (a caller
// that skipped release_stream_cache), so blocks leave the cache through
// return_blocks, which synchronises the device and frees them without naming
// any stream.  The cache is never destroyed: freeing blocks at exit would race
// the runtime's teardown.
struct CachedBlock {
    int dev;
    hipStream_t stream;
    size_t bytes;
    void* ptr;
};
using BlockList = std::list<CachedBlock>;  // oldest first
struct BlockCache {
    std::mutex mu;
    BlockList order;
    std::map<std::pair<int, hipStream_t>, std::multimap<size_t, BlockList::iterator>> free;
    std::map<int, size_t> held;  // bytes cached per device
    size_t limit = kDefaultCacheLimit;
};
BlockCache& block_cache() {
    static BlockCache* c = new BlockCache;
    return *c;
}
size_t block_size(size_t bytes) { return (bytes + 511) & ~size_t(511); }

// Unlinks one cached block (the cache's mutex held).
void unlink_block(BlockCache& c, BlockList::iterator it) {
    auto key = std::make_pair(it->dev, it->stream);
    auto list = c.free.find(key);
    if (list != c.free.end()) {
        auto range = list->second.equal_range(it->bytes);
        for (auto m = range.first; m != range.second; ++m)
            if (m->second == it) {
                list->second.erase(m);
                break;
            }
        if (list->second.empty()) c.free.erase(list);
    }
    c.held[it->dev] -= it->bytes;
    c.order.erase(it);
}

void* take_cached(int dev, hipStream_t stream, size_t need, size_t* got) {
    BlockCache& c = block_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    auto list = c.free.find({dev, stream});
    if (list == c.free.end()) return nullptr;
    auto it = list->second.lower_bound(need);
    if (it == list->second.end() || it->first > need + need / 4) return nullptr;
    BlockList::iterator b = it->second;
    void* p = b->ptr;
    *got = b->bytes;
    unlink_block(c, b);
    return p;
}

// Makes `dev` current for a scope and restores the caller's device after it,
// also when a HIP call in between throws.
class DeviceGuard {
  public:
    DeviceGuard() {
        hip_check(hipGetDevice(&saved_), "hipGetDevice");
        current_ = saved_;
    }
    ~DeviceGuard() {
        if (current_ != saved_) (void)hipSetDevice(saved_);
    }
    void set(int dev) {
        if (dev == current_) return;
        hip_check(hipSetDevice(dev), "hipSetDevice");
        current_ = dev;
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

  private:
    int saved_ = 0;
    int current_ = 0;
};

// Hands blocks back to HIP: per device, one device synchronisation (every
// user of a block, on whatever stream, has then finished) and a hipFree per
// block.  No stream handle is used, so blocks of destroyed streams are freed
// like any other.  Every block is attempted; the first failure is thrown after
// the caller's device is restored.
void return_blocks(std::vector<CachedBlock> blocks) {
    if (blocks.empty()) return;
    std::stable_sort(blocks.begin(), blocks.end(),
                     [](const CachedBlock& a, const CachedBlock& b) { return a.dev < b.dev; });
    DeviceGuard guard;
    std::string first_error;
    auto note = [&](hipError_t e, const char* what) {
        if (e != hipSuccess && first_error.empty())
            first_error = std::string(what) + ": " + hipGetErrorString(e);
    };
    int synced = -1;
    for (const CachedBlock& b : blocks) {
        try {
            guard.set(b.dev);
        } catch (const std::exception& e) {
            if (first_error.empty()) first_error = e.what();
            continue;
        }
        if (synced != b.dev) {
            note(hipDeviceSynchronize(), "hipDeviceSynchronize");
            synced = b.dev;
        }
        note(hipFree(b.ptr), "hipFree");
    }
    if (!first_error.empty()) fail(first_error);
}
}  // namespace

Storage::Storage(size_t bytes, hipStream_t stream) : bytes_(bytes), stream_(stream) {
    if (bytes == 0) return;
    if ((arena_ = capture_arena(stream))) {
        ptr_ = arena_->take(bytes);
        return;
    }
    hip_check(hipGetDevice(&device_), "hipGetDevice");
    const size_t need = block_size(bytes);
    if ((ptr_ = take_cached(device_, stream, need, &block_))) return;
    retain_pool_memory();
    hipError_t e = hipMallocAsync(&ptr_, need, stream);
    if (e == hipErrorOutOfMemory && g_narenas.load() == 0) {
        // The pool is out of memory, possibly to blocks this cache holds for
        // other sizes or streams: hand them all back and try once more.  Not
        // while any stream is being captured: the device synchronisation and
        // frees of release_cached_memory would invalidate that capture.
        (void)hipGetLastError();
        release_cached_memory();
        e = hipMallocAsync(&ptr_, need, stream);
    }
    hip_check(e, "hipMallocAsync");
    block_ = need;
}

Storage::~Storage() {
    if (!ptr_ || arena_) return;  // arena memory goes with the arena
    if (auto a = capture_arena(stream_)) {
        a->defer_free(ptr_);  // a free on a capturing stream would be recorded
        return;
    }
    std::vector<CachedBlock> evicted;
    {
        BlockCache& c = block_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        if (block_ > c.limit && g_narenas.load() == 0) {  // too big to cache: back to the pool
            evicted.push_back({device_, stream_, block_, ptr_});
        } else {
            c.order.push_back({device_, stream_, block_, ptr_});
            c.free[{device_, stream_}].emplace(block_, std::prev(c.order.end()));
            size_t& held = c.held[device_];
            held += block_;
            // No frees while a capture is recorded anywhere (a free call can
            // invalidate it); the next free after the capture trims the cache.
            const bool capturing = g_narenas.load() != 0;
            for (auto it = c.order.begin(); !capturing && held > c.limit && it != c.order.end();) {
                auto next = std::next(it);
                if (it->dev == device_) {
                    evicted.push_back(*it);
                    unlink_block(c, it);
                }
                it = next;
            }
        }
    }
    try {
        return_blocks(std::move(evicted));
    } catch (...) {  // a destructor must not throw; a block that failed is lost to the pool
    }
}

void release_cached_memory() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::vector<CachedBlock> blocks;
    {
        BlockCache& c = block_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        for (auto it = c.order.begin(); it != c.order.end();) {
            auto next = std::next(it);
            if (it->dev == dev) {
                blocks.push_back(*it);
                unlink_block(c, it);
            }
            it = next;
        }
    }
    return_blocks(std::move(blocks));
}

void release_stream_cache(hipStream_t stream) {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::vector<CachedBlock> blocks;
    {
        BlockCache& c = block_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        for (auto it = c.order.begin(); it != c.order.end();) {
            auto next = std::next(it);
            // a created stream's handle names one device; the null stream is
            // the current device's
            if (it->stream == stream && (stream != nullptr || it->dev == dev)) {
                blocks.push_back(*it);
                unlink_block(c, it);
            }
            it = next;
        }
    }
    return_blocks(std::move(blocks));
}

size_t cached_bytes() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    BlockCache& c = block_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.held.find(dev);
    return it == c.held.end() ? 0 : it->second;
}

void set_cache_limit(size_t bytes) {
    std::vector<CachedBlock> evicted;
    {
        BlockCache& c = block_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        c.limit = bytes;
        for (auto it = c.order.begin(); it != c.order.end();) {
            auto next = std::next(it);
            if (c.held[it->dev] > c.limit) {
                evicted.push_back(*it);
                unlink_block(c, it);
            }
            it = next;
        }
    }
    return_blocks(std::move(evicted));
}

size_t cache_limit() {
    BlockCache& c = block_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    return c.limit;
}

Tensor Tensor::empty(const std::vector<int64_t>& shape, Dtype dt) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dt;
    t.storage_ = std::make_shared<Storage>(static_cast<size_t>(count(shape)) * dtype_size(dt),
                                           current_stream());
    return t;
}

namespace {
void no_fill_under_capture(const char* what) {
    if (capture_arena(current_stream()))
        fail(std::string(what) + ": not available while the current stream is captured into a "
             "graph (no memset nodes in captured graphs); create the tensor before the capture");
}
}  // namespace

Tensor Tensor::zeros(const std::vector<int64_t>& shape, Dtype dt) {
    no_fill_under_capture("ag::Tensor::zeros");
    Tensor t = empty(shape, dt);
    if (t.nbytes())
        hip_check(hipMemsetAsync(t.data(), 0, t.nbytes(), current_stream()), "hipMemsetAsync");
    return t;
}

Tensor Tensor::ones(const std::vector<int64_t>& shape, Dtype dt) {
    no_fill_under_capture("ag::Tensor::ones");
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

Tensor Tensor::full(const std::vector<int64_t>& shape, float value, Dtype dt) {
    Tensor t = empty(shape, dt);
    const int rc = agk_fill(t.data(), t.numel(), value, dt == Dtype::Float32 ? AGK_F32 : AGK_BF16,
                            reinterpret_cast<agk_stream_t>(current_stream()));
    internal::agk_check(rc, "ag::Tensor::full");
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
