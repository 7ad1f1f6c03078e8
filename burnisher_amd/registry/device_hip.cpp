// device_hip.cpp -- Burnisher's device boundary (include/burnisher/device.h) on HIP, for a ROCm
// build of the reference runtime: it takes the place of src/cuda/device.cu and of
// src/core/device_stub.cpp, and makes Device::CUDA mean "the MI355X" to Tensor, DeviceWeights
// and every model graph.
//
// The contract is the reference's (device.cu:60-200):
//   - every allocation is ZEROED, so device and host (calloc) tensors start alike;
//   - live and peak bytes count what the runtime asked for (not the driver's slack), and
//     reset_peak() restarts the high-water mark at the live total;
//   - freed blocks are kept by exact size and handed to the next allocation of that size while
//     the device keeps a headroom free, because a forward allocates the same shapes each time;
//   - all work is ordered on the default stream, which is what makes reusing a block safe.
// Zero-filling uses an asynchronous memset on the default stream: it is ordered before every
// later kernel on that stream, so the host does not wait for it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>

#include "burnisher/device.h"

namespace burnisher {
namespace device {
namespace {

// Blocks are cached only while at least this much device memory stays free; an allocation that
// leaves less returns the cache to the driver first.
constexpr size_t kHeadroom = size_t{4} << 30;

struct Pool {
    std::mutex mu;
    size_t live = 0, peak = 0;
    std::multimap<size_t, void*> cached;    // size -> free block
    std::map<void*, size_t> owned;          // block -> size, for every live block
    // The driver's free bytes as of the last fresh allocation, moved by this pool's own frees
    // since: a release decides between caching and freeing on it without a driver query (each
    // query is a system call, and a forward releases every intermediate).
    size_t free_est = 0;
};

// Leaked on purpose: Tensor deleters can run after static destruction.
Pool& pool() {
    static Pool* p = new Pool();
    return *p;
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("hip ") + what + ": " + hipGetErrorString(e));
}

size_t free_bytes() {
    size_t f = 0, t = 0;
    return hipMemGetInfo(&f, &t) == hipSuccess ? f : 0;
}

void drop_cache_locked(Pool& p) {
    for (auto& kv : p.cached) {
        (void)hipFree(kv.second);
        p.free_est += kv.first;
    }
    p.cached.clear();
}

}  // namespace

bool available() {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

void* alloc(size_t bytes) {
    Pool& p = pool();
    void* ptr = nullptr;
    {
        std::lock_guard<std::mutex> lock(p.mu);
        auto it = p.cached.find(bytes);
        if (it != p.cached.end()) {
            ptr = it->second;
            p.cached.erase(it);
        }
    }
    if (!ptr) {
        if (hipMalloc(&ptr, bytes) != hipSuccess) {
            (void)hipGetLastError();
            std::lock_guard<std::mutex> lock(p.mu);
            drop_cache_locked(p);
            ptr = nullptr;
            check(hipMalloc(&ptr, bytes), "hipMalloc");
        }
        const size_t f = free_bytes();
        std::lock_guard<std::mutex> lock(p.mu);
        p.free_est = f;
        if (f < kHeadroom) {
            drop_cache_locked(p);
            p.free_est = free_bytes();
        }
    }
    check(hipMemsetAsync(ptr, 0, bytes, nullptr), "hipMemsetAsync (zero fill)");
    std::lock_guard<std::mutex> lock(p.mu);
    p.live += bytes;
    p.peak = std::max(p.peak, p.live);
    p.owned[ptr] = bytes;
    return ptr;
}

void release(void* ptr) {
    if (!ptr) return;
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    auto it = p.owned.find(ptr);
    if (it == p.owned.end()) {
        (void)hipFree(ptr);
        return;
    }
    const size_t bytes = it->second;
    p.owned.erase(it);
    p.live -= std::min(p.live, bytes);
    if (p.free_est >= kHeadroom) {
        p.cached.emplace(bytes, ptr);
    } else {
        (void)hipFree(ptr);
        p.free_est += bytes;
    }
}

void copy_to_device(void* dst, const void* src, size_t bytes) {
    check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "memcpy H2D");
}

void copy_to_host(void* dst, const void* src, size_t bytes) {
    check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "memcpy D2H");
}

void synchronize() { check(hipDeviceSynchronize(), "synchronize"); }

void* alloc_pinned(size_t bytes) {
    void* ptr = nullptr;
    check(hipHostMalloc(&ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
    return ptr;
}

void release_pinned(void* ptr) {
    if (ptr) (void)hipHostFree(ptr);
}

size_t allocated_bytes() {
    std::lock_guard<std::mutex> lock(pool().mu);
    return pool().live;
}

size_t peak_allocated_bytes() {
    std::lock_guard<std::mutex> lock(pool().mu);
    return pool().peak;
}

void reset_peak() {
    std::lock_guard<std::mutex> lock(pool().mu);
    pool().peak = pool().live;
}

}  // namespace device
}  // namespace burnisher
