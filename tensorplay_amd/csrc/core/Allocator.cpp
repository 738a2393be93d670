#include "Allocator.h"

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <mutex>
#include <unordered_map>

#include "CachingAllocatorCore.h"
#include "Exception.h"

namespace tensorplay {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) TP_THROW(RuntimeError, std::string(what) + ": " + hipGetErrorString(e));
}

// Runtime calls of one device for CachingAllocatorCore.
struct HipBackend {
    using Event = hipEvent_t;
    int dev = 0;

    void* raw_alloc(size_t n) {
        DeviceGuard guard(Device(DeviceType::ROCm, dev));
        void* p = nullptr;
        const hipError_t e = hipMalloc(&p, n);
        if (e == hipErrorOutOfMemory) {
            (void)hipGetLastError();
            return nullptr;
        }
        hip_check(e, "hipMalloc");
        return p;
    }
    void raw_free(void* p) {
        DeviceGuard guard(Device(DeviceType::ROCm, dev));
        (void)hipFree(p);
    }
    Event record(void* stream) {
        DeviceGuard guard(Device(DeviceType::ROCm, dev));
        hipEvent_t e = nullptr;
        hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags");
        hip_check(hipEventRecord(e, static_cast<hipStream_t>(stream)), "hipEventRecord");
        return e;
    }
    bool done(Event e) {
        const hipError_t r = hipEventQuery(e);
        if (r == hipErrorNotReady) {
            (void)hipGetLastError();
            return false;
        }
        hip_check(r, "hipEventQuery");
        return true;
    }
    void destroy(Event e) { (void)hipEventDestroy(e); }
    void wait_all() {
        DeviceGuard guard(Device(DeviceType::ROCm, dev));
        (void)hipDeviceSynchronize();
    }
};

using DeviceCache = CachingAllocatorCore<HipBackend>;

class ROCmAllocators {
public:
    DeviceCache& of(int dev) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = caches_.find(dev);
        if (it == caches_.end()) it = caches_.emplace(dev, new DeviceCache(HipBackend{dev})).first;
        return *it->second;  // never erased: blocks outlive any lookup
    }
    std::vector<DeviceCache*> all() {
        std::lock_guard<std::mutex> g(mu_);
        std::vector<DeviceCache*> v;
        for (auto& kv : caches_) v.push_back(kv.second);
        return v;
    }

private:
    std::mutex mu_;
    std::unordered_map<int, DeviceCache*> caches_;
};

ROCmAllocators& rocm_allocators() {
    static ROCmAllocators* a = new ROCmAllocators();  // outlives every tensor
    return *a;
}

// The current stream of each device, per host thread.
thread_local std::unordered_map<int, void*> t_streams;

}  // namespace

std::shared_ptr<void> allocate(size_t nbytes, const Device& device) {
    if (device.is_cpu()) {
        size_t n = (nbytes + 63) / 64 * 64;
        void* p = std::aligned_alloc(64, n ? n : 64);
        if (!p) TP_THROW(RuntimeError, "host allocation failed");
        return std::shared_ptr<void>(p, [](void* q) { std::free(q); });
    }
    size_t size = nbytes;
    const int dev = device.index;
    DeviceCache& cache = rocm_allocators().of(dev);
    void* p = cache.allocate(size, currentStream(dev));
    if (!p) TP_THROW(RuntimeError, "hipMalloc: out of memory allocating " + std::to_string(size) + " bytes");
    return std::shared_ptr<void>(p, [&cache](void* q) { cache.free(q); });
}

void recordStream(void* block, int device_index, void* stream) {
    rocm_allocators().of(device_index).record_stream(block, stream);
}

AllocatorStats allocatorStats(int device_index) {
    const CacheStats c = rocm_allocators().of(device_index).stats();
    AllocatorStats s;
    s.allocated_bytes = c.allocated_bytes;
    s.cached_bytes = c.cached_bytes;
    s.pending_bytes = c.pending_bytes;
    s.device_allocs = c.device_allocs;
    s.requests = c.requests;
    s.leaked_bytes = c.leaked_bytes;
    return s;
}

void emptyCache() {
    for (DeviceCache* c : rocm_allocators().all()) c->release_all();
}

void releaseStreamBlocks(int device_index, void* stream) { rocm_allocators().of(device_index).release_stream(stream); }

int rocmDeviceCount() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

void* currentStream(int device_index) {
    auto it = t_streams.find(device_index);
    return it == t_streams.end() ? nullptr : it->second;
}

void setCurrentStream(int device_index, void* stream) { t_streams[device_index] = stream; }

void synchronize(int device_index) {
    DeviceGuard guard(Device(DeviceType::ROCm, device_index));
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

DeviceGuard::DeviceGuard(const Device& d) {
    if (!d.is_rocm()) return;
    int cur = 0;
    hip_check(hipGetDevice(&cur), "hipGetDevice");
    if (cur != d.index) {
        hip_check(hipSetDevice(d.index), "hipSetDevice");
        prev_ = cur;
    }
}

DeviceGuard::~DeviceGuard() {
    if (prev_ >= 0) (void)hipSetDevice(prev_);
}

}  // namespace tensorplay
