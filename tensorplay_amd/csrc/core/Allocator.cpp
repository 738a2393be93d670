#include "Allocator.h"

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "Exception.h"

namespace tensorplay {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) TP_THROW(RuntimeError, std::string(what) + ": " + hipGetErrorString(e));
}

// Size classes: 512 B granularity below 1 MiB, 2 MiB granularity above.
size_t round_size(size_t n) {
    if (n == 0) n = 1;
    const size_t small = 512, large = 2u << 20;
    return n < (1u << 20) ? (n + small - 1) / small * small : (n + large - 1) / large * large;
}

struct DeviceCache {
    std::unordered_map<size_t, std::vector<void*>> free_blocks;
    AllocatorStats stats;
};

class ROCmCachingAllocator {
public:
    void* allocate(size_t& size, int dev) {
        size = round_size(size);
        {
            std::lock_guard<std::mutex> g(mu_);
            auto& c = caches_[dev];
            c.stats.requests++;
            auto it = c.free_blocks.find(size);
            if (it != c.free_blocks.end() && !it->second.empty()) {
                void* p = it->second.back();
                it->second.pop_back();
                c.stats.cached_bytes -= (int64_t)size;
                c.stats.allocated_bytes += (int64_t)size;
                return p;
            }
        }
        DeviceGuard guard(Device(DeviceType::ROCm, dev));
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, size);
        if (e == hipErrorOutOfMemory) {
            (void)hipGetLastError();
            release_all(dev);
            e = hipMalloc(&p, size);
        }
        hip_check(e, "hipMalloc");
        std::lock_guard<std::mutex> g(mu_);
        auto& c = caches_[dev];
        c.stats.device_allocs++;
        c.stats.allocated_bytes += (int64_t)size;
        return p;
    }

    void free(void* p, size_t size, int dev) {
        std::lock_guard<std::mutex> g(mu_);
        auto& c = caches_[dev];
        c.free_blocks[size].push_back(p);
        c.stats.allocated_bytes -= (int64_t)size;
        c.stats.cached_bytes += (int64_t)size;
    }

    void release_all(int dev) {
        std::vector<void*> blocks;
        {
            std::lock_guard<std::mutex> g(mu_);
            auto& c = caches_[dev];
            for (auto& kv : c.free_blocks) {
                for (void* p : kv.second) blocks.push_back(p);
                c.stats.cached_bytes -= (int64_t)(kv.first * kv.second.size());
            }
            c.free_blocks.clear();
        }
        if (blocks.empty()) return;
        DeviceGuard guard(Device(DeviceType::ROCm, dev));
        (void)hipDeviceSynchronize();
        for (void* p : blocks) (void)hipFree(p);
    }

    void release_everything() {
        std::vector<int> devs;
        {
            std::lock_guard<std::mutex> g(mu_);
            for (auto& kv : caches_) devs.push_back(kv.first);
        }
        for (int d : devs) release_all(d);
    }

    AllocatorStats stats(int dev) {
        std::lock_guard<std::mutex> g(mu_);
        return caches_[dev].stats;
    }

private:
    std::mutex mu_;
    std::unordered_map<int, DeviceCache> caches_;
};

ROCmCachingAllocator& rocm_allocator() {
    static ROCmCachingAllocator* a = new ROCmCachingAllocator();  // outlives every tensor
    return *a;
}

std::mutex g_stream_mu;
std::unordered_map<int, void*> g_streams;

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
    void* p = rocm_allocator().allocate(size, dev);
    return std::shared_ptr<void>(p, [size, dev](void* q) { rocm_allocator().free(q, size, dev); });
}

AllocatorStats allocatorStats(int device_index) { return rocm_allocator().stats(device_index); }

void emptyCache() { rocm_allocator().release_everything(); }

int rocmDeviceCount() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

void* currentStream(int device_index) {
    std::lock_guard<std::mutex> g(g_stream_mu);
    auto it = g_streams.find(device_index);
    return it == g_streams.end() ? nullptr : it->second;
}

void setCurrentStream(int device_index, void* stream) {
    std::lock_guard<std::mutex> g(g_stream_mu);
    g_streams[device_index] = stream;
}

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
