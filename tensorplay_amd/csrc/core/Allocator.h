// Memory for tensors.  CPU: aligned host allocations.  ROCm: a caching
// allocator over hipMalloc (the reference's CUDA allocator allocates and frees
// on every call, /root/reference/p10/src/backend/cuda/CUDAAllocator.cpp:70-89;
// here freed blocks are kept per device and size class and handed out again,
// so steady-state reductions never reach hipMalloc).
//
// Blocks are reused in stream order on the device's current stream; work that
// runs on several streams at once must synchronise before memory is freed.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>

#include "Device.h"

namespace tensorplay {

struct AllocatorStats {
    int64_t allocated_bytes = 0;   // handed out to tensors now
    int64_t cached_bytes = 0;      // held in free lists
    int64_t device_allocs = 0;     // hipMalloc calls
    int64_t requests = 0;          // allocate() calls
};

// Returns memory that frees itself (back to the cache) when the last owner drops it.
std::shared_ptr<void> allocate(size_t nbytes, const Device& device);
AllocatorStats allocatorStats(int device_index);
void emptyCache();  // releases every cached (free) ROCm block

// ROCm runtime helpers used by the core.
int rocmDeviceCount();                       // 0 when no GPU/driver
void* currentStream(int device_index);       // hipStream_t (nullptr = default stream)
void setCurrentStream(int device_index, void* stream);
void synchronize(int device_index);          // hipDeviceSynchronize on that device

class DeviceGuard {
public:
    explicit DeviceGuard(const Device& d);
    ~DeviceGuard();

private:
    int prev_ = -1;
};

}  // namespace tensorplay
