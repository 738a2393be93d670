// Memory for tensors.  CPU: aligned host allocations.  ROCm: a caching
// allocator over hipMalloc (the reference's CUDA allocator allocates and frees
// on every call, /root/reference/p10/src/backend/cuda/CUDAAllocator.cpp:70-89;
// here freed blocks are kept per device, stream and size class and handed out
// again, so steady-state reductions never reach hipMalloc).
//
// Streams: each host thread has its own current stream per device
// (setCurrentStream; the default stream until set).  A block belongs to the
// stream that was current when it was allocated and is reused only on that
// stream, in stream order.  A tensor whose memory is also used on another
// stream is marked with recordStream(); when it is freed, its block waits for
// that stream's queued work (an event) before any reuse.  Free lists are keyed
// by the stream handle and a destroyed stream's handle may be given to a new
// stream: call releaseStreamBlocks(device, stream) before destroying a stream
// that allocated tensors (it drains the device and frees that stream's blocks).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>

#include "Device.h"

namespace tensorplay {

struct AllocatorStats {
    int64_t allocated_bytes = 0;   // handed out to tensors now
    int64_t cached_bytes = 0;      // held in free lists
    int64_t pending_bytes = 0;     // freed, waiting for another stream's work
    int64_t device_allocs = 0;     // hipMalloc calls
    int64_t requests = 0;          // allocate() calls
    int64_t leaked_bytes = 0;      // dropped because the runtime failed while freeing
};

// Returns memory that frees itself (back to the cache) when the last owner drops it.
std::shared_ptr<void> allocate(size_t nbytes, const Device& device);
AllocatorStats allocatorStats(int device_index);
void emptyCache();  // releases every cached (free) ROCm block
// Drains the device and returns every block owned by `stream` to the runtime
// (call before destroying that stream).
void releaseStreamBlocks(int device_index, void* stream);
// Marks the ROCm block that starts at `block` as used on `stream` as well.
void recordStream(void* block, int device_index, void* stream);

// ROCm runtime helpers used by the core.
int rocmDeviceCount();                       // 0 when no GPU/driver
void* currentStream(int device_index);       // this thread's hipStream_t (nullptr = default stream)
void setCurrentStream(int device_index, void* stream);  // for the calling thread only
void synchronize(int device_index);          // hipDeviceSynchronize on that device

class DeviceGuard {
public:
    explicit DeviceGuard(const Device& d);
    ~DeviceGuard();

private:
    int prev_ = -1;
};

}  // namespace tensorplay
