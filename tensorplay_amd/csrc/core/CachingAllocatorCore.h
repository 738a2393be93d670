// Stream-aware caching of device blocks, independent of the device runtime.
//
// The reference allocates and frees device memory on every call
// (/root/reference/p10/src/backend/cuda/CUDAAllocator.cpp:70-89), so a freed
// block is never handed out again while a kernel still uses it.  A caching
// allocator keeps freed blocks and must give the same guarantee itself:
//
//  * every block belongs to the stream it was allocated on (the caller's
//    current stream).  Work on that stream is ordered, so a block freed by the
//    host can go straight back to that stream's free list: the next kernel
//    that receives it runs after every kernel queued before the free;
//  * a block used on other streams as well (record_stream) is not reusable
//    when the host frees it: the allocator records an event on each of those
//    streams and keeps the block pending until every event has completed;
//  * allocation on stream B never returns a block of stream A's free list.
//
// Backend supplies the runtime calls; the ROCm build uses hipMalloc and hip
// events (Allocator.cpp), the CPU test drives the same logic with mock streams
// and events whose completion the test controls.
//
//   void* Backend::raw_alloc(size_t)        nullptr when out of memory
//   void  Backend::raw_free(void*)
//   Event Backend::record(Stream)            an event after the stream's queued work
//   bool  Backend::done(Event)               true once it has completed
//   void  Backend::destroy(Event)
//   void  Backend::wait_all()                every queued kernel has finished
//
// free() runs inside a tensor's deleter, possibly while the process exits, so
// it never throws: if recording an event fails it waits for the whole device
// instead (the block is then idle and goes straight to its free list), and if
// that fails too the block is dropped (kept out of every list, counted in
// leaked_bytes) rather than handed out again unsafely.
//
// Free lists are keyed by the stream handle.  A runtime may give a destroyed
// stream's handle to a new stream, so before destroying a stream that
// allocated blocks, call release_stream(s): it drains the device and returns
// every block owned by `s` to the runtime.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

namespace tensorplay {

struct CacheStats {
    int64_t allocated_bytes = 0;  // handed out now
    int64_t cached_bytes = 0;     // reusable, in free lists
    int64_t pending_bytes = 0;    // freed, waiting for other streams' events
    int64_t device_allocs = 0;    // raw_alloc calls that succeeded
    int64_t requests = 0;         // allocate() calls
    int64_t leaked_bytes = 0;     // dropped by free() after the runtime failed (never reused)
};

template <class Backend>
class CachingAllocatorCore {
public:
    using Stream = void*;
    using Event = typename Backend::Event;

    explicit CachingAllocatorCore(Backend be = Backend()) : be_(std::move(be)) {}

    // Size classes: 512 B granularity below 1 MiB, 2 MiB granularity above.
    static size_t round_size(size_t n) {
        if (n == 0) n = 1;
        const size_t small = 512, large = size_t(2) << 20;
        return n < (size_t(1) << 20) ? (n + small - 1) / small * small : (n + large - 1) / large * large;
    }

    // Returns a block of at least `size` bytes for use on `stream`, or nullptr
    // when even a fresh raw allocation fails.  `size` is rounded in place.
    void* allocate(size_t& size, Stream stream) {
        size = round_size(size);
        {
            std::lock_guard<std::mutex> g(mu_);
            stats_.requests++;
            collect_pending_locked();
            if (void* p = take_locked(size, stream)) return p;
        }
        void* p = be_.raw_alloc(size);
        if (!p) {
            // out of memory: wait for every pending block, return the cache
            // to the runtime, and try once more
            release_all();
            p = be_.raw_alloc(size);
            if (!p) return nullptr;
        }
        std::lock_guard<std::mutex> g(mu_);
        stats_.device_allocs++;
        stats_.allocated_bytes += (int64_t)size;
        live_[p] = Live{size, stream, {}};
        return p;
    }

    // Marks the block at `p` as used on `stream` too: its reuse then waits for
    // the work queued on `stream` up to the free.
    void record_stream(void* p, Stream stream) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = live_.find(p);
        if (it == live_.end() || stream == it->second.stream) return;
        for (Stream s : it->second.uses)
            if (s == stream) return;
        it->second.uses.push_back(stream);
    }

    void free(void* p) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) return;
        Live b = std::move(it->second);
        live_.erase(it);
        stats_.allocated_bytes -= (int64_t)b.size;
        if (b.uses.empty()) {
            free_[{b.stream, b.size}].push_back(p);
            stats_.cached_bytes += (int64_t)b.size;
            return;
        }
        Pending pd{p, b.size, b.stream, {}};
        try {
            for (Stream s : b.uses) pd.events.push_back(be_.record(s));
        } catch (...) {
            for (const Event& e : pd.events) destroy_quietly(e);
            try {
                be_.wait_all();  // nothing queued anywhere still uses the block
                free_[{b.stream, b.size}].push_back(p);
                stats_.cached_bytes += (int64_t)b.size;
            } catch (...) {
                stats_.leaked_bytes += (int64_t)b.size;
            }
            return;
        }
        pending_.push_back(std::move(pd));
        stats_.pending_bytes += (int64_t)b.size;
    }

    // Returns every block owned by `stream` (free or pending) to the runtime,
    // after draining the device.  Call it before destroying a stream that
    // allocated blocks: its handle may be reused by a later stream.
    void release_stream(Stream stream) {
        be_.wait_all();
        std::vector<void*> blocks;
        {
            std::lock_guard<std::mutex> g(mu_);
            collect_pending_locked();  // all events have completed
            for (auto it = free_.begin(); it != free_.end();) {
                if (it->first.first != stream) {
                    ++it;
                    continue;
                }
                for (void* q : it->second) blocks.push_back(q);
                stats_.cached_bytes -= (int64_t)(it->first.second * it->second.size());
                it = free_.erase(it);
            }
        }
        for (void* q : blocks) be_.raw_free(q);
    }

    // Returns every cached block to the runtime (pending ones after their
    // events complete: the device is drained first).
    void release_all() {
        std::vector<void*> blocks;
        {
            std::lock_guard<std::mutex> g(mu_);
            if (free_.empty() && pending_.empty()) return;
        }
        be_.wait_all();
        {
            std::lock_guard<std::mutex> g(mu_);
            collect_pending_locked();  // all events have completed
            for (auto& kv : free_) {
                for (void* p : kv.second) blocks.push_back(p);
                stats_.cached_bytes -= (int64_t)(kv.first.second * kv.second.size());
            }
            free_.clear();
        }
        for (void* p : blocks) be_.raw_free(p);
    }

    CacheStats stats() {
        std::lock_guard<std::mutex> g(mu_);
        return stats_;
    }

    Backend& backend() { return be_; }

private:
    void destroy_quietly(const Event& e) {
        try {
            be_.destroy(e);
        } catch (...) {
        }
    }

    struct Live {
        size_t size;
        Stream stream;              // allocation stream: the block's owner
        std::vector<Stream> uses;   // other streams recorded with record_stream
    };
    struct Pending {
        void* p;
        size_t size;
        Stream stream;
        std::vector<Event> events;
    };

    void* take_locked(size_t size, Stream stream) {
        auto it = free_.find({stream, size});
        if (it == free_.end() || it->second.empty()) return nullptr;
        void* p = it->second.back();
        it->second.pop_back();
        stats_.cached_bytes -= (int64_t)size;
        stats_.allocated_bytes += (int64_t)size;
        live_[p] = Live{size, stream, {}};
        return p;
    }

    // Moves pending blocks whose events have all completed to their owner
    // stream's free list.
    void collect_pending_locked() {
        for (size_t i = 0; i < pending_.size();) {
            Pending& pd = pending_[i];
            bool all = true;
            for (const Event& e : pd.events)
                if (!be_.done(e)) { all = false; break; }
            if (!all) { ++i; continue; }
            for (const Event& e : pd.events) be_.destroy(e);
            free_[{pd.stream, pd.size}].push_back(pd.p);
            stats_.pending_bytes -= (int64_t)pd.size;
            stats_.cached_bytes += (int64_t)pd.size;
            pending_[i] = std::move(pending_.back());
            pending_.pop_back();
        }
    }

    Backend be_;
    std::mutex mu_;
    std::map<std::pair<Stream, size_t>, std::vector<void*>> free_;
    std::unordered_map<void*, Live> live_;
    std::vector<Pending> pending_;
    CacheStats stats_;
};

}  // namespace tensorplay
