// CPU test of CachingAllocatorCore's stream rules with mock streams and
// events (no GPU).  Streams are plain ids; an event is "done" only when the
// test completes it, so the test can hold a stream's work "in flight".
#include <cstdio>
#include <cstdlib>
#include <set>
#include <stdexcept>
#include <vector>

#include "CachingAllocatorCore.h"

using namespace tensorplay;

struct MockBackend {
    using Event = int;
    std::vector<bool>* ev_done;         // event id -> completed
    std::vector<void*>* stream_of_ev;   // event id -> stream it was recorded on
    size_t* budget;                     // bytes raw_alloc may still hand out
    std::set<void*>* raw_live;
    int* waits;
    bool* fail_record;  // record() throws (a failing runtime)
    bool* fail_wait;    // wait_all() throws too

    void* raw_alloc(size_t n) {
        if (n > *budget) return nullptr;
        *budget -= n;
        void* p = std::malloc(n);
        raw_live->insert(p);
        return p;
    }
    void raw_free(void* p) {
        raw_live->erase(p);
        std::free(p);
    }
    Event record(void* s) {
        if (*fail_record) throw std::runtime_error("record failed");
        ev_done->push_back(false);
        stream_of_ev->push_back(s);
        return (int)ev_done->size() - 1;
    }
    bool done(Event e) { return (*ev_done)[e]; }
    void destroy(Event) {}
    void wait_all() {
        if (*fail_wait) throw std::runtime_error("wait failed");
        ++*waits;
        for (size_t i = 0; i < ev_done->size(); ++i) (*ev_done)[i] = true;
    }
};

static int failures = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);          \
            ++failures;                                                       \
        }                                                                     \
    } while (0)

int main() {
    std::vector<bool> ev;
    std::vector<void*> ev_stream;
    size_t budget = 1 << 30;
    std::set<void*> raw;
    int waits = 0;
    bool fail_record = false, fail_wait = false;
    CachingAllocatorCore<MockBackend> a(MockBackend{&ev, &ev_stream, &budget, &raw, &waits, &fail_record, &fail_wait});
    void* A = (void*)0xA;
    void* B = (void*)0xB;

    // 1. a block freed on stream A is reused on A, never on B
    size_t n = 1000;
    void* pa = a.allocate(n, A);
    CHECK(n == 1024);
    a.free(pa);
    size_t m = 1000;
    void* pb = a.allocate(m, B);
    CHECK(pb != pa);
    size_t k = 1000;
    void* pa2 = a.allocate(k, A);
    CHECK(pa2 == pa);
    CHECK(a.stats().device_allocs == 2);

    // 2. a block also used on B (record_stream) waits for B's event after the free
    a.record_stream(pa2, B);
    a.free(pa2);
    CHECK(ev.size() == 1 && ev_stream[0] == B);
    CHECK(a.stats().pending_bytes == 1024);
    size_t k2 = 1000;
    void* q = a.allocate(k2, A);          // B's work still in flight
    CHECK(q != pa2);
    size_t k3 = 1000;
    void* q2 = a.allocate(k3, B);         // another stream never takes it
    CHECK(q2 != pa2);
    ev[0] = true;                          // B's work has completed
    size_t k4 = 1000;
    void* q3 = a.allocate(k4, B);
    CHECK(q3 != pa2);                     // completed, but owned by A
    size_t k5 = 1000;
    void* q4 = a.allocate(k5, A);
    CHECK(q4 == pa2);                     // now back on A's free list
    CHECK(a.stats().pending_bytes == 0);

    // 3. recording the owner stream itself, or twice, adds nothing to wait for
    a.record_stream(q4, A);
    a.free(q4);
    CHECK(a.stats().pending_bytes == 0);
    size_t k6 = 1000;
    CHECK(a.allocate(k6, A) == q4);
    a.record_stream(q4, B);
    a.record_stream(q4, B);
    a.free(q4);
    CHECK(ev.size() == 2);

    // 4. out of memory: wait for the device, return the cache, retry once
    for (void* p : {pb, q, q2, q3}) a.free(p);
    const int64_t cached = a.stats().cached_bytes;
    CHECK(cached == 4 * 1024);
    budget = 0;
    size_t big = 3 << 20;
    void* none = a.allocate(big, A);
    CHECK(none == nullptr);               // nothing to release can satisfy it
    CHECK(waits == 1);
    CHECK(a.stats().cached_bytes == 0 && a.stats().pending_bytes == 0);
    budget = 8 << 20;
    size_t big2 = 3 << 20;
    void* pbig = a.allocate(big2, A);
    CHECK(pbig != nullptr && big2 == (4u << 20));
    a.free(pbig);
    a.release_all();
    CHECK(raw.empty());
    CHECK(a.stats().allocated_bytes == 0);

    // 5. free() never throws: a failing event record falls back to draining the
    // device (the block becomes reusable on its owner stream) ...
    size_t s5 = 1000;
    void* r5 = a.allocate(s5, A);
    a.record_stream(r5, B);
    fail_record = true;
    const int w0 = waits;
    a.free(r5);  // must not throw
    CHECK(waits == w0 + 1);
    CHECK(a.stats().pending_bytes == 0 && a.stats().cached_bytes == 1024);
    fail_record = false;
    size_t s6 = 1000;
    CHECK(a.allocate(s6, A) == r5);
    // ... and when draining fails too, the block is dropped, never reused
    a.record_stream(r5, B);
    fail_record = fail_wait = true;
    a.free(r5);
    fail_record = fail_wait = false;
    CHECK(a.stats().leaked_bytes == 1024);
    size_t s7 = 1000;
    CHECK(a.allocate(s7, A) != r5);

    // 6. release_stream returns one stream's blocks (free and pending) to the
    // runtime and keeps the other streams' cache
    a.release_all();
    size_t s8 = 1000, s9 = 1000, s10 = 1000;
    void* xa = a.allocate(s8, A);
    void* xb = a.allocate(s9, B);
    void* xa2 = a.allocate(s10, A);
    a.record_stream(xa2, B);
    a.free(xa);
    a.free(xb);
    a.free(xa2);  // pending on B's event
    CHECK(a.stats().pending_bytes == 1024);
    a.release_stream(A);
    CHECK(raw.count(xa) == 0 && raw.count(xa2) == 0 && raw.count(xb) == 1);
    CHECK(a.stats().cached_bytes == 1024 && a.stats().pending_bytes == 0);
    size_t s11 = 1000;
    CHECK(a.allocate(s11, B) == xb);
    // the test's own cleanup: blocks still handed out, and the dropped one
    for (void* p : std::vector<void*>(raw.begin(), raw.end())) {
        raw.erase(p);
        std::free(p);
    }

    std::printf(failures ? "FAILED %d\n" : "OK\n", failures);
    return failures ? 1 : 0;
}
