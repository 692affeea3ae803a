// Host unit test of the library's caching pools (namitorch_amd/csrc/nt_pool.cpp):
// block rounding, stream-ordered reuse, reuse gated by events of other
// streams, the waste bound, out-of-memory trimming, statistics, error codes,
// and the page-locked host pool.  The device services are fakes (heap memory,
// events completed by hand), so it runs without a GPU under AddressSanitizer
// and UBSan (tests/test_host_tables.py builds and runs it).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <set>
#include <string>
#include <vector>

#include "../../include/namitorch_amd.h"
#include "../../namitorch_amd/csrc/nt_pool.hpp"

using namespace nt;

static int failures = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
            ++failures;                                                          \
        }                                                                        \
    } while (0)

struct FakeEvent {
    void *stream;
    bool done;
};

// Heap-backed device and host memory with a per-device capacity; events
// complete only when the test says so (or the device is synchronized).
class FakeOps final : public PoolOps {
  public:
    uint64_t capacity = uint64_t(1) << 40;
    uint64_t used = 0;
    int device_allocs = 0, device_frees = 0, host_allocs = 0, host_frees = 0, syncs = 0;
    bool fail_events = false;
    std::set<void *> device_live, host_live;
    std::set<FakeEvent *> events;
    std::vector<std::pair<void *, uint64_t>> sizes;

    ~FakeOps() override {
        for (void *p : device_live) std::free(p);
        for (void *p : host_live) std::free(p);
        for (FakeEvent *e : events) delete e;
    }
    int device_alloc(int32_t, uint64_t bytes, void **out, std::string &error) override {
        if (used + bytes > capacity) {
            error = "fake: out of memory";
            return 1;
        }
        *out = std::malloc(bytes);
        used += bytes;
        sizes.emplace_back(*out, bytes);
        device_live.insert(*out);
        ++device_allocs;
        return 0;
    }
    void device_free(int32_t, void *ptr) override {
        CHECK(device_live.erase(ptr) == 1);
        for (auto &entry : sizes)
            if (entry.first == ptr) {
                used -= entry.second;
                entry.first = nullptr;
            }
        std::free(ptr);
        ++device_frees;
    }
    int host_alloc(uint64_t bytes, void **out, std::string &) override {
        *out = std::malloc(bytes);
        host_live.insert(*out);
        ++host_allocs;
        return 0;
    }
    void host_free(void *ptr) override {
        CHECK(host_live.erase(ptr) == 1);
        std::free(ptr);
        ++host_frees;
    }
    void *event_record(int32_t, void *stream) override {
        if (fail_events) return nullptr;
        FakeEvent *e = new FakeEvent{stream, false};
        events.insert(e);
        return e;
    }
    bool event_done(void *event) override {
        CHECK(events.count(static_cast<FakeEvent *>(event)) == 1);
        return static_cast<FakeEvent *>(event)->done;
    }
    void event_destroy(void *event) override {
        CHECK(events.erase(static_cast<FakeEvent *>(event)) == 1);
        delete static_cast<FakeEvent *>(event);
    }
    void device_synchronize(int32_t) override {
        ++syncs;
        for (FakeEvent *e : events) e->done = true;
    }
    void complete(void *stream) {
        for (FakeEvent *e : events)
            if (e->stream == stream) e->done = true;
    }
};

static void *S(uintptr_t id) { return reinterpret_cast<void *>(id); }

static void test_rounding() {
    CHECK(DevicePool::rounded(0) == 512);
    CHECK(DevicePool::rounded(1) == 512);
    CHECK(DevicePool::rounded(512) == 512);
    CHECK(DevicePool::rounded(513) == 1024);
    CHECK(DevicePool::rounded(uint64_t(1) << 20) == uint64_t(1) << 20);
    CHECK(DevicePool::rounded((uint64_t(1) << 20) + 1) == uint64_t(2) << 20);
    CHECK(DevicePool::rounded(uint64_t(3) << 20) == uint64_t(4) << 20);
}

static void test_stream_ordered_reuse() {
    FakeOps ops;
    std::string error;
    {
        DevicePool pool(ops);
        void *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr;
        CHECK(pool.allocate(0, 1000, S(1), &a, error) == NT_OK && a != nullptr);
        uint64_t in_use = 0, reserved = 0;
        pool.stats(0, &in_use, &reserved);
        CHECK(in_use == 1024 && reserved == 1024);
        CHECK(pool.release(a, error) == NT_OK);
        pool.stats(0, &in_use, &reserved);
        CHECK(in_use == 0 && reserved == 1024);
        CHECK(pool.allocate(0, 900, S(2), &b, error) == NT_OK && b != a);     // another stream: a new block
        CHECK(pool.allocate(0, 900, S(1), &c, error) == NT_OK && c == a);     // its own stream: reused
        CHECK(ops.device_allocs == 2);
        // Waste bound: a 4096-byte idle block does not serve a 1024-byte request.
        void *big = nullptr;
        CHECK(pool.allocate(0, 4096, S(1), &big, error) == NT_OK);
        CHECK(pool.release(big, error) == NT_OK);
        CHECK(pool.allocate(0, 1000, S(1), &d, error) == NT_OK && d != big);
        void *again = nullptr;
        CHECK(pool.allocate(0, 3000, S(1), &again, error) == NT_OK && again == big);   // 3072: within 2x
        // Devices do not share blocks.
        void *other = nullptr;
        CHECK(pool.release(again, error) == NT_OK);
        CHECK(pool.allocate(1, 4096, S(1), &other, error) == NT_OK && other != big);
        for (void *p : {b, c, d, other}) CHECK(pool.release(p, error) == NT_OK);
    }
    CHECK(ops.events.empty());
}

static void test_other_streams_gate_reuse() {
    FakeOps ops;
    std::string error;
    {
        DevicePool pool(ops);
        void *a = nullptr, *b = nullptr;
        CHECK(pool.allocate(0, 2048, S(1), &a, error) == NT_OK);
        CHECK(pool.record(a, S(7), error) == NT_OK);
        CHECK(pool.record(a, S(7), error) == NT_OK);        // once per stream
        CHECK(pool.record(a, S(1), error) == NT_OK);        // the allocation stream itself: nothing to do
        CHECK(pool.release(a, error) == NT_OK);
        CHECK(ops.events.size() == 1);                      // one event, on stream 7
        CHECK(pool.allocate(0, 2048, S(1), &b, error) == NT_OK && b != a);   // stream 7 not done yet
        ops.complete(S(7));
        void *c = nullptr;
        CHECK(pool.allocate(0, 2048, S(1), &c, error) == NT_OK && c == a);   // now reusable
        CHECK(ops.events.empty());                          // the settled event was released
        // A stream that cannot be tracked keeps the block out of the pool.
        CHECK(pool.record(c, S(9), error) == NT_OK);
        ops.fail_events = true;
        CHECK(pool.release(c, error) == NT_OK);
        ops.fail_events = false;
        uint64_t in_use = 0, reserved = 0;
        pool.stats(0, &in_use, &reserved);
        CHECK(in_use == 2048 && reserved == 2048);          // b live; a's block is gone from the books
        CHECK(pool.release(b, error) == NT_OK);
    }
    CHECK(ops.events.empty());
}

static void test_out_of_memory_trims() {
    FakeOps ops;
    ops.capacity = 8192;
    std::string error;
    {
        DevicePool pool(ops);
        void *a = nullptr, *b = nullptr, *c = nullptr;
        CHECK(pool.allocate(0, 4096, S(1), &a, error) == NT_OK);
        CHECK(pool.record(a, S(2), error) == NT_OK);
        CHECK(pool.allocate(0, 4096, S(1), &b, error) == NT_OK);
        CHECK(pool.release(a, error) == NT_OK);              // idle, waiting for stream 2
        CHECK(pool.release(b, error) == NT_OK);              // idle
        // 8 KiB on another stream: nothing idle fits that stream, the device is
        // full, so the pool waits for the device, frees both idle blocks and retries.
        CHECK(pool.allocate(0, 8192, S(3), &c, error) == NT_OK);
        CHECK(ops.syncs == 1 && ops.device_frees == 2);
        uint64_t in_use = 0, reserved = 0;
        pool.stats(0, &in_use, &reserved);
        CHECK(in_use == 8192 && reserved == 8192);
        void *d = nullptr;
        CHECK(pool.allocate(0, 512, S(3), &d, error) == NT_ERR_HIP && d == nullptr);
        CHECK(error.find("out of memory") != std::string::npos && error.find("8192 in use") != std::string::npos);
        CHECK(pool.release(c, error) == NT_OK);
        pool.trim(0);
        pool.stats(0, &in_use, &reserved);
        CHECK(in_use == 0 && reserved == 0 && ops.used == 0);
    }
    CHECK(ops.events.empty());
}

static void test_errors() {
    FakeOps ops;
    std::string error;
    DevicePool pool(ops);
    int local = 0;
    CHECK(pool.release(&local, error) == NT_ERR_VALUE && error.find("not a live allocation") != std::string::npos);
    CHECK(pool.record(&local, S(1), error) == NT_ERR_VALUE);
    CHECK(pool.release(nullptr, error) == NT_OK);
    CHECK(pool.allocate(0, 16, S(1), nullptr, error) == NT_ERR_VALUE);
    void *p = &local;
    CHECK(pool.allocate(-1, 16, S(1), &p, error) == NT_ERR_VALUE && p == nullptr);
    CHECK(pool.allocate(0, uint64_t(1) << 63, S(1), &p, error) == NT_ERR_VALUE);
    void *a = nullptr;
    CHECK(pool.allocate(0, 16, S(1), &a, error) == NT_OK);
    CHECK(pool.release(a, error) == NT_OK);
    CHECK(pool.release(a, error) == NT_ERR_VALUE);          // a second free is refused
}

static void test_host_pool() {
    CHECK(HostPool::rounded(0) == 4096 && HostPool::rounded(4096) == 4096 && HostPool::rounded(4097) == 8192);
    CHECK(HostPool::rounded(uint64_t(3) << 20) == uint64_t(4) << 20);
    FakeOps ops;
    std::string error;
    {
        HostPool pool(ops, 16384);
        void *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr;
        CHECK(pool.take(100, &a, error) == NT_OK && ops.host_allocs == 1);
        pool.give(a, 100, {ops.event_record(0, S(1))});
        CHECK(pool.take(100, &b, error) == NT_OK && b != a);  // a's copy is still pending
        ops.complete(S(1));
        CHECK(pool.take(3000, &c, error) == NT_OK && c == a); // settled, same 4 KiB class: reused
        CHECK(pool.take(5000, &d, error) == NT_OK && d != b); // 8 KiB class: a new buffer
        pool.give(b, 100, {});
        pool.give(c, 100, {});
        CHECK(pool.idle_count() == 2 && pool.idle_bytes() == 8192);
        pool.give(d, 5000, {});                               // 16 KiB idle: at the budget, nothing released
        CHECK(pool.idle_count() == 3 && ops.host_frees == 0);
        void *e = nullptr;
        CHECK(pool.take(1, &e, error) == NT_OK);
        pool.give(e, 9000, {});                               // a 16 KiB class: over budget, the largest settled goes
        CHECK(ops.host_frees == 1 && pool.idle_bytes() <= 16384);
        void *f = nullptr;
        CHECK(pool.take(10, &f, error) == NT_OK);
        pool.give(f, 10, {ops.event_record(0, S(5))});        // unsettled buffers are never released
        pool.give(nullptr, 8, {ops.event_record(0, S(1))});   // nothing to keep; the event is released
    }
    CHECK(ops.events.empty());
}

static void test_retired_stream_blocks_serve_every_stream() {
    FakeOps ops;
    std::string error;
    {
        DevicePool pool(ops);
        void *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr, *e = nullptr, *f = nullptr;
        CHECK(pool.allocate(0, 4096, S(5), &a, error) == NT_OK);
        CHECK(pool.allocate(0, 4096, S(5), &b, error) == NT_OK);
        CHECK(pool.allocate(0, 8192, S(5), &c, error) == NT_OK);
        CHECK(pool.record(c, S(6), error) == NT_OK);
        CHECK(pool.release(a, error) == NT_OK);          // idle on stream 5 before it is destroyed
        CHECK(pool.release(c, error) == NT_OK);          // idle, also waiting for stream 6
        pool.retire_stream(S(5));
        CHECK(pool.release(b, error) == NT_OK);          // freed after the destroy
        // Another stream reuses both 4 KiB blocks; nothing new is allocated.
        CHECK(pool.allocate(0, 4096, S(7), &d, error) == NT_OK && (d == a || d == b));
        CHECK(pool.allocate(0, 4096, S(8), &e, error) == NT_OK && (e == a || e == b) && e != d);
        CHECK(ops.device_allocs == 3);
        // The 8 KiB block still waits for stream 6.
        CHECK(pool.allocate(0, 8192, S(7), &f, error) == NT_OK && f != c);
        ops.complete(S(6));
        void *g = nullptr;
        CHECK(pool.allocate(0, 8192, S(9), &g, error) == NT_OK && g == c);
        // A block handed to stream 7 belongs to stream 7 from then on.
        CHECK(pool.release(d, error) == NT_OK);
        void *h = nullptr;
        CHECK(pool.allocate(0, 4096, S(8), &h, error) == NT_OK && h != d);
        // A handle that names a new stream again is ordinary: its blocks stay with it.
        pool.revive_stream(S(5));
        void *k = nullptr, *l = nullptr;
        CHECK(pool.allocate(0, 1024, S(5), &k, error) == NT_OK);
        CHECK(pool.release(k, error) == NT_OK);
        CHECK(pool.allocate(0, 1024, S(7), &l, error) == NT_OK && l != k);
        for (void *p : {e, f, g, h, l}) CHECK(pool.release(p, error) == NT_OK);
    }
    CHECK(ops.events.empty());
}

int main() {
    test_rounding();
    test_stream_ordered_reuse();
    test_other_streams_gate_reuse();
    test_out_of_memory_trims();
    test_retired_stream_blocks_serve_every_stream();
    test_errors();
    test_host_pool();
    if (failures == 0) std::printf("pools: all checks passed\n");
    return failures == 0 ? 0 : 1;
}
