// nt_pool.hpp — stream-ordered caching pools for device memory and
// page-locked host memory (plain C++: the device services come through
// PoolOps, HIP in the library and fakes in the host unit test).
//
// Device pool.  A block is allocated on a stream; freeing it returns it to
// the pool for reuse by later allocations on that same stream, which stream
// order already places after every use queued on it.  A block used on other
// streams as well (record) is reused only after an event recorded on each of
// those streams at free time has completed.  Blocks are never handed across
// streams, so the pool never synchronizes, except when the device runs out
// of memory: then idle blocks are released (after one device-wide wait) and
// the allocation is retried.  A stream destroyed after all its work completed
// (retire_stream) leaves its blocks to every stream: its idle blocks, and
// those freed later, are reused by allocations on any stream once their
// events of other streams have completed.
//
// Host pool.  Page-locked buffers are kept after use: releasing page-locked
// memory waits for the whole device.  Sizes are rounded up to a power of two
// (at least 4 KiB) so buffers of similar requests are shared.  A buffer comes
// back with the events after which no queued copy touches it, and is handed
// out again only when they have all completed.  Idle buffers beyond a byte
// budget are released (the largest settled first), which waits for the
// device, so the budget is set well above what a process keeps in flight.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace nt {

// Device services the pools need.  Streams and events are opaque handles.
class PoolOps {
  public:
    virtual ~PoolOps() = default;
    // 0: allocated; 1: out of memory; negative: another failure (message in `error`).
    virtual int device_alloc(int32_t device, uint64_t bytes, void **out, std::string &error) = 0;
    virtual void device_free(int32_t device, void *ptr) = 0;
    virtual int host_alloc(uint64_t bytes, void **out, std::string &error) = 0;
    virtual void host_free(void *ptr) = 0;
    // A new event recorded on `stream` of `device` (NULL on failure).
    virtual void *event_record(int32_t device, void *stream) = 0;
    virtual bool event_done(void *event) = 0;
    virtual void event_destroy(void *event) = 0;
    virtual void device_synchronize(int32_t device) = 0;
};

class DevicePool {
  public:
    explicit DevicePool(PoolOps &ops) : ops_(ops) {}
    DevicePool(const DevicePool &) = delete;
    DevicePool &operator=(const DevicePool &) = delete;
    ~DevicePool();

    // Block sizes: 512-byte steps up to 1 MiB, 2 MiB steps above (0 bytes: one step).
    static uint64_t rounded(uint64_t bytes);

    // Status codes are the C ABI's (NT_OK, NT_ERR_VALUE, NT_ERR_HIP ...).
    int32_t allocate(int32_t device, uint64_t bytes, void *stream, void **out, std::string &error);
    // `stream` will also use the live block at `ptr`.
    int32_t record(void *ptr, void *stream, std::string &error);
    int32_t release(void *ptr, std::string &error);
    // `stream` was destroyed after all its work completed: its blocks need no
    // ordering after it any more.  revive_stream: the handle names a new
    // stream again.
    void retire_stream(void *stream);
    void revive_stream(void *stream);
    void stats(int32_t device, uint64_t *in_use, uint64_t *reserved);
    // Return every idle block whose pending events have completed (waits for the device first).
    void trim(int32_t device);

  private:
    struct Block {
        void *ptr = nullptr;
        uint64_t size = 0;
        int32_t device = 0;
        void *stream = nullptr;                 // allocation stream: reuse happens only on it
        bool any_stream = false;                // its allocation stream was retired: any stream may reuse it
        std::vector<void *> also_used;          // streams recorded with record()
        std::vector<void *> pending;            // events to complete before reuse
    };
    struct Pool {
        std::multimap<uint64_t, Block *> idle;  // by size
        uint64_t reserved = 0;                  // bytes obtained from the device
        uint64_t in_use = 0;                    // bytes handed out
    };
    bool settled(Block *b);
    void trim_locked(int32_t device, Pool &pool);

    PoolOps &ops_;
    std::mutex lock_;
    std::map<int32_t, Pool> pools_;
    std::unordered_map<void *, Block *> live_;
    std::vector<void *> retired_;               // destroyed stream handles not handed out again
};

class HostPool {
  public:
    explicit HostPool(PoolOps &ops, uint64_t keep_bytes = uint64_t(1) << 30) : ops_(ops), keep_bytes_(keep_bytes) {}
    HostPool(const HostPool &) = delete;
    HostPool &operator=(const HostPool &) = delete;
    ~HostPool();

    // The size class of a request: the next power of two, at least 4 KiB.
    static uint64_t rounded(uint64_t bytes);
    // A buffer of at least `bytes` (an idle settled one of the same class when there is one).
    int32_t take(uint64_t bytes, void **out, std::string &error);
    // `ptr` (taken for `bytes`) is free once every event in `after` has
    // completed; the pool owns those events from here on.
    void give(void *ptr, uint64_t bytes, std::vector<void *> after);
    size_t idle_count();
    uint64_t idle_bytes();

  private:
    struct Idle {
        void *ptr;
        uint64_t size;
        std::vector<void *> after;
    };
    bool settled(Idle &idle);

    PoolOps &ops_;
    uint64_t keep_bytes_;
    uint64_t idle_bytes_ = 0;
    std::mutex lock_;
    std::vector<Idle> idle_;
};

}  // namespace nt
