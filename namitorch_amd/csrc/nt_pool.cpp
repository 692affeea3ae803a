// nt_pool.cpp — the caching pools of nt_pool.hpp.
#include "nt_pool.hpp"

#include "../../include/namitorch_amd.h"

namespace nt {

namespace {
constexpr uint64_t kSmallRound = 512;                  // blocks up to 1 MiB: 512-byte steps
constexpr uint64_t kLargeRound = uint64_t(2) << 20;    // larger blocks: 2 MiB steps
constexpr uint64_t kSmallLimit = uint64_t(1) << 20;
}  // namespace

// ---- device pool ------------------------------------------------------------------------
DevicePool::~DevicePool() {
    // Device memory is not returned (the library's pools live until the
    // process ends); the bookkeeping and pending events are released.
    for (auto &entry : pools_)
        for (auto &idle : entry.second.idle) {
            for (void *event : idle.second->pending) ops_.event_destroy(event);
            delete idle.second;
        }
    for (auto &entry : live_) delete entry.second;
}

uint64_t DevicePool::rounded(uint64_t bytes) {
    if (bytes == 0) bytes = 1;
    const uint64_t step = bytes <= kSmallLimit ? kSmallRound : kLargeRound;
    return (bytes + step - 1) / step * step;
}

bool DevicePool::settled(Block *b) {
    for (void *event : b->pending)
        if (!ops_.event_done(event)) return false;
    for (void *event : b->pending) ops_.event_destroy(event);
    b->pending.clear();
    return true;
}

void DevicePool::trim_locked(int32_t device, Pool &pool) {
    ops_.device_synchronize(device);
    for (auto it = pool.idle.begin(); it != pool.idle.end();) {
        Block *b = it->second;
        if (settled(b)) {
            ops_.device_free(b->device, b->ptr);
            pool.reserved -= b->size;
            delete b;
            it = pool.idle.erase(it);
        } else {
            ++it;
        }
    }
}

int32_t DevicePool::allocate(int32_t device, uint64_t bytes, void *stream, void **out, std::string &error) {
    if (out == nullptr) {
        error = "nt_malloc: output pointer is NULL";
        return NT_ERR_VALUE;
    }
    *out = nullptr;
    if (device < 0) {
        error = "nt_malloc: invalid device";
        return NT_ERR_VALUE;
    }
    if (bytes > (uint64_t(1) << 62)) {
        error = "nt_malloc: size out of range";
        return NT_ERR_VALUE;
    }
    const uint64_t size = rounded(bytes);
    std::lock_guard<std::mutex> guard(lock_);
    Pool &pool = pools_[device];
    // Smallest idle block of this stream (or of a retired one) that fits and
    // wastes at most half of itself.
    for (auto it = pool.idle.lower_bound(size); it != pool.idle.end() && it->first <= 2 * size; ++it) {
        Block *b = it->second;
        if (b->device != device || (b->stream != stream && !b->any_stream) || !settled(b)) continue;
        pool.idle.erase(it);
        b->stream = stream;
        b->any_stream = false;
        b->also_used.clear();
        live_[b->ptr] = b;
        pool.in_use += b->size;
        *out = b->ptr;
        return NT_OK;
    }
    void *ptr = nullptr;
    int status = ops_.device_alloc(device, size, &ptr, error);
    if (status == 1) {
        trim_locked(device, pool);
        status = ops_.device_alloc(device, size, &ptr, error);
    }
    if (status != 0) {
        error += " (" + std::to_string(size) + " bytes; " + std::to_string(pool.in_use) + " in use, " +
                 std::to_string(pool.reserved) + " reserved)";
        return NT_ERR_HIP;
    }
    Block *b = new Block;
    b->ptr = ptr;
    b->size = size;
    b->device = device;
    b->stream = stream;
    live_[ptr] = b;
    pool.reserved += size;
    pool.in_use += size;
    *out = ptr;
    return NT_OK;
}

int32_t DevicePool::record(void *ptr, void *stream, std::string &error) {
    std::lock_guard<std::mutex> guard(lock_);
    auto it = live_.find(ptr);
    if (it == live_.end()) {
        error = "nt_record_stream: not a live allocation of this library";
        return NT_ERR_VALUE;
    }
    Block *b = it->second;
    if (stream == b->stream) return NT_OK;
    for (void *known : b->also_used)
        if (known == stream) return NT_OK;
    b->also_used.push_back(stream);
    return NT_OK;
}

int32_t DevicePool::release(void *ptr, std::string &error) {
    if (ptr == nullptr) return NT_OK;
    std::lock_guard<std::mutex> guard(lock_);
    auto it = live_.find(ptr);
    if (it == live_.end()) {
        error = "nt_free: not a live allocation of this library";
        return NT_ERR_VALUE;
    }
    Block *b = it->second;
    live_.erase(it);
    Pool &pool = pools_[b->device];
    pool.in_use -= b->size;
    for (void *other : b->also_used) {
        void *event = ops_.event_record(b->device, other);
        if (event == nullptr) {
            // The other stream cannot be tracked: keep the block out of the
            // pool for good (its memory may still be read).
            for (void *pending : b->pending) ops_.event_destroy(pending);
            pool.reserved -= b->size;
            delete b;
            return NT_OK;
        }
        b->pending.push_back(event);
    }
    b->also_used.clear();
    for (void *gone : retired_)
        if (gone == b->stream) b->any_stream = true;
    pool.idle.emplace(b->size, b);
    return NT_OK;
}

void DevicePool::retire_stream(void *stream) {
    std::lock_guard<std::mutex> guard(lock_);
    for (auto &entry : pools_)
        for (auto &idle : entry.second.idle)
            if (idle.second->stream == stream) idle.second->any_stream = true;
    for (void *gone : retired_)
        if (gone == stream) return;
    retired_.push_back(stream);
}

void DevicePool::revive_stream(void *stream) {
    std::lock_guard<std::mutex> guard(lock_);
    for (auto it = retired_.begin(); it != retired_.end(); ++it)
        if (*it == stream) {
            retired_.erase(it);
            return;
        }
}

void DevicePool::stats(int32_t device, uint64_t *in_use, uint64_t *reserved) {
    std::lock_guard<std::mutex> guard(lock_);
    const Pool &pool = pools_[device];
    if (in_use) *in_use = pool.in_use;
    if (reserved) *reserved = pool.reserved;
}

void DevicePool::trim(int32_t device) {
    std::lock_guard<std::mutex> guard(lock_);
    trim_locked(device, pools_[device]);
}

// ---- host pool ----------------------------------------------------------------------------
HostPool::~HostPool() {
    // Buffers are not returned (the library's pools live until the process
    // ends); pending events are released.
    for (Idle &idle : idle_)
        for (void *event : idle.after) ops_.event_destroy(event);
}

bool HostPool::settled(Idle &idle) {
    for (void *event : idle.after)
        if (!ops_.event_done(event)) return false;
    for (void *event : idle.after) ops_.event_destroy(event);
    idle.after.clear();
    return true;
}

uint64_t HostPool::rounded(uint64_t bytes) {
    uint64_t size = 4096;
    while (size < bytes && size < (uint64_t(1) << 62)) size <<= 1;
    return size;
}

int32_t HostPool::take(uint64_t bytes, void **out, std::string &error) {
    if (out == nullptr) {
        error = "host pool: output pointer is NULL";
        return NT_ERR_VALUE;
    }
    *out = nullptr;
    const uint64_t size = rounded(bytes);
    {
        std::lock_guard<std::mutex> guard(lock_);
        for (size_t k = 0; k < idle_.size(); ++k) {
            if (idle_[k].size != size || !settled(idle_[k])) continue;
            *out = idle_[k].ptr;
            idle_bytes_ -= size;
            idle_.erase(idle_.begin() + (std::ptrdiff_t)k);
            return NT_OK;
        }
    }
    return ops_.host_alloc(size, out, error) == 0 ? NT_OK : NT_ERR_HIP;
}

void HostPool::give(void *ptr, uint64_t bytes, std::vector<void *> after) {
    if (ptr == nullptr) {
        for (void *event : after) ops_.event_destroy(event);
        return;
    }
    const uint64_t size = rounded(bytes);
    std::lock_guard<std::mutex> guard(lock_);
    idle_.push_back(Idle{ptr, size, std::move(after)});
    idle_bytes_ += size;
    // Over budget: release settled buffers, largest first.
    while (idle_bytes_ > keep_bytes_) {
        size_t pick = idle_.size();
        for (size_t k = 0; k < idle_.size(); ++k)
            if ((pick == idle_.size() || idle_[k].size > idle_[pick].size) && settled(idle_[k])) pick = k;
        if (pick == idle_.size()) break;
        ops_.host_free(idle_[pick].ptr);
        idle_bytes_ -= idle_[pick].size;
        idle_.erase(idle_.begin() + (std::ptrdiff_t)pick);
    }
}

size_t HostPool::idle_count() {
    std::lock_guard<std::mutex> guard(lock_);
    return idle_.size();
}

uint64_t HostPool::idle_bytes() {
    std::lock_guard<std::mutex> guard(lock_);
    return idle_bytes_;
}

}  // namespace nt
