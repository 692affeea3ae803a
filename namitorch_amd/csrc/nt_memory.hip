// nt_memory.hip — device memory, streams, events, copies, fills and casts of
// the C ABI, so a host layer can run the optimizer step with no other GPU
// framework.  The reference gets these from CuPy (backends/_cuda_memory.py,
// backends/_cuda_execution.py, backends/cuda/__init__.py:87-153); here they
// are the library's own.
//
// Allocation is a per-device caching pool ordered by streams, the way CuPy's
// and PyTorch's pools work: a block is allocated on a stream; freeing it
// returns it to the pool for reuse by later allocations on that same stream,
// which stream order already places after every use queued on it.  A block
// used on other streams as well (nt_record_stream) is reused only after an
// event recorded on each of those streams at free time has completed.
// Blocks are never handed across streams, so the pool never synchronizes.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "nt_internal.hpp"

namespace nt {
namespace {

constexpr uint64_t kSmallRound = 512;                  // blocks up to 1 MiB: 512-byte steps
constexpr uint64_t kLargeRound = uint64_t(2) << 20;    // larger blocks: 2 MiB steps
constexpr uint64_t kSmallLimit = uint64_t(1) << 20;

struct Block {
    void *ptr = nullptr;
    uint64_t size = 0;
    int32_t device = 0;
    hipStream_t stream = nullptr;                       // allocation stream: reuse happens only on it
    std::vector<hipStream_t> also_used;                 // streams recorded with nt_record_stream
    std::vector<hipEvent_t> pending;                    // events to complete before reuse
};

struct Pool {
    std::multimap<uint64_t, Block *> free_blocks;       // by size
    uint64_t reserved = 0;                              // bytes obtained from hipMalloc
    uint64_t in_use = 0;                                // bytes handed out
};

std::mutex g_lock;
std::map<int32_t, Pool> g_pools;
std::unordered_map<void *, Block *> g_live;

uint64_t rounded(uint64_t bytes) {
    if (bytes == 0) bytes = 1;
    const uint64_t step = bytes <= kSmallLimit ? kSmallRound : kLargeRound;
    return (bytes + step - 1) / step * step;
}

// True when every pending event of a free block has completed (those events
// are then released).
bool settled(Block *b) {
    for (size_t k = 0; k < b->pending.size(); ++k) {
        const hipError_t status = hipEventQuery(b->pending[k]);
        if (status == hipErrorNotReady) return false;
        if (status != hipSuccess) (void)hipGetLastError();
    }
    for (hipEvent_t e : b->pending) (void)hipEventDestroy(e);
    b->pending.clear();
    return true;
}

// Release every free block of `pool` that has settled (after a device-wide wait).
void trim(int32_t device, Pool &pool) {
    (void)hipDeviceSynchronize();
    for (auto it = pool.free_blocks.begin(); it != pool.free_blocks.end();) {
        Block *b = it->second;
        if (settled(b)) {
            (void)hipFree(b->ptr);
            pool.reserved -= b->size;
            delete b;
            it = pool.free_blocks.erase(it);
        } else {
            ++it;
        }
    }
    (void)hipGetLastError();
    (void)device;
}

}  // namespace

// ---- element kernels: fill a bit pattern, cast between float types ------------------
__global__ __launch_bounds__(kBlock) void fill_pattern_kernel(uint8_t *out, uint64_t count, int32_t itemsize,
                                                              uint64_t pattern) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < count; i += stride) {
        switch (itemsize) {
            case 1: out[i] = (uint8_t)pattern; break;
            case 2: reinterpret_cast<uint16_t *>(out)[i] = (uint16_t)pattern; break;
            case 4: reinterpret_cast<uint32_t *>(out)[i] = (uint32_t)pattern; break;
            default: reinterpret_cast<uint64_t *>(out)[i] = pattern; break;
        }
    }
}

// out[i] = in[i] converted with one rounding (round to nearest even): the
// value widens exactly to fp64, then rounds once to the output type.
template <class I, class O>
__global__ __launch_bounds__(kBlock) void cast_kernel(const typename I::raw *in, typename O::raw *out, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        out[i] = O::from_f64(widen64<I>(in[i]));
}

template <class I>
static int32_t launch_cast(const void *in, void *out, int32_t out_dtype, uint64_t n, dim3 grid, hipStream_t s) {
    const auto *src = static_cast<const typename I::raw *>(in);
    switch (out_dtype) {
        case NT_F32: cast_kernel<I, TF32><<<grid, dim3(kBlock), 0, s>>>(src, (float *)out, n); break;
        case NT_F16: cast_kernel<I, TF16><<<grid, dim3(kBlock), 0, s>>>(src, (uint16_t *)out, n); break;
        case NT_BF16: cast_kernel<I, TBF16><<<grid, dim3(kBlock), 0, s>>>(src, (uint16_t *)out, n); break;
        case NT_F64: cast_kernel<I, TF64><<<grid, dim3(kBlock), 0, s>>>(src, (double *)out, n); break;
        default: return fail(NT_ERR_TYPE, "nt_cast: unsupported output dtype");
    }
    return NT_OK;
}

static dim3 element_grid(uint64_t n) {
    uint64_t blocks = (n + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    return dim3((unsigned)(blocks ? blocks : 1));
}

}  // namespace nt

using namespace nt;

extern "C" {

// ---- memory -------------------------------------------------------------------------
int32_t nt_malloc(int32_t device, uint64_t bytes, void *stream, void **out) {
    clear_error();
    if (out == nullptr) return fail(NT_ERR_VALUE, "nt_malloc: output pointer is NULL");
    if (device < 0) return fail(NT_ERR_VALUE, "nt_malloc: invalid device");
    *out = nullptr;
    const uint64_t size = rounded(bytes);
    hipStream_t s = (hipStream_t)stream;
    std::lock_guard<std::mutex> lock(g_lock);
    Pool &pool = g_pools[device];
    // Smallest free block of this stream that fits and wastes at most half of itself.
    for (auto it = pool.free_blocks.lower_bound(size); it != pool.free_blocks.end() && it->first <= 2 * size; ++it) {
        Block *b = it->second;
        if (b->device != device || b->stream != s || !settled(b)) continue;
        pool.free_blocks.erase(it);
        b->also_used.clear();
        g_live[b->ptr] = b;
        pool.in_use += b->size;
        *out = b->ptr;
        return NT_OK;
    }
    DeviceGuard guard(device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    void *ptr = nullptr;
    hipError_t status = hipMalloc(&ptr, size);
    if (status == hipErrorOutOfMemory || status == hipErrorMemoryAllocation) {
        (void)hipGetLastError();
        trim(device, pool);
        status = hipMalloc(&ptr, size);
    }
    if (status != hipSuccess)
        return hip_check(status, ("hipMalloc(" + std::to_string(size) + " bytes; " + std::to_string(pool.in_use) +
                                  " in use, " + std::to_string(pool.reserved) + " reserved)").c_str());
    Block *b = new Block;
    b->ptr = ptr;
    b->size = size;
    b->device = device;
    b->stream = s;
    g_live[ptr] = b;
    pool.reserved += size;
    pool.in_use += size;
    *out = ptr;
    return NT_OK;
}

int32_t nt_record_stream(void *ptr, void *stream) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_lock);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) return fail(NT_ERR_VALUE, "nt_record_stream: not a live allocation of this library");
    Block *b = it->second;
    hipStream_t s = (hipStream_t)stream;
    if (s != b->stream) {
        for (hipStream_t known : b->also_used)
            if (known == s) return NT_OK;
        b->also_used.push_back(s);
    }
    return NT_OK;
}

int32_t nt_free(void *ptr) {
    clear_error();
    if (ptr == nullptr) return NT_OK;
    std::lock_guard<std::mutex> lock(g_lock);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) return fail(NT_ERR_VALUE, "nt_free: not a live allocation of this library");
    Block *b = it->second;
    g_live.erase(it);
    Pool &pool = g_pools[b->device];
    pool.in_use -= b->size;
    if (!b->also_used.empty()) {
        DeviceGuard guard(b->device);
        for (hipStream_t other : b->also_used) {
            hipEvent_t e = nullptr;
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess ||
                hipEventRecord(e, other) != hipSuccess) {
                // Cannot track the other stream: keep the block out of the pool.
                (void)hipGetLastError();
                if (e) (void)hipEventDestroy(e);
                for (hipEvent_t p : b->pending) (void)hipEventDestroy(p);
                pool.reserved -= b->size;
                delete b;          // leaked on purpose: its memory may still be read
                return NT_OK;
            }
            b->pending.push_back(e);
        }
        b->also_used.clear();
    }
    pool.free_blocks.emplace(b->size, b);
    return NT_OK;
}

int32_t nt_memory_stats(int32_t device, uint64_t *in_use, uint64_t *reserved) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_lock);
    const Pool &pool = g_pools[device];
    if (in_use) *in_use = pool.in_use;
    if (reserved) *reserved = pool.reserved;
    return NT_OK;
}

int32_t nt_empty_cache(int32_t device) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_lock);
    DeviceGuard guard(device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    trim(device, g_pools[device]);
    return NT_OK;
}

int32_t nt_host_alloc(uint64_t bytes, void **out) {
    clear_error();
    if (out == nullptr) return fail(NT_ERR_VALUE, "nt_host_alloc: output pointer is NULL");
    *out = nullptr;
    NT_HIP_TRY(hipHostMalloc(out, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
    return NT_OK;
}

int32_t nt_host_free(void *ptr) {
    clear_error();
    if (ptr != nullptr) NT_HIP_TRY(hipHostFree(ptr), "hipHostFree");
    return NT_OK;
}

// ---- streams and events -----------------------------------------------------------------
int32_t nt_stream_create(int32_t device, void **out) {
    clear_error();
    if (out == nullptr) return fail(NT_ERR_VALUE, "nt_stream_create: output pointer is NULL");
    DeviceGuard guard(device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    hipStream_t s = nullptr;
    NT_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *out = s;
    return NT_OK;
}

int32_t nt_stream_destroy(void *stream) {
    clear_error();
    if (stream != nullptr) NT_HIP_TRY(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
    return NT_OK;
}

int32_t nt_stream_wait_event(void *stream, void *event) {
    clear_error();
    if (event == nullptr) return fail(NT_ERR_VALUE, "nt_stream_wait_event: NULL event");
    NT_HIP_TRY(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0), "hipStreamWaitEvent");
    return NT_OK;
}

int32_t nt_event_create(int32_t timing, void **out) {
    clear_error();
    if (out == nullptr) return fail(NT_ERR_VALUE, "nt_event_create: output pointer is NULL");
    hipEvent_t e = nullptr;
    NT_HIP_TRY(hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming), "hipEventCreate");
    *out = e;
    return NT_OK;
}

int32_t nt_event_destroy(void *event) {
    clear_error();
    if (event != nullptr) NT_HIP_TRY(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
    return NT_OK;
}

int32_t nt_event_record(void *event, void *stream) {
    clear_error();
    if (event == nullptr) return fail(NT_ERR_VALUE, "nt_event_record: NULL event");
    NT_HIP_TRY(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
    return NT_OK;
}

int32_t nt_event_synchronize(void *event) {
    clear_error();
    if (event == nullptr) return fail(NT_ERR_VALUE, "nt_event_synchronize: NULL event");
    NT_HIP_TRY(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
    return NT_OK;
}

int32_t nt_event_query(void *event, int32_t *done) {
    clear_error();
    if (event == nullptr || done == nullptr) return fail(NT_ERR_VALUE, "nt_event_query: NULL argument");
    const hipError_t status = hipEventQuery((hipEvent_t)event);
    if (status == hipErrorNotReady) {
        (void)hipGetLastError();
        *done = 0;
        return NT_OK;
    }
    NT_HIP_TRY(status, "hipEventQuery");
    *done = 1;
    return NT_OK;
}

int32_t nt_event_elapsed(void *start, void *stop, float *milliseconds) {
    clear_error();
    if (start == nullptr || stop == nullptr || milliseconds == nullptr)
        return fail(NT_ERR_VALUE, "nt_event_elapsed: NULL argument");
    NT_HIP_TRY(hipEventElapsedTime(milliseconds, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsedTime");
    return NT_OK;
}

// ---- copies, fills, casts -------------------------------------------------------------------
int32_t nt_memcpy_async(void *dst, const void *src, uint64_t bytes, int32_t kind, void *stream) {
    clear_error();
    if (bytes == 0) return NT_OK;
    if (dst == nullptr || src == nullptr) return fail(NT_ERR_VALUE, "memcpy with NULL pointer");
    hipMemcpyKind direction;
    switch (kind) {
        case NT_COPY_H2D: direction = hipMemcpyHostToDevice; break;
        case NT_COPY_D2H: direction = hipMemcpyDeviceToHost; break;
        case NT_COPY_D2D: direction = hipMemcpyDeviceToDevice; break;
        default: return fail(NT_ERR_VALUE, "nt_memcpy_async: unknown copy kind");
    }
    NT_HIP_TRY(hipMemcpyAsync(dst, src, bytes, direction, (hipStream_t)stream), "hipMemcpyAsync");
    return NT_OK;
}

int32_t nt_fill(void *ptr, uint64_t count, int32_t itemsize, uint64_t pattern, void *stream) {
    clear_error();
    if (itemsize != 1 && itemsize != 2 && itemsize != 4 && itemsize != 8)
        return fail(NT_ERR_VALUE, "nt_fill: itemsize must be 1, 2, 4 or 8");
    if (count == 0) return NT_OK;
    if (ptr == nullptr) return fail(NT_ERR_VALUE, "nt_fill: NULL array");
    if ((uintptr_t)ptr % (uintptr_t)itemsize != 0) return fail(NT_ERR_VALUE, "nt_fill: array not aligned to its items");
    fill_pattern_kernel<<<element_grid(count), dim3(kBlock), 0, (hipStream_t)stream>>>(static_cast<uint8_t *>(ptr),
                                                                                        count, itemsize, pattern);
    NT_LAUNCH_CHECK("fill_pattern_kernel launch");
    return NT_OK;
}

int32_t nt_cast(const void *in, int32_t in_dtype, void *out, int32_t out_dtype, uint64_t count, void *stream) {
    clear_error();
    if (count == 0) return NT_OK;
    if (in == nullptr || out == nullptr) return fail(NT_ERR_VALUE, "nt_cast: NULL array");
    const dim3 grid = element_grid(count);
    hipStream_t s = (hipStream_t)stream;
    int32_t rc;
    switch (in_dtype) {
        case NT_F32: rc = launch_cast<TF32>(in, out, out_dtype, count, grid, s); break;
        case NT_F16: rc = launch_cast<TF16>(in, out, out_dtype, count, grid, s); break;
        case NT_BF16: rc = launch_cast<TBF16>(in, out, out_dtype, count, grid, s); break;
        case NT_F64: rc = launch_cast<TF64>(in, out, out_dtype, count, grid, s); break;
        default: return fail(NT_ERR_TYPE, "nt_cast: unsupported input dtype");
    }
    if (rc != NT_OK) return rc;
    NT_LAUNCH_CHECK("cast_kernel launch");
    return NT_OK;
}

int32_t nt_pointer_device(const void *ptr, int32_t *device) {
    clear_error();
    if (ptr == nullptr || device == nullptr) return fail(NT_ERR_VALUE, "nt_pointer_device: NULL argument");
    hipPointerAttribute_t attributes{};
    const hipError_t status = hipPointerGetAttributes(&attributes, ptr);
    if (status != hipSuccess) {
        (void)hipGetLastError();
        return fail(NT_ERR_VALUE, "nt_pointer_device: not a device pointer");
    }
    if (attributes.type != hipMemoryTypeDevice) return fail(NT_ERR_VALUE, "nt_pointer_device: not device memory");
    *device = attributes.device;
    return NT_OK;
}

int32_t nt_stream_capturing(void *stream, int32_t *capturing) {
    clear_error();
    if (capturing == nullptr) return fail(NT_ERR_VALUE, "nt_stream_capturing: NULL argument");
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hipError_t err = hipStreamIsCapturing((hipStream_t)stream, &status);
    if (err == hipErrorStreamCaptureImplicit) {
        // The null stream was queried while another stream captures in a
        // mode that forbids null-stream work: report that as a capture.
        (void)hipGetLastError();
        *capturing = 1;
        return NT_OK;
    }
    NT_HIP_TRY(err, "hipStreamIsCapturing");
    *capturing = status == hipStreamCaptureStatusActive ? 1 : 0;
    return NT_OK;
}

}  // extern "C"
