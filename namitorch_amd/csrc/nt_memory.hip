// nt_memory.hip — device memory, streams, events, copies, fills and casts of
// the C ABI, so a host layer can run the optimizer step with no other GPU
// framework.  The reference gets these from CuPy (backends/_cuda_memory.py,
// backends/_cuda_execution.py, backends/cuda/__init__.py:87-153); here they
// are the library's own.
//
// Memory comes from the stream-ordered caching pools of nt_pool.hpp, with
// HIP as their device services.  The pools live until the process ends
// (they are never destroyed, so no HIP call runs during static teardown).
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <thread>
#include <unordered_set>

#include "nt_internal.hpp"
#include "nt_pool.hpp"

namespace nt {
namespace {

// Streams that nt_stream_destroy has destroyed, each after waiting for all
// its work, until HIP hands the same handle out again (nt_stream_create).
// A plan or pool block used on such a stream may be released later (objects
// are finalized in any order when a reference cycle is collected): its
// release needs no ordering after that stream, and an event must not be
// recorded on a destroyed handle.
struct DestroyedStreams {
    std::mutex lock;
    std::unordered_set<void *> handles;
};

DestroyedStreams &destroyed_streams() {
    static DestroyedStreams *streams = new DestroyedStreams();   // never destroyed, like the pools
    return *streams;
}

}  // namespace

bool stream_destroyed(void *stream) {
    if (stream == nullptr) return false;
    DestroyedStreams &d = destroyed_streams();
    std::lock_guard<std::mutex> guard(d.lock);
    return d.handles.count(stream) != 0;
}

namespace {

class HipOps final : public PoolOps {
  public:
    int device_alloc(int32_t device, uint64_t bytes, void **out, std::string &error) override {
        DeviceGuard guard(device);
        if (!guard.ok()) {
            error = "hipSetDevice failed";
            return -1;
        }
        const hipError_t status = hipMalloc(out, bytes);
        if (status == hipSuccess) return 0;
        (void)hipGetLastError();
        error = std::string("hipMalloc: ") + hipGetErrorName(status);
        return (status == hipErrorOutOfMemory || status == hipErrorMemoryAllocation) ? 1 : -1;
    }
    void device_free(int32_t device, void *ptr) override {
        DeviceGuard guard(device);
        if (hipFree(ptr) != hipSuccess) (void)hipGetLastError();
    }
    int host_alloc(uint64_t bytes, void **out, std::string &error) override {
        const hipError_t status = hipHostMalloc(out, bytes, hipHostMallocDefault);
        if (status == hipSuccess) return 0;
        (void)hipGetLastError();
        error = std::string("hipHostMalloc: ") + hipGetErrorName(status);
        return -1;
    }
    void host_free(void *ptr) override {
        if (hipHostFree(ptr) != hipSuccess) (void)hipGetLastError();
    }
    void *event_record(int32_t device, void *stream) override {
        DeviceGuard guard(device);
        hipEvent_t event = nullptr;
        if (hipEventCreateWithFlags(&event, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        // A destroyed stream's work has completed: an event never recorded
        // reads as complete.
        if (stream_destroyed(stream)) return event;
        if (hipEventRecord(event, (hipStream_t)stream) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipEventDestroy(event);
            return nullptr;
        }
        return event;
    }
    bool event_done(void *event) override {
        const hipError_t status = hipEventQuery((hipEvent_t)event);
        if (status == hipErrorNotReady) {
            (void)hipGetLastError();
            return false;
        }
        if (status != hipSuccess) (void)hipGetLastError();   // a failed event cannot guard anything
        return true;
    }
    void event_destroy(void *event) override {
        if (hipEventDestroy((hipEvent_t)event) != hipSuccess) (void)hipGetLastError();
    }
    void device_synchronize(int32_t device) override {
        DeviceGuard guard(device);
        if (hipDeviceSynchronize() != hipSuccess) (void)hipGetLastError();
    }
};

}  // namespace

PoolOps &hip_pool_ops() {
    static HipOps *ops = new HipOps();       // never destroyed
    return *ops;
}

DevicePool &device_pool() {
    static DevicePool *pool = new DevicePool(hip_pool_ops());
    return *pool;
}

HostPool &host_pool() {
    static HostPool *pool = new HostPool(hip_pool_ops());
    return *pool;
}


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
    std::string error;
    const int32_t rc = device_pool().allocate(device, bytes, stream, out, error);
    return rc == NT_OK ? NT_OK : fail(rc, error);
}

int32_t nt_record_stream(void *ptr, void *stream) {
    clear_error();
    std::string error;
    const int32_t rc = device_pool().record(ptr, stream, error);
    return rc == NT_OK ? NT_OK : fail(rc, error);
}

int32_t nt_free(void *ptr) {
    clear_error();
    std::string error;
    const int32_t rc = device_pool().release(ptr, error);
    return rc == NT_OK ? NT_OK : fail(rc, error);
}

int32_t nt_memory_stats(int32_t device, uint64_t *in_use, uint64_t *reserved) {
    clear_error();
    device_pool().stats(device, in_use, reserved);
    return NT_OK;
}

int32_t nt_empty_cache(int32_t device) {
    clear_error();
    if (device < 0) return fail(NT_ERR_VALUE, "nt_empty_cache: invalid device");
    device_pool().trim(device);
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

int32_t nt_mirror_alloc(int32_t count, nt_amp_mirror **out) {
    clear_error();
    if (out == nullptr) return fail(NT_ERR_VALUE, "nt_mirror_alloc: output pointer is NULL");
    *out = nullptr;
    if (count < 1 || count > (1 << 20)) return fail(NT_ERR_VALUE, "nt_mirror_alloc: count must be in [1, 2**20]");
    void *memory = nullptr;
    const size_t bytes = (size_t)count * sizeof(nt_amp_mirror);
    NT_HIP_TRY(hipHostMalloc(&memory, bytes, hipHostMallocCoherent), "hipHostMalloc(coherent)");
    std::memset(memory, 0, bytes);
    *out = static_cast<nt_amp_mirror *>(memory);
    return NT_OK;
}

// Wait until the kernel queued on `stream` to fill `mirror` has set its
// flag.  The flag is polled; every 64 polls the stream is queried, and once
// all its work has completed with the flag still clear, no queued kernel was
// going to write it (an error, not a hang).  Nothing is recorded on the
// stream, so waiting adds no marker to it.
int32_t nt_mirror_wait(const nt_amp_mirror *mirror, void *stream) {
    clear_error();
    if (mirror == nullptr) return fail(NT_ERR_VALUE, "nt_mirror_wait: mirror is NULL");
    for (uint32_t poll = 1;; ++poll) {
        if (__atomic_load_n(&mirror->ready, __ATOMIC_ACQUIRE) != 0) return NT_OK;
        if (poll % 64u == 0u) {
            bool idle = stream_destroyed(stream);
            if (!idle) {
                const hipError_t status = hipStreamQuery((hipStream_t)stream);
                if (status == hipSuccess) {
                    idle = true;
                } else if (status == hipErrorNotReady) {
                    (void)hipGetLastError();
                } else {
                    return hip_check(status, "hipStreamQuery");
                }
            }
            if (idle) {
                if (__atomic_load_n(&mirror->ready, __ATOMIC_ACQUIRE) != 0) return NT_OK;
                return fail(NT_ERR_RUNTIME, "nt_mirror_wait: the stream completed without writing the mirror");
            }
            std::this_thread::yield();
        } else {
            __builtin_ia32_pause();
        }
    }
}

int32_t nt_mirror_free(nt_amp_mirror *mirrors) {
    clear_error();
    if (mirrors != nullptr) NT_HIP_TRY(hipHostFree(mirrors), "hipHostFree");
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
    {
        DestroyedStreams &d = destroyed_streams();
        std::lock_guard<std::mutex> lock(d.lock);
        d.handles.erase(s);                         // the handle is live again
    }
    device_pool().revive_stream(s);
    *out = s;
    return NT_OK;
}

int32_t nt_stream_destroy(void *stream) {
    clear_error();
    if (stream == nullptr) return NT_OK;
    // Everything queued on the stream completes first, so the plans and pool
    // blocks that were used on it need no ordering after it any more.
    NT_HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    NT_HIP_TRY(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
    {
        DestroyedStreams &d = destroyed_streams();
        std::lock_guard<std::mutex> lock(d.lock);
        d.handles.insert(stream);
    }
    // Its pool blocks become reusable on every stream.
    device_pool().retire_stream(stream);
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
