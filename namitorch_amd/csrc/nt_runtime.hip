// nt_runtime.hip — error reporting, device helpers and multi-tensor plans.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "nt_internal.hpp"
#include "nt_pool.hpp"
#include "nt_tables.hpp"

namespace nt {

static thread_local std::string g_last_error;

int32_t fail(int32_t code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

int32_t hip_check(hipError_t err, const char *what) {
    if (err == hipSuccess) return NT_OK;
    // Consume the runtime's per-thread last error, so that a later launch
    // check (hipGetLastError) reports that launch and not this failure.
    (void)hipGetLastError();
    return fail(NT_ERR_HIP, std::string(what) + ": " + hipGetErrorName(err) + " (" +
                                hipGetErrorString(err) + ")");
}

DeviceGuard::DeviceGuard(int32_t device) {
    err_ = hipGetDevice(&prev_);
    if (err_ != hipSuccess) {
        ok_ = false;
        prev_ = -1;
        return;
    }
    if (prev_ != device) {
        err_ = hipSetDevice(device);
        ok_ = (err_ == hipSuccess);
    }
}

DeviceGuard::~DeviceGuard() {
    int cur = -1;
    if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_ && hipSetDevice(prev_) != hipSuccess)
        (void)hipGetLastError();
}

Xform make_xform(const nt_grad_xform *x) {
    Xform r{};
    r.scale = 1.0f;
    r.inv_scale = 1.0f;
    r.clip_coef = 1.0;
    if (x == nullptr) return r;
    r.scale = x->scale;
    if (x->unscale) {
        // Dividing by a power of two equals multiplying by its exact inverse
        // (both round the same real number once), so use the multiply then.
        int e = 0;
        float m = frexpf(x->scale, &e);
        float inv = ldexpf(1.0f, 1 - e);
        bool pow2 = (m == 0.5f) && inv != 0.0f && (double)inv * (double)x->scale == 1.0;
        r.unscale = pow2 ? 2 : 1;
        r.inv_scale = pow2 ? inv : 1.0f;
    }
    r.clip = x->clip ? 1 : 0;
    r.clip_coef = x->clip_coef;
    return r;
}

int32_t check_plan(const nt_plan *plan) {
    if (plan == nullptr) return fail(NT_ERR_VALUE, "multi-tensor plan is NULL");
    return NT_OK;
}

int32_t check_no_incoming(const nt_plan *plan, const char *entry) {
    if (plan->n_incoming == 0) return NT_OK;
    return fail(NT_ERR_VALUE, std::string(entry) +
                                  ": the plan has incoming gradients (column 5); add them into the stored "
                                  "gradients first (nt_grad_accumulate) or clear the column");
}

}  // namespace nt

using namespace nt;

extern "C" {

const char *nt_last_error(void) { return g_last_error.c_str(); }

int32_t nt_abi_version(void) { return 4; }

int32_t nt_hip_version(int32_t *built, int32_t *runtime) {
    clear_error();
    if (built == nullptr || runtime == nullptr) return fail(NT_ERR_VALUE, "nt_hip_version: NULL output");
    *built = HIP_VERSION;
    int version = 0;
    NT_HIP_TRY(hipRuntimeGetVersion(&version), "hipRuntimeGetVersion");
    *runtime = version;
    return NT_OK;
}

int32_t nt_device_count(int32_t *count) {
    clear_error();
    if (count == nullptr) return fail(NT_ERR_VALUE, "count is NULL");
    int c = 0;
    hipError_t err = hipGetDeviceCount(&c);
    if (err == hipErrorNoDevice) c = 0;
    else NT_HIP_TRY(err, "hipGetDeviceCount");
    *count = c;
    return NT_OK;
}

int32_t nt_device_arch(int32_t device, char *buf, int32_t len) {
    clear_error();
    if (buf == nullptr || len <= 0) return fail(NT_ERR_VALUE, "arch buffer is empty");
    hipDeviceProp_t prop;
    NT_HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    std::strncpy(buf, prop.gcnArchName, (size_t)len - 1);
    buf[len - 1] = '\0';
    return NT_OK;
}

int32_t nt_set_device(int32_t device) {
    clear_error();
    NT_HIP_TRY(hipSetDevice(device), "hipSetDevice");
    return NT_OK;
}

int32_t nt_get_device(int32_t *device) {
    clear_error();
    if (device == nullptr) return fail(NT_ERR_VALUE, "device output pointer is NULL");
    int d = 0;
    NT_HIP_TRY(hipGetDevice(&d), "hipGetDevice");
    *device = d;
    return NT_OK;
}

int32_t nt_stream_synchronize(void *stream) {
    clear_error();
    NT_HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return NT_OK;
}

int32_t nt_memcpy_d2h(void *dst, const void *src, uint64_t bytes, void *stream) {
    clear_error();
    if (bytes == 0) return NT_OK;
    if (dst == nullptr || src == nullptr) return fail(NT_ERR_VALUE, "memcpy with NULL pointer");
    NT_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync(D2H)");
    NT_HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return NT_OK;
}

int32_t nt_memcpy_h2d(void *dst, const void *src, uint64_t bytes, void *stream) {
    clear_error();
    if (bytes == 0) return NT_OK;
    if (dst == nullptr || src == nullptr) return fail(NT_ERR_VALUE, "memcpy with NULL pointer");
    NT_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync(H2D)");
    NT_HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return NT_OK;
}

int32_t nt_plan_create(int32_t device, const nt_mt_tensor *tensors, int32_t n,
                       const nt_mt_layout *layout, int64_t chunk, void *stream, nt_plan **out) {
    clear_error();
    if (out == nullptr) return fail(NT_ERR_VALUE, "plan output pointer is NULL");
    *out = nullptr;
    PlanTables tables;
    std::string error;
    int32_t built = build_plan_tables(tensors, n, layout, chunk, tables, error);
    if (built != NT_OK) return fail(built, error);
    const std::vector<DevTensor> &host = tables.tensors;
    const std::vector<Task> &tasks = tables.tasks;
    const uint64_t total = tables.numel;
    const uint32_t max_slot = tables.max_slot;
    chunk = tables.chunk;

    DeviceGuard guard(device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");

    nt_plan *plan = new nt_plan{};
    plan->device = device;
    plan->ntensors = n;
    plan->layout = *layout;
    plan->numel = total;
    plan->chunk = chunk;
    plan->ntasks = (int64_t)tasks.size();
    plan->max_slot = max_slot;
    plan->npartials = plan->ntasks > 0 ? (plan->ntasks + kPrepassTasks - 1) / kPrepassTasks : 1;
    plan->nstage2 = plan->npartials > kFinalizeDirect ? (plan->npartials + kStage2Span - 1) / kStage2Span : 0;
    int64_t grid = plan->ntasks < 4096 ? plan->ntasks : 4096;
    plan->pow_grid = (int32_t)(grid > 0 ? grid : 1);

    plan->flags.reserve((size_t)n);
    for (int32_t t = 0; t < n; ++t) plan->flags.push_back(host[(size_t)t].flags);

    hipStream_t s = (hipStream_t)stream;
    plan->stream = s;
    // Device tables from the library's pool (ordered on the creation
    // stream); the staging copy of the tables and the pointer ring share
    // one page-locked buffer from the host pool.
    auto cleanup = [&](int32_t rc) {
        (void)hipStreamSynchronize(s);     // nothing queued may still read what is returned below
        std::string ignored;
        for (void *block : {(void *)plan->d_tensors, (void *)plan->d_tasks, (void *)plan->d_partials,
                            (void *)plan->d_partials2, (void *)plan->d_pow_partials})
            if (block) (void)device_pool().release(block, ignored);
        for (int r = 0; r < kRingSlots; ++r)
            if (plan->ring_events[r]) (void)hipEventDestroy(plan->ring_events[r]);
        if (plan->h_staging) host_pool().give(plan->h_staging, plan->host_bytes, {});
        delete plan;
        (void)hipGetLastError();
        return rc;
    };
    const size_t tensor_bytes = host.size() * sizeof(DevTensor);
    const size_t task_bytes = (tasks.empty() ? 1 : tasks.size()) * sizeof(Task);
    const size_t ring_bytes = (size_t)kRingSlots * host.size() * sizeof(void *);
    auto take = [&](void **out, size_t bytes, const char *what) {
        const int32_t code = device_pool().allocate(device, bytes, stream, out, error);
        return code == NT_OK ? NT_OK : fail(code, std::string(what) + ": " + error);
    };
    int32_t rc;
    if ((rc = take((void **)&plan->d_tensors, tensor_bytes, "plan tensors")) != NT_OK) return cleanup(rc);
    if ((rc = take((void **)&plan->d_tasks, task_bytes, "plan tasks")) != NT_OK) return cleanup(rc);
    if ((rc = take((void **)&plan->d_partials, (size_t)plan->npartials * sizeof(Partial), "plan partials")) != NT_OK)
        return cleanup(rc);
    if ((rc = take((void **)&plan->d_partials2, (size_t)(plan->nstage2 > 0 ? plan->nstage2 : 1) * sizeof(Partial),
                   "plan partials")) != NT_OK)
        return cleanup(rc);
    if ((rc = take((void **)&plan->d_pow_partials, (size_t)plan->pow_grid * sizeof(double), "plan partials")) != NT_OK)
        return cleanup(rc);
    plan->host_bytes = tensor_bytes + task_bytes + ring_bytes;
    if (host_pool().take(plan->host_bytes, &plan->h_staging, error) != NT_OK)
        return cleanup(fail(NT_ERR_HIP, "plan staging: " + error));
    plan->h_ring = static_cast<char *>(plan->h_staging) + tensor_bytes + task_bytes;
    for (int r = 0; r < kRingSlots; ++r)
        if ((rc = hip_check(hipEventCreateWithFlags(&plan->ring_events[r], hipEventDisableTiming), "hipEventCreate(plan ring)")) != NT_OK) return cleanup(rc);
    char *staging = static_cast<char *>(plan->h_staging);
    std::memcpy(staging, host.data(), tensor_bytes);
    if (!tasks.empty()) std::memcpy(staging + tensor_bytes, tasks.data(), tasks.size() * sizeof(Task));
    if ((rc = hip_check(hipMemcpyAsync(plan->d_tensors, staging, tensor_bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync(plan tensors)")) != NT_OK) return cleanup(rc);
    if (!tasks.empty() &&
        (rc = hip_check(hipMemcpyAsync(plan->d_tasks, staging + tensor_bytes, tasks.size() * sizeof(Task), hipMemcpyHostToDevice, s), "hipMemcpyAsync(plan tasks)")) != NT_OK)
        return cleanup(rc);
    *out = plan;
    return NT_OK;
}

int32_t nt_plan_destroy(nt_plan *plan) {
    clear_error();
    if (plan == nullptr) return NT_OK;
    DeviceGuard guard(plan->device);
    // Kernels queued with this plan may still read its tables: the device
    // blocks return to the pool in the order of every stream that used the
    // plan, and the page-locked buffer once each of those streams has passed
    // this point.  Nothing waits here.
    std::string ignored;
    for (void *block : {(void *)plan->d_tensors, (void *)plan->d_tasks, (void *)plan->d_partials,
                        (void *)plan->d_partials2, (void *)plan->d_pow_partials}) {
        if (block == nullptr) continue;
        for (hipStream_t other : plan->others) (void)device_pool().record(block, other, ignored);
        (void)device_pool().release(block, ignored);
    }
    std::vector<void *> after;
    bool tracked = true;
    for (size_t k = 0; k <= plan->others.size() && tracked; ++k) {
        void *event = hip_pool_ops().event_record(plan->device, k == 0 ? plan->stream : plan->others[k - 1]);
        if (event == nullptr) tracked = false;
        else after.push_back(event);
    }
    if (!tracked) {
        // A stream could not be tracked: wait for the device instead.
        for (void *event : after) hip_pool_ops().event_destroy(event);
        after.clear();
        (void)hipDeviceSynchronize();
    }
    host_pool().give(plan->h_staging, plan->host_bytes, std::move(after));
    // The ring's events were recorded on the plan's streams.  When one of
    // those streams is already destroyed (a reference cycle finalized it
    // first), the four events are left to the process rather than destroyed.
    bool streams_alive = !stream_destroyed(plan->stream);
    for (hipStream_t other : plan->others) streams_alive = streams_alive && !stream_destroyed(other);
    if (streams_alive)
        for (int r = 0; r < kRingSlots; ++r) (void)hipEventDestroy(plan->ring_events[r]);
    delete plan;
    (void)hipGetLastError();   // teardown is best effort; leave no error for a later launch check
    return NT_OK;
}

int32_t nt_plan_set_pointers(nt_plan *plan, int32_t column, const void *const *pointers, int32_t n, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if (n == 0 && plan->ntensors == 0) return NT_OK;
    std::string error;
    rc = check_pointer_column(plan->layout, plan->flags, column, pointers, n, error);
    if (rc != NT_OK) return fail(rc, error);
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    // The slot's previous upload must have left it before it is rewritten.
    const int32_t slot = plan->ring_next;
    plan->ring_next = (slot + 1) % kRingSlots;
    if (plan->ring_used[slot]) NT_HIP_TRY(hipEventSynchronize(plan->ring_events[slot]), "hipEventSynchronize(plan ring)");
    const void **ring = static_cast<const void **>(plan->h_ring) + (size_t)slot * n;
    std::memcpy(ring, pointers, (size_t)n * sizeof(void *));
    hipStream_t s = (hipStream_t)stream;
    // Strided copy into column `column` of every descriptor, ordered on the
    // stream after the kernels already queued with the old pointers.
    char *dst = reinterpret_cast<char *>(plan->d_tensors) + column_offset(column);
    NT_HIP_TRY(hipMemcpy2DAsync(dst, sizeof(DevTensor), ring, sizeof(void *), sizeof(void *), (size_t)n,
                                hipMemcpyHostToDevice, s), "hipMemcpy2DAsync(plan pointers)");
    NT_HIP_TRY(hipEventRecord(plan->ring_events[slot], s), "hipEventRecord(plan ring)");
    plan->ring_used[slot] = true;
    if (column == kIncomingColumn) {
        int32_t set = 0;
        for (int32_t t = 0; t < n; ++t) set += pointers[t] != nullptr;
        plan->n_incoming = set;
    }
    return NT_OK;
}

int32_t nt_plan_info(const nt_plan *plan, uint64_t *numel, int32_t *tensors, int64_t *tasks) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if (numel) *numel = plan->numel;
    if (tensors) *tensors = plan->ntensors;
    if (tasks) *tasks = plan->ntasks;
    return NT_OK;
}

}  // extern "C"
