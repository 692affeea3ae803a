// nt_internal.hpp — host-side internals shared by the library's .hip files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include <vector>

#include "nt_common.hpp"

struct nt_plan {
    int32_t device;
    int32_t ntensors;
    nt_mt_layout layout;
    uint64_t numel;
    int64_t chunk;               // elements per workgroup task
    int64_t ntasks;
    int64_t npartials;           // pre-pass workgroups = partial slots
    int64_t nstage2;             // stage-2 workgroups (0: finalize reads the partials directly)
    int32_t pow_grid;            // workgroups of the general p-norm pass
    uint32_t max_slot;           // largest coefficient slot any tensor selects
    nt::DevTensor *d_tensors;    // [ntensors]
    nt::Task *d_tasks;           // [ntasks]
    nt::Partial *d_partials;     // [npartials]
    nt::Partial *d_partials2;    // [max(nstage2, 1)]
    double *d_pow_partials;      // [pow_grid] (general p-norm)
    void *h_staging;             // pinned host copy of the tables (async upload source)
    // Pointer-column updates (nt_plan_set_pointers): per-tensor alignment
    // flags as computed at creation, and a small ring of pinned slots, each
    // reused only after the copy that read it has completed.
    std::vector<uint32_t> flags;
    void *h_ring;                // kRingSlots x ntensors pointers
    hipEvent_t ring_events[nt::kRingSlots];
    bool ring_used[nt::kRingSlots];
    int32_t ring_next;
    // Descriptors whose incoming-gradient column is set: only nt_amp_prepass
    // and nt_adamw_mt (16/32-bit gradients) read that column; every other
    // entry point refuses such a plan rather than ignore the addend.
    int32_t n_incoming;
    // Streams the plan has been used on: the creation stream and any other
    // stream passed to an entry point with this plan.  Its memory returns to
    // the library's pools in their order when the plan is destroyed.
    hipStream_t stream;
    std::vector<hipStream_t> others;
    uint64_t host_bytes;         // h_staging and h_ring share one page-locked buffer of this size
};

namespace nt {

// This workgroup's slice; false when it starts past the end of its tensor
// (the last task of a tensor may be short).  `per_xcd` as in xcd_grouped.
__device__ __forceinline__ bool task_slice(const DevTensor *__restrict__ tensors, const Task *__restrict__ tasks,
                                           int64_t chunk, int32_t shift, const DevTensor *&d, Slice &slice,
                                           uint32_t per_xcd = 0u) {
    const uint32_t b = xcd_grouped(blockIdx.x, gridDim.x, per_xcd);
    const Task task = tasks[b >> shift];
    d = &tensors[task.tensor];
    return slice_of(task, b & ((1u << shift) - 1u), d->numel, chunk, shift, slice);
}

// log2(chunk / slice) when that is a power of two in [1, 64] and the grid
// stays below 2**31 workgroups, else 0 (one workgroup per task).
inline int32_t split_shift(const nt_plan *plan, int64_t slice) {
    if (plan->chunk % slice != 0) return 0;
    const int64_t parts = plan->chunk / slice;
    if (parts > 64 || (parts & (parts - 1)) != 0) return 0;
    int32_t shift = 0;
    while ((int64_t(1) << shift) < parts) ++shift;
    if (plan->ntasks > (int64_t(0x7fffffff) >> shift)) return 0;
    return shift;
}

// Record `msg` as this thread's last error and return `code`.
int32_t fail(int32_t code, const std::string &msg);
// Convert a HIP status into NT_ERR_HIP with context; NT_OK on success.
int32_t hip_check(hipError_t err, const char *what);
// Clear this thread's last error.
void clear_error();

// Scoped switch to `device` (restores the caller's current device).
class DeviceGuard {
  public:
    explicit DeviceGuard(int32_t device);
    ~DeviceGuard();
    bool ok() const { return ok_; }
    hipError_t error() const { return err_; }

  private:
    int prev_ = -1;
    bool ok_ = true;
    hipError_t err_ = hipSuccess;
};

// Device-side transform parameters from a host nt_grad_xform (ctrl ignored).
Xform make_xform(const nt_grad_xform *x);

// The library's caching pools (nt_pool.hpp) over HIP; they live until the process ends.
class PoolOps;
class DevicePool;
class HostPool;
PoolOps &hip_pool_ops();
DevicePool &device_pool();
HostPool &host_pool();

// Validate a plan pointer.
int32_t check_plan(const nt_plan *plan);

// True when `stream` was destroyed by nt_stream_destroy (after all its work
// completed) and its handle has not been handed out again.
bool stream_destroyed(void *stream);

// Remember that `stream` uses `plan` (see nt_plan::others).
inline void note_stream(nt_plan *plan, void *stream) {
    const hipStream_t s = (hipStream_t)stream;
    if (s == plan->stream) return;
    for (hipStream_t known : plan->others)
        if (known == s) return;
    plan->others.push_back(s);
}
// NT_ERR_VALUE (naming `entry`) when the plan has incoming gradients set.
int32_t check_no_incoming(const nt_plan *plan, const char *entry);

}  // namespace nt

#define NT_HIP_TRY(expr, what)                                   \
    do {                                                         \
        int32_t nt_rc_ = nt::hip_check((expr), (what));          \
        if (nt_rc_ != NT_OK) return nt_rc_;                      \
    } while (0)

#define NT_LAUNCH_CHECK(what) NT_HIP_TRY(hipGetLastError(), what)
