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
};

namespace nt {

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

// Validate a plan pointer.
int32_t check_plan(const nt_plan *plan);

}  // namespace nt

#define NT_HIP_TRY(expr, what)                                   \
    do {                                                         \
        int32_t nt_rc_ = nt::hip_check((expr), (what));          \
        if (nt_rc_ != NT_OK) return nt_rc_;                      \
    } while (0)

#define NT_LAUNCH_CHECK(what) NT_HIP_TRY(hipGetLastError(), what)
