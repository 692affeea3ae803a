// nt_layout.hpp — device-table layouts shared by the kernels and the
// host-side plan builder (plain C++: no HIP headers, so the builder can also
// be compiled by the host compiler for its unit test).
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace nt {

// One descriptor per tensor of a multi-tensor plan (64 bytes, one cache line
// of the scalar data cache).
struct alignas(64) DevTensor {
    void *param;
    void *grad;
    void *exp_avg;
    void *exp_avg_sq;
    void *model_copy;
    uint64_t numel;
    uint32_t slot;
    uint32_t flags;       // bit 0: every role pointer is 16-byte aligned
    // A gradient of the grad dtype still to be added to `grad` (the last
    // micro-batch's accumulation, deferred): the kernels that take it use
    // round(grad + incoming) as the gradient and do not write `grad`.
    // NULL: none.
    const void *incoming;
};
static_assert(sizeof(DevTensor) == 64, "descriptor layout");
static_assert(offsetof(DevTensor, param) == 0 && offsetof(DevTensor, grad) == 8 && offsetof(DevTensor, exp_avg) == 16 &&
                  offsetof(DevTensor, exp_avg_sq) == 24 && offsetof(DevTensor, model_copy) == 32 &&
                  offsetof(DevTensor, incoming) == 56,
              "pointer columns of the descriptor (nt_plan_set_pointers)");
constexpr uint32_t kAligned16 = 1u;
constexpr int32_t kIncomingColumn = 5;
// Byte offset of pointer column c (0 param .. 4 model_copy, 5 incoming).
constexpr size_t column_offset(int32_t c) { return c == kIncomingColumn ? offsetof(DevTensor, incoming) : (size_t)c * 8; }

// One task per `chunk` consecutive elements of one tensor; workgroup i of a
// multi-tensor launch processes task i.
struct Task {
    uint32_t tensor;
    uint32_t chunk;
};
static_assert(sizeof(Task) == 8, "task layout");

constexpr int64_t kChunkQuantum = 2048;   // chunk sizes are multiples of this (16-byte aligned starts)
constexpr int64_t kDefaultChunk = 4096;

// The workgroup -> element arithmetic of the kernels, plain integer code
// that also builds with the host compiler (its unit test checks it at full
// grid sizes).
#if defined(__HIPCC__)
#define NT_LAYOUT_FN __host__ __device__ inline __attribute__((always_inline))
#else
#define NT_LAYOUT_FN inline
#endif

// ---- split launches ----------------------------------------------------------------------
// A plan task of `chunk` elements may run on 2**shift workgroups, each taking
// a slice of chunk >> shift elements: workgroup b covers slice
// (b mod 2**shift) of task (b >> shift).  Streaming kernels use it to pick
// the workgroup shape that moves their read/write mix fastest while the task
// map stays as built.
struct Slice {
    uint64_t start, end;
};

// The dispatcher deals the workgroups of a grid to the eight XCDs in turn
// (workgroup b runs on XCD b mod 8).  With per_xcd > 0 the grid's work is
// renumbered so that it is walked in groups of 8 * per_xcd workgroups and,
// within a group, each XCD takes one contiguous run of per_xcd (a short last
// group is split the same way, the first n mod 8 XCDs taking one more): each
// XCD then streams contiguous address ranges while the group front still
// moves through memory in order.  A bijection on [0, n); per_xcd == 0 keeps
// the launch order.
NT_LAYOUT_FN uint32_t xcd_grouped(uint32_t b, uint32_t n, uint32_t per_xcd) {
    if (per_xcd == 0u) return b;
    const uint32_t size = 8u * per_xcd;
    const uint32_t base = b / size * size;
    const uint32_t m = n - base < size ? n - base : size, w = b - base;
    const uint32_t q = m / 8u, r = m % 8u, x = w % 8u;
    return base + x * q + (x < r ? x : r) + w / 8u;
}

// Slice `part` of `task` in a tensor of `numel` elements; false when it
// starts past the tensor's end (the last task of a tensor may be short).
NT_LAYOUT_FN bool slice_of(const Task &task, uint32_t part, uint64_t numel, int64_t chunk, int32_t shift,
                           Slice &slice) {
    const uint64_t width = (uint64_t)chunk >> shift;
    slice.start = (uint64_t)task.chunk * (uint64_t)chunk + (uint64_t)part * width;
    slice.end = slice.start + width < numel ? slice.start + width : numel;
    return slice.start < numel;
}

}  // namespace nt
