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

}  // namespace nt
