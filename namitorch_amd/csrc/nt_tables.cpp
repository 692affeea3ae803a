// nt_tables.cpp — host-side construction and validation of multi-tensor
// plan tables (see nt_tables.hpp).
#include "nt_tables.hpp"

namespace nt {

size_t dtype_size(int32_t dtype) {
    switch (dtype) {
        case NT_F32: return 4;
        case NT_F16:
        case NT_BF16: return 2;
        case NT_F64: return 8;
        default: return 0;
    }
}

bool valid_dtype(int32_t dtype, bool allow_none) {
    return (allow_none && dtype == NT_DTYPE_NONE) || dtype == NT_F32 || dtype == NT_F16 || dtype == NT_BF16 ||
           dtype == NT_F64;
}

int32_t build_plan_tables(const nt_mt_tensor *tensors, int32_t n, const nt_mt_layout *layout, int64_t chunk,
                          PlanTables &out, std::string &error) {
    if (layout == nullptr) {
        error = "plan layout is NULL";
        return NT_ERR_VALUE;
    }
    if (n < 0 || (n > 0 && tensors == nullptr)) {
        error = "plan tensor table is invalid";
        return NT_ERR_VALUE;
    }
    if (!valid_dtype(layout->param_dtype, true) || !valid_dtype(layout->grad_dtype, false) ||
        !valid_dtype(layout->state_dtype, true) || !valid_dtype(layout->copy_dtype, true)) {
        error = "plan layout names an unsupported dtype code";
        return NT_ERR_TYPE;
    }
    if (chunk == 0) chunk = kDefaultChunk;
    if (chunk < kChunkQuantum || chunk % kChunkQuantum != 0 || chunk > (int64_t)1 << 30) {
        error = "plan chunk must be a positive multiple of 2048 elements, at most 2**30";
        return NT_ERR_VALUE;
    }
    out = PlanTables{};
    out.chunk = chunk;
    out.tensors.assign(n > 0 ? (size_t)n : 1, DevTensor{});
    const size_t sizes[5] = {dtype_size(layout->param_dtype), dtype_size(layout->grad_dtype),
                             dtype_size(layout->state_dtype), dtype_size(layout->state_dtype),
                             dtype_size(layout->copy_dtype)};
    for (int32_t t = 0; t < n; ++t) {
        const nt_mt_tensor &s = tensors[t];
        if (s.grad == nullptr && s.numel > 0) {
            error = "plan tensor " + std::to_string(t) + " has no gradient";
            return NT_ERR_VALUE;
        }
        if (s.slot >= NT_MAX_SLOTS) {
            error = "plan tensor " + std::to_string(t) + " selects a coefficient slot >= 16";
            return NT_ERR_VALUE;
        }
        DevTensor d{};
        d.param = s.param;
        d.grad = s.grad;
        d.exp_avg = s.exp_avg;
        d.exp_avg_sq = s.exp_avg_sq;
        d.model_copy = s.model_copy;
        d.numel = s.numel;
        d.slot = s.slot;
        if (s.slot > out.max_slot) out.max_slot = s.slot;
        bool aligned = true;
        const void *pointers[5] = {s.param, s.grad, s.exp_avg, s.exp_avg_sq, s.model_copy};
        for (int r = 0; r < 5; ++r) {
            if (pointers[r] == nullptr) continue;
            const uintptr_t p = (uintptr_t)pointers[r];
            if (p % 16 != 0) aligned = false;
            if (sizes[r] != 0 && p % sizes[r] != 0) {
                error = "plan tensor " + std::to_string(t) + " has a pointer not aligned to its dtype";
                return NT_ERR_VALUE;
            }
        }
        d.flags = aligned ? kAligned16 : 0u;
        out.tensors[(size_t)t] = d;
        const uint64_t chunks = (s.numel + (uint64_t)chunk - 1) / (uint64_t)chunk;
        if (chunks > 0xffffffffull) {
            error = "tensor too large for the task map";
            return NT_ERR_VALUE;
        }
        if (out.tasks.size() + chunks > 0x7fffffffull) {
            error = "too many workgroup tasks";
            return NT_ERR_VALUE;
        }
        out.numel += s.numel;
        for (uint64_t c = 0; c < chunks; ++c) out.tasks.push_back(Task{(uint32_t)t, (uint32_t)c});
    }
    return NT_OK;
}

int32_t check_pointer_column(const nt_mt_layout &layout, const std::vector<uint32_t> &flags, int32_t column,
                             const void *const *pointers, int32_t n, std::string &error) {
    if (column < 0 || column > kIncomingColumn) {
        error = "nt_plan_set_pointers: column must be 0..5";
        return NT_ERR_VALUE;
    }
    if (n != (int32_t)flags.size() || (n > 0 && pointers == nullptr)) {
        error = "nt_plan_set_pointers: one pointer per plan tensor is required";
        return NT_ERR_VALUE;
    }
    const int32_t dtypes[6] = {layout.param_dtype, layout.grad_dtype, layout.state_dtype, layout.state_dtype,
                               layout.copy_dtype, layout.grad_dtype};
    const size_t size = dtype_size(dtypes[column]);
    if (size == 0) {
        error = "nt_plan_set_pointers: the plan layout has no such column";
        return NT_ERR_VALUE;
    }
    if (column == kIncomingColumn && size == 8) {
        error = "nt_plan_set_pointers: incoming gradients are not supported for float64 gradients";
        return NT_ERR_TYPE;
    }
    for (int32_t t = 0; t < n; ++t) {
        const uintptr_t p = (uintptr_t)pointers[t];
        if (p == 0) {
            if (column == kIncomingColumn) continue;       // no incoming gradient for this tensor
            error = "nt_plan_set_pointers: pointer " + std::to_string(t) + " is NULL";
            return NT_ERR_VALUE;
        }
        if (p % size != 0 || ((flags[(size_t)t] & kAligned16) && p % 16 != 0)) {
            error = "nt_plan_set_pointers: pointer " + std::to_string(t) + " breaks the alignment the plan was built for";
            return NT_ERR_VALUE;
        }
    }
    return NT_OK;
}

}  // namespace nt
