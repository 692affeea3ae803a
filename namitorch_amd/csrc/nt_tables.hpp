// nt_tables.hpp — host-side construction and validation of multi-tensor
// plan tables (plain C++; linked into the library and into the host unit
// test under AddressSanitizer/UBSan).
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/namitorch_amd.h"
#include "nt_layout.hpp"

namespace nt {

struct PlanTables {
    std::vector<DevTensor> tensors;   // one per tensor (a single zero entry for n == 0)
    std::vector<Task> tasks;          // tensor-major, chunk-minor
    uint64_t numel = 0;
    uint32_t max_slot = 0;
    int64_t chunk = 0;
};

// Bytes per element of a dtype code (0 for NT_DTYPE_NONE or unknown codes).
size_t dtype_size(int32_t dtype);
bool valid_dtype(int32_t dtype, bool allow_none);

// Validates the plan request and builds its descriptor table and task map.
// Returns NT_OK, or an NT_ERR_* code with the message in `error`.
int32_t build_plan_tables(const nt_mt_tensor *tensors, int32_t n, const nt_mt_layout *layout, int64_t chunk,
                          PlanTables &out, std::string &error);

// Checks a replacement pointer column (nt_plan_set_pointers): one non-NULL
// pointer per tensor, aligned to the column's dtype and, where the tensor's
// descriptor was built 16-byte aligned, to 16 bytes.
int32_t check_pointer_column(const nt_mt_layout &layout, const std::vector<uint32_t> &flags, int32_t column,
                             const void *const *pointers, int32_t n, std::string &error);

}  // namespace nt
