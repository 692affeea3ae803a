// Host unit test of the multi-tensor plan builder (namitorch_amd/csrc/nt_tables.cpp):
// descriptor packing, task maps, alignment flags, error codes and pointer-column
// checks.  Built by tests/test_host_tables.py with g++ and AddressSanitizer/UBSan;
// runs without a GPU (the pointers are never dereferenced).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../namitorch_amd/csrc/nt_tables.hpp"

using namespace nt;

static int failures = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
            ++failures;                                                          \
        }                                                                        \
    } while (0)

static void *ptr(uintptr_t value) { return reinterpret_cast<void *>(value); }

static nt_mt_tensor tensor(uintptr_t param, uintptr_t grad, uintptr_t m, uintptr_t v, uint64_t numel, uint32_t slot) {
    nt_mt_tensor t{};
    t.param = ptr(param);
    t.grad = ptr(grad);
    t.exp_avg = ptr(m);
    t.exp_avg_sq = ptr(v);
    t.model_copy = nullptr;
    t.numel = numel;
    t.slot = slot;
    return t;
}

static void test_packing_and_tasks() {
    const nt_mt_layout layout{NT_F32, NT_F32, NT_F32, NT_DTYPE_NONE};
    std::vector<nt_mt_tensor> rows = {
        tensor(0x10000, 0x20000, 0x30000, 0x40000, 10000, 0),   // 3 tasks of 4096 (last partial)
        tensor(0x50000, 0x60000, 0x70000, 0x80000, 4096, 1),    // exactly one task
        tensor(0x90000, 0xa0000, 0xb0000, 0xc0000, 0, 2),       // empty: no task
        tensor(0xd0004, 0xe0000, 0xf0000, 0xf8000, 1, 3),       // 4-byte aligned only
    };
    PlanTables out;
    std::string error;
    CHECK(build_plan_tables(rows.data(), (int32_t)rows.size(), &layout, 0, out, error) == NT_OK);
    CHECK(out.chunk == kDefaultChunk);
    CHECK(out.numel == 10000 + 4096 + 0 + 1);
    CHECK(out.max_slot == 3);
    CHECK(out.tensors.size() == 4);
    CHECK(out.tasks.size() == 3 + 1 + 0 + 1);
    const uint32_t want[][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 0}, {3, 0}};
    for (size_t i = 0; i < out.tasks.size() && i < 5; ++i)
        CHECK(out.tasks[i].tensor == want[i][0] && out.tasks[i].chunk == want[i][1]);
    CHECK(out.tensors[0].flags == kAligned16 && out.tensors[1].flags == kAligned16);
    CHECK(out.tensors[3].flags == 0u);
    CHECK(out.tensors[0].param == ptr(0x10000) && out.tensors[0].grad == ptr(0x20000));
    CHECK(out.tensors[1].slot == 1 && out.tensors[1].numel == 4096);
}

static void test_chunks() {
    const nt_mt_layout layout{NT_DTYPE_NONE, NT_BF16, NT_DTYPE_NONE, NT_DTYPE_NONE};
    nt_mt_tensor row = tensor(0, 0x1000, 0, 0, 1 << 20, 0);
    PlanTables out;
    std::string error;
    CHECK(build_plan_tables(&row, 1, &layout, 8192, out, error) == NT_OK);
    CHECK(out.tasks.size() == (1u << 20) / 8192);
    for (int64_t bad : {int64_t(1000), int64_t(2047), int64_t(3000), (int64_t(1) << 31)}) {
        CHECK(build_plan_tables(&row, 1, &layout, bad, out, error) == NT_ERR_VALUE);
        CHECK(error.find("multiple of 2048") != std::string::npos);
    }
    // Zero tensors: a valid empty plan with one placeholder descriptor.
    CHECK(build_plan_tables(nullptr, 0, &layout, 0, out, error) == NT_OK);
    CHECK(out.tasks.empty() && out.tensors.size() == 1 && out.numel == 0);
}

static void test_errors() {
    const nt_mt_layout layout{NT_F32, NT_F16, NT_F32, NT_DTYPE_NONE};
    PlanTables out;
    std::string error;
    nt_mt_tensor no_grad = tensor(0x1000, 0, 0x2000, 0x3000, 5, 0);
    CHECK(build_plan_tables(&no_grad, 1, &layout, 0, out, error) == NT_ERR_VALUE);
    CHECK(error == "plan tensor 0 has no gradient");
    nt_mt_tensor slot = tensor(0x1000, 0x2000, 0x3000, 0x4000, 5, NT_MAX_SLOTS);
    CHECK(build_plan_tables(&slot, 1, &layout, 0, out, error) == NT_ERR_VALUE);
    CHECK(error.find("slot >= 16") != std::string::npos);
    nt_mt_tensor odd = tensor(0x1002, 0x2000, 0x3000, 0x4000, 5, 0);      // fp32 param at 2-byte alignment
    CHECK(build_plan_tables(&odd, 1, &layout, 0, out, error) == NT_ERR_VALUE);
    CHECK(error.find("not aligned to its dtype") != std::string::npos);
    nt_mt_tensor half = tensor(0x1000, 0x2002, 0x3000, 0x4000, 5, 0);     // fp16 grad at 2 bytes: fine
    CHECK(build_plan_tables(&half, 1, &layout, 0, out, error) == NT_OK);
    CHECK(out.tensors[0].flags == 0u);
    const nt_mt_layout bad_dtype{NT_F32, 7, NT_F32, NT_DTYPE_NONE};
    CHECK(build_plan_tables(&half, 1, &bad_dtype, 0, out, error) == NT_ERR_TYPE);
    const nt_mt_layout no_grad_dtype{NT_F32, NT_DTYPE_NONE, NT_F32, NT_DTYPE_NONE};
    CHECK(build_plan_tables(&half, 1, &no_grad_dtype, 0, out, error) == NT_ERR_TYPE);
    CHECK(build_plan_tables(nullptr, 2, &layout, 0, out, error) == NT_ERR_VALUE);
    CHECK(build_plan_tables(&half, 1, nullptr, 0, out, error) == NT_ERR_VALUE);
    nt_mt_tensor huge = tensor(0x1000, 0x2000, 0x3000, 0x4000, (uint64_t(1) << 32) * 4096, 0);
    CHECK(build_plan_tables(&huge, 1, &layout, 0, out, error) == NT_ERR_VALUE);
}

static void test_pointer_columns() {
    const nt_mt_layout layout{NT_F32, NT_BF16, NT_F32, NT_DTYPE_NONE};
    const std::vector<uint32_t> flags = {kAligned16, 0u};
    std::string error;
    const void *good[2] = {ptr(0x10010), ptr(0x20002)};
    CHECK(check_pointer_column(layout, flags, 1, good, 2, error) == NT_OK);
    const void *misaligned[2] = {ptr(0x10008), ptr(0x20002)};            // tensor 0 was built 16-byte aligned
    CHECK(check_pointer_column(layout, flags, 1, misaligned, 2, error) == NT_ERR_VALUE);
    CHECK(error.find("pointer 0 breaks the alignment") != std::string::npos);
    const void *odd[2] = {ptr(0x10010), ptr(0x20001)};                   // bf16 at 1 byte
    CHECK(check_pointer_column(layout, flags, 1, odd, 2, error) == NT_ERR_VALUE);
    const void *null_ptr[2] = {ptr(0x10010), nullptr};
    CHECK(check_pointer_column(layout, flags, 1, null_ptr, 2, error) == NT_ERR_VALUE);
    CHECK(check_pointer_column(layout, flags, 1, good, 1, error) == NT_ERR_VALUE);   // wrong count
    CHECK(check_pointer_column(layout, flags, 4, good, 2, error) == NT_ERR_VALUE);   // no copy column
    CHECK(check_pointer_column(layout, flags, 6, good, 2, error) == NT_ERR_VALUE);   // no such column
    CHECK(check_pointer_column(layout, flags, 0, good, 2, error) == NT_ERR_VALUE);   // fp32 param at 2 bytes
    // Column 5: incoming gradients of the grad dtype; NULL means none.
    CHECK(check_pointer_column(layout, flags, 5, good, 2, error) == NT_OK);
    CHECK(check_pointer_column(layout, flags, 5, null_ptr, 2, error) == NT_OK);
    const void *none[2] = {nullptr, nullptr};
    CHECK(check_pointer_column(layout, flags, 5, none, 2, error) == NT_OK);
    CHECK(check_pointer_column(layout, flags, 5, misaligned, 2, error) == NT_ERR_VALUE);
    CHECK(check_pointer_column(layout, flags, 5, odd, 2, error) == NT_ERR_VALUE);
    const nt_mt_layout f64{NT_F64, NT_F64, NT_F64, NT_DTYPE_NONE};
    const void *wide[2] = {ptr(0x10010), ptr(0x20008)};
    CHECK(check_pointer_column(f64, flags, 1, wide, 2, error) == NT_OK);
    CHECK(check_pointer_column(f64, flags, 5, wide, 2, error) == NT_ERR_TYPE);    // float64: not supported
    // Column 5 sits after numel/slot/flags in the descriptor.
    CHECK(column_offset(5) == offsetof(DevTensor, incoming) && column_offset(5) == 56 && column_offset(4) == 32);
}

// Fixed-seed random tensor lists: every tensor's elements are covered by its
// tasks exactly once, tasks are tensor-major and chunk-minor, the element
// count adds up, and the 16-byte flag is set exactly when every pointer is
// 16-byte aligned.
static void test_random_lists() {
    uint64_t state = 0x9e3779b97f4a7c15ull;
    auto next = [&state](uint64_t bound) {
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        return (state >> 33) % bound;
    };
    const nt_mt_layout layout{NT_F32, NT_BF16, NT_F32, NT_BF16};
    const uint64_t sizes[5] = {4, 2, 4, 4, 2};
    const uint64_t edges[] = {0, 1, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 8193};
    const int64_t chunks[] = {0, 2048, 4096, 6144, 8192};
    for (int round = 0; round < 300; ++round) {
        const int n = 1 + (int)next(12);
        std::vector<nt_mt_tensor> rows;
        std::vector<bool> aligned;
        for (int t = 0; t < n; ++t) {
            const uint64_t numel = next(3) == 0 ? edges[next(10)] : next(50000);
            uintptr_t pointer[5];
            bool all16 = true;
            for (int c = 0; c < 5; ++c) {
                const uint64_t offset = next(2) == 0 ? 16 * next(4) : sizes[c] * next(8);
                pointer[c] = (uintptr_t)(0x1000000ull * (uint64_t)(5 * t + c + 1) + offset);
                all16 = all16 && pointer[c] % 16 == 0;
            }
            rows.push_back(tensor(pointer[0], pointer[1], pointer[2], pointer[3], numel, (uint32_t)next(NT_MAX_SLOTS)));
            rows.back().model_copy = ptr(pointer[4]);
            aligned.push_back(all16);
        }
        const int64_t requested = chunks[next(5)];
        PlanTables out;
        std::string error;
        CHECK(build_plan_tables(rows.data(), n, &layout, requested, out, error) == NT_OK);
        const uint64_t chunk = (uint64_t)out.chunk;
        CHECK(chunk == (requested == 0 ? (uint64_t)kDefaultChunk : (uint64_t)requested));
        uint64_t total = 0;
        size_t task = 0;
        for (int t = 0; t < n; ++t) {
            const uint64_t numel = rows[(size_t)t].numel;
            total += numel;
            uint64_t covered = 0;
            for (uint64_t c = 0; c * chunk < numel; ++c, ++task) {
                CHECK(task < out.tasks.size());
                if (task >= out.tasks.size()) return;
                CHECK(out.tasks[task].tensor == (uint32_t)t && out.tasks[task].chunk == (uint32_t)c);
                covered += std::min(chunk, numel - c * chunk);
            }
            CHECK(covered == numel);
            CHECK((out.tensors[(size_t)t].flags == kAligned16) == aligned[(size_t)t]);
            CHECK(out.tensors[(size_t)t].numel == numel && out.tensors[(size_t)t].slot == rows[(size_t)t].slot);
        }
        CHECK(task == out.tasks.size());
        CHECK(out.numel == total);
    }
}

int main() {
    test_packing_and_tasks();
    test_chunks();
    test_errors();
    test_pointer_columns();
    test_random_lists();
    if (failures == 0) std::printf("plan tables: all checks passed\n");
    return failures == 0 ? 0 : 1;
}
