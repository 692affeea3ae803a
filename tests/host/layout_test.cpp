// Host unit test of the kernels' workgroup -> element arithmetic
// (namitorch_amd/csrc/nt_layout.hpp): the XCD-grouped renumbering of the
// grid and the split of plan tasks into slices.  Built by
// tests/test_host_tables.py with g++ and AddressSanitizer/UBSan; no GPU.
//
// xcd_grouped acts on each group of 8 * per_xcd workgroups separately, so it
// is a bijection on [0, n) for every n exactly when it is one on every group
// size m in [1, 8 * per_xcd]: that is checked exhaustively, with each XCD's
// share of a group a contiguous run.
#include <cstdio>
#include <vector>

#include "../../namitorch_amd/csrc/nt_layout.hpp"

using namespace nt;

static int failures = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
            ++failures;                                                          \
        }                                                                        \
    } while (0)

// The last group of a grid of n = base + m workgroups (base a multiple of
// 8 * per_xcd): a bijection onto [base, n), one contiguous run per XCD.
static void check_group(uint32_t base, uint32_t m, uint32_t per_xcd) {
    const uint32_t n = base + m;
    std::vector<int> hits(m, 0);
    std::vector<uint32_t> low(8, 0xffffffffu), high(8, 0u), count(8, 0u);
    for (uint32_t w = 0; w < m; ++w) {
        const uint32_t to = xcd_grouped(base + w, n, per_xcd);
        CHECK(to >= base && to < n);
        if (to < base || to >= n) return;
        hits[to - base] += 1;
        const uint32_t x = w % 8u;                // the XCD workgroup base + w runs on
        low[x] = to < low[x] ? to : low[x];
        high[x] = to > high[x] ? to : high[x];
        count[x] += 1;
    }
    for (uint32_t i = 0; i < m; ++i) CHECK(hits[i] == 1);
    for (uint32_t x = 0; x < 8u && x < m; ++x) CHECK(high[x] - low[x] + 1u == count[x]);
}

static void test_xcd_grouped_is_a_bijection() {
    const uint32_t per_xcd_values[] = {1, 2, 3, 7, 64, 256};
    for (uint32_t per_xcd : per_xcd_values) {
        const uint32_t size = 8u * per_xcd;
        for (uint32_t m = 1; m <= size; ++m) check_group(0u, m, per_xcd);
        // The same shapes at the top of the grid range (grids stay below 2**31).
        const uint32_t top = (0x7fffffffu / size - 1u) * size;
        for (uint32_t m : {1u, 7u, 9u, size - 1u, size})
            if (m <= size) check_group(top, m, per_xcd);
        check_group(size, size, per_xcd);
        // Full groups: every XCD's run has per_xcd workgroups, in XCD order.
        for (uint32_t w = 0; w < size; ++w)
            CHECK(xcd_grouped(w, 3u * size, per_xcd) == (w % 8u) * per_xcd + w / 8u);
    }
    for (uint32_t b : {0u, 1u, 77u, 0x7ffffffeu}) CHECK(xcd_grouped(b, 0x7fffffffu, 0u) == b);
}

static void test_slices_cover_each_element_once() {
    uint64_t state = 0x2545f4914f6cdd1dull;
    auto next = [&state](uint64_t bound) {
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        return (state >> 33) % bound;
    };
    for (int round = 0; round < 400; ++round) {
        const int64_t chunk = kChunkQuantum * (int64_t)(1 + next(8));
        int32_t shift = (int32_t)next(7);
        while (shift > 0 && ((chunk >> shift) << shift) != chunk) --shift;   // the launches split evenly only
        const uint64_t numel = next(4) == 0 ? (uint64_t)chunk * next(5) + next(3) : next(200000);
        const uint64_t tasks = (numel + (uint64_t)chunk - 1) / (uint64_t)chunk;
        uint64_t expected = 0;
        for (uint64_t t = 0; t < tasks; ++t) {
            for (uint32_t part = 0; part < (1u << shift); ++part) {
                Slice slice{};
                const bool live = slice_of(Task{0u, (uint32_t)t}, part, numel, chunk, shift, slice);
                if (!live) {
                    CHECK(slice.start >= numel);
                    continue;
                }
                CHECK(slice.start == expected);                   // ascending, no gap, no overlap
                CHECK(slice.end > slice.start && slice.end <= numel);
                CHECK(slice.end - slice.start <= (uint64_t)(chunk >> shift));
                expected = slice.end;
            }
        }
        CHECK(expected == numel);
    }
}

int main() {
    test_xcd_grouped_is_a_bijection();
    test_slices_cover_each_element_once();
    if (failures != 0) {
        std::printf("%d checks failed\n", failures);
        return 1;
    }
    std::printf("all checks passed\n");
    return 0;
}
