// Host unit test of the GradScaler / clip decisions (namitorch_amd/csrc/nt_scaler.hpp),
// the code one lane of the finalize and combine kernels runs: the loss-scale
// state machine of the reference's GradScaler.update (amp.py:225-233), its fp32
// rounding and clamping (_scale_value, amp.py:114-119), the norm and clip
// decision of clip_grad_norm_ (optim/clip_grad.py:63-79,106-107) and the
// multi-optimizer combine.  Built by tests/test_host_tables.py with g++ and
// AddressSanitizer/UBSan; no GPU involved.  Expected values are written out by
// hand from those rules (scale sequences, nearest-fp32 values), not recomputed
// with the header's formulas.
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "../../namitorch_amd/csrc/nt_scaler.hpp"

using namespace nt;

static int failures = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
            ++failures;                                                          \
        }                                                                        \
    } while (0)

static nt_amp_ctrl fresh(float scale) {
    nt_amp_ctrl c{};
    c.scale = scale;
    c.scale_used = scale;
    c.clip_coef = 1.0;
    return c;
}

// One finalize over finite statistics (found = 0) or a NaN/inf iteration
// (found = 1), with the scaler update on.
static void iterate(nt_amp_ctrl &c, int found, double growth, double backoff, int interval) {
    nt_amp_ctrl next = carried_ctrl(c);
    decide_iteration(next, 4.0, 1.0, 0, found, 2.0, -1.0, NT_FINALIZE_SCALER_UPDATE, growth, backoff, interval);
    c = next;
}

static void test_growth_and_backoff_sequence() {
    // Interval 3, growth 2, backoff 0.5 from 65536.  Pattern and the scale /
    // tracker after each update, tabulated from the reference's rules.
    const int found[] = {0, 0, 0, 1, 0, 0, 1, 0, 0, 0, 0};
    const float scale[] = {65536, 65536, 131072, 65536, 65536, 65536, 32768, 32768, 32768, 65536, 65536};
    const int tracker[] = {1, 2, 0, 0, 1, 2, 0, 1, 2, 0, 1};
    nt_amp_ctrl c = fresh(65536.0f);
    float before = c.scale;
    for (int i = 0; i < 11; ++i) {
        iterate(c, found[i], 2.0, 0.5, 3);
        CHECK(c.scale == scale[i]);
        CHECK(c.growth_tracker == tracker[i]);
        CHECK(c.scale_used == before);       // the iteration divides by the scale it started with
        CHECK(c.skip == found[i]);
        CHECK(c.found_inf == found[i]);
        before = c.scale;
    }
    CHECK(c.iterations == 11);
    CHECK(c.skipped == 2);
}

static void test_interval_one_grows_every_clean_iteration() {
    nt_amp_ctrl c = fresh(1.0f);
    for (int i = 0; i < 5; ++i) iterate(c, 0, 2.0, 0.5, 1);
    CHECK(c.scale == 32.0f);
    CHECK(c.growth_tracker == 0);
}

static void test_fp32_rounding_of_the_product() {
    // The factor multiplies in fp64 and the product rounds once to fp32:
    // 3 * 1.1 = 3.3000000000000003, nearest fp32 3.29999995f = 0x1.a66666p+1
    // (an fp32 product 3.0f * 1.1f would give 0x1.a66668p+1).
    nt_amp_ctrl c = fresh(3.0f);
    iterate(c, 0, 1.1, 0.5, 1);
    CHECK(c.scale == 0x1.a66666p+1f);
    // 3 * 0.9 = 2.7, nearest fp32 0x1.59999ap+1 (fp32 product: 0x1.599998p+1).
    c = fresh(3.0f);
    iterate(c, 1, 2.0, 0.9, 1);
    CHECK(c.scale == 0x1.59999ap+1f);
}

static void test_clamps() {
    // Backoff below float32 tiny stops at tiny; never a subnormal or zero.
    nt_amp_ctrl c = fresh(FLT_MIN);
    iterate(c, 1, 2.0, 0.5, 1);
    CHECK(c.scale == FLT_MIN);
    c = fresh(2.0f * FLT_MIN);
    iterate(c, 1, 2.0, 0.125, 1);
    CHECK(c.scale == FLT_MIN);
    // Growth above float32 max stops at max; never inf.
    c = fresh(0x1p127f);
    iterate(c, 0, 2.0, 0.5, 1);
    CHECK(c.scale == FLT_MAX);
    iterate(c, 0, 2.0, 0.5, 1);
    CHECK(c.scale == FLT_MAX);
    CHECK(std::isfinite(c.scale));
}

static void test_no_update_flag_keeps_the_scaler_state() {
    nt_amp_ctrl c = fresh(1024.0f);
    c.growth_tracker = 5;
    nt_amp_ctrl next = carried_ctrl(c);
    decide_iteration(next, 1.0, 1.0, 0, 1, 2.0, -1.0, 0, 2.0, 0.5, 6);
    CHECK(next.scale == 1024.0f);
    CHECK(next.growth_tracker == 5);
    CHECK(next.skip == 1);            // the skip decision does not depend on the update
    CHECK(next.iterations == 1 && next.skipped == 1);
    // A block finalized in place (no carry) divides by its current scale,
    // whatever an earlier iteration left in scale_used.
    nt_amp_ctrl in_place = fresh(2048.0f);
    in_place.scale_used = 4096.0f;
    decide_iteration(in_place, 1.0, 1.0, 0, 0, 2.0, -1.0, NT_FINALIZE_SCALER_UPDATE, 2.0, 0.5, 2000);
    CHECK(in_place.scale_used == 2048.0f);
}

static void test_carried_ctrl_clears_the_iteration() {
    nt_amp_ctrl s{};
    s.sumsq = 9.0;
    s.amax = 3.0;
    s.norm = 3.0;
    s.clip_coef = 0.25;
    s.scale = 512.0f;
    s.scale_used = 1024.0f;
    s.found_inf = 1;
    s.has_nan = 1;
    s.clip = 1;
    s.skip = 1;
    s.growth_tracker = 7;
    s.iterations = 40;
    s.skipped = 3;
    const nt_amp_ctrl c = carried_ctrl(s);
    CHECK(c.scale == 512.0f && c.scale_used == 512.0f);
    CHECK(c.growth_tracker == 7 && c.iterations == 40 && c.skipped == 3);
    CHECK(c.sumsq == 0.0 && c.amax == 0.0 && c.norm == 0.0 && c.clip_coef == 1.0);
    CHECK(c.found_inf == 0 && c.has_nan == 0 && c.clip == 0 && c.skip == 0);
}

static nt_amp_ctrl decide(double sumsq, double amax, int nan, int inf, double norm_type, double max_norm, int flags) {
    nt_amp_ctrl c = fresh(1.0f);
    decide_iteration(c, sumsq, amax, nan, inf, norm_type, max_norm, flags, 2.0, 0.5, 2000);
    return c;
}

static void test_norm_and_clip_decisions() {
    // 2-norm from the fp64 sum of squares: sqrt(16) = 4 > 1 clips.
    nt_amp_ctrl c = decide(16.0, 3.0, 0, 0, 2.0, 1.0, 0);
    CHECK(c.norm == 4.0);
    CHECK(c.clip == 1);
    CHECK(c.clip_coef < 0.25 && c.clip_coef > 0.2499999);   // 1 / (4 + 1e-6)
    // A norm equal to max_norm still clips (coefficient max / (max + 1e-6) < 1).
    c = decide(1.0, 1.0, 0, 0, 2.0, 1.0, 0);
    CHECK(c.clip == 1);
    // A norm below max_norm does not; the coefficient is still reported.
    c = decide(0.25, 0.5, 0, 0, 2.0, 1.0, 0);
    CHECK(c.norm == 0.5 && c.clip == 0 && c.clip_coef > 1.99 && c.clip_coef < 2.0);
    // No max_norm (negative): coefficient 1, no clip, the norm still computed.
    c = decide(16.0, 3.0, 0, 0, 2.0, -1.0, 0);
    CHECK(c.norm == 4.0 && c.clip == 0 && c.clip_coef == 1.0);
    // Infinity norm: the max |g|, whatever the sum of squares says.
    c = decide(16.0, 3.0, 0, 0, INFINITY, 10.0, 0);
    CHECK(c.norm == 3.0 && c.clip == 0);
    // All-zero gradients: norm 0, no clip.
    c = decide(0.0, 0.0, 0, 0, 2.0, 1.0, 0);
    CHECK(c.norm == 0.0 && c.clip == 0 && c.found_inf == 0);
    // NaN seen: norm NaN, skip, no clip (NaN < 1 is false).
    c = decide(16.0, 3.0, 1, 0, 2.0, 1.0, 0);
    CHECK(std::isnan(c.norm) && c.has_nan == 1 && c.found_inf == 1 && c.skip == 1 && c.clip == 0);
    // inf seen: norm inf, coefficient 0 clips unless clipping waits for finite grads.
    c = decide(16.0, 3.0, 0, 1, 2.0, 1.0, 0);
    CHECK(std::isinf(c.norm) && c.has_nan == 0 && c.found_inf == 1 && c.skip == 1);
    CHECK(c.clip_coef == 0.0 && c.clip == 1);
    c = decide(16.0, 3.0, 0, 1, 2.0, 1.0, NT_FINALIZE_CLIP_IF_FINITE);
    CHECK(c.clip == 0);
    // NaN and inf together: NaN wins.
    c = decide(16.0, 3.0, 1, 1, 2.0, 1.0, 0);
    CHECK(std::isnan(c.norm));
    // The statistics are kept in the block.
    c = decide(16.0, 3.0, 0, 0, 2.0, 1.0, 0);
    CHECK(c.sumsq == 16.0 && c.amax == 3.0);
}

static void test_combine() {
    nt_amp_ctrl carry = fresh(256.0f);
    carry.growth_tracker = 1;
    carry.iterations = 9;
    nt_amp_ctrl a = carry, b = carry, d = carry;
    a.sumsq = 9.0;  a.amax = 3.0;
    b.sumsq = 16.0; b.amax = 2.0;
    d.sumsq = 0.0;  d.amax = 0.0;
    const nt_amp_ctrl *blocks[] = {&a, &b, &d};
    // Finite: one global 2-norm sqrt(9 + 16) = 5 over all, one scaler update
    // (tracker 1 -> 2 == interval: growth).
    nt_amp_ctrl shared = combined_decisions(blocks, 3, carry, 2.0, 2.5, NT_FINALIZE_SCALER_UPDATE, 2.0, 0.5, 2);
    CHECK(shared.norm == 5.0 && shared.amax == 3.0 && shared.clip == 1);
    CHECK(shared.scale == 512.0f && shared.scale_used == 256.0f && shared.growth_tracker == 0);
    CHECK(shared.iterations == 10);
    nt_amp_ctrl out = combined_block(shared, b);
    CHECK(out.sumsq == 16.0 && out.amax == 2.0);          // its own statistics
    CHECK(out.norm == 5.0 && out.clip == 1 && out.scale == 512.0f && out.skip == 0);
    // One optimizer saw inf: every block gets the backoff, only that one skips.
    b.found_inf = 1;
    shared = combined_decisions(blocks, 3, carry, 2.0, 2.5, NT_FINALIZE_SCALER_UPDATE, 2.0, 0.5, 2);
    CHECK(std::isinf(shared.norm) && shared.found_inf == 1);
    CHECK(shared.scale == 128.0f && shared.growth_tracker == 0 && shared.skipped == 1);
    CHECK(combined_block(shared, a).skip == 0);
    CHECK(combined_block(shared, b).skip == 1);
    CHECK(combined_block(shared, d).skip == 0);
    CHECK(combined_block(shared, a).found_inf == 0);
    // NaN in another block makes the shared norm NaN.
    d.has_nan = 1;
    d.found_inf = 1;
    shared = combined_decisions(blocks, 3, carry, 2.0, 2.5, 0, 2.0, 0.5, 2);
    CHECK(std::isnan(shared.norm) && shared.has_nan == 1);
    CHECK(shared.scale == 256.0f);                          // no update flag
    CHECK(combined_block(shared, a).has_nan == 0 && combined_block(shared, d).has_nan == 1);
}

int main() {
    test_growth_and_backoff_sequence();
    test_interval_one_grows_every_clean_iteration();
    test_fp32_rounding_of_the_product();
    test_clamps();
    test_no_update_flag_keeps_the_scaler_state();
    test_carried_ctrl_clears_the_iteration();
    test_norm_and_clip_decisions();
    test_combine();
    if (failures != 0) {
        std::printf("%d checks failed\n", failures);
        return 1;
    }
    std::printf("all checks passed\n");
    return 0;
}
