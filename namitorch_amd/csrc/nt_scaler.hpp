// nt_scaler.hpp — the per-iteration decisions of the GradScaler / clip path:
// the global norm, the clip decision, the skip flag and the loss-scale state
// machine, made by one lane of the finalize and combine kernels from the
// iteration's merged statistics.
//
// Plain arithmetic on an nt_amp_ctrl block, with no device intrinsics, so the
// same code also compiles with a host compiler: the host unit test
// (tests/host/scaler_test.cpp) drives it with g++ under the sanitizers.
#pragma once

#include <stdint.h>

#include "../../include/namitorch_amd.h"

#if defined(__HIPCC__)
#define NT_SCALER_FN __host__ __device__ inline __attribute__((always_inline))
#else
#define NT_SCALER_FN inline
#endif

namespace nt {

// Reference scaler update (amp.py:225-233): on a non-finite iteration the
// scale is multiplied by `backoff` and the tracker restarts; otherwise the
// tracker counts clean iterations and every `interval`-th multiplies the
// scale by `growth`.  The factors apply in fp64 to the fp32 scale, clamped to
// [float32 tiny, float32 max] and rounded to fp32 (_scale_value, amp.py:114-119).
NT_SCALER_FN void scaler_update(nt_amp_ctrl *c, int found, double growth, double backoff, int interval) {
    const double tiny = 1.1754943508222875e-38;    // float32 tiny
    const double fmax = 3.4028234663852886e+38;    // float32 max
    if (found) {
        double s = (double)c->scale * backoff;
        c->scale = (float)(s > tiny ? s : tiny);
        c->growth_tracker = 0;
    } else {
        c->growth_tracker += 1;
        if (c->growth_tracker == interval) {
            double s = (double)c->scale * growth;
            c->scale = (float)(s < fmax ? s : fmax);
            c->growth_tracker = 0;
        }
    }
}

// A new iteration's block continuing `s`'s scaler state: scale,
// growth_tracker, iterations and skipped carry over, every per-iteration
// field starts cleared (clip_coef 1).
NT_SCALER_FN nt_amp_ctrl carried_ctrl(const nt_amp_ctrl &s) {
    nt_amp_ctrl c{};
    c.scale = s.scale;
    c.scale_used = s.scale;
    c.growth_tracker = s.growth_tracker;
    c.iterations = s.iterations;
    c.skipped = s.skipped;
    c.clip_coef = 1.0;
    return c;
}

// One iteration's decisions from its merged statistics (fp64 sum of squares
// and max |g'| of the finite unscaled gradients, NaN/inf seen), starting
// from `c` (the carried scaler state): the norm, the clip decision, the skip
// flag and, with NT_FINALIZE_SCALER_UPDATE, the scaler update.
NT_SCALER_FN void decide_iteration(nt_amp_ctrl &c, double sumsq, double amax, int32_t nan, int32_t inf,
                                   double norm_type, double max_norm, int32_t flags, double growth,
                                   double backoff, int32_t interval) {
    // _total_norm (optim/clip_grad.py:63-79): the max-abs prescale is
    // non-finite or zero => return it; else scale * total^(1/p).
    double norm;
    if (nan) norm = __builtin_nan("");
    else if (inf) norm = __builtin_inf();
    else if (amax == 0.0 || __builtin_isinf(norm_type)) norm = amax;
    else norm = __builtin_sqrt(sumsq);   // p == 2; other p: nt_grad_norm_pow
    c.sumsq = sumsq;
    c.amax = amax;
    c.norm = norm;
    c.has_nan = nan;
    c.found_inf = nan | inf;
    if (max_norm >= 0.0) {
        c.clip_coef = max_norm / (norm + 1e-6);
        c.clip = c.clip_coef < 1.0 ? 1 : 0;
        if ((flags & NT_FINALIZE_CLIP_IF_FINITE) && c.found_inf) c.clip = 0;
    } else {
        c.clip_coef = 1.0;
        c.clip = 0;
    }
    c.skip = c.found_inf;
    c.scale_used = c.scale;
    c.iterations += 1;
    c.skipped += c.found_inf;
    if (flags & NT_FINALIZE_SCALER_UPDATE) scaler_update(&c, c.found_inf, growth, backoff, interval);
}

// Several optimizers in one scaler iteration: block[0..n) hold each one's
// finalized statistics.  Their sums add in block order, the maxima and the
// NaN/inf flags combine, and one set of decisions (global norm and clip, one
// scaler update over all) is made from `carry`'s scaler state.
NT_SCALER_FN nt_amp_ctrl combined_decisions(const nt_amp_ctrl *const *block, int32_t n, const nt_amp_ctrl &carry,
                                            double norm_type, double max_norm, int32_t flags, double growth,
                                            double backoff, int32_t interval) {
    double sumsq = 0.0, amax = 0.0;
    int32_t nan = 0, inf = 0;
    for (int32_t i = 0; i < n; ++i) {
        const nt_amp_ctrl &b = *block[i];
        sumsq += b.sumsq;
        amax = b.amax > amax ? b.amax : amax;
        nan |= b.has_nan;
        inf |= b.found_inf;          // with has_nan somewhere, the norm is NaN whatever inf says
    }
    nt_amp_ctrl c = carried_ctrl(carry);
    decide_iteration(c, sumsq, amax, nan, inf, norm_type, max_norm, flags, growth, backoff, interval);
    return c;
}

// One optimizer's block after the combine: the shared decisions, with its
// own statistics and its own skip flag (GradScaler.step checks its own
// optimizer's gradients, amp.py:209-217).
NT_SCALER_FN nt_amp_ctrl combined_block(const nt_amp_ctrl &shared, const nt_amp_ctrl &own) {
    nt_amp_ctrl out = shared;
    out.sumsq = own.sumsq;
    out.amax = own.amax;
    out.found_inf = own.found_inf;
    out.has_nan = own.has_nan;
    out.skip = own.found_inf;
    return out;
}

}  // namespace nt
