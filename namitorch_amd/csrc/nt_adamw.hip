// nt_adamw.hip — AdamW update kernels for gfx950.
//
// Element arithmetic follows the reference operation for operation
// (backends/cuda/adamw.py:15-25, identical to the NumPy path of
// optim/adam.py:35-42 + optim/_common.py:67-73):
//
//   g   = maximize ? -g : g
//   g   = g + wd*p                      (Adam only: coupled L2 decay)
//   m   = (b1*m) + (c1*g)
//   v   = (b2*v) + ((c2*g)*g)
//   if update_parameter:
//     p   = (wd != 0) ? p*decay : p      (AdamW only: decoupled decay)
//     p   = p - lr*((m/bc1) / (sqrt(v/bc2) + eps))
//
// Every operation rounds to fp32 (no FMA contraction, IEEE divide and
// sqrt), so results are bit-identical to NumPy on the same inputs.  For
// float16 parameters each operation additionally rounds to fp16, which is
// what NumPy's float16 ufuncs compute; float64 parameters use fp64.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "nt_internal.hpp"

namespace nt {

// Rounding policy after every arithmetic operation.
struct RoundF32 {
    __device__ static float r(float x) { return x; }
};
struct RoundF16 {
    __device__ static float r(float x) { return TF16::round_f32(x); }
};

template <class R>
__device__ __forceinline__ void adamw_elem(float &p, float g, float &m, float &v,
                                           const nt_adamw_coefs &c) {
    if (c.maximize) g = -g;
    if (c.coupled_weight_decay && c.weight_decay != 0.0f) g = R::r(g + R::r(c.weight_decay * p));
    m = R::r(R::r(c.beta1 * m) + R::r(c.complement1 * g));
    v = R::r(R::r(c.beta2 * v) + R::r(R::r(c.complement2 * g) * g));
    if (c.update_parameter) {
        float value = p;
        if (!c.coupled_weight_decay && c.weight_decay != 0.0f) value = R::r(value * c.decay_factor);
        float corrected = R::r(m / c.correction1);
        float denominator = R::r(R::r(__builtin_sqrtf(R::r(v / c.correction2))) + c.eps);
        p = R::r(value - R::r(c.lr * R::r(corrected / denominator)));
    }
}

__device__ __forceinline__ void adamw_elem64(double &p, double g, double &m, double &v,
                                             const nt_adamw_coefs64 &c) {
    if (c.maximize) g = -g;
    if (c.coupled_weight_decay && c.weight_decay != 0.0) g = g + c.weight_decay * p;
    m = c.beta1 * m + c.complement1 * g;
    v = c.beta2 * v + (c.complement2 * g) * g;
    if (c.update_parameter) {
        double value = p;
        if (!c.coupled_weight_decay && c.weight_decay != 0.0) value *= c.decay_factor;
        double corrected = m / c.correction1;
        double denominator = __builtin_sqrt(v / c.correction2) + c.eps;
        p = value - c.lr * (corrected / denominator);
    }
}

// ---- per-tensor kernel: the reference kernel's ABI ------------------------------
// One workgroup per kChunk elements; each thread handles kUnroll groups of 4
// elements per iteration (each group contiguous across the workgroup) with
// 128-bit global accesses when all four pointers are 16-byte aligned.
constexpr uint64_t kChunk = 4096;

__global__ __launch_bounds__(kBlock) void adamw_f32_kernel(
    float *__restrict__ param, const float *__restrict__ grad, float *__restrict__ m1,
    float *__restrict__ m2, nt_adamw_coefs c, uint64_t count, int vectorized) {
    const uint64_t start = (uint64_t)blockIdx.x * kChunk;
    const uint64_t end = min(start + kChunk, count);
    const bool update = c.update_parameter != 0;
    uint64_t scalar_from = start;
    if (vectorized) {
        const uint64_t vend = start + ((end - start) & ~(uint64_t)(kVec - 1));
        for (uint64_t base = start + (uint64_t)threadIdx.x * kVec; base < vend; base += kTile) {
            float p[kUnroll][kVec], g[kUnroll][kVec], a[kUnroll][kVec], b[kUnroll][kVec];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const uint64_t i = base + (uint64_t)u * kBlock * kVec;
                if (i < vend) {
                    Vec4IO<TF32, true>::load(grad, i, g[u]);
                    Vec4IO<TF32, true>::load(m1, i, a[u]);
                    Vec4IO<TF32, true>::load(m2, i, b[u]);
                    if (update) Vec4IO<TF32, true>::load(param, i, p[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const uint64_t i = base + (uint64_t)u * kBlock * kVec;
                if (i < vend) {
#pragma unroll
                    for (int k = 0; k < kVec; ++k) adamw_elem<RoundF32>(p[u][k], g[u][k], a[u][k], b[u][k], c);
                    Vec4IO<TF32, true>::store(m1, i, a[u]);
                    Vec4IO<TF32, true>::store(m2, i, b[u]);
                    if (update) Vec4IO<TF32, true>::store(param, i, p[u]);
                }
            }
        }
        scalar_from = vend;
    }
    for (uint64_t i = scalar_from + threadIdx.x; i < end; i += kBlock) {
        float p = update ? param[i] : 0.0f, a = m1[i], b = m2[i];
        adamw_elem<RoundF32>(p, grad[i], a, b, c);
        m1[i] = a;
        m2[i] = b;
        if (update) param[i] = p;
    }
}

// ---- multi-tensor kernel ------------------------------------------------------------
struct MtArgs {
    nt_adamw_coefs slots[NT_MAX_SLOTS];
    Xform xf;
    const nt_amp_ctrl *ctrl;
    int64_t chunk;
    int32_t honor_skip;
    int32_t split_shift;     // each task runs on 2**split_shift workgroups
    uint32_t xcd_group;      // workgroups per XCD per group of the grid order (xcd_grouped), 0: launch order
};

struct MtArgs64 {
    nt_adamw_coefs64 slots[NT_MAX_SLOTS];
    Xform xf;
    const nt_amp_ctrl *ctrl;
    int64_t chunk;
    int32_t honor_skip;
};

// Transform parameters from the device control block (sync-free path).
__device__ __forceinline__ bool xform_from_ctrl(const nt_amp_ctrl *ctrl, int honor_skip, Xform &xf) {
    if (ctrl == nullptr) return true;
    if (honor_skip && ctrl->skip) return false;
    if (xf.unscale) {
        const float s = ctrl->scale_used;
        const uint32_t b = f32_bits(s);
        const uint32_t e = (b >> 23) & 0xffu;
        xf.scale = s;
        if ((b & 0x807fffffu) == 0u && e >= 1u && e <= 253u) {
            xf.unscale = 2;                       // power of two: exact inverse
            xf.inv_scale = bits_f32((254u - e) << 23);
        } else {
            xf.unscale = 1;
        }
    }
    xf.clip = ctrl->clip;
    xf.clip_coef = ctrl->clip_coef;
    return true;
}

// One whole kPassSlice-element slice on one wave, one 4-element group per
// lane, for the common case: an aligned tensor without a deferred addend,
// Adam/AdamW without maximize or coupled decay, the parameter updated, fp32
// rounding.  The gradient transform is fixed at compile time (UNSCALE as
// Xform::unscale, CLIP), so the element code has no branches on it.  The
// arithmetic is the general path's (adamw_mt_kernel) for those settings,
// operation for operation.
template <class P, class G, class S, class C, bool HAS_COPY, int UNSCALE, bool CLIP>
__device__ __forceinline__ void lean_slice(const DevTensor &d, const nt_adamw_coefs &c, const Xform &xf,
                                           uint64_t start) {
    auto *pp = reinterpret_cast<typename P::raw *>(d.param);
    auto *gp = reinterpret_cast<const typename G::raw *>(d.grad);
    auto *ap = reinterpret_cast<typename S::raw *>(d.exp_avg);
    auto *bp = reinterpret_cast<typename S::raw *>(d.exp_avg_sq);
    auto *cp = reinterpret_cast<typename C::raw *>(d.model_copy);
    const uint64_t i = start + (uint64_t)threadIdx.x * kVec;
    float p[kVec], g[kVec], a[kVec], b[kVec];
    Vec4IO<G, true>::load(gp, i, g);
    Vec4IO<S, true>::load(ap, i, a);
    Vec4IO<S, true>::load(bp, i, b);
    Vec4IO<P, true>::load(pp, i, p);
    const bool decay = c.weight_decay != 0.0f;
#pragma unroll
    for (int k = 0; k < kVec; ++k) {
        float gk = g[k];
        if constexpr (UNSCALE == 1) gk = G::round_f32(gk / xf.scale);
        if constexpr (UNSCALE == 2) gk = G::round_f32(gk * xf.inv_scale);
        if constexpr (CLIP) gk = G::to_f32(G::from_f64((double)gk * xf.clip_coef));
        a[k] = (c.beta1 * a[k]) + (c.complement1 * gk);
        b[k] = (c.beta2 * b[k]) + ((c.complement2 * gk) * gk);
        const float value = decay ? p[k] * c.decay_factor : p[k];
        const float corrected = a[k] / c.correction1;
        const float denominator = __builtin_sqrtf(b[k] / c.correction2) + c.eps;
        p[k] = value - c.lr * (corrected / denominator);
    }
    Vec4IO<S, true>::store(ap, i, a);
    Vec4IO<S, true>::store(bp, i, b);
    Vec4IO<P, true>::store(pp, i, p);
    if constexpr (HAS_COPY) Vec4IO<C, true>::store(cp, i, p);
}

template <class P, class G, class S, class C, bool HAS_COPY, bool CLIP>
__device__ __forceinline__ void lean_slice_unscale(const DevTensor &d, const nt_adamw_coefs &c, const Xform &xf,
                                                   uint64_t start) {
    if (xf.unscale == 2) lean_slice<P, G, S, C, HAS_COPY, 2, CLIP>(d, c, xf, start);
    else if (xf.unscale == 1) lean_slice<P, G, S, C, HAS_COPY, 1, CLIP>(d, c, xf, start);
    else lean_slice<P, G, S, C, HAS_COPY, 0, CLIP>(d, c, xf, start);
}

// BLOCK lanes per workgroup, UNROLL 4-element groups in flight per lane;
// each workgroup takes one slice of a task (task_slice).  A whole one-wave
// slice in the common case runs lean_slice; everything else (tensor tails,
// unaligned tensors, deferred addends, maximize, coupled decay, lr == 0,
// fp16 rounding, the whole-task shape) the general loop below.
template <class P, class G, class S, class C, class R, bool HAS_COPY, int BLOCK, int UNROLL>
__global__ __launch_bounds__(BLOCK) void adamw_mt_kernel(const DevTensor *__restrict__ tensors,
                                                         const Task *__restrict__ tasks, MtArgs args) {
    constexpr int kTileElems = BLOCK * kVec * UNROLL;
    Xform xf = args.xf;
    if (!xform_from_ctrl(args.ctrl, args.honor_skip, xf)) return;
    const DevTensor *dp;
    Slice slice;
    if (!task_slice(tensors, tasks, args.chunk, args.split_shift, dp, slice, args.xcd_group)) return;
    const DevTensor d = *dp;
    const nt_adamw_coefs c = args.slots[d.slot];
    const uint64_t start = slice.start, end = slice.end;
    if constexpr (BLOCK == 64 && UNROLL == 1 && std::is_same<R, RoundF32>::value) {
        if (end - start == (uint64_t)kPassSlice && (d.flags & kAligned16) != 0u && d.incoming == nullptr &&
            !c.maximize && !c.coupled_weight_decay && c.update_parameter) {
            if (xf.clip) lean_slice_unscale<P, G, S, C, HAS_COPY, true>(d, c, xf, start);
            else lean_slice_unscale<P, G, S, C, HAS_COPY, false>(d, c, xf, start);
            return;
        }
    }

    auto *pp = reinterpret_cast<typename P::raw *>(d.param);
    auto *gp = reinterpret_cast<const typename G::raw *>(d.grad);
    auto *ap = reinterpret_cast<typename S::raw *>(d.exp_avg);
    auto *bp = reinterpret_cast<typename S::raw *>(d.exp_avg_sq);
    auto *cp = reinterpret_cast<typename C::raw *>(d.model_copy);
    // A deferred accumulation: the gradient is round(grad + incoming).
    const auto *ip = reinterpret_cast<const typename G::raw *>(d.incoming);
    const bool update = c.update_parameter != 0;
    const bool read_param = update || (c.coupled_weight_decay && c.weight_decay != 0.0f);

    uint64_t scalar_from = start;
    if (d.flags & kAligned16) {
        const uint64_t vend = start + ((end - start) & ~(uint64_t)(kVec - 1));
        // All groups of an iteration are loaded first, then updated, then
        // stored stream by stream (fewer read/write turnarounds per wave).
        for (uint64_t base = start + (uint64_t)threadIdx.x * kVec; base < vend; base += kTileElems) {
            float p[UNROLL][kVec], g[UNROLL][kVec], h[UNROLL][kVec], a[UNROLL][kVec], b[UNROLL][kVec];
            bool ok[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint64_t i = base + (uint64_t)u * BLOCK * kVec;
                ok[u] = i < vend;
                if (ok[u]) {
                    Vec4IO<G, true>::load(gp, i, g[u]);
                    if (ip != nullptr) Vec4IO<G, true>::load(ip, i, h[u]);
                    Vec4IO<S, true>::load(ap, i, a[u]);
                    Vec4IO<S, true>::load(bp, i, b[u]);
                    if (read_param) Vec4IO<P, true>::load(pp, i, p[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                if (ok[u]) {
#pragma unroll
                    for (int k = 0; k < kVec; ++k) {
                        const float gs = ip != nullptr ? G::round_f32(g[u][k] + h[u][k]) : g[u][k];
                        const float gk = clip_one<G>(unscale_one<G>(gs, xf), xf);
                        adamw_elem<R>(p[u][k], gk, a[u][k], b[u][k], c);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
                if (ok[u]) Vec4IO<S, true>::store(ap, base + (uint64_t)u * BLOCK * kVec, a[u]);   // rounds to S
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
                if (ok[u]) Vec4IO<S, true>::store(bp, base + (uint64_t)u * BLOCK * kVec, b[u]);
            if (update) {
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    if (ok[u]) Vec4IO<P, true>::store(pp, base + (uint64_t)u * BLOCK * kVec, p[u]);
                if constexpr (HAS_COPY) {
#pragma unroll
                    for (int u = 0; u < UNROLL; ++u)
                        if (ok[u]) Vec4IO<C, true>::store(cp, base + (uint64_t)u * BLOCK * kVec, p[u]);   // RNE copy
                }
            }
        }
        scalar_from = vend;
    }
    for (uint64_t i = scalar_from + threadIdx.x; i < end; i += BLOCK) {
        float p = read_param ? load1<P>(pp, i) : 0.0f;
        float a = load1<S>(ap, i), b = load1<S>(bp, i);
        float g = load1<G>(gp, i);
        if (ip != nullptr) g = G::round_f32(g + load1<G>(ip, i));
        g = clip_one<G>(unscale_one<G>(g, xf), xf);
        adamw_elem<R>(p, g, a, b, c);
        store1<S>(ap, i, a);
        store1<S>(bp, i, b);
        if (update) {
            store1<P>(pp, i, p);
            if constexpr (HAS_COPY) store1<C>(cp, i, p);
        }
    }
}

// float64 parameters, grads and states (array path).
__global__ __launch_bounds__(kBlock) void adamw_mt_f64_kernel(const DevTensor *__restrict__ tensors,
                                                              const Task *__restrict__ tasks, MtArgs64 args) {
    Xform xf = args.xf;
    if (!xform_from_ctrl(args.ctrl, args.honor_skip, xf)) return;
    const Task task = tasks[blockIdx.x];
    const DevTensor d = tensors[task.tensor];
    const nt_adamw_coefs64 c = args.slots[d.slot];
    const uint64_t start = (uint64_t)task.chunk * (uint64_t)args.chunk;
    const uint64_t end = min(start + (uint64_t)args.chunk, d.numel);
    double *pp = reinterpret_cast<double *>(d.param);
    const double *gp = reinterpret_cast<const double *>(d.grad);
    double *ap = reinterpret_cast<double *>(d.exp_avg);
    double *bp = reinterpret_cast<double *>(d.exp_avg_sq);
    for (uint64_t i = start + threadIdx.x; i < end; i += kBlock) {
        double g = gp[i];
        if (xf.unscale) g = g / (double)xf.scale;
        if (xf.clip) g = g * xf.clip_coef;
        double p = (c.update_parameter || c.coupled_weight_decay) ? pp[i] : 0.0, a = ap[i], b = bp[i];
        adamw_elem64(p, g, a, b, c);
        ap[i] = a;
        bp[i] = b;
        if (c.update_parameter) pp[i] = p;
    }
}

// Dummy trait for "no model copy".
struct TNone {
    using raw = uint16_t;
    static constexpr int code = NT_DTYPE_NONE;
    __device__ static float to_f32(raw) { return 0.0f; }
    __device__ static raw from_f32(float) { return 0; }
    __device__ static float round_f32(float x) { return x; }
};

// Occupancy cap of the one-wave pass for layouts with fp32 moments.  Each
// workgroup reserves this many bytes of LDS that it never touches, so at most
// 160 KiB / bytes one-wave workgroups are resident on a CU of the MI355X,
// against 32 without it (8 waves per SIMD at the pass's 38-42 VGPRs).  With
// 16 to 20 waves per CU in flight instead of 32, these mixes (28 bytes per
// element of which 16 read) stream faster; bf16 moments (20 bytes per element)
// stream slower with any cap.  Timed against no cap on the same buffers in
// one process (fused steps, four rounds):
//   all fp32 (GPT-2-124M):                 10240 B (16 per CU) -2.1 %
//   fp16 gradients, GPT-2 AMP:              9216 B (17 per CU) -3.2 %
//   bf16 gradients, Llama-7B and its 1/8:   8192 B (20 per CU) -1.0 % / -2.1 %
//   bf16 moments, GPT-1.3B and its 1/8:     5 KiB level, 6-12 KiB +1.5 to +30 %
template <class P, class G, class S>
constexpr size_t pass_lds_cap() {
    if constexpr (!std::is_same<P, TF32>::value || !std::is_same<S, TF32>::value) return 0;
    else if constexpr (std::is_same<G, TF16>::value) return 9216;
    else if constexpr (std::is_same<G, TBF16>::value) return 8192;
    else return 10240;
}

// Launch shape of the pass.  A task whose size is a power-of-two multiple of
// kPassSlice is split over one-wave workgroups of kPassSlice elements, one
// 4-element group per lane: many short workgroups stream the pass's
// read/write mix faster than fewer long ones.  Other task sizes run whole
// tasks on kBlock lanes with kPass2Unroll groups in flight per lane.
//
// The all-float32 layout without a model copy (p, g, m, v) walks its grid in
// XCD groups of kFp32XcdGroup workgroups per XCD: measured against the launch
// order on the same buffers, 1.5 % faster on the GPT-2 list (five runs, -2.8 to
// +0.1 %) and 3-7 % on flat 4-64 M-element tensors, while the 16-bit layouts
// measured up to 5 % slower with any grouping, so they keep the launch order.
template <class P, class G, class S, class C, class R, bool HAS_COPY>
static int32_t launch_mt(nt_plan *plan, const MtArgs &args, hipStream_t stream) {
    MtArgs a = args;
    a.split_shift = split_shift(plan, kPassSlice);
    constexpr bool all_fp32 = std::is_same<P, TF32>::value && std::is_same<G, TF32>::value &&
                              std::is_same<S, TF32>::value && !HAS_COPY;
    a.xcd_group = all_fp32 && a.split_shift > 0 ? kFp32XcdGroup : 0u;
    if (a.split_shift > 0) {
        static_assert(kPassSlice == 64 * kVec, "one 4-element group per lane of one wave");
        adamw_mt_kernel<P, G, S, C, R, HAS_COPY, 64, 1><<<dim3((unsigned)(plan->ntasks << a.split_shift)), dim3(64),
                                                          pass_lds_cap<P, G, S>(), stream>>>(plan->d_tensors,
                                                                                             plan->d_tasks, a);
    } else {
        adamw_mt_kernel<P, G, S, C, R, HAS_COPY, kBlock, kPass2Unroll><<<dim3((unsigned)plan->ntasks), dim3(kBlock), 0,
                                                                         stream>>>(plan->d_tensors, plan->d_tasks, a);
    }
    NT_LAUNCH_CHECK("adamw_mt_kernel launch");
    return NT_OK;
}

template <class G, class S>
static int32_t dispatch_copy(nt_plan *plan, const MtArgs &args, hipStream_t stream) {
    switch (plan->layout.copy_dtype) {
        case NT_DTYPE_NONE: return launch_mt<TF32, G, S, TNone, RoundF32, false>(plan, args, stream);
        case NT_BF16: return launch_mt<TF32, G, S, TBF16, RoundF32, true>(plan, args, stream);
        case NT_F16: return launch_mt<TF32, G, S, TF16, RoundF32, true>(plan, args, stream);
        case NT_F32: return launch_mt<TF32, G, S, TF32, RoundF32, true>(plan, args, stream);
        default: return fail(NT_ERR_TYPE, "unsupported model-copy dtype for fp32 AdamW");
    }
}

template <class G>
static int32_t dispatch_state(nt_plan *plan, const MtArgs &args, hipStream_t stream) {
    switch (plan->layout.state_dtype) {
        case NT_F32: return dispatch_copy<G, TF32>(plan, args, stream);
        case NT_BF16: return dispatch_copy<G, TBF16>(plan, args, stream);
        default: return fail(NT_ERR_TYPE, "unsupported optimizer-state dtype for fp32 AdamW");
    }
}

// The dtype combinations the pass is built for, checked before anything is
// launched (also for an empty plan, so a bad layout fails the same way for
// every parameter list).
static int32_t check_mt_layout(const nt_mt_layout &L) {
    if (L.param_dtype == NT_DTYPE_NONE) return fail(NT_ERR_VALUE, "nt_adamw_mt: plan has no parameters");
    if (L.param_dtype == NT_F64) {
        if (L.grad_dtype != NT_F64 || L.state_dtype != NT_F64 || L.copy_dtype != NT_DTYPE_NONE)
            return fail(NT_ERR_TYPE, "float64 AdamW requires float64 grads and states");
        return NT_OK;
    }
    if (L.param_dtype == NT_F16) {
        // float16 parameters: NumPy float16 arithmetic, states and grads float16.
        if (L.grad_dtype != NT_F16 || L.state_dtype != NT_F16 || L.copy_dtype != NT_DTYPE_NONE)
            return fail(NT_ERR_TYPE, "float16 AdamW requires float16 grads and states");
        return NT_OK;
    }
    if (L.param_dtype != NT_F32) return fail(NT_ERR_TYPE, "unsupported parameter dtype");
    if (L.grad_dtype != NT_F32 && L.grad_dtype != NT_F16 && L.grad_dtype != NT_BF16)
        return fail(NT_ERR_TYPE, "unsupported gradient dtype for fp32 AdamW");
    if (L.state_dtype != NT_F32 && L.state_dtype != NT_BF16)
        return fail(NT_ERR_TYPE, "unsupported optimizer-state dtype for fp32 AdamW");
    if (L.copy_dtype != NT_DTYPE_NONE && L.copy_dtype != NT_BF16 && L.copy_dtype != NT_F16 && L.copy_dtype != NT_F32)
        return fail(NT_ERR_TYPE, "unsupported model-copy dtype for fp32 AdamW");
    return NT_OK;
}

}  // namespace nt

using namespace nt;

extern "C" {

int32_t nt_adamw_f32(float *parameter, const float *gradient, float *exp_avg, float *exp_avg_sq, float lr,
                     float beta1, float beta2, float complement1, float complement2, float eps,
                     float weight_decay, float decay_factor, float correction1, float correction2,
                     int32_t maximize, int32_t update_parameter, uint64_t count, void *stream) {
    clear_error();
    if (count == 0) return NT_OK;
    if (gradient == nullptr || exp_avg == nullptr || exp_avg_sq == nullptr || (update_parameter && parameter == nullptr))
        return fail(NT_ERR_VALUE, "nt_adamw_f32: NULL array");
    nt_adamw_coefs c{lr, beta1, beta2, complement1, complement2, eps, weight_decay, decay_factor,
                     correction1, correction2, maximize ? 1 : 0, update_parameter ? 1 : 0, 0, 0};
    const int vectorized = ((((uintptr_t)parameter | (uintptr_t)gradient | (uintptr_t)exp_avg |
                               (uintptr_t)exp_avg_sq) & 15u) == 0) ? 1 : 0;
    const uint64_t blocks = (count + kChunk - 1) / kChunk;
    if (blocks > 0x7fffffffull) return fail(NT_ERR_VALUE, "nt_adamw_f32: tensor too large");
    adamw_f32_kernel<<<dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)stream>>>(
        parameter, gradient, exp_avg, exp_avg_sq, c, count, vectorized);
    NT_LAUNCH_CHECK("adamw_f32_kernel launch");
    return NT_OK;
}

int32_t nt_adamw_mt(nt_plan *plan, const void *slots, int32_t nslots, const nt_grad_xform *xform, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if (nslots < 1 || nslots > NT_MAX_SLOTS || slots == nullptr)
        return fail(NT_ERR_VALUE, "nt_adamw_mt: 1..16 coefficient slots required");
    if ((uint32_t)nslots <= plan->max_slot)
        return fail(NT_ERR_VALUE, "nt_adamw_mt: the plan selects coefficient slot " + std::to_string(plan->max_slot) +
                                      " but only " + std::to_string(nslots) + " slots were given");
    const nt_mt_layout &L = plan->layout;
    if ((rc = check_mt_layout(L)) != NT_OK) return rc;
    if (plan->ntasks == 0) return NT_OK;
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;

    if (L.param_dtype == NT_F64) {
        MtArgs64 a{};
        const nt_adamw_coefs64 *src = static_cast<const nt_adamw_coefs64 *>(slots);
        for (int i = 0; i < nslots; ++i) a.slots[i] = src[i];
        a.xf = make_xform(xform);
        a.ctrl = xform ? xform->ctrl : nullptr;
        a.honor_skip = xform ? xform->honor_skip : 0;
        a.chunk = plan->chunk;
        adamw_mt_f64_kernel<<<dim3((unsigned)plan->ntasks), dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks, a);
        NT_LAUNCH_CHECK("adamw_mt_f64_kernel launch");
        return NT_OK;
    }

    MtArgs a{};
    const nt_adamw_coefs *src = static_cast<const nt_adamw_coefs *>(slots);
    for (int i = 0; i < nslots; ++i) a.slots[i] = src[i];
    a.xf = make_xform(xform);
    a.ctrl = xform ? xform->ctrl : nullptr;
    a.honor_skip = xform ? xform->honor_skip : 0;
    a.chunk = plan->chunk;

    if (L.param_dtype == NT_F16) return launch_mt<TF16, TF16, TF16, TNone, RoundF16, false>(plan, a, s);
    switch (L.grad_dtype) {
        case NT_F32: return dispatch_state<TF32>(plan, a, s);
        case NT_F16: return dispatch_state<TF16>(plan, a, s);
        case NT_BF16: return dispatch_state<TBF16>(plan, a, s);
        default: return fail(NT_ERR_TYPE, "unsupported gradient dtype for fp32 AdamW");
    }
}

}  // extern "C"
