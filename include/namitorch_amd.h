/*
 * namitorch_amd.h — C ABI of the MI355X (gfx950) optimizer-step library.
 *
 * This is the drop-in boundary for NamiTorch's optimizer-step hot path:
 * AdamW.step(), GradScaler unscale_/finite-check/update and clip_grad_norm_.
 * Every entry point takes plain pointers, sizes and a hipStream_t passed as
 * `void*`; no framework types cross the boundary.  Callers (the Python host
 * layer in namitorch_amd/, through ctypes) own every tensor buffer: memory
 * from the library's caching allocator (nt_malloc) or from any other
 * allocator.  The library also owns multi-tensor plans (descriptor table,
 * task map and reduction workspace), released by nt_plan_destroy().
 *
 * Status codes: 0 = OK; a negative code names the exception class the
 * Python layer raises, with the message from nt_last_error() (per thread).
 *
 * Reference citations are paths under renderityai/NamiTorch.
 */
#ifndef NAMITORCH_AMD_H
#define NAMITORCH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define NT_OK 0
#define NT_ERR_VALUE (-1)   /* ValueError  */
#define NT_ERR_TYPE (-2)    /* TypeError   */
#define NT_ERR_RUNTIME (-3) /* RuntimeError (contract violations)   */
#define NT_ERR_HIP (-4)     /* RuntimeError (HIP runtime failure)   */

/* ---- storage dtype codes ----------------------------------------------- */
#define NT_DTYPE_NONE (-1)
#define NT_F32 0
#define NT_F16 1
#define NT_BF16 2
#define NT_F64 3

/* ---- nt_amp_finalize flags --------------------------------------------- */
#define NT_FINALIZE_SCALER_UPDATE 1   /* advance scale/growth tracker (amp.py:225-233) */
#define NT_FINALIZE_CLIP_IF_FINITE 2  /* clip only when no grad is non-finite (runner.py:249) */

/* ---- nt_grad_norm_pow flags -------------------------------------------- */
/* p = 2 only: run the prescaled sum only when max|g| lies outside
 * [2^-480, 2^480], where the finalize's sqrt(sum g^2) can overflow or lose
 * bits in fp64 (float64 gradients); otherwise leave the block unchanged. */
#define NT_NORM_POW_GUARD 1

/* ---- nt_tensor_scalar operations --------------------------------------- */
#define NT_OP_MUL 0
#define NT_OP_DIV 1

/* ---- multi-tensor plan limits ------------------------------------------ */
#define NT_MAX_SLOTS 16     /* coefficient sets per nt_adamw_mt launch */
#define NT_MAX_COMBINE 8    /* control blocks per nt_amp_combine call */

/*
 * One tensor of a multi-tensor plan.  `param` is the array the update is
 * computed on (fp32 master weights in master mode, else the parameter
 * itself); `model_copy` is an optional low-precision copy written in the same
 * pass (NULL when absent).  Unused roles are NULL (a grad-only plan for
 * clip_grad_norm_ has only `grad`).  `slot` selects the coefficient set.
 */
typedef struct nt_mt_tensor {
    void *param;
    void *grad;
    void *exp_avg;
    void *exp_avg_sq;
    void *model_copy;
    uint64_t numel;
    uint32_t slot;
    uint32_t reserved;
} nt_mt_tensor; /* 56 bytes; padded to 64 on device */

/* Storage dtypes of the roles; identical for every tensor of one plan. */
typedef struct nt_mt_layout {
    int32_t param_dtype;  /* NT_F32 (master or plain), NT_F16, NT_F64 */
    int32_t grad_dtype;   /* NT_F32, NT_F16, NT_BF16, NT_F64 */
    int32_t state_dtype;  /* NT_F32, NT_BF16 (or the param dtype) */
    int32_t copy_dtype;   /* NT_DTYPE_NONE, NT_F16, NT_BF16 */
} nt_mt_layout;

/*
 * The ten AdamW coefficients, each already rounded to the parameter dtype
 * on the host exactly as the reference does (optim/adam.py:82-86 via
 * optim/_common.py:39-47), plus the two launch flags of the reference kernel
 * (backends/cuda/adamw.py:7-11).  `coupled_weight_decay` selects the
 * reference's Adam (L2 term added to the gradient, optim/_common.py:62-63)
 * instead of AdamW's decoupled decay.
 */
typedef struct nt_adamw_coefs {
    float lr, beta1, beta2, complement1, complement2;
    float eps, weight_decay, decay_factor, correction1, correction2;
    int32_t maximize;
    int32_t update_parameter;
    int32_t coupled_weight_decay;
    int32_t reserved;
} nt_adamw_coefs; /* 56 bytes */

/* fp64 twin for float64 parameters (array path only). */
typedef struct nt_adamw_coefs64 {
    double lr, beta1, beta2, complement1, complement2;
    double eps, weight_decay, decay_factor, correction1, correction2;
    int32_t maximize;
    int32_t update_parameter;
    int32_t coupled_weight_decay;
    int32_t reserved;
} nt_adamw_coefs64; /* 96 bytes */

/*
 * Device-resident control block of one AMP/clip iteration.  Written by
 * nt_amp_finalize(); read by nt_adamw_mt() when a grad transform points at it.
 */
typedef struct nt_amp_ctrl {
    double sumsq;          /* sum of squares of the (unscaled) grads, fp64;
                              undefined when found_inf is set */
    double amax;           /* max |g| over finite grads, fp64 */
    double norm;           /* global grad norm (fp64), reference semantics */
    double clip_coef;      /* max_norm / (norm + 1e-6) */
    float scale;           /* loss scale of the next iteration */
    float scale_used;      /* loss scale this iteration's grads divide by */
    int32_t found_inf;     /* any unscaled grad non-finite */
    int32_t has_nan;       /* any unscaled grad NaN */
    int32_t clip;          /* clip_coef < 1: pass 2 multiplies by clip_coef */
    int32_t skip;          /* pass 2 leaves params/states untouched */
    int32_t growth_tracker;
    int32_t iterations;    /* finalize calls since the block was reset */
    int32_t skipped;       /* of which found non-finite grads */
    int32_t reserved;
} nt_amp_ctrl; /* 72 bytes */

/*
 * Page-locked host mirror of one control block.  nt_amp_finalize and
 * nt_amp_combine, given a mirror, store the block's final contents in
 * `ctrl` and then set `ready` to 1 with a system-scope release, so the
 * host reads the iteration's decisions (skip, scale, norm) without an event
 * on the launch stream: the host clears `ready` before the launch and reads
 * `ctrl` once `ready` is 1.  Mirrors come from nt_mirror_alloc
 * (fine-grained page-locked memory, which the device writes through to the
 * host).  No reference counterpart: the reference reads these values with
 * blocking device-to-host copies (amp.py:152-167, .item()).
 */
typedef struct nt_amp_mirror {
    nt_amp_ctrl ctrl;
    int32_t ready;
    int32_t reserved;
} nt_amp_mirror; /* 80 bytes */

/*
 * How pass 2 turns a stored grad into the one AdamW consumes.  With
 * `ctrl == NULL` the host-known values below are used: unscale divides by
 * `scale` in fp32 and rounds to the grad dtype (amp.py:190-191); clip
 * multiplies in fp64 by `clip_coef` and rounds to the grad dtype
 * (optim/clip_grad.py:111).  With `ctrl != NULL` the scale, clip flag, clip
 * coefficient and skip flag are read from that device block instead
 * (scale_used, clip, clip_coef, skip).
 */
typedef struct nt_grad_xform {
    float scale;
    int32_t unscale;
    double clip_coef;
    int32_t clip;
    int32_t honor_skip;    /* with ctrl: skip the update when ctrl->skip */
    const nt_amp_ctrl *ctrl;
} nt_grad_xform;

typedef struct nt_plan nt_plan; /* opaque multi-tensor plan */

/* ---- library / device -------------------------------------------------- */

/* Thread-local message of the last failing call ("" if none). */
const char *nt_last_error(void);

/* ABI version of this library (bumped when a struct layout or an entry
 * point's signature changes). */
int32_t nt_abi_version(void);

/* HIP_VERSION of the headers the library was compiled with, and that of the
 * HIP runtime it is bound to in this process (hipRuntimeGetVersion; both
 * major * 10^7 + minor * 10^5 + patch). */
int32_t nt_hip_version(int32_t *built, int32_t *runtime);

/* Number of visible HIP devices. */
int32_t nt_device_count(int32_t *count);

/* Name of the gfx target of `device` (e.g. "gfx950") into buf[len]. */
int32_t nt_device_arch(int32_t device, char *buf, int32_t len);

/* The calling thread's current device: entry points that take only
 * pointers and a stream queue on the null stream of this device when
 * `stream` is NULL (replaces the device scope `cupy.cuda.Device(...)` that
 * the reference's CUDA calls run in, backends/_cuda_execution.py:132). */
int32_t nt_set_device(int32_t device);
int32_t nt_get_device(int32_t *device);

/* Wait for all work queued on `stream`. */
int32_t nt_stream_synchronize(void *stream);

/* Copy `bytes` between host and device on `stream` and wait for it. */
int32_t nt_memcpy_d2h(void *dst, const void *src, uint64_t bytes, void *stream);
int32_t nt_memcpy_h2d(void *dst, const void *src, uint64_t bytes, void *stream);

/* ---- device memory, streams, events (nt_memory.hip) ---------------------
 * The services the reference takes from CuPy (its memory pool and OOM
 * report, backends/_cuda_memory.py:24-94; streams and event-ordered
 * lifetimes, backends/_cuda_execution.py:21-137; transfers,
 * backends/cuda/__init__.py:87-153), owned by the library so a host layer
 * needs no other GPU framework.
 *
 * nt_malloc: `bytes` of device memory on `device` for use on `stream`, from
 * a caching pool: a freed block is reused only by later allocations on the
 * stream it was allocated on (stream order makes that safe); a block also
 * used on other streams (nt_record_stream) is reused once an event recorded
 * on each of them at nt_free has completed.  An out-of-memory hipMalloc
 * releases the cached blocks and retries; the error names the bytes in use
 * and reserved.  nt_empty_cache releases every cached block (waits for the
 * device). */
#define NT_COPY_H2D 1
#define NT_COPY_D2H 2
#define NT_COPY_D2D 3
int32_t nt_malloc(int32_t device, uint64_t bytes, void *stream, void **out);
int32_t nt_free(void *ptr);
int32_t nt_record_stream(void *ptr, void *stream);
int32_t nt_memory_stats(int32_t device, uint64_t *in_use, uint64_t *reserved);
int32_t nt_empty_cache(int32_t device);
/* Page-locked host memory (hipHostMalloc). */
int32_t nt_host_alloc(uint64_t bytes, void **out);
int32_t nt_host_free(void *ptr);
/* `count` zeroed control-block mirrors in one fine-grained page-locked
 * allocation (hipHostMallocCoherent); nt_mirror_free releases it. */
int32_t nt_mirror_alloc(int32_t count, nt_amp_mirror **out);
int32_t nt_mirror_free(nt_amp_mirror *mirrors);
/* Wait for `mirror`'s flag, set by a kernel queued on `stream`: polls the
 * flag, querying the stream every 64 polls; NT_ERR_RUNTIME when all the
 * stream's work completed and the flag is still clear.  Records nothing on
 * the stream. */
int32_t nt_mirror_wait(const nt_amp_mirror *mirror, void *stream);
/* Streams are created at the default priority and do not synchronize with
 * the null stream.  nt_stream_destroy waits for the stream's work first;
 * plans and pool blocks that were used on it may still be destroyed or
 * freed afterwards, in any order. */
int32_t nt_stream_create(int32_t device, void **out);
int32_t nt_stream_destroy(void *stream);
int32_t nt_stream_wait_event(void *stream, void *event);
/* Events (`timing` != 0 for nt_event_elapsed); nt_event_query sets *done to
 * 1 once the recorded work has completed, else 0. */
int32_t nt_event_create(int32_t timing, void **out);
int32_t nt_event_destroy(void *event);
int32_t nt_event_record(void *event, void *stream);
int32_t nt_event_synchronize(void *event);
int32_t nt_event_query(void *event, int32_t *done);
int32_t nt_event_elapsed(void *start, void *stop, float *milliseconds);
/* Asynchronous copy of `bytes` (NT_COPY_*) ordered on `stream`. */
int32_t nt_memcpy_async(void *dst, const void *src, uint64_t bytes, int32_t kind, void *stream);
/* Write `count` items of `itemsize` bytes (1, 2, 4, 8), each the low bytes
 * of `pattern`: Tensor.fill_/zero_ and zero-initialized state
 * (optim/_common.py:50-54) without hipMemset, so it can be captured. */
int32_t nt_fill(void *ptr, uint64_t count, int32_t itemsize, uint64_t pattern, void *stream);
/* out[i] = in[i] converted between NT_F32/NT_F16/NT_BF16/NT_F64 with one
 * rounding to nearest even, as NumPy's astype (Tensor.to(dtype),
 * tensor.py:1252-1287 on device arrays). */
int32_t nt_cast(const void *in, int32_t in_dtype, void *out, int32_t out_dtype,
                uint64_t count, void *stream);
/* Device ordinal of a device pointer (NT_ERR_VALUE for host memory):
 * backend.adamw.supports's "array on this device" check
 * (backends/cuda/adamw.py:33-46) for arrays handed over by address. */
int32_t nt_pointer_device(const void *ptr, int32_t *device);
/* *capturing = 1 while `stream` is being captured into a HIP graph: the
 * guard of backends/_graph_capture.py:12-14. */
int32_t nt_stream_capturing(void *stream, int32_t *capturing);

/* ---- per-tensor AdamW: the reference kernel's own ABI ------------------ */

/*
 * Replaces `namitorch_adamw_float32` (backends/cuda/adamw.py:7-28, launched
 * by AdamWCUDAKernel.run, backends/cuda/adamw.py:54-73): one fp32 tensor,
 * same arguments in the same order, plus the stream.  Returns NT_OK with
 * nothing launched for count == 0.
 */
int32_t nt_adamw_f32(float *parameter, const float *gradient, float *exp_avg,
                     float *exp_avg_sq, float lr, float beta1, float beta2,
                     float complement1, float complement2, float eps,
                     float weight_decay, float decay_factor, float correction1,
                     float correction2, int32_t maximize,
                     int32_t update_parameter, uint64_t count, void *stream);

/* ---- multi-tensor plans ------------------------------------------------ */

/*
 * Build a plan over `n` tensors on `device`: uploads the descriptor table
 * and a workgroup->(tensor, chunk) task map.  Replaces the per-parameter
 * Python loop of _FirstOrderOptimizer.step (optim/_common.py:165-166) and
 * the per-gradient loops of GradScaler.unscale_/_finite (amp.py:152-192)
 * and _total_norm (optim/clip_grad.py:63-79) with one launch per pass.
 * `chunk` is the elements per workgroup task (0 = default).  The tables
 * live in memory of the library's pools and are staged in page-locked host
 * memory, copied asynchronously on `stream`, so creation does not wait for
 * queued work.  nt_plan_destroy() does not wait either: the plan's memory
 * returns to the pools in the order of every stream the plan was used on
 * (those streams must still exist when the plan is destroyed).
 */
int32_t nt_plan_create(int32_t device, const nt_mt_tensor *tensors, int32_t n,
                       const nt_mt_layout *layout, int64_t chunk,
                       void *stream, nt_plan **out);
int32_t nt_plan_destroy(nt_plan *plan);

/*
 * Replace one pointer column of every descriptor of `plan`: column 0 param,
 * 1 grad, 2 exp_avg, 3 exp_avg_sq, 4 model_copy, 5 incoming; `pointers[n]`
 * with n the plan's tensor count.
 *
 * Column 5 (incoming, NULL allowed per tensor, grad dtype, not float64)
 * defers the last micro-batch's gradient accumulation into the step
 * (Tensor._accumulate_grad, tensor.py:443-450, autograd.py:198-205): for a
 * tensor with an incoming pointer, nt_amp_prepass and nt_adamw_mt use
 * round_to_grad_dtype(grad + incoming) as its gradient, the value the
 * accumulation would have stored, and do not write `grad`.  nt_grad_apply,
 * nt_grad_norm_pow, nt_grad_zero and nt_grad_accumulate refuse a plan with
 * any incoming pointer set (NT_ERR_VALUE).  The update is a copy queued on `stream` after the
 * work already queued there, so kernels launched earlier keep the old
 * pointers.  Lets one plan serve gradients that are reallocated every step
 * (Optimizer.zero_grad(set_to_none=True), optim/optimizer.py:197-206, then a
 * new backward) without rebuilding its tables.  A pointer must keep the
 * alignment the plan was built with (NT_ERR_VALUE otherwise; build a new
 * plan then).  Calls on one plan must use one stream.  No reference
 * counterpart: the reference passes arrays per launch.
 */
int32_t nt_plan_set_pointers(nt_plan *plan, int32_t column, const void *const *pointers, int32_t n,
                             void *stream);

/* Elements, tensors and workgroup tasks in a plan. */
int32_t nt_plan_info(const nt_plan *plan, uint64_t *numel, int32_t *tensors,
                     int64_t *tasks);

/*
 * Pass 2: multi-tensor AdamW over every tensor of `plan` in one launch.
 * `slots[nslots]` holds the coefficient sets tensors select by `slot`
 * (fp32 params: nt_adamw_coefs; fp64 params: nt_adamw_coefs64).  The
 * element arithmetic is the reference's, operation for operation and
 * without FMA contraction (backends/cuda/adamw.py:15-25 ==
 * optim/adam.py:35-42 + optim/_common.py:67-73).  `xform` may be NULL.
 * A tensor's incoming gradient (plan column 5) is added to its gradient
 * first.
 */
int32_t nt_adamw_mt(nt_plan *plan, const void *slots, int32_t nslots,
                    const nt_grad_xform *xform, void *stream);

/*
 * Pass 1 of an AMP/clip iteration over the grads of `plan`: per element
 * g' = to_grad_dtype(f32(g) / scale) when `unscale` (amp.py:190-191),
 * finiteness of g' (amp.py:152-167) and the fp64 sum of squares and max of
 * |g'| (optim/clip_grad.py:63-79).  Writes per-workgroup partials into the
 * plan's workspace; grads are not written.  With `ctrl != NULL` the scale
 * is read from ctrl->scale on the device (the sync-free path).  A tensor's
 * incoming gradient (plan column 5) is added to its gradient first.
 */
int32_t nt_amp_prepass(nt_plan *plan, float scale, int32_t unscale,
                       const nt_amp_ctrl *ctrl, void *stream);

/*
 * Stage 2: reduce the partials of the last nt_amp_prepass in a fixed order
 * into `ctrl` (device memory).  norm_type 2 or +inf; other norm types call
 * nt_grad_norm_pow afterwards.  With `max_norm >= 0` also computes
 * clip_coef = max_norm / (norm + 1e-6) and clip = clip_coef < 1
 * (optim/clip_grad.py:106-107); with NT_FINALIZE_CLIP_IF_FINITE the clip
 * is also withheld when any grad is non-finite, as the reference training
 * loop only clips after a finite unscale_ (training/runner.py:249).  Always
 * sets skip = found_inf and scale_used = scale.  With
 * NT_FINALIZE_SCALER_UPDATE the GradScaler state machine of amp.py:225-233
 * then runs on the device, advancing ctrl->scale and ctrl->growth_tracker.
 * `carry` (may be NULL; never equal to `ctrl`): the scaler state starts
 * from *carry as nt_ctrl_carry(ctrl, carry) would set it, so a new
 * iteration's block needs no carry launch; with NULL it starts from *ctrl.
 * The pre-pass of such an iteration reads the scale from `carry`'s block.
 * `mirror` (may be NULL) receives a host copy of the finished block.
 */
int32_t nt_amp_finalize(nt_plan *plan, nt_amp_ctrl *ctrl, const nt_amp_ctrl *carry,
                        double norm_type, double max_norm, int32_t flags,
                        double growth_factor, double backoff_factor,
                        int32_t growth_interval, nt_amp_mirror *mirror, void *stream);

/*
 * One GradScaler iteration over several optimizers (amp.py:169-233 called
 * for each optimizer, then update() once).  `blocks[0..n)` (device memory,
 * 1 <= n <= NT_MAX_COMBINE, pairwise distinct) hold each optimizer's
 * statistics from nt_amp_prepass + nt_amp_finalize with max_norm < 0 and no
 * flags; `carry` is the previous iteration's block they all carried from.
 * The sums of squares add in block order and the maxima and NaN/inf flags
 * combine into the norm of all their gradients (norm_type 2 or +inf), from
 * which the clip decision is taken as nt_amp_finalize takes it
 * (NT_FINALIZE_CLIP_IF_FINITE: no clip when any optimizer's gradients are
 * non-finite, the reference loop clipping only after every unscale_
 * returned True, training/runner.py:248-249); NT_FINALIZE_SCALER_UPDATE
 * runs one scaler update, backing off when any optimizer found a non-finite
 * gradient (amp.py:224-233).  Every block then holds the global norm, clip
 * flag and coefficient and the new scaler state, and keeps its own
 * sumsq/amax/found_inf/has_nan with skip = its own found_inf: each
 * optimizer's step checks only its own gradients (GradScaler.step,
 * amp.py:209-217).  No single reference function: it is the composition the
 * reference runs on the host.  `mirrors` (may be NULL, else n entries, each
 * may be NULL) receive host copies of the finished blocks.
 */
int32_t nt_amp_combine(nt_amp_ctrl *const *blocks, int32_t n, const nt_amp_ctrl *carry,
                       double norm_type, double max_norm, int32_t flags,
                       double growth_factor, double backoff_factor,
                       int32_t growth_interval, nt_amp_mirror *const *mirrors, void *stream);

/*
 * General p-norm (0 < p < inf) of optim/clip_grad.py:70-79: sum over
 * grads of (|g'|/amax)^p in fp64, with amax from the previous prepass
 * already in `ctrl`; leaves the norm in ctrl->norm, the raw sum in
 * ctrl->sumsq and, with max_norm >= 0, the clip coefficient.  A
 * non-finite or zero amax leaves the block as nt_amp_finalize wrote it.
 * p = 2 is the finalize's own case except for float64 gradients whose
 * squares leave the fp64 range: NT_NORM_POW_GUARD runs the pass only then,
 * deciding on the device (no host round trip).
 */
int32_t nt_grad_norm_pow(nt_plan *plan, nt_amp_ctrl *ctrl, double norm_type,
                         double max_norm, float scale, int32_t unscale,
                         int32_t scale_from_ctrl, int32_t flags, void *stream);

/*
 * Write the transformed grads back in place: the deferred form of
 * GradScaler.unscale_'s grad.copy_(grad / scale) (amp.py:191) and of
 * clip_grad_norm_'s grad.copy_(f64(grad) * coef) (optim/clip_grad.py:111).
 */
int32_t nt_grad_apply(nt_plan *plan, const nt_grad_xform *xform,
                      void *stream);

/* Set ctrl->scale / growth_tracker and clear every other field (a kernel,
 * not a memset, so the call can be captured in a HIP graph). */
int32_t nt_ctrl_reset(nt_amp_ctrl *ctrl, float scale, int32_t growth_tracker,
                      void *stream);

/* Start a new iteration's block: dst takes src's scaler state (scale,
 * growth_tracker, iterations, skipped); every per-iteration field of dst is
 * cleared.  dst and src may not alias. */
int32_t nt_ctrl_carry(nt_amp_ctrl *dst, const nt_amp_ctrl *src, void *stream);

/* ---- gradient producer edges ------------------------------------------- */

/*
 * Zero every gradient of `plan` in one launch: Optimizer.zero_grad with
 * set_to_none=False (optim/optimizer.py:197-206, grad.zero_() per
 * parameter).  Gradients are the plan's `grad` column (layout.grad_dtype).
 */
int32_t nt_grad_zero(nt_plan *plan, void *stream);

/*
 * Accumulate incoming gradients into stored ones for every tensor of
 * `plan` in one launch: Tensor._accumulate_grad (tensor.py:443-450) over
 * autograd.accumulate_gradient (autograd.py:198-205).  Stored gradients are
 * the `grad` column (layout.grad_dtype), incoming ones the `param` column
 * (layout.param_dtype).  Each incoming value is cast to the stored dtype
 * (round to nearest even) and added in the stored dtype, as NumPy does;
 * with `assign` != 0 the cast value replaces the stored one (the first
 * gradient of a leaf).
 */
int32_t nt_grad_accumulate(nt_plan *plan, int32_t assign, void *stream);

/*
 * nt_amp_prepass followed by nt_amp_finalize over one flat gradient buffer
 * grad[count] of `grad_dtype` (NT_F32, NT_F16, NT_BF16) on `device`,
 * allocating nothing: no plan, no hipMalloc, no library allocation.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation), e.g. over a flat gradient bucket.  Arguments and the block
 * written to `ctrl` mean what they mean for that pair (unscale by `scale`,
 * or by carry->scale when `carry` is given; norm_type 2 or +inf only).  The
 * per-workgroup partials live in a fixed 64 KiB device array of the library
 * (4096 partials), one per GPU, held until the process ends; count is at
 * most 2**40 elements (NT_ERR_VALUE beyond, nothing launched).  Every call
 * on one GPU shares that array: calls that overlap on one GPU (on different
 * streams, or from several threads) race and must be serialized by the
 * caller.  Nothing in it needs clearing between calls: each call writes all
 * the partials it reads.
 */
int32_t nt_amp_flat_stats_noalloc(int32_t device, const void *grad, int32_t grad_dtype,
                                  uint64_t count, float scale, int32_t unscale,
                                  nt_amp_ctrl *ctrl, const nt_amp_ctrl *carry,
                                  double norm_type, double max_norm, int32_t flags,
                                  double growth_factor, double backoff_factor,
                                  int32_t growth_interval, void *stream);

/* ---- small single-array kernels ---------------------------------------- */

/*
 * out[i] = in[i] * operand (NT_OP_MUL) or in[i] / operand (NT_OP_DIV),
 * computed in `out_dtype` and rounded once to it: Tensor.__mul__ and
 * Tensor.__truediv__ with a scalar operand (tensor.py:814-823 through
 * _binary_operation, tensor.py:634-646, and binary_forward,
 * _backend.py:54-72).  The caller promotes as the reference does
 * (dtype.py:99-109, 204-208: a Python float is float32, so a float16 loss
 * times the loss scale is float32) and passes the operand already rounded
 * to `out_dtype`; `in_dtype` must widen exactly into `out_dtype`.  This is
 * GradScaler.scale (amp.py:137-138: loss * self._scale) and the training
 * loop's loss / grad_accum_steps (training/runner.py:246).  With
 * `ctrl != NULL` the operand is ctrl->scale (the loss scale held on the
 * device after a fused step).
 */
int32_t nt_tensor_scalar(const void *in, int32_t in_dtype, void *out,
                         int32_t out_dtype, double operand, int32_t op,
                         const nt_amp_ctrl *ctrl, uint64_t count, void *stream);

/*
 * *flag = 1 if any element of `array` is < 0 (the exp_avg_sq check of
 * _check_state, optim/_common.py:114-115); `flag` is device memory and is
 * cleared first.
 */
int32_t nt_any_negative(const void *array, int32_t dtype, uint64_t count,
                        int32_t *flag, void *stream);

/* ---- measurement ------------------------------------------------------- */

/*
 * Streaming probe, no counterpart in the reference: a measurement aid for
 * benchmarks.  It moves `count` elements through `nreads` read and
 * `nwrites` write streams with the pass's access pattern (one-wave
 * workgroups of 256 elements, one nontemporal group of four elements per
 * lane: 16 bytes for fp32 streams, 8 bytes for 16-bit streams; reads before
 * writes) and
 * one add per written element, so its bandwidth is the ceiling of that
 * read/write mix on the device.  The last `nreads16` read and `nwrites16`
 * write streams are 16-bit (bfloat16), the others fp32.  Supported
 * (nreads, nreads16, nwrites, nwrites16): (0,0,1,0) (0,0,3,0) (1,0,0,0)
 * (1,0,1,0) (2,0,2,0) (4,0,0,0) (4,0,3,0) (5,0,4,0), and the pass mixes
 * (4,3,4,3) (C4: fp32 master + three bf16 streams each way) and (4,1,4,1)
 * (C3/C5: three fp32 streams + one 16-bit stream each way).  `count` is a
 * positive multiple of 4096, every stream holds `count` elements and is
 * 16-byte aligned; a read-only probe passes one fp32 write stream that is
 * written only if the sum of the reads has one particular NaN bit pattern.
 */
int32_t nt_stream_probe(const void *const *reads, int32_t nreads, int32_t nreads16,
                        void *const *writes, int32_t nwrites, int32_t nwrites16,
                        uint64_t count, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NAMITORCH_AMD_H */
