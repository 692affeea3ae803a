// nt_grad.hip — gradient producer edges of the optimizer step: zeroing every
// gradient of a plan in one launch (Optimizer.zero_grad(set_to_none=False))
// and accumulating incoming gradients into the stored ones
// (Tensor._accumulate_grad → autograd.accumulate_gradient) for all leaves
// in one launch.
//
// Accumulation follows NumPy exactly: the incoming value is cast to the
// stored dtype (round to nearest even; float64 → float16/bfloat16 rounds
// once, through round-to-odd float32), then the two values are added in the
// stored dtype.  For float16 that is what NumPy's half add does: widen both
// to float32, add in float32, round the sum to float16.  bfloat16 (no NumPy
// counterpart) is treated the same way.
#include <hip/hip_runtime.h>

#include "nt_internal.hpp"

namespace nt {

// ---- zero ------------------------------------------------------------------------------
// 16-byte zero stores where the tensor is aligned; a slice is one store per
// lane of a kBlock-lane workgroup (write-only streams run fastest that way).
template <class T>
constexpr int64_t zero_slice() { return (int64_t)kBlock * (16 / (int64_t)sizeof(T)); }

template <class T>
__global__ __launch_bounds__(kBlock) void grad_zero_kernel(const DevTensor *__restrict__ tensors,
                                                           const Task *__restrict__ tasks, int64_t chunk,
                                                           int32_t shift) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(1))) u32x4 gu32x4;
    constexpr int kPer = 16 / (int)sizeof(T);           // elements per 16-byte store
    const DevTensor *dp;
    Slice slice;
    if (!task_slice(tensors, tasks, chunk, shift, dp, slice)) return;
    const DevTensor &d = *dp;
    const uint64_t start = slice.start, end = slice.end;
    T *g = reinterpret_cast<T *>(d.grad);
    uint64_t scalar_from = start;
    if (d.flags & kAligned16) {
        const uint64_t vend = start + ((end - start) / kPer) * kPer;
        const u32x4 zero = {0u, 0u, 0u, 0u};
        for (uint64_t i = start + (uint64_t)threadIdx.x * kPer; i < vend; i += (uint64_t)kBlock * kPer)
            __builtin_nontemporal_store(zero, (gu32x4 *)(g + i));
        scalar_from = vend;
    }
    for (uint64_t i = scalar_from + threadIdx.x; i < end; i += kBlock) g[i] = T(0);
}

// ---- accumulate (stored dtype D, incoming dtype S; 16-bit and fp32) ----------------------
template <class D, class S, bool ASSIGN>
__device__ __forceinline__ float accumulate_one(float stored, float incoming) {
    const float converted = D::round_f32(incoming);      // S value (exact in fp32) cast to D
    if constexpr (ASSIGN) return converted;
    return D::round_f32(stored + converted);
}

// A slice is one kTile iteration: kUnroll 4-element groups per lane.  For
// this read-read-write mix that ran faster than one-wave slices or one
// group per lane.
template <class D, class S, bool ASSIGN>
__global__ __launch_bounds__(kBlock) void grad_accumulate_kernel(const DevTensor *__restrict__ tensors,
                                                                 const Task *__restrict__ tasks, int64_t chunk,
                                                                 int32_t shift) {
    const DevTensor *dp;
    Slice slice;
    if (!task_slice(tensors, tasks, chunk, shift, dp, slice)) return;
    const DevTensor &d = *dp;
    const uint64_t start = slice.start, end = slice.end;
    auto *dst = reinterpret_cast<typename D::raw *>(d.grad);
    const auto *src = reinterpret_cast<const typename S::raw *>(d.param);
    uint64_t scalar_from = start;
    if (d.flags & kAligned16) {
        const uint64_t vend = start + ((end - start) & ~(uint64_t)(kVec - 1));
        for (uint64_t base = start + (uint64_t)threadIdx.x * kVec; base < vend; base += kTile) {
            float a[kUnroll][kVec], b[kUnroll][kVec];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const uint64_t i = base + (uint64_t)u * kBlock * kVec;
                if (i < vend) {
                    Vec4IO<S, true>::load(src, i, b[u]);
                    if constexpr (!ASSIGN) Vec4IO<D, true>::load(dst, i, a[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const uint64_t i = base + (uint64_t)u * kBlock * kVec;
                if (i < vend) {
#pragma unroll
                    for (int k = 0; k < kVec; ++k)
                        a[u][k] = accumulate_one<D, S, ASSIGN>(ASSIGN ? 0.0f : a[u][k], b[u][k]);
                    Vec4IO<D, true>::store(dst, i, a[u]);
                }
            }
        }
        scalar_from = vend;
    }
    for (uint64_t i = scalar_from + threadIdx.x; i < end; i += kBlock) {
        const float stored = ASSIGN ? 0.0f : load1<D>(dst, i);
        store1<D>(dst, i, accumulate_one<D, S, ASSIGN>(stored, load1<S>(src, i)));
    }
}

// ---- accumulate with float64 on either side (per element) --------------------------------
__device__ __forceinline__ double load_any(const void *base, int32_t dtype, uint64_t i) {
    switch (dtype) {
        case NT_F64: return reinterpret_cast<const double *>(base)[i];
        case NT_F32: return (double)reinterpret_cast<const float *>(base)[i];
        case NT_F16: return (double)f16_to_f32(reinterpret_cast<const uint16_t *>(base)[i]);
        default: return (double)bf16_to_f32(reinterpret_cast<const uint16_t *>(base)[i]);
    }
}

// Cast a float64 value to `dtype` (single rounding) and return it as float64.
__device__ __forceinline__ double round_to(double v, int32_t dtype) {
    switch (dtype) {
        case NT_F64: return v;
        case NT_F32: return (double)(float)v;
        case NT_F16: return (double)TF16::to_f32(TF16::from_f64(v));
        default: return (double)TBF16::to_f32(TBF16::from_f64(v));
    }
}

__device__ __forceinline__ void store_any(void *base, int32_t dtype, uint64_t i, double v) {
    switch (dtype) {
        case NT_F64: reinterpret_cast<double *>(base)[i] = v; break;
        case NT_F32: reinterpret_cast<float *>(base)[i] = (float)v; break;
        case NT_F16: reinterpret_cast<uint16_t *>(base)[i] = TF16::from_f64(v); break;
        default: reinterpret_cast<uint16_t *>(base)[i] = TBF16::from_f64(v); break;
    }
}

__global__ __launch_bounds__(kBlock) void grad_accumulate_any_kernel(const DevTensor *__restrict__ tensors,
                                                                     const Task *__restrict__ tasks, int64_t chunk,
                                                                     int32_t dst_dtype, int32_t src_dtype,
                                                                     int32_t assign) {
    const Task task = tasks[blockIdx.x];
    const DevTensor &d = tensors[task.tensor];
    const uint64_t start = (uint64_t)task.chunk * (uint64_t)chunk;
    const uint64_t end = min(start + (uint64_t)chunk, d.numel);
    for (uint64_t i = start + threadIdx.x; i < end; i += kBlock) {
        const double converted = round_to(load_any(d.param, src_dtype, i), dst_dtype);
        double value = converted;
        if (!assign) {
            const double stored = load_any(d.grad, dst_dtype, i);
            // float64 adds in float64; the narrower dtypes add in float32 and
            // round once, as above (both operands are exact in float32).
            value = dst_dtype == NT_F64 ? stored + converted : (double)((float)stored + (float)converted);
        }
        store_any(d.grad, dst_dtype, i, value);
    }
}

template <class D, class S>
static void launch_accumulate(const nt_plan *plan, hipStream_t s, bool assign) {
    const int32_t shift = split_shift(plan, kTile);
    const dim3 grid((unsigned)(plan->ntasks << shift));
    if (assign)
        grad_accumulate_kernel<D, S, true><<<grid, dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks, plan->chunk, shift);
    else
        grad_accumulate_kernel<D, S, false><<<grid, dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks, plan->chunk, shift);
}

template <class D>
static bool dispatch_source(int32_t src, const nt_plan *plan, hipStream_t s, bool assign) {
    switch (src) {
        case NT_F32: launch_accumulate<D, TF32>(plan, s, assign); return true;
        case NT_F16: launch_accumulate<D, TF16>(plan, s, assign); return true;
        case NT_BF16: launch_accumulate<D, TBF16>(plan, s, assign); return true;
        default: return false;
    }
}

template <class T>
static void launch_zero(const nt_plan *plan, hipStream_t s) {
    const int32_t shift = split_shift(plan, zero_slice<T>());
    grad_zero_kernel<T><<<dim3((unsigned)(plan->ntasks << shift)), dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks,
                                                                                       plan->chunk, shift);
}

}  // namespace nt

using namespace nt;

extern "C" {

int32_t nt_grad_zero(nt_plan *plan, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if ((rc = check_no_incoming(plan, "nt_grad_zero")) != NT_OK) return rc;
    if (plan->ntasks == 0) return NT_OK;
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    switch (plan->layout.grad_dtype) {
        case NT_F32: launch_zero<uint32_t>(plan, s); break;
        case NT_F16:
        case NT_BF16: launch_zero<uint16_t>(plan, s); break;
        case NT_F64: launch_zero<uint64_t>(plan, s); break;
        default: return fail(NT_ERR_TYPE, "nt_grad_zero: unsupported gradient dtype");
    }
    NT_LAUNCH_CHECK("grad_zero_kernel launch");
    return NT_OK;
}

int32_t nt_grad_accumulate(nt_plan *plan, int32_t assign, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if ((rc = check_no_incoming(plan, "nt_grad_accumulate")) != NT_OK) return rc;
    const int32_t dst = plan->layout.grad_dtype, src = plan->layout.param_dtype;
    if (src == NT_DTYPE_NONE) return fail(NT_ERR_VALUE, "nt_grad_accumulate: the plan has no incoming gradients");
    if (plan->ntasks == 0) return NT_OK;
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)plan->ntasks);
    const DevTensor *t = plan->d_tensors;
    const Task *k = plan->d_tasks;
    bool launched = false;
    if (dst != NT_F64 && src != NT_F64) {
        switch (dst) {
            case NT_F32: launched = dispatch_source<TF32>(src, plan, s, assign != 0); break;
            case NT_F16: launched = dispatch_source<TF16>(src, plan, s, assign != 0); break;
            case NT_BF16: launched = dispatch_source<TBF16>(src, plan, s, assign != 0); break;
            default: break;
        }
    } else {
        grad_accumulate_any_kernel<<<grid, dim3(kBlock), 0, s>>>(t, k, plan->chunk, dst, src, assign != 0);
        launched = true;
    }
    if (!launched) return fail(NT_ERR_TYPE, "nt_grad_accumulate: unsupported gradient dtypes");
    NT_LAUNCH_CHECK("grad_accumulate_kernel launch");
    return NT_OK;
}

}  // extern "C"
