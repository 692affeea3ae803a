// nt_common.hpp — device helpers shared by the optimizer-step kernels.
//
// Storage types, exact conversions and 128-bit vector I/O for gfx950.
// All arithmetic here must round exactly like NumPy on the host: the library
// is compiled with -ffp-contract=off (no FMA contraction), correctly rounded
// fp32 divide/sqrt and fp32 denormals preserved.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/namitorch_amd.h"
#include "nt_layout.hpp"

namespace nt {

constexpr int kBlock = 256;        // threads per workgroup (4 wave64s)
constexpr int kVec = 4;            // elements per vector access
constexpr int kUnroll = 2;         // independent vector groups per thread per iteration
constexpr int kTile = kBlock * kVec * kUnroll;   // elements per workgroup iteration
constexpr int kPass2Unroll = 4;    // groups in flight per lane in the multi-tensor AdamW pass
constexpr int kPass2Tile = kBlock * kVec * kPass2Unroll;
constexpr int kPassSlice = 256;    // elements per one-wave workgroup of the split multi-tensor pass
constexpr uint32_t kFp32XcdGroup = 256;   // workgroups per XCD per group, all-float32 pass layout
// Gradient bytes the pre-pass leaves resident in the MI355X's 256 MB Infinity
// Cache (MALL) for the AdamW pass that follows it: the pre-pass reads its last
// tasks, up to this many bytes, with temporal loads (which allocate in the
// MALL) and the rest nontemporally (which do not).  The pass's own accesses are
// nontemporal, so they find those gradients still resident.  Timed against
// 128-4096 MiB windows at either end of the task list (same buffers, one
// process): a 320 MiB window at the end was the best or level on every layout.
constexpr uint64_t kMallKeepBytes = 320ull << 20;

// ---- bit casts ---------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bits_f32(uint32_t b) { return __builtin_bit_cast(float, b); }

// ---- bfloat16 (stored as uint16 bit patterns) ---------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// Round-to-nearest-even fp32 -> bf16.  NaN stays NaN (quieted, sign kept).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// ---- float16 (stored as uint16 bit patterns) ----------------------------------
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// v_cvt_f16_f32: round to nearest even, overflow to inf.  The operand is
// made opaque first: otherwise the compiler folds a producing multiply and
// this conversion into one v_fma_mixlo_f16 with a +0 addend, which turns a
// -0 product into +0 (NumPy's float16 arithmetic, an fp32 operation rounded
// once to fp16, keeps -0).  Every fp16 result is therefore the fp32 value of
// its operation rounded once.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    __asm__("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// fp64 -> fp32 with round-to-odd: truncate toward zero, then force the last
// bit to 1 when the conversion was inexact.  A second rounding of this value
// to a format with at least two fewer significand bits (fp16: 11, bf16: 8,
// against fp32's 24) equals a single correct rounding from fp64, which is
// what NumPy's direct float64 -> float16 cast produces.
__device__ __forceinline__ float f64_to_f32_odd(double d) {
    float f = (float)d;                      // round to nearest even
    double back = (double)f;
    if (back != d && d == d) {               // inexact and not NaN
        uint32_t b = f32_bits(f);
        if (__builtin_fabs(back) > __builtin_fabs(d)) b -= 1u;  // undo rounding away from zero
        b |= 1u;
        f = bits_f32(b);
    }
    return f;
}

// ---- storage type traits -----------------------------------------------------
// Each trait: `raw` storage type, exact widening to fp32/fp64, rounding of an
// fp32 (or fp64) value to the storage format and back.
struct TF32 {
    using raw = float;
    static constexpr int code = NT_F32;
    __device__ static float to_f32(raw x) { return x; }
    __device__ static raw from_f32(float x) { return x; }
    __device__ static float round_f32(float x) { return x; }
    __device__ static raw from_f64(double x) { return (float)x; }
};
struct TF16 {
    using raw = uint16_t;
    static constexpr int code = NT_F16;
    __device__ static float to_f32(raw x) { return f16_to_f32(x); }
    __device__ static raw from_f32(float x) { return f32_to_f16(x); }
    __device__ static float round_f32(float x) { return f16_to_f32(f32_to_f16(x)); }
    __device__ static raw from_f64(double x) { return f32_to_f16(f64_to_f32_odd(x)); }
};
struct TBF16 {
    using raw = uint16_t;
    static constexpr int code = NT_BF16;
    __device__ static float to_f32(raw x) { return bf16_to_f32(x); }
    __device__ static raw from_f32(float x) { return f32_to_bf16(x); }
    __device__ static float round_f32(float x) { return bf16_to_f32(f32_to_bf16(x)); }
    __device__ static raw from_f64(double x) { return f32_to_bf16(f64_to_f32_odd(x)); }
};
struct TF64 {
    using raw = double;
    static constexpr int code = NT_F64;
    __device__ static raw from_f64(double x) { return x; }
};

// Exact widening of a stored value to fp64.
template <class T>
__device__ __forceinline__ double widen64(typename T::raw x) {
    if constexpr (T::code == NT_F64) return x;
    else return (double)T::to_f32(x);
}

// ---- 4-element vector I/O ------------------------------------------------------
// Loads/stores of 4 consecutive elements at a 4-element-aligned index: one
// dwordx4 for fp32, one dwordx2 for 16-bit types.  A wave's instruction
// covers 64 consecutive groups, i.e. whole cache lines.  Pointers are cast
// to the global address space (global_load/global_store instead of flat),
// and streams touched once per step use nontemporal accesses.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) f32x4 gf32x4;
typedef __attribute__((address_space(1))) u32x2 gu32x2;

template <bool NT, class V, class G>
__device__ __forceinline__ V gload(const void *p) {
    const G *q = (const G *)(p);
    if constexpr (NT) return __builtin_nontemporal_load(q);
    else return *q;
}
template <bool NT, class V, class G>
__device__ __forceinline__ void gstore(void *p, V v) {
    G *q = (G *)(p);
    if constexpr (NT) __builtin_nontemporal_store(v, q);
    else *q = v;
}

template <class T, bool NT> struct Vec4IO;

template <bool NT> struct Vec4IO<TF32, NT> {
    __device__ static void load(const float *base, uint64_t i, float (&out)[4]) {
        f32x4 a = gload<NT, f32x4, gf32x4>(base + i);
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    }
    __device__ static void store(float *base, uint64_t i, const float (&in)[4]) {
        gstore<NT, f32x4, gf32x4>(base + i, f32x4{in[0], in[1], in[2], in[3]});
    }
};

template <class T, bool NT> struct Vec4IO16 {
    __device__ static void load(const uint16_t *base, uint64_t i, float (&out)[4]) {
        u32x2 w = gload<NT, u32x2, gu32x2>(base + i);
        out[0] = T::to_f32((uint16_t)(w.x & 0xffffu));
        out[1] = T::to_f32((uint16_t)(w.x >> 16));
        out[2] = T::to_f32((uint16_t)(w.y & 0xffffu));
        out[3] = T::to_f32((uint16_t)(w.y >> 16));
    }
    // Rounds each float to T (values already representable store exactly).
    __device__ static void store(uint16_t *base, uint64_t i, const float (&in)[4]) {
        u32x2 w = {(uint32_t)T::from_f32(in[0]) | ((uint32_t)T::from_f32(in[1]) << 16),
                   (uint32_t)T::from_f32(in[2]) | ((uint32_t)T::from_f32(in[3]) << 16)};
        gstore<NT, u32x2, gu32x2>(base + i, w);
    }
};
template <bool NT> struct Vec4IO<TF16, NT> : Vec4IO16<TF16, NT> {};
template <bool NT> struct Vec4IO<TBF16, NT> : Vec4IO16<TBF16, NT> {};

// Scalar element access for tails and unaligned tensors.
template <class T>
__device__ __forceinline__ float load1(const typename T::raw *base, uint64_t i) {
    return T::to_f32(base[i]);
}
template <class T>
__device__ __forceinline__ void store1(typename T::raw *base, uint64_t i, float v) {
    base[i] = T::from_f32(v);
}

// ---- device descriptor / task tables: nt_layout.hpp ------------------------------
constexpr int kRingSlots = 4;        // pinned slots per plan for pointer-column updates
static_assert(kTile == kChunkQuantum, "plan chunks are whole workgroup tiles");

// Per-workgroup partial of the grad pre-pass: float64 sum of squares of the
// finite (unscaled) grads and max |g| as a double that is +inf when some
// grad is infinite and NaN when some grad is NaN.
struct alignas(16) Partial {
    double sumsq;
    double amax;
};
constexpr int kPrepassTasks = 8;        // 4096-element tasks per pre-pass workgroup
constexpr int kPrepassUnroll = 4;       // 4-element groups in flight per lane
constexpr int kPrepassTile = kBlock * kVec * kPrepassUnroll;
constexpr int64_t kStage2Span = 4096;   // partials per stage-2 workgroup
constexpr int64_t kFinalizeDirect = 4096;  // at most this many partials: no stage 2

// ---- grad transform (unscale then clip), exactly as stored grads would be -------
// g' = to_G(f32(g) / scale)           (amp.py:190-191; division or an exact
//                                      multiply by 1/scale for powers of two)
// g''= to_G(f64(g') * clip_coef)      (optim/clip_grad.py:111)
struct Xform {
    float scale;
    float inv_scale;
    double clip_coef;
    int32_t unscale;      // 0: none, 1: divide, 2: multiply by exact inverse
    int32_t clip;
};

template <class G>
__device__ __forceinline__ float unscale_one(float g, const Xform &x) {
    if (x.unscale == 1) return G::round_f32(g / x.scale);
    if (x.unscale == 2) return G::round_f32(g * x.inv_scale);
    return g;
}
template <class G>
__device__ __forceinline__ float clip_one(float g, const Xform &x) {
    if (!x.clip) return g;
    return G::to_f32(G::from_f64((double)g * x.clip_coef));
}

// ---- wavefront / workgroup reductions (fixed order => deterministic) --------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        double o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
    return v;
}

}  // namespace nt
