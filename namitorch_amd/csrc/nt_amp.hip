// nt_amp.hip — gradient pre-pass (unscale + finite check + fp64 norm partials),
// the single-workgroup finalize, the general p-norm, in-place grad apply and
// small helpers of the GradScaler path.
//
// Reductions are deterministic: every workgroup writes its partial to a
// fixed slot and one workgroup reduces the slots in a fixed order.  No
// atomics are used.
#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "nt_internal.hpp"
#include "nt_scaler.hpp"

namespace nt {

struct Acc {
    double sumsq = 0.0;
    double amax = 0.0;
    int nan = 0;
    int inf = 0;
    __device__ void add(float g) {
        if (__builtin_isfinite(g)) {
            const double d = (double)g;
            sumsq = __builtin_fma(d, d, sumsq);
            const double a = __builtin_fabs(d);
            amax = a > amax ? a : amax;
        } else if (g != g) {
            nan = 1;
        } else {
            inf = 1;
        }
    }
    __device__ void add64(double g) {
        if (__builtin_isfinite(g)) {
            sumsq = __builtin_fma(g, g, sumsq);
            const double a = __builtin_fabs(g);
            amax = a > amax ? a : amax;
        } else if (g != g) {
            nan = 1;
        } else {
            inf = 1;
        }
    }
};

// Reduce an Acc over the workgroup; thread 0 gets the result.
__device__ Acc block_reduce(Acc a) {
    __shared__ double s_sum[kBlock / 64];
    __shared__ double s_max[kBlock / 64];
    __shared__ int s_flags[kBlock / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double s = wave_sum(a.sumsq);
    double m = wave_max(a.amax);
    int f = wave_or(a.nan | (a.inf << 1));
    if (lane == 0) {
        s_sum[wave] = s;
        s_max[wave] = m;
        s_flags[wave] = f;
    }
    __syncthreads();
    Acc r;
    if (threadIdx.x == 0) {
        double ts = 0.0, tm = 0.0;
        int tf = 0;
        for (int w = 0; w < kBlock / 64; ++w) {
            ts += s_sum[w];
            tm = s_max[w] > tm ? s_max[w] : tm;
            tf |= s_flags[w];
        }
        r.sumsq = ts;
        r.amax = tm;
        r.nan = tf & 1;
        r.inf = (tf >> 1) & 1;
    }
    return r;
}

__device__ __forceinline__ float ctrl_scale_inv(float s, int &mode, float &inv) {
    const uint32_t b = f32_bits(s);
    const uint32_t e = (b >> 23) & 0xffu;
    if ((b & 0x807fffffu) == 0u && e >= 1u && e <= 253u) {
        mode = 2;
        inv = bits_f32((254u - e) << 23);
    } else {
        mode = 1;
        inv = 1.0f;
    }
    return s;
}

// ---- pre-pass ------------------------------------------------------------------
// One workgroup per kPrepassTasks consecutive tasks.  Per element g' (the
// unscaled grad, rounded to its dtype) it keeps
//   * the max of |g'| as fp32 bits: integer order equals magnitude order for
//     finite values, +inf is 0x7f800000 and any NaN is above it, so one
//     unsigned max yields amax, "some inf" and "some NaN" together;
//   * the fp64 sum of g'^2 over finite g'.  For fp16/bf16 grads g'*g' is exact
//     in fp32 whenever the fp32 exponent of g' lies in [-63, 62] (at most 11
//     significant bits squared, result normal), so only the fp64 add remains;
//     other groups take the fp64 fma path.
struct PAcc {
    double sumsq = 0.0;
    uint32_t amax_bits = 0;
};

__device__ __forceinline__ void pacc_wide(PAcc &a, float g) {
    const uint32_t b = f32_bits(g) & 0x7fffffffu;
    a.amax_bits = b > a.amax_bits ? b : a.amax_bits;
    if (b < 0x7f800000u) {
        const double d = (double)g;
        a.sumsq = __builtin_fma(d, d, a.sumsq);
    }
}

// fp32 exponent field of g in [64, 189] (or g == 0): g*g exact and normal in fp32.
__device__ __forceinline__ bool square_exact(float g) {
    const uint32_t b = f32_bits(g) & 0x7fffffffu;
    const uint32_t e = b >> 23;
    return b == 0u || (e - 64u) <= 125u;
}

// fp16: every finite fp16 squares exactly into a normal fp32, so the fast
// accumulation is always exact (non-finite values only set the flags).
// bf16 (raw mode): accumulates the squares of the stored values; exactness is
// checked per workgroup from the min/max magnitudes afterwards.
template <class G>
__device__ __forceinline__ void pacc_fast(PAcc &a, uint32_t &mn, const float (&g)[kPrepassUnroll][kVec]) {
#pragma unroll
    for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
        for (int k = 0; k < kVec; ++k) {
            const uint32_t b = f32_bits(g[u][k]) & 0x7fffffffu;
            a.amax_bits = b > a.amax_bits ? b : a.amax_bits;
            if constexpr (G::code == NT_BF16) {
                const uint32_t z = b - 1u;                // 0 wraps to the top: ignored by min
                mn = z < mn ? z : mn;
            }
            a.sumsq += (double)(g[u][k] * g[u][k]);
        }
}

__device__ __forceinline__ void pacc_fast1(PAcc &a, uint32_t &mn, float v, bool track_min) {
    const uint32_t b = f32_bits(v) & 0x7fffffffu;
    a.amax_bits = b > a.amax_bits ? b : a.amax_bits;
    if (track_min) {
        const uint32_t z = b - 1u;
        mn = z < mn ? z : mn;
    }
    a.sumsq += (double)(v * v);
}

// Wave-uniform max/min of a u32 (every lane gets the result).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

__device__ __forceinline__ double amax_from_bits(uint32_t bits) { return (double)bits_f32(bits); }

// Fixed-order combination of two partials: sums add, a NaN max wins, else the
// larger max (+inf included).
__device__ __forceinline__ Partial merge_partial(Partial a, Partial b) {
    Partial r;
    r.sumsq = a.sumsq + b.sumsq;
    r.amax = (a.amax != a.amax) ? a.amax : ((b.amax != b.amax) ? b.amax : (b.amax > a.amax ? b.amax : a.amax));
    return r;
}

// Per-workgroup combination of the waves' partials without a barrier: each
// wave's lane 0 parks its partial in LDS and bumps a workgroup counter; the
// last wave to arrive combines the slots in wave order (deterministic) and
// writes the workgroup's partial.  Waves never wait for each other.
struct WaveJoin {
    Partial slot[kBlock / 64];
    uint32_t arrived;
};

__device__ __forceinline__ void wave_join_init(WaveJoin &j) {
    if (threadIdx.x == 0) j.arrived = 0u;
    __syncthreads();
}

__device__ __forceinline__ void wave_join_finish(WaveJoin &j, Partial mine, Partial *out) {
    if ((threadIdx.x & 63) != 0) return;
    const int wave = threadIdx.x >> 6;
    j.slot[wave] = mine;
    const uint32_t before = __hip_atomic_fetch_add(&j.arrived, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (before != (uint32_t)(kBlock / 64 - 1)) return;
    Partial r = j.slot[0];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w) r = merge_partial(r, j.slot[w]);
    *out = r;
}

// g <- round_G(g + h) elementwise: Tensor._accumulate_grad's add in the
// gradient dtype (both operands already of that dtype; NumPy's float16 add
// widens to float32 and rounds once, and so does bfloat16 here).
template <class G>
__device__ __forceinline__ void add_incoming(float (&g)[kPrepassUnroll][kVec], const float (&h)[kPrepassUnroll][kVec]) {
#pragma unroll
    for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
        for (int k = 0; k < kVec; ++k) g[u][k] = G::round_f32(g[u][k] + h[u][k]);
}

// ---- whole-task loads with a chosen cache policy ----------------------------------
// A whole, aligned pre-pass task is read through a buffer resource over its
// bytes, so the cache policy is an immediate of each load instruction:
// temporal loads allocate in the MALL (the gradients stay resident for the
// AdamW pass that follows), nontemporal ones do not.  (The same choice made
// between two ordinary loads is not kept: the compiler merges loads that
// differ only in their nontemporal marking.)
constexpr int kCpolNontemporal = 2;     // the nt bit of the cache-policy operand

template <class T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t task_rsrc(const T *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T *>(base), (short)0, (int)(kPrepassTile * sizeof(T)),
                                             0x00020000);
}

// The kPrepassUnroll pairs of 32-bit words of this lane (4 16-bit values each).
__device__ __forceinline__ void task_words(__amdgpu_buffer_rsrc_t r, u32x2 (&w)[kPrepassUnroll], bool keep) {
    const int lane = (int)threadIdx.x * kVec * 2;
    if (keep) {
#pragma unroll
        for (int u = 0; u < kPrepassUnroll; ++u)
            w[u] = __builtin_amdgcn_raw_buffer_load_b64(r, lane + u * kBlock * kVec * 2, 0, 0);
    } else {
#pragma unroll
        for (int u = 0; u < kPrepassUnroll; ++u)
            w[u] = __builtin_amdgcn_raw_buffer_load_b64(r, lane + u * kBlock * kVec * 2, 0, kCpolNontemporal);
    }
}

// This lane's kPrepassUnroll groups of 4 values, widened to fp32.
template <class G>
__device__ __forceinline__ void task_values(__amdgpu_buffer_rsrc_t r, float (&g)[kPrepassUnroll][kVec], bool keep) {
    if constexpr (sizeof(typename G::raw) == 2) {
        u32x2 w[kPrepassUnroll];
        task_words(r, w, keep);
#pragma unroll
        for (int u = 0; u < kPrepassUnroll; ++u) {
            g[u][0] = G::to_f32((uint16_t)(w[u].x & 0xffffu));
            g[u][1] = G::to_f32((uint16_t)(w[u].x >> 16));
            g[u][2] = G::to_f32((uint16_t)(w[u].y & 0xffffu));
            g[u][3] = G::to_f32((uint16_t)(w[u].y >> 16));
        }
    } else {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 w[kPrepassUnroll];
        const int lane = (int)threadIdx.x * kVec * 4;
        if (keep) {
#pragma unroll
            for (int u = 0; u < kPrepassUnroll; ++u)
                w[u] = __builtin_amdgcn_raw_buffer_load_b128(r, lane + u * kBlock * kVec * 4, 0, 0);
        } else {
#pragma unroll
            for (int u = 0; u < kPrepassUnroll; ++u)
                w[u] = __builtin_amdgcn_raw_buffer_load_b128(r, lane + u * kBlock * kVec * 4, 0, kCpolNontemporal);
        }
#pragma unroll
        for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
            for (int k = 0; k < kVec; ++k) g[u][k] = bits_f32(w[u][k]);
    }
}

// No raw-word visitor (prepass_visit's default).
struct NoRaw {};

// Visits the elements of this workgroup's tasks: vec(g) for each group of
// kPrepassUnroll x 4 loaded values (missing ones 0), one(value) for
// tail/unaligned elements.  With a `raw` visitor, whole aligned tasks of
// tensors without a deferred addend hand it the kPrepassUnroll pairs of
// 32-bit words as loaded (4 16-bit values per pair, in memory order) instead.
// Task entries and descriptors are read at workgroup-uniform addresses, so
// they come through scalar loads with no LDS staging or barrier; every wave
// covers its lanes' share of each task.
template <class G, class Vec, class One, class Raw = NoRaw>
__device__ __forceinline__ void prepass_visit(const DevTensor *__restrict__ tensors, const Task *__restrict__ tasks,
                                              int64_t first, int ntask, int64_t chunk, int64_t keep_from, Vec vec,
                                              One one, Raw raw = Raw()) {
    for (int j = 0; j < ntask; ++j) {
        // Tasks from keep_from on are read with temporal loads (keep_from_task).
        const bool keep = first + j >= keep_from;
        const Task task = tasks[first + j];
        const DevTensor d = tensors[task.tensor];
        const uint64_t start = (uint64_t)task.chunk * (uint64_t)chunk;
        const auto *gp = reinterpret_cast<const typename G::raw *>(d.grad);
        // A deferred accumulation: the gradient is round(grad + incoming).
        const auto *ip = reinterpret_cast<const typename G::raw *>(d.incoming);
        // A whole, aligned 4096-element task (all but tensor tails): straight
        // code with the kPrepassUnroll loads issued back to back.  The
        // branches are workgroup-uniform.
        if (chunk == kPrepassTile && (d.flags & kAligned16) != 0u && start + (uint64_t)kPrepassTile <= d.numel) {
            if constexpr (!std::is_same<Raw, NoRaw>::value) {
                if (ip == nullptr) {
                    u32x2 w[kPrepassUnroll];
                    task_words(task_rsrc(gp + start), w, keep);
                    // All loads issue before any of them is consumed.
                    __builtin_amdgcn_sched_barrier(0);
                    raw(w);
                    continue;
                }
            }
            float g[kPrepassUnroll][kVec];
            task_values<G>(task_rsrc(gp + start), g, keep);
            if (ip != nullptr) {
                float h[kPrepassUnroll][kVec];
                task_values<G>(task_rsrc(ip + start), h, keep);
                add_incoming<G>(g, h);
            }
            vec(g);
            continue;
        }
        const uint64_t end = min(start + (uint64_t)chunk, d.numel);
        uint64_t scalar_from = start;
        if (d.flags & kAligned16) {
            const uint64_t vend = start + ((end - start) & ~(uint64_t)(kVec - 1));
            for (uint64_t base = start + (uint64_t)threadIdx.x * kVec; base < vend; base += kPrepassTile) {
                float g[kPrepassUnroll][kVec], h[kPrepassUnroll][kVec];
#pragma unroll
                for (int u = 0; u < kPrepassUnroll; ++u) {
                    const uint64_t i = base + (uint64_t)u * kBlock * kVec;
                    if (i < vend) {
                        Vec4IO<G, true>::load(gp, i, g[u]);
                        if (ip != nullptr) Vec4IO<G, true>::load(ip, i, h[u]);
                    } else {
#pragma unroll
                        for (int k = 0; k < kVec; ++k) g[u][k] = h[u][k] = 0.0f;
                    }
                }
                if (ip != nullptr) add_incoming<G>(g, h);
                vec(g);
            }
            scalar_from = vend;
        }
        for (uint64_t i = scalar_from + threadIdx.x; i < end; i += kBlock) {
            float v = load1<G>(gp, i);
            if (ip != nullptr) v = G::round_f32(v + load1<G>(ip, i));
            one(v);
        }
    }
}

// fp16 gradients under a power-of-two unscale whose inverse is itself an
// fp16 value (2**-24 .. 2**15): the fp16 product g * inv is the exact product
// rounded once to fp16, which is what round_f16(f32(g) * inv) gives, so two
// values are unscaled per packed instruction.  Each square is exact in fp32
// and the fp64 sum adds them in pacc_fast's order (per lane: group by group,
// values in memory order).  |h| bit patterns order like magnitudes in fp16 as
// in fp32 (+inf 0x7c00, every NaN above), so the maximum runs on packed
// 16-bit lanes and is widened to fp32 bits once at the end.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void pacc_f16_word(PAcc &a, ushort2_t &max2, half2_t inv2, uint32_t word) {
    const half2_t h = __builtin_bit_cast(half2_t, word) * inv2;
    const ushort2_t bits = __builtin_bit_cast(ushort2_t, h) & (ushort2_t)(0x7fff);
    max2 = __builtin_elementwise_max(max2, bits);
    // h*h + 0 (exact, so equal to h*h): one mixed-precision fma from the fp16 halves.
    const float h0 = (float)h.x, h1 = (float)h.y;
    a.sumsq += (double)__builtin_fmaf(h0, h0, 0.0f);
    a.sumsq += (double)__builtin_fmaf(h1, h1, 0.0f);
}

// Runs body(unscale, raw): unscale is the per-value form for the generic
// paths, raw the packed form for whole aligned tasks.
template <class Body>
__device__ __forceinline__ void visit_f16(half2_t inv2, ushort2_t &max2, PAcc &acc, Body body) {
    const float inv = (float)inv2.x;
    body([inv](float g) { return TF16::round_f32(g * inv); },
         [&](const u32x2 (&w)[kPrepassUnroll]) {
#pragma unroll
             for (int u = 0; u < kPrepassUnroll; ++u) {
                 pacc_f16_word(acc, max2, inv2, w[u].x);
                 pacc_f16_word(acc, max2, inv2, w[u].y);
             }
         });
}

template <class G>
__global__ __launch_bounds__(kBlock) void prepass_kernel(const DevTensor *__restrict__ tensors,
                                                         const Task *__restrict__ tasks, int64_t ntasks,
                                                         int64_t chunk, int64_t keep_from, Xform xf,
                                                         const nt_amp_ctrl *ctrl, Partial *__restrict__ partials) {
    __shared__ WaveJoin join;
    wave_join_init(join);
    if (ctrl != nullptr && xf.unscale) xf.scale = ctrl_scale_inv(ctrl->scale, xf.unscale, xf.inv_scale);
    const int64_t first = (int64_t)blockIdx.x * kPrepassTasks;
    const int64_t left = ntasks - first;
    const int ntask = left < (int64_t)kPrepassTasks ? (int)(left > 0 ? left : 0) : kPrepassTasks;

    PAcc acc;
    uint32_t mn = 0xffffffffu;
    // Raw mode (bf16): no unscale, or an exact power-of-two scale >= 1.  The
    // squares of the stored values are summed and the sum rescaled by
    // inv_scale^2 at the end.  That equals the sum over the unscaled values
    // when every unscaled value stays a normal bf16 and every stored square is
    // exact in fp32, which each wave checks from its own magnitude range; a
    // wave that fails the check recomputes its elements one by one.
    const bool raw = G::code == NT_BF16 && (xf.unscale == 0 || (xf.unscale == 2 && xf.inv_scale <= 1.0f));
    if (raw) {
        prepass_visit<G>(tensors, tasks, first, ntask, chunk, keep_from,
                         [&](const float (&g)[kPrepassUnroll][kVec]) { pacc_fast<G>(acc, mn, g); },
                         [&](float v) { pacc_fast1(acc, mn, v, true); });
        const uint32_t mx = wave_max_u32(acc.amax_bits);
        const uint32_t wmn = wave_min_u32(mn);
        // fp32 exponent field: stored square exact and normal for [64, 189];
        // unscaled value (by 2^-k) a normal bf16 for >= k + 1.
        const uint32_t k = xf.unscale ? 127u - ((f32_bits(xf.inv_scale) >> 23) & 0xffu) : 0u;
        const uint32_t lo = k + 1u > 64u ? k + 1u : 64u;
        const bool finite = mx < 0x7f800000u;
        const bool any_nonzero = wmn != 0xffffffffu;
        const uint32_t emax = mx >> 23, emin = (wmn + 1u) >> 23;
        const bool redo = finite && (emax > 189u || (any_nonzero && emin < lo));   // wave-uniform
        Partial mine;
        if (redo) {
            acc = PAcc();
            prepass_visit<G>(tensors, tasks, first, ntask, chunk, keep_from,
                             [&](const float (&g)[kPrepassUnroll][kVec]) {
#pragma unroll
                                 for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
                                     for (int k = 0; k < kVec; ++k) pacc_wide(acc, unscale_one<G>(g[u][k], xf));
                             },
                             [&](float v) { pacc_wide(acc, unscale_one<G>(v, xf)); });
            mine = Partial{wave_sum(acc.sumsq), amax_from_bits(wave_max_u32(acc.amax_bits))};
        } else {
            mine = Partial{wave_sum(acc.sumsq), amax_from_bits(mx)};
            if (xf.unscale) {
                const double inv = (double)xf.inv_scale;
                mine.sumsq *= inv * inv;       // exact: a power of two
                mine.amax *= inv;
            }
        }
        wave_join_finish(join, mine, partials + blockIdx.x);
        return;
    }
    // Per-element path: unscale and round each value, then accumulate.  The
    // unscale mode is the same for the whole grid; each mode has its own
    // element loop, so no element pays a test of it (the compiler does not
    // hoist the test out of the unrolled loop by itself).
    auto visit = [&](auto unscale) {
        prepass_visit<G>(tensors, tasks, first, ntask, chunk, keep_from,
                         [&](const float (&g)[kPrepassUnroll][kVec]) {
                             float h[kPrepassUnroll][kVec];
#pragma unroll
                             for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
                                 for (int k = 0; k < kVec; ++k) h[u][k] = unscale(g[u][k]);
                             if constexpr (G::code == NT_F16) {
                                 pacc_fast<G>(acc, mn, h);
                             } else {
#pragma unroll
                                 for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
                                     for (int k = 0; k < kVec; ++k) pacc_wide(acc, h[u][k]);
                             }
                         },
                         [&](float v) { pacc_wide(acc, unscale(v)); });
    };
    if constexpr (G::code == NT_F16) {
        const uint32_t e = f32_bits(xf.inv_scale) >> 23;
        if (xf.unscale == 2 && e >= 127u - 24u && e <= 127u + 15u) {
            // inv = 2**(e - 127) is an fp16 value: the packed path.
            const half2_t inv2 = {(_Float16)xf.inv_scale, (_Float16)xf.inv_scale};
            ushort2_t max2 = {0, 0};
            visit_f16(inv2, max2, acc, [&](auto unscale, auto raw) {
                prepass_visit<G>(tensors, tasks, first, ntask, chunk, keep_from,
                                 [&](const float (&g)[kPrepassUnroll][kVec]) {
                                     float h[kPrepassUnroll][kVec];
#pragma unroll
                                     for (int u = 0; u < kPrepassUnroll; ++u)
#pragma unroll
                                         for (int k = 0; k < kVec; ++k) h[u][k] = unscale(g[u][k]);
                                     pacc_fast<G>(acc, mn, h);
                                 },
                                 [&](float v) { pacc_wide(acc, unscale(v)); }, raw);
            });
            const uint32_t m16 = max2.x > max2.y ? max2.x : max2.y;
            const uint32_t wide = f32_bits(f16_to_f32((uint16_t)m16));
            acc.amax_bits = wide > acc.amax_bits ? wide : acc.amax_bits;
            const Partial mine{wave_sum(acc.sumsq), amax_from_bits(wave_max_u32(acc.amax_bits))};
            wave_join_finish(join, mine, partials + blockIdx.x);
            return;
        }
    }
    // The three cases of unscale_one.
    if (xf.unscale == 2) {
        const float inv = xf.inv_scale;
        visit([inv](float g) { return G::round_f32(g * inv); });
    } else if (xf.unscale == 1) {
        const float scale = xf.scale;
        visit([scale](float g) { return G::round_f32(g / scale); });
    } else {
        visit([](float g) { return g; });
    }
    const Partial mine{wave_sum(acc.sumsq), amax_from_bits(wave_max_u32(acc.amax_bits))};
    wave_join_finish(join, mine, partials + blockIdx.x);
}

__global__ __launch_bounds__(kBlock) void prepass_f64_kernel(const DevTensor *__restrict__ tensors,
                                                             const Task *__restrict__ tasks, int64_t ntasks,
                                                             int64_t chunk, Xform xf, const nt_amp_ctrl *ctrl,
                                                             Partial *__restrict__ partials) {
    __shared__ WaveJoin join;
    wave_join_init(join);
    const double scale = (ctrl != nullptr) ? (double)ctrl->scale : (double)xf.scale;
    Acc acc;
    for (int j = 0; j < kPrepassTasks; ++j) {
        const int64_t t = (int64_t)blockIdx.x * kPrepassTasks + j;
        if (t >= ntasks) break;
        const Task task = tasks[t];
        const DevTensor d = tensors[task.tensor];
        const uint64_t start = (uint64_t)task.chunk * (uint64_t)chunk;
        const uint64_t end = min(start + (uint64_t)chunk, d.numel);
        const double *gp = reinterpret_cast<const double *>(d.grad);
        for (uint64_t i = start + threadIdx.x; i < end; i += kBlock) {
            double g = gp[i];
            if (xf.unscale) g = g / scale;
            acc.add64(g);
        }
    }
    const double s = wave_sum(acc.sumsq);
    const double m = wave_max(acc.amax);
    const int f = wave_or(acc.nan | (acc.inf << 1));
    const Partial mine{s, (f & 1) ? __builtin_nan("") : ((f & 2) ? __builtin_inf() : m)};
    wave_join_finish(join, mine, partials + blockIdx.x);
}

// Fixed-order reduction of partials[begin, end) over one workgroup.
__device__ Acc reduce_partials(const Partial *__restrict__ partials, int64_t begin, int64_t end) {
    Acc acc;
    for (int64_t i = begin + threadIdx.x; i < end; i += kBlock) {
        const Partial p = partials[i];
        acc.sumsq += p.sumsq;
        if (p.amax != p.amax) acc.nan = 1;
        else if (__builtin_isinf(p.amax)) acc.inf = 1;
        else acc.amax = p.amax > acc.amax ? p.amax : acc.amax;
    }
    return block_reduce(acc);
}

__global__ __launch_bounds__(kBlock) void stage2_kernel(const Partial *__restrict__ partials, int64_t n,
                                                        Partial *__restrict__ out) {
    const int64_t begin = (int64_t)blockIdx.x * kStage2Span;
    const int64_t end = min(begin + kStage2Span, n);
    Acc r = reduce_partials(partials, begin, end);
    if (threadIdx.x == 0) {
        const double amax = r.nan ? __builtin_nan("") : (r.inf ? __builtin_inf() : r.amax);
        out[blockIdx.x] = Partial{r.sumsq, amax};
    }
}

// Host copy of a finished block: the block's bytes go to the page-locked
// mirror (fine-grained memory: the stores reach host memory, no device cache
// keeps them), then a system-scope release orders them before `ready` = 1,
// which the host reads before the block.
__device__ __forceinline__ void publish(nt_amp_mirror *mirror, const nt_amp_ctrl &c) {
    mirror->ctrl = c;
    __hip_atomic_store(&mirror->ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// `carry` (optional): start from carried_ctrl(*carry) instead of *ctrl, so a
// new iteration's block needs no separate carry kernel.  `mirror` (optional):
// publish the finished block to the host.
__global__ __launch_bounds__(kBlock) void finalize_kernel(const Partial *__restrict__ partials, int64_t n,
                                                          nt_amp_ctrl *ctrl, const nt_amp_ctrl *carry,
                                                          double norm_type, double max_norm,
                                                          int32_t flags, double growth, double backoff,
                                                          int32_t interval, nt_amp_mirror *mirror) {
    Acc r = reduce_partials(partials, 0, n);
    if (threadIdx.x != 0) return;
    nt_amp_ctrl c = carry != nullptr ? carried_ctrl(*carry) : *ctrl;
    decide_iteration(c, r.sumsq, r.amax, r.nan, r.inf, norm_type, max_norm, flags, growth, backoff, interval);
    *ctrl = c;
    if (mirror != nullptr) publish(mirror, c);
}

// Several optimizers in one scaler iteration: blocks[0..n) hold each one's
// finalized statistics.  Their sums add in block order, the maxima and the
// NaN/inf flags combine, and one set of decisions (global norm and clip,
// one scaler update over all) goes into every block, which keeps its own
// statistics and skip flag.
struct CombineBlocks {
    nt_amp_ctrl *block[NT_MAX_COMBINE];
    nt_amp_mirror *mirror[NT_MAX_COMBINE];   // NULL: no host copy of that block
};

__global__ void combine_kernel(CombineBlocks blocks, int32_t n, const nt_amp_ctrl *carry, double norm_type,
                               double max_norm, int32_t flags, double growth, double backoff, int32_t interval) {
    if (threadIdx.x != 0) return;
    const nt_amp_ctrl c = combined_decisions(blocks.block, n, *carry, norm_type, max_norm, flags, growth, backoff,
                                             interval);
    for (int32_t i = 0; i < n; ++i) {
        const nt_amp_ctrl out = combined_block(c, *blocks.block[i]);
        *blocks.block[i] = out;
        if (blocks.mirror[i] != nullptr) publish(blocks.mirror[i], out);
    }
}

// With `guard`, the p = 2 prescaled pass runs only when the finalize's
// sqrt(sum of g^2) may have lost accuracy: fp64 squares overflow above 2^511
// and fall below the normal range under 2^-511, so the direct sum is kept
// while max|g'| lies in [2^-480, 2^480] (float32, float16 and bfloat16
// gradients always do).
__device__ __forceinline__ bool direct_norm_exact(double amax) {
    return amax >= 0x1p-480 && amax <= 0x1p480;
}

// (|g'|/amax)^p: NumPy's power with exponent 2 is the plain square.
__device__ __forceinline__ double pow_term(double a, double p) { return p == 2.0 ? a * a : pow(a, p); }

// General p-norm second pass: sum of (|g'|/amax)^p in fp64
// (optim/clip_grad.py:73-76).
template <class G>
__global__ __launch_bounds__(kBlock) void norm_pow_kernel(const DevTensor *__restrict__ tensors,
                                                          const Task *__restrict__ tasks, int64_t ntasks,
                                                          int64_t chunk, Xform xf, const nt_amp_ctrl *ctrl,
                                                          int32_t scale_from_ctrl, double p, int32_t guard,
                                                          double *__restrict__ partials) {
    const double s = ctrl->amax;
    // The finalize already holds the norm when the prescale is non-finite or
    // zero (clip_grad.py:71-72), and with `guard` when the direct sum is exact.
    if (ctrl->found_inf || !(s > 0.0) || (guard && direct_norm_exact(s))) return;
    if (scale_from_ctrl && xf.unscale) xf.scale = ctrl_scale_inv(ctrl->scale_used, xf.unscale, xf.inv_scale);
    double acc = 0.0;
    for (int64_t t = blockIdx.x; t < ntasks; t += gridDim.x) {
        const Task task = tasks[t];
        const DevTensor d = tensors[task.tensor];
        const uint64_t start = (uint64_t)task.chunk * (uint64_t)chunk;
        const uint64_t end = min(start + (uint64_t)chunk, d.numel);
        const auto *gp = reinterpret_cast<const typename G::raw *>(d.grad);
        for (uint64_t i = start + threadIdx.x; i < end; i += kBlock) {
            const double a = __builtin_fabs((double)unscale_one<G>(load1<G>(gp, i), xf)) / s;
            acc += pow_term(a, p);
        }
    }
    Acc in;
    in.sumsq = acc;
    Acc r = block_reduce(in);
    if (threadIdx.x == 0) partials[blockIdx.x] = r.sumsq;
}

// float64 gradients: unscale divides in fp64 (amp.py:190-191 on a float64
// array), then the same prescaled terms.
__global__ __launch_bounds__(kBlock) void norm_pow_f64_kernel(const DevTensor *__restrict__ tensors,
                                                              const Task *__restrict__ tasks, int64_t ntasks,
                                                              int64_t chunk, Xform xf, const nt_amp_ctrl *ctrl,
                                                              int32_t scale_from_ctrl, double p, int32_t guard,
                                                              double *__restrict__ partials) {
    const double s = ctrl->amax;
    if (ctrl->found_inf || !(s > 0.0) || (guard && direct_norm_exact(s))) return;
    const double scale = scale_from_ctrl ? (double)ctrl->scale_used : (double)xf.scale;
    double acc = 0.0;
    for (int64_t t = blockIdx.x; t < ntasks; t += gridDim.x) {
        const Task task = tasks[t];
        const DevTensor d = tensors[task.tensor];
        const uint64_t start = (uint64_t)task.chunk * (uint64_t)chunk;
        const uint64_t end = min(start + (uint64_t)chunk, d.numel);
        const double *gp = reinterpret_cast<const double *>(d.grad);
        for (uint64_t i = start + threadIdx.x; i < end; i += kBlock) {
            double g = gp[i];
            if (xf.unscale) g = g / scale;
            acc += pow_term(__builtin_fabs(g) / s, p);
        }
    }
    Acc in;
    in.sumsq = acc;
    Acc r = block_reduce(in);
    if (threadIdx.x == 0) partials[blockIdx.x] = r.sumsq;
}

__global__ __launch_bounds__(kBlock) void norm_pow_finalize_kernel(const double *__restrict__ partials, int32_t n,
                                                                   nt_amp_ctrl *ctrl, double p, double max_norm,
                                                                   int32_t guard) {
    {
        // Same early exits as the pass (block-uniform, before any partial is read).
        const double s = ctrl->amax;
        if (ctrl->found_inf || !(s > 0.0) || (guard && direct_norm_exact(s))) return;
    }
    Acc acc;
    for (int32_t i = threadIdx.x; i < n; i += kBlock) acc.sumsq += partials[i];
    Acc r = block_reduce(acc);
    if (threadIdx.x != 0) return;
    nt_amp_ctrl c = *ctrl;
    const double s = c.amax;
    double total = r.sumsq;
    double result = s * pow(total, 1.0 / p);
    if (!__builtin_isfinite(result)) result = exp(log(s) + log(total) / p);
    c.norm = result;
    c.sumsq = total;    // the raw sum, for combining several plans on the host
    if (max_norm >= 0.0) {
        c.clip_coef = max_norm / (result + 1e-6);
        c.clip = c.clip_coef < 1.0 ? 1 : 0;
    }
    *ctrl = c;
}

// In-place grad transform: g <- clip(unscale(g)).  One slice (task_slice)
// per workgroup: kBlock lanes with UNROLL 4-element groups each.  fp32
// gradients run 1024-element slices with one group per lane; 16-bit ones,
// whose f64 clip rounding costs twice the ALU work per byte, keep whole
// tasks with two groups per lane in flight (both measured fastest).
template <class G> struct ApplyShape {
    static constexpr int unroll = G::code == NT_F32 ? 1 : 2;
    static constexpr int64_t slice = G::code == NT_F32 ? (int64_t)kBlock * kVec : 0;   // 0: whole tasks
};

template <class G, int UNROLL = ApplyShape<G>::unroll, int BLOCK = kBlock>
__global__ __launch_bounds__(BLOCK) void grad_apply_kernel(const DevTensor *__restrict__ tensors,
                                                           const Task *__restrict__ tasks, int64_t chunk, Xform xf,
                                                           const nt_amp_ctrl *ctrl, int32_t shift) {
    if (ctrl != nullptr) {
        if (xf.unscale) xf.scale = ctrl_scale_inv(ctrl->scale_used, xf.unscale, xf.inv_scale);
        xf.clip = ctrl->clip;
        xf.clip_coef = ctrl->clip_coef;
    }
    if (!xf.unscale && !xf.clip) return;
    const DevTensor *dp;
    Slice slice;
    if (!task_slice(tensors, tasks, chunk, shift, dp, slice)) return;
    const DevTensor &d = *dp;
    const uint64_t start = slice.start, end = slice.end;
    auto *gp = reinterpret_cast<typename G::raw *>(d.grad);
    uint64_t scalar_from = start;
    if (d.flags & kAligned16) {
        const uint64_t vend = start + ((end - start) & ~(uint64_t)(kVec - 1));
        for (uint64_t base = start + (uint64_t)threadIdx.x * kVec; base < vend; base += (uint64_t)BLOCK * kVec * UNROLL) {
            float g[UNROLL][kVec];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint64_t i = base + (uint64_t)u * BLOCK * kVec;
                if (i < vend) Vec4IO<G, true>::load(gp, i, g[u]);
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint64_t i = base + (uint64_t)u * BLOCK * kVec;
                if (i < vend) {
#pragma unroll
                    for (int k = 0; k < kVec; ++k) g[u][k] = clip_one<G>(unscale_one<G>(g[u][k], xf), xf);
                    Vec4IO<G, true>::store(gp, i, g[u]);
                }
            }
        }
        scalar_from = vend;
    }
    for (uint64_t i = scalar_from + threadIdx.x; i < end; i += BLOCK)
        store1<G>(gp, i, clip_one<G>(unscale_one<G>(load1<G>(gp, i), xf), xf));
}

__global__ __launch_bounds__(kBlock) void grad_apply_f64_kernel(const DevTensor *__restrict__ tensors,
                                                                const Task *__restrict__ tasks, int64_t chunk,
                                                                Xform xf, const nt_amp_ctrl *ctrl) {
    double scale = xf.scale;
    if (ctrl != nullptr) {
        scale = ctrl->scale_used;
        xf.clip = ctrl->clip;
        xf.clip_coef = ctrl->clip_coef;
    }
    if (!xf.unscale && !xf.clip) return;
    const Task task = tasks[blockIdx.x];
    const DevTensor d = tensors[task.tensor];
    const uint64_t start = (uint64_t)task.chunk * (uint64_t)chunk;
    const uint64_t end = min(start + (uint64_t)chunk, d.numel);
    double *gp = reinterpret_cast<double *>(d.grad);
    for (uint64_t i = start + threadIdx.x; i < end; i += kBlock) {
        double g = gp[i];
        if (xf.unscale) g = g / scale;
        if (xf.clip) g = g * xf.clip_coef;
        gp[i] = g;
    }
}

__global__ void ctrl_carry_kernel(nt_amp_ctrl *dst, const nt_amp_ctrl *src) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    *dst = carried_ctrl(*src);
}

__global__ void ctrl_reset_kernel(nt_amp_ctrl *ctrl, float scale, int32_t tracker) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    nt_amp_ctrl c{};
    c.scale = scale;
    c.scale_used = scale;
    c.growth_tracker = tracker;
    c.clip_coef = 1.0;
    *ctrl = c;
}

// out = to_O(widen(in) op operand).  The operand is already a value of the
// output (compute) dtype, and the input widens exactly into it, so one fp64
// operation followed by one rounding is the compute dtype's correctly
// rounded product or quotient: a product of two values of at most 24
// significant bits is exact in fp64, and a quotient rounded to fp64 and then
// to a format of p <= 24 bits rounds innocuously (53 >= 2p + 2).
template <class I, class O>
__global__ __launch_bounds__(kBlock) void tensor_scalar_kernel(const typename I::raw *in, typename O::raw *out,
                                                               double operand, const nt_amp_ctrl *ctrl,
                                                               int32_t op, uint64_t n) {
    const double s = ctrl != nullptr ? (double)ctrl->scale : operand;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kBlock) {
        const double x = widen64<I>(in[i]);
        out[i] = O::from_f64(op == NT_OP_DIV ? x / s : x * s);
    }
}

template <class I>
static int32_t launch_tensor_scalar(const void *in, void *out, int32_t out_dtype, double operand,
                                    const nt_amp_ctrl *ctrl, int32_t op, uint64_t n, dim3 grid, hipStream_t s) {
    const auto *src = static_cast<const typename I::raw *>(in);
    switch (out_dtype) {
        case NT_F32: tensor_scalar_kernel<I, TF32><<<grid, dim3(kBlock), 0, s>>>(src, (float *)out, operand, ctrl, op, n); break;
        case NT_F16: tensor_scalar_kernel<I, TF16><<<grid, dim3(kBlock), 0, s>>>(src, (uint16_t *)out, operand, ctrl, op, n); break;
        case NT_BF16: tensor_scalar_kernel<I, TBF16><<<grid, dim3(kBlock), 0, s>>>(src, (uint16_t *)out, operand, ctrl, op, n); break;
        case NT_F64: tensor_scalar_kernel<I, TF64><<<grid, dim3(kBlock), 0, s>>>(src, (double *)out, operand, ctrl, op, n); break;
        default: return fail(NT_ERR_TYPE, "nt_tensor_scalar: unsupported output dtype");
    }
    return NT_OK;
}

__global__ void clear_flag_kernel(int32_t *flag) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *flag = 0;
}

// Any element < 0 sets *flag = 1 (plain stores of the same value; -0.0 and
// NaN are not negative, as with NumPy's less(array, 0)).
template <class T>
__global__ __launch_bounds__(kBlock) void any_negative_kernel(const typename T::raw *a, uint64_t n, int32_t *flag) {
    int found = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kBlock)
        found |= (T::to_f32(a[i]) < 0.0f) ? 1 : 0;
    if (found) *flag = 1;
}
__global__ __launch_bounds__(kBlock) void any_negative_f64_kernel(const double *a, uint64_t n, int32_t *flag) {
    int found = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kBlock)
        found |= (a[i] < 0.0) ? 1 : 0;
    if (found) *flag = 1;
}

template <template <class> class K, class... Args>
static int32_t grad_dispatch(int32_t gdt, dim3 grid, hipStream_t s, Args... args) {
    switch (gdt) {
        case NT_F32: K<TF32>::launch(grid, s, args...); break;
        case NT_F16: K<TF16>::launch(grid, s, args...); break;
        case NT_BF16: K<TBF16>::launch(grid, s, args...); break;
        default: return fail(NT_ERR_TYPE, "unsupported gradient dtype");
    }
    return NT_OK;
}

// First pre-pass task read with temporal loads: the plan's last tasks that
// hold at most kMallKeepBytes of gradient data (counting a deferred addend
// stream too), so the AdamW pass re-reads them from the MALL.
static int64_t keep_from_task(const nt_plan *plan) {
    const int32_t gdt = plan->layout.grad_dtype;
    const uint64_t size = gdt == NT_F16 || gdt == NT_BF16 ? 2u : 4u;
    const uint64_t per_task = (uint64_t)plan->chunk * size * (plan->n_incoming > 0 ? 2u : 1u);
    const int64_t keep = (int64_t)(kMallKeepBytes / per_task);
    return plan->ntasks > keep ? plan->ntasks - keep : 0;
}

template <class G> struct PrepassL {
    template <class... A> static void launch(dim3 g, hipStream_t s, A... a) {
        prepass_kernel<G><<<g, dim3(kBlock), 0, s>>>(a...);
    }
};
template <class G> struct NormPowL {
    template <class... A> static void launch(dim3 g, hipStream_t s, A... a) {
        norm_pow_kernel<G><<<g, dim3(kBlock), 0, s>>>(a...);
    }
};
template <class G> struct ApplyL {
    // Grid: the plan's tasks, each split as ApplyShape<G> says.
    static void launch(dim3, hipStream_t s, const nt_plan *plan, Xform xf, const nt_amp_ctrl *ctrl) {
        const int32_t shift = ApplyShape<G>::slice ? split_shift(plan, ApplyShape<G>::slice) : 0;
        grad_apply_kernel<G><<<dim3((unsigned)(plan->ntasks << shift)), dim3(kBlock), 0, s>>>(
            plan->d_tensors, plan->d_tasks, plan->chunk, xf, ctrl, shift);
    }
};

static uint64_t small_grid(uint64_t n) {
    uint64_t b = (n + kBlock - 1) / kBlock;
    if (b > 1024) b = 1024;
    return b ? b : 1;
}

// ---- plan-free pre-pass over one flat gradient buffer, allocating nothing ----------
// nt_amp_flat_stats_noalloc's per-workgroup partials live in `scratch`, a
// fixed device array of this file: every GPU holds its own copy for the life
// of the process.  Host code never uses the array's name as an address; it
// resolves the device address once per device (hipGetSymbolAddress, with that
// device current) and passes that pointer to the kernels.
constexpr int kFlatPartials = 4096;                          // 64 KiB of partials
constexpr int kFlatUnroll = 4;                               // 4-element groups per lane per iteration
constexpr uint64_t kFlatMaxCount = uint64_t(1) << 40;
constexpr int kFlatMaxDevices = 64;
static __device__ __align__(256) Partial scratch[kFlatPartials];

static std::mutex g_scratch_lock;
static Partial *g_scratch_address[kFlatMaxDevices] = {};

// Device address of `scratch` on `device` (which must be current).
static int32_t flat_scratch(int32_t device, Partial **out) {
    std::lock_guard<std::mutex> lock(g_scratch_lock);
    if (g_scratch_address[device] == nullptr) {
        void *address = nullptr;
        NT_HIP_TRY(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_scratch_address[device] = static_cast<Partial *>(address);
    }
    *out = g_scratch_address[device];
    return NT_OK;
}

// Grid-stride pass over grad[0, count): each workgroup writes one partial
// (fp64 sum of squares of the finite unscaled values, max |g'| with inf/NaN
// encoded) to partials[blockIdx.x]; the grid never exceeds kFlatPartials.
template <class G>
__global__ __launch_bounds__(kBlock) void flat_prepass_kernel(const typename G::raw *__restrict__ grad, uint64_t count,
                                                              int32_t aligned, Xform xf, const nt_amp_ctrl *carry,
                                                              Partial *__restrict__ partials) {
    __shared__ WaveJoin join;
    wave_join_init(join);
    if (carry != nullptr && xf.unscale) xf.scale = ctrl_scale_inv(carry->scale, xf.unscale, xf.inv_scale);
    PAcc acc;
    uint64_t scalar_from = 0;
    if (aligned) {
        const uint64_t vend = count & ~(uint64_t)(kVec - 1);
        const uint64_t stride = (uint64_t)gridDim.x * kBlock * kVec * kFlatUnroll;
        for (uint64_t base = (uint64_t)blockIdx.x * kBlock * kVec * kFlatUnroll + (uint64_t)threadIdx.x * kVec;
             base < vend; base += stride) {
            float g[kFlatUnroll][kVec];
#pragma unroll
            for (int u = 0; u < kFlatUnroll; ++u) {
                const uint64_t i = base + (uint64_t)u * kBlock * kVec;
                if (i < vend) {
                    Vec4IO<G, true>::load(grad, i, g[u]);
                } else {
#pragma unroll
                    for (int k = 0; k < kVec; ++k) g[u][k] = 0.0f;     // adds nothing to either statistic
                }
            }
#pragma unroll
            for (int u = 0; u < kFlatUnroll; ++u)
#pragma unroll
                for (int k = 0; k < kVec; ++k) pacc_wide(acc, unscale_one<G>(g[u][k], xf));
        }
        scalar_from = vend;
    }
    for (uint64_t i = scalar_from + (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * kBlock)
        pacc_wide(acc, unscale_one<G>(load1<G>(grad, i), xf));
    const Partial mine{wave_sum(acc.sumsq), amax_from_bits(wave_max_u32(acc.amax_bits))};
    wave_join_finish(join, mine, partials + blockIdx.x);
}

template <class G>
static void launch_flat_prepass(dim3 grid, hipStream_t s, const void *grad, uint64_t count, int32_t aligned,
                                Xform xf, const nt_amp_ctrl *carry, Partial *partials) {
    flat_prepass_kernel<G><<<grid, dim3(kBlock), 0, s>>>(static_cast<const typename G::raw *>(grad), count, aligned,
                                                         xf, carry, partials);
}

}  // namespace nt

using namespace nt;

extern "C" {

int32_t nt_amp_prepass(nt_plan *plan, float scale, int32_t unscale, const nt_amp_ctrl *ctrl, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if (unscale && ctrl == nullptr && !(scale > 0.0f && __builtin_isfinite(scale)))
        return fail(NT_ERR_VALUE, "loss scale must be finite and positive");
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    nt_grad_xform hx{};
    hx.scale = unscale ? scale : 1.0f;
    hx.unscale = unscale ? 1 : 0;
    Xform xf = make_xform(unscale && ctrl == nullptr ? &hx : nullptr);
    if (unscale && ctrl != nullptr) xf.unscale = 1;  // scale read on the device
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)plan->npartials);
    if (plan->layout.grad_dtype == NT_F64) {
        prepass_f64_kernel<<<grid, dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks, plan->ntasks, plan->chunk,
                                                         xf, ctrl, plan->d_partials);
    } else {
        rc = grad_dispatch<PrepassL>(plan->layout.grad_dtype, grid, s, (const DevTensor *)plan->d_tensors,
                                     (const Task *)plan->d_tasks, plan->ntasks, plan->chunk, keep_from_task(plan),
                                     xf, ctrl, plan->d_partials);
        if (rc != NT_OK) return rc;
    }
    NT_LAUNCH_CHECK("prepass_kernel launch");
    if (plan->nstage2 > 0) {
        stage2_kernel<<<dim3((unsigned)plan->nstage2), dim3(kBlock), 0, s>>>(plan->d_partials, plan->npartials,
                                                                            plan->d_partials2);
        NT_LAUNCH_CHECK("stage2_kernel launch");
    }
    return NT_OK;
}

int32_t nt_amp_finalize(nt_plan *plan, nt_amp_ctrl *ctrl, const nt_amp_ctrl *carry, double norm_type,
                        double max_norm, int32_t flags, double growth_factor, double backoff_factor,
                        int32_t growth_interval, nt_amp_mirror *mirror, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if (ctrl == nullptr) return fail(NT_ERR_VALUE, "control block is NULL");
    if (carry == ctrl) return fail(NT_ERR_VALUE, "nt_amp_finalize: carry and ctrl must be different blocks");
    if (!(norm_type > 0.0)) return fail(NT_ERR_VALUE, "norm_type must be positive or positive infinity.");
    if (flags & ~(NT_FINALIZE_SCALER_UPDATE | NT_FINALIZE_CLIP_IF_FINITE))
        return fail(NT_ERR_VALUE, "nt_amp_finalize: unknown flags");
    if ((flags & NT_FINALIZE_SCALER_UPDATE) &&
        (growth_interval <= 0 || !(growth_factor > 1.0) || !(backoff_factor > 0.0 && backoff_factor < 1.0)))
        return fail(NT_ERR_VALUE, "invalid GradScaler growth/backoff settings");
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    const Partial *src = plan->nstage2 > 0 ? plan->d_partials2 : plan->d_partials;
    const int64_t count = plan->nstage2 > 0 ? plan->nstage2 : plan->npartials;
    finalize_kernel<<<dim3(1), dim3(kBlock), 0, (hipStream_t)stream>>>(
        src, count, ctrl, carry, norm_type, max_norm, flags, growth_factor,
        backoff_factor, growth_interval, mirror);
    NT_LAUNCH_CHECK("finalize_kernel launch");
    return NT_OK;
}

int32_t nt_amp_combine(nt_amp_ctrl *const *blocks, int32_t n, const nt_amp_ctrl *carry, double norm_type,
                       double max_norm, int32_t flags, double growth_factor, double backoff_factor,
                       int32_t growth_interval, nt_amp_mirror *const *mirrors, void *stream) {
    clear_error();
    if (blocks == nullptr || n < 1 || n > NT_MAX_COMBINE)
        return fail(NT_ERR_VALUE, "nt_amp_combine: 1 to " + std::to_string(NT_MAX_COMBINE) + " control blocks required");
    if (carry == nullptr) return fail(NT_ERR_VALUE, "nt_amp_combine: carry block is NULL");
    CombineBlocks list{};
    for (int32_t i = 0; i < n; ++i) {
        if (blocks[i] == nullptr) return fail(NT_ERR_VALUE, "control block is NULL");
        if (blocks[i] == carry) return fail(NT_ERR_VALUE, "nt_amp_combine: carry and a combined block must differ");
        for (int32_t j = 0; j < i; ++j)
            if (blocks[j] == blocks[i]) return fail(NT_ERR_VALUE, "nt_amp_combine: a control block is listed twice");
        list.block[i] = blocks[i];
        list.mirror[i] = mirrors != nullptr ? mirrors[i] : nullptr;
    }
    if (!(norm_type == 2.0 || (__builtin_isinf(norm_type) && norm_type > 0.0)))
        return fail(NT_ERR_VALUE, "nt_amp_combine: norm_type must be 2 or positive infinity");
    if (flags & ~(NT_FINALIZE_SCALER_UPDATE | NT_FINALIZE_CLIP_IF_FINITE))
        return fail(NT_ERR_VALUE, "nt_amp_combine: unknown flags");
    if ((flags & NT_FINALIZE_SCALER_UPDATE) &&
        (growth_interval <= 0 || !(growth_factor > 1.0) || !(backoff_factor > 0.0 && backoff_factor < 1.0)))
        return fail(NT_ERR_VALUE, "invalid GradScaler growth/backoff settings");
    combine_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>(list, n, carry, norm_type, max_norm, flags,
                                                                  growth_factor, backoff_factor, growth_interval);
    NT_LAUNCH_CHECK("combine_kernel launch");
    return NT_OK;
}

int32_t nt_grad_norm_pow(nt_plan *plan, nt_amp_ctrl *ctrl, double norm_type, double max_norm, float scale,
                         int32_t unscale, int32_t scale_from_ctrl, int32_t flags, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if ((rc = check_no_incoming(plan, "nt_grad_norm_pow")) != NT_OK) return rc;
    if (ctrl == nullptr) return fail(NT_ERR_VALUE, "control block is NULL");
    if (!(norm_type > 0.0) || __builtin_isinf(norm_type))
        return fail(NT_ERR_VALUE, "nt_grad_norm_pow needs a finite positive norm_type");
    if (flags & ~NT_NORM_POW_GUARD) return fail(NT_ERR_VALUE, "nt_grad_norm_pow: unknown flags");
    const int32_t guard_on = (flags & NT_NORM_POW_GUARD) ? 1 : 0;
    if (guard_on && norm_type != 2.0) return fail(NT_ERR_VALUE, "nt_grad_norm_pow: the guard applies to norm_type 2 only");
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    nt_grad_xform hx{};
    hx.scale = unscale ? scale : 1.0f;
    hx.unscale = unscale ? 1 : 0;
    Xform xf = make_xform(unscale && !scale_from_ctrl ? &hx : nullptr);
    if (unscale && scale_from_ctrl) xf.unscale = 1;
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)plan->pow_grid);
    if (plan->layout.grad_dtype == NT_F64) {
        norm_pow_f64_kernel<<<grid, dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks, plan->ntasks, plan->chunk,
                                                          xf, ctrl, scale_from_ctrl, norm_type, guard_on,
                                                          plan->d_pow_partials);
    } else {
        rc = grad_dispatch<NormPowL>(plan->layout.grad_dtype, grid, s, (const DevTensor *)plan->d_tensors,
                                     (const Task *)plan->d_tasks, plan->ntasks, plan->chunk, xf,
                                     (const nt_amp_ctrl *)ctrl, scale_from_ctrl, norm_type, guard_on,
                                     plan->d_pow_partials);
        if (rc != NT_OK) return rc;
    }
    NT_LAUNCH_CHECK("norm_pow_kernel launch");
    norm_pow_finalize_kernel<<<dim3(1), dim3(kBlock), 0, s>>>(plan->d_pow_partials, plan->pow_grid, ctrl,
                                                              norm_type, max_norm, guard_on);
    NT_LAUNCH_CHECK("norm_pow_finalize_kernel launch");
    return NT_OK;
}

int32_t nt_grad_apply(nt_plan *plan, const nt_grad_xform *xform, void *stream) {
    clear_error();
    int32_t rc = check_plan(plan);
    if (rc != NT_OK) return rc;
    if ((rc = check_no_incoming(plan, "nt_grad_apply")) != NT_OK) return rc;
    if (xform == nullptr || plan->ntasks == 0) return NT_OK;
    note_stream(plan, stream);
    DeviceGuard guard(plan->device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    Xform xf = make_xform(xform);
    const nt_amp_ctrl *ctrl = xform->ctrl;
    if (ctrl != nullptr) xf.unscale = xform->unscale ? 1 : 0;
    hipStream_t s = (hipStream_t)stream;
    if (plan->layout.grad_dtype == NT_F64) {
        grad_apply_f64_kernel<<<dim3((unsigned)plan->ntasks), dim3(kBlock), 0, s>>>(plan->d_tensors, plan->d_tasks,
                                                                                    plan->chunk, xf, ctrl);
    } else {
        rc = grad_dispatch<ApplyL>(plan->layout.grad_dtype, dim3(), s, (const nt_plan *)plan, xf, ctrl);
        if (rc != NT_OK) return rc;
    }
    NT_LAUNCH_CHECK("grad_apply_kernel launch");
    return NT_OK;
}

int32_t nt_ctrl_reset(nt_amp_ctrl *ctrl, float scale, int32_t growth_tracker, void *stream) {
    clear_error();
    if (ctrl == nullptr) return fail(NT_ERR_VALUE, "control block is NULL");
    ctrl_reset_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>(ctrl, scale, growth_tracker);
    NT_LAUNCH_CHECK("ctrl_reset_kernel launch");
    return NT_OK;
}

int32_t nt_ctrl_carry(nt_amp_ctrl *dst, const nt_amp_ctrl *src, void *stream) {
    clear_error();
    if (dst == nullptr || src == nullptr) return fail(NT_ERR_VALUE, "control block is NULL");
    if (dst == src) return fail(NT_ERR_VALUE, "nt_ctrl_carry: dst and src alias");
    ctrl_carry_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>(dst, src);
    NT_LAUNCH_CHECK("ctrl_carry_kernel launch");
    return NT_OK;
}

int32_t nt_tensor_scalar(const void *in, int32_t in_dtype, void *out, int32_t out_dtype, double operand,
                         int32_t op, const nt_amp_ctrl *ctrl, uint64_t count, void *stream) {
    clear_error();
    if (op != NT_OP_MUL && op != NT_OP_DIV) return fail(NT_ERR_VALUE, "nt_tensor_scalar: unknown operation");
    if (out_dtype != NT_F32 && out_dtype != NT_F16 && out_dtype != NT_BF16 && out_dtype != NT_F64)
        return fail(NT_ERR_TYPE, "nt_tensor_scalar: unsupported output dtype");
    if (count == 0) return NT_OK;
    if (in == nullptr || out == nullptr) return fail(NT_ERR_VALUE, "nt_tensor_scalar: NULL array");
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)small_grid(count));
    int32_t rc;
    switch (in_dtype) {
        case NT_F32: rc = launch_tensor_scalar<TF32>(in, out, out_dtype, operand, ctrl, op, count, grid, s); break;
        case NT_F16: rc = launch_tensor_scalar<TF16>(in, out, out_dtype, operand, ctrl, op, count, grid, s); break;
        case NT_BF16: rc = launch_tensor_scalar<TBF16>(in, out, out_dtype, operand, ctrl, op, count, grid, s); break;
        case NT_F64: rc = launch_tensor_scalar<TF64>(in, out, out_dtype, operand, ctrl, op, count, grid, s); break;
        default: return fail(NT_ERR_TYPE, "nt_tensor_scalar: unsupported input dtype");
    }
    if (rc != NT_OK) return rc;
    NT_LAUNCH_CHECK("tensor_scalar_kernel launch");
    return NT_OK;
}

int32_t nt_any_negative(const void *array, int32_t dtype, uint64_t count, int32_t *flag, void *stream) {
    clear_error();
    if (flag == nullptr) return fail(NT_ERR_VALUE, "nt_any_negative: NULL flag");
    hipStream_t s = (hipStream_t)stream;
    clear_flag_kernel<<<dim3(1), dim3(64), 0, s>>>(flag);
    NT_LAUNCH_CHECK("clear_flag_kernel launch");
    if (count == 0) return NT_OK;
    if (array == nullptr) return fail(NT_ERR_VALUE, "nt_any_negative: NULL array");
    dim3 grid((unsigned)small_grid(count));
    switch (dtype) {
        case NT_F32: any_negative_kernel<TF32><<<grid, dim3(kBlock), 0, s>>>((const float *)array, count, flag); break;
        case NT_F16: any_negative_kernel<TF16><<<grid, dim3(kBlock), 0, s>>>((const uint16_t *)array, count, flag); break;
        case NT_BF16: any_negative_kernel<TBF16><<<grid, dim3(kBlock), 0, s>>>((const uint16_t *)array, count, flag); break;
        case NT_F64: any_negative_f64_kernel<<<grid, dim3(kBlock), 0, s>>>((const double *)array, count, flag); break;
        default: return fail(NT_ERR_TYPE, "nt_any_negative: unsupported dtype");
    }
    NT_LAUNCH_CHECK("any_negative_kernel launch");
    return NT_OK;
}

}  // extern "C"

extern "C" {

int32_t nt_amp_flat_stats_noalloc(int32_t device, const void *grad, int32_t grad_dtype, uint64_t count, float scale,
                                  int32_t unscale, nt_amp_ctrl *ctrl, const nt_amp_ctrl *carry, double norm_type,
                                  double max_norm, int32_t flags, double growth_factor, double backoff_factor,
                                  int32_t growth_interval, void *stream) {
    clear_error();
    if (device < 0 || device >= kFlatMaxDevices) return fail(NT_ERR_VALUE, "nt_amp_flat_stats_noalloc: invalid device");
    if (ctrl == nullptr) return fail(NT_ERR_VALUE, "control block is NULL");
    if (carry == ctrl) return fail(NT_ERR_VALUE, "nt_amp_flat_stats_noalloc: carry and ctrl must be different blocks");
    if (!(norm_type == 2.0 || (__builtin_isinf(norm_type) && norm_type > 0.0)))
        return fail(NT_ERR_VALUE, "nt_amp_flat_stats_noalloc: norm_type must be 2 or +inf");
    if (flags & ~(NT_FINALIZE_SCALER_UPDATE | NT_FINALIZE_CLIP_IF_FINITE))
        return fail(NT_ERR_VALUE, "nt_amp_flat_stats_noalloc: unknown flags");
    if ((flags & NT_FINALIZE_SCALER_UPDATE) &&
        (growth_interval <= 0 || !(growth_factor > 1.0) || !(backoff_factor > 0.0 && backoff_factor < 1.0)))
        return fail(NT_ERR_VALUE, "invalid GradScaler growth/backoff settings");
    if (grad_dtype != NT_F32 && grad_dtype != NT_F16 && grad_dtype != NT_BF16)
        return fail(NT_ERR_TYPE, "nt_amp_flat_stats_noalloc: gradients must be float32, float16 or bfloat16");
    if (count > kFlatMaxCount)
        return fail(NT_ERR_VALUE, "nt_amp_flat_stats_noalloc: count " + std::to_string(count) +
                                      " exceeds the maximum of 2**40 elements");
    if (count > 0 && grad == nullptr) return fail(NT_ERR_VALUE, "nt_amp_flat_stats_noalloc: NULL gradient buffer");
    if (unscale && carry == nullptr && !(scale > 0.0f && __builtin_isfinite(scale)))
        return fail(NT_ERR_VALUE, "loss scale must be finite and positive");
    DeviceGuard guard(device);
    if (!guard.ok()) return hip_check(guard.error(), "hipSetDevice");
    Partial *partials = nullptr;
    int32_t rc = flat_scratch(device, &partials);
    if (rc != NT_OK) return rc;
    nt_grad_xform hx{};
    hx.scale = unscale ? scale : 1.0f;
    hx.unscale = unscale ? 1 : 0;
    Xform xf = make_xform(unscale && carry == nullptr ? &hx : nullptr);
    if (unscale && carry != nullptr) xf.unscale = 1;   // scale read from the carry block on the device
    const uint64_t per_group = (uint64_t)kBlock * kVec * kFlatUnroll;
    uint64_t groups = (count + per_group - 1) / per_group;
    if (groups > (uint64_t)kFlatPartials) groups = kFlatPartials;
    const uintptr_t alignment = grad_dtype == NT_F32 ? 16u : 8u;
    const int32_t aligned = ((uintptr_t)grad % alignment) == 0 ? 1 : 0;
    hipStream_t s = (hipStream_t)stream;
    if (groups > 0) {
        const dim3 grid((unsigned)groups);
        switch (grad_dtype) {
            case NT_F32: launch_flat_prepass<TF32>(grid, s, grad, count, aligned, xf, carry, partials); break;
            case NT_F16: launch_flat_prepass<TF16>(grid, s, grad, count, aligned, xf, carry, partials); break;
            default: launch_flat_prepass<TBF16>(grid, s, grad, count, aligned, xf, carry, partials); break;
        }
        NT_LAUNCH_CHECK("flat_prepass_kernel launch");
    }
    finalize_kernel<<<dim3(1), dim3(kBlock), 0, s>>>(partials, (int64_t)groups, ctrl, carry, norm_type, max_norm,
                                                     flags, growth_factor, backoff_factor, growth_interval, nullptr);
    NT_LAUNCH_CHECK("finalize_kernel launch");
    return NT_OK;
}

}  // extern "C"
