// nt_probe_shapes.hip — the AdamW pass's in-place read/write mixes under
// different launch shapes, for a benchmark to compare against the shape the
// pass uses (measurement only; no counterpart in the reference).
//
// Mix 0 is the float32 pass (read p, g, m, v; write p, m, v in place: 28
// bytes per element), mix 1 the GPT-1.3B pass (read an fp32 master and
// bfloat16 g, m, v; write the master, m, v in place and a bfloat16 copy: 20
// bytes per element).  Every element gets AdamW-like arithmetic (moment
// updates, a square root and a divide), so the loads cannot be dropped.
//
// Shapes: one tile of BLOCK x 4 x UNROLL elements per workgroup (the pass:
// BLOCK 64, UNROLL 1), optionally with the tile order made contiguous per XCD;
// persistent grids of `per_cu` workgroups per compute unit walking the tiles,
// optionally software-pipelined (the next tile's loads issued before this
// tile's stores); gfx950 direct-to-LDS loads; ordinary (temporal) loads.
#include <hip/hip_runtime.h>

#include "nt_internal.hpp"

namespace nt {
namespace {

struct ShapeBuffers {
    float *p;
    const void *g;
    void *m;
    void *v;
    uint16_t *copy;
};

template <bool NT>
__device__ __forceinline__ f32x4 load_f32(const void *base, uint64_t i) {
    return gload<NT, f32x4, gf32x4>(static_cast<const float *>(base) + i);
}
template <bool NT>
__device__ __forceinline__ f32x4 load_bf16(const void *base, uint64_t i) {
    const u32x2 w = gload<NT, u32x2, gu32x2>(static_cast<const uint16_t *>(base) + i);
    return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                 __uint_as_float(w.y & 0xffff0000u)};
}
__device__ __forceinline__ u32x2 to_bf16x4(f32x4 v) {
    return u32x2{(uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16),
                 (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16)};
}

__device__ __forceinline__ void update(f32x4 &p, f32x4 g, f32x4 &m, f32x4 &v) {
    m = m * 0.9f + g * 0.1f;
    v = v * 0.999f + (g * 0.001f) * g;
    const f32x4 d = {__builtin_sqrtf(v.x) + 1e-8f, __builtin_sqrtf(v.y) + 1e-8f, __builtin_sqrtf(v.z) + 1e-8f,
                     __builtin_sqrtf(v.w) + 1e-8f};
    p = p * 0.9999f - (m / d) * 0.001f;
}

template <int MIX, bool NT>
__device__ __forceinline__ void load_all(const ShapeBuffers &b, uint64_t i, f32x4 &p, f32x4 &g, f32x4 &m, f32x4 &v) {
    if constexpr (MIX == 0) {
        g = load_f32<NT>(b.g, i);
        m = load_f32<NT>(b.m, i);
        v = load_f32<NT>(b.v, i);
    } else {
        g = load_bf16<NT>(b.g, i);
        m = load_bf16<NT>(b.m, i);
        v = load_bf16<NT>(b.v, i);
    }
    p = load_f32<NT>(b.p, i);
}

template <int MIX, bool NT>
__device__ __forceinline__ void store_all(const ShapeBuffers &b, uint64_t i, f32x4 p, f32x4 m, f32x4 v) {
    if constexpr (MIX == 0) {
        gstore<NT, f32x4, gf32x4>(static_cast<float *>(b.m) + i, m);
        gstore<NT, f32x4, gf32x4>(static_cast<float *>(b.v) + i, v);
        gstore<NT, f32x4, gf32x4>(b.p + i, p);
    } else {
        gstore<NT, u32x2, gu32x2>(static_cast<uint16_t *>(b.m) + i, to_bf16x4(m));
        gstore<NT, u32x2, gu32x2>(static_cast<uint16_t *>(b.v) + i, to_bf16x4(v));
        gstore<NT, f32x4, gf32x4>(b.p + i, p);
        gstore<NT, u32x2, gu32x2>(b.copy + i, to_bf16x4(p));
    }
}

template <int MIX, int BLOCK, int UNROLL, bool XCD, bool NT>
__global__ __launch_bounds__(BLOCK) void shape_tiles_kernel(ShapeBuffers b, uint32_t ntiles) {
    uint32_t t = blockIdx.x;
    if constexpr (XCD) t = (t % 8u) * (ntiles / 8u) + t / 8u;    // workgroups reach XCDs round robin
    const uint64_t base = (uint64_t)t * (BLOCK * kVec * UNROLL) + (uint64_t)threadIdx.x * kVec;
    f32x4 p[UNROLL], g[UNROLL], m[UNROLL], v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) load_all<MIX, NT>(b, base + (uint64_t)u * BLOCK * kVec, p[u], g[u], m[u], v[u]);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) update(p[u], g[u], m[u], v[u]);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) store_all<MIX, NT>(b, base + (uint64_t)u * BLOCK * kVec, p[u], m[u], v[u]);
}

template <int MIX, int BLOCK, int UNROLL, bool PIPE>
__global__ __launch_bounds__(BLOCK) void shape_persistent_kernel(ShapeBuffers b, uint32_t ntiles) {
    constexpr uint64_t kTile = (uint64_t)BLOCK * kVec * UNROLL;
    uint32_t t = blockIdx.x;
    if (t >= ntiles) return;
    uint64_t base = (uint64_t)t * kTile + (uint64_t)threadIdx.x * kVec;
    f32x4 p[UNROLL], g[UNROLL], m[UNROLL], v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) load_all<MIX, true>(b, base + (uint64_t)u * BLOCK * kVec, p[u], g[u], m[u], v[u]);
    while (true) {
        const uint32_t next = t + gridDim.x;
        const uint64_t following = (uint64_t)next * kTile + (uint64_t)threadIdx.x * kVec;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) update(p[u], g[u], m[u], v[u]);
        if constexpr (PIPE) {
            f32x4 p2[UNROLL], g2[UNROLL], m2[UNROLL], v2[UNROLL];
            if (next < ntiles) {
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    load_all<MIX, true>(b, following + (uint64_t)u * BLOCK * kVec, p2[u], g2[u], m2[u], v2[u]);
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) store_all<MIX, true>(b, base + (uint64_t)u * BLOCK * kVec, p[u], m[u], v[u]);
            if (next >= ntiles) return;
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                p[u] = p2[u];
                g[u] = g2[u];
                m[u] = m2[u];
                v[u] = v2[u];
            }
        } else {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) store_all<MIX, true>(b, base + (uint64_t)u * BLOCK * kVec, p[u], m[u], v[u]);
            if (next >= ntiles) return;
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
                load_all<MIX, true>(b, following + (uint64_t)u * BLOCK * kVec, p[u], g[u], m[u], v[u]);
        }
        t = next;
        base = following;
    }
}

// Mix 0 with its four reads through gfx950's direct-to-LDS loads (16 bytes per
// lane, nontemporal, into the wave's own 4 KiB of LDS), read back after the
// wave's loads have landed.
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;
__global__ __launch_bounds__(64) void shape_lds_kernel(ShapeBuffers b) {
    __shared__ __attribute__((aligned(16))) float staged[4][64 * kVec];
    const uint64_t i = (uint64_t)blockIdx.x * (64 * kVec) + (uint64_t)threadIdx.x * kVec;
    constexpr int kNontemporal = 2;
    __builtin_amdgcn_global_load_lds((global_void *)(static_cast<const float *>(b.g) + i), (lds_void *)&staged[0][0],
                                     16, 0, kNontemporal);
    __builtin_amdgcn_global_load_lds((global_void *)(static_cast<float *>(b.m) + i), (lds_void *)&staged[1][0], 16, 0,
                                     kNontemporal);
    __builtin_amdgcn_global_load_lds((global_void *)(static_cast<float *>(b.v) + i), (lds_void *)&staged[2][0], 16, 0,
                                     kNontemporal);
    __builtin_amdgcn_global_load_lds((global_void *)(b.p + i), (lds_void *)&staged[3][0], 16, 0, kNontemporal);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    f32x4 g = *(const f32x4 *)&staged[0][threadIdx.x * kVec];
    f32x4 m = *(const f32x4 *)&staged[1][threadIdx.x * kVec];
    f32x4 v = *(const f32x4 *)&staged[2][threadIdx.x * kVec];
    f32x4 p = *(const f32x4 *)&staged[3][threadIdx.x * kVec];
    update(p, g, m, v);
    store_all<0, true>(b, i, p, m, v);
}

typedef void (*ShapeLaunch)(const ShapeBuffers &, uint64_t count, uint32_t persistent_grid, hipStream_t);

template <int MIX, int BLOCK, int UNROLL, bool XCD, bool NT>
void launch_tiles(const ShapeBuffers &b, uint64_t count, uint32_t, hipStream_t s) {
    const uint32_t ntiles = (uint32_t)(count / (BLOCK * kVec * UNROLL));
    shape_tiles_kernel<MIX, BLOCK, UNROLL, XCD, NT><<<dim3(ntiles), dim3(BLOCK), 0, s>>>(b, ntiles);
}
template <int MIX, int BLOCK, int UNROLL, bool PIPE>
void launch_persistent(const ShapeBuffers &b, uint64_t count, uint32_t grid, hipStream_t s) {
    const uint32_t ntiles = (uint32_t)(count / (BLOCK * kVec * UNROLL));
    shape_persistent_kernel<MIX, BLOCK, UNROLL, PIPE><<<dim3(grid < ntiles ? grid : ntiles), dim3(BLOCK), 0, s>>>(b, ntiles);
}
void launch_lds(const ShapeBuffers &b, uint64_t count, uint32_t, hipStream_t s) {
    shape_lds_kernel<<<dim3((uint32_t)(count / (64 * kVec))), dim3(64), 0, s>>>(b);
}

// Indexed by NT_SHAPE_* (see the header); nullptr where a shape has no variant for the mix.
template <int MIX>
constexpr ShapeLaunch kShapes[] = {
    launch_tiles<MIX, 64, 1, false, true>,  launch_tiles<MIX, 64, 1, true, true>,
    launch_tiles<MIX, 64, 2, false, true>,  launch_tiles<MIX, 128, 1, false, true>,
    launch_tiles<MIX, 256, 1, false, true>, launch_tiles<MIX, 256, 2, false, true>,
    launch_tiles<MIX, 512, 1, false, true>, launch_persistent<MIX, 64, 1, false>,
    launch_persistent<MIX, 64, 1, true>,    launch_persistent<MIX, 256, 1, true>,
    launch_persistent<MIX, 64, 2, true>,    MIX == 0 ? launch_lds : nullptr,
    launch_tiles<MIX, 64, 1, false, false>,
};
constexpr int kShapeCount = sizeof(kShapes<0>) / sizeof(kShapes<0>[0]);

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int32_t nt_stream_probe_shape(int32_t mix, int32_t shape, void *const *streams, uint64_t count, int32_t per_cu,
                              void *stream) {
    clear_error();
    if (mix != 0 && mix != 1) return fail(NT_ERR_VALUE, "nt_stream_probe_shape: mix must be 0 or 1");
    if (shape < 0 || shape >= kShapeCount) return fail(NT_ERR_VALUE, "nt_stream_probe_shape: unknown shape");
    const ShapeLaunch launch = mix == 0 ? kShapes<0>[shape] : kShapes<1>[shape];
    if (launch == nullptr) return fail(NT_ERR_VALUE, "nt_stream_probe_shape: this shape has no variant for this mix");
    if (count == 0 || count % 8192 != 0 || count / 256 > 0xffffffffull)
        return fail(NT_ERR_VALUE, "nt_stream_probe_shape: count must be a positive multiple of 8192 below 2**40");
    if (per_cu < 1 || per_cu > 64) return fail(NT_ERR_VALUE, "nt_stream_probe_shape: per_cu must be in [1, 64]");
    if (streams == nullptr) return fail(NT_ERR_VALUE, "nt_stream_probe_shape: NULL stream table");
    const int nstreams = mix == 0 ? 4 : 5;
    for (int k = 0; k < nstreams; ++k)
        if (streams[k] == nullptr || (uintptr_t)streams[k] % 16 != 0)
            return fail(NT_ERR_VALUE, "nt_stream_probe_shape: streams must be 16-byte aligned");
    ShapeBuffers b{static_cast<float *>(streams[0]), streams[1], streams[2], streams[3],
                   mix == 1 ? static_cast<uint16_t *>(streams[4]) : nullptr};
    int device = 0, units = 0;
    NT_HIP_TRY(hipGetDevice(&device), "hipGetDevice");
    NT_HIP_TRY(hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
    launch(b, count, (uint32_t)units * (uint32_t)per_cu, (hipStream_t)stream);
    NT_LAUNCH_CHECK("nt_stream_probe_shape launch");
    return NT_OK;
}

}  // extern "C"
