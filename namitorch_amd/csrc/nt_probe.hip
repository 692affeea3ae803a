// nt_probe.hip — streaming probe: the memory access pattern of the
// multi-tensor AdamW pass with the arithmetic reduced to one add per stream,
// so that a benchmark can report the bandwidth each access mix reaches on
// the device next to what the pass reaches.
//
// Each workgroup is one wave covering 256 consecutive elements of every
// stream (like a slice of a pass task), each lane one group of four elements
// with nontemporal accesses: 16 bytes for fp32 streams and 8 bytes for
// 16-bit streams, as the pass issues them.  All reads come first, then the
// writes grouped by stream.  Write stream w receives read stream (w mod R) plus
// read stream R-1 (1.0 when there are no reads), so every read is used and
// nothing is optimised away; 16-bit streams hold bfloat16 values, read
// exactly and written truncated to their upper 16 bits.
#include <hip/hip_runtime.h>

#include "nt_internal.hpp"

namespace nt {

constexpr int kProbeMax = 8;
constexpr int kProbeLanes = 64;
constexpr int kProbeUnroll = 1;
constexpr int kProbeSlice = kProbeLanes * kVec * kProbeUnroll;   // elements per workgroup
static_assert(kProbeSlice == kPassSlice, "the probe streams like the split pass");
constexpr uint64_t kProbeQuantum = 4096;                        // count granularity of the entry point

struct ProbeArgs {
    const void *reads[kProbeMax];
    void *writes[kProbeMax];
};

__device__ __forceinline__ f32x4 bf16x4_to_f32(u32x2 w) {
    return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                 __uint_as_float(w.y & 0xffff0000u)};
}

__device__ __forceinline__ u32x2 f32x4_to_bf16_trunc(f32x4 v) {
    return u32x2{(__float_as_uint(v.x) >> 16) | (__float_as_uint(v.y) & 0xffff0000u),
                 (__float_as_uint(v.z) >> 16) | (__float_as_uint(v.w) & 0xffff0000u)};
}

// R read streams of which the last R16 are 16-bit; W write streams of which
// the last W16 are 16-bit.
template <int R, int R16, int W, int W16>
__global__ __launch_bounds__(kProbeLanes) void stream_probe_kernel(ProbeArgs args) {
    constexpr int R32 = R - R16, W32 = W - W16;
    const uint64_t start = (uint64_t)blockIdx.x * kProbeSlice + (uint64_t)threadIdx.x * kVec;
    f32x4 in[R > 0 ? R : 1][kProbeUnroll];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            const uint64_t i = start + (uint64_t)u * kProbeLanes * kVec;
            if (r < R32)
                in[r][u] = gload<true, f32x4, gf32x4>(static_cast<const float *>(args.reads[r]) + i);
            else
                in[r][u] = bf16x4_to_f32(gload<true, u32x2, gu32x2>(static_cast<const uint16_t *>(args.reads[r]) + i));
        }
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            const uint64_t i = start + (uint64_t)u * kProbeLanes * kVec;
            f32x4 value = {1.0f, 1.0f, 1.0f, 1.0f};
            if constexpr (R > 0) value = in[w % R][u] + in[R - 1][u];
            if (w < W32)
                gstore<true, f32x4, gf32x4>(static_cast<float *>(args.writes[w]) + i, value);
            else
                gstore<true, u32x2, gu32x2>(static_cast<uint16_t *>(args.writes[w]) + i, f32x4_to_bf16_trunc(value));
        }
    if constexpr (W == 0 && R > 0) {
        // Read-only probe: keep the loads alive with a store nobody reads
        // unless the sum has an impossible bit pattern.
        f32x4 sum = in[0][0];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int u = 0; u < kProbeUnroll; ++u) sum += in[r][u];
        if (__builtin_bit_cast(uint32_t, sum.x) == 0x7fbadbadu)
            static_cast<float *>(args.writes[kProbeMax - 1])[start] = sum.y;
    }
}

template <int R, int R16, int W, int W16>
static void launch_probe(dim3 grid, hipStream_t s, const ProbeArgs &args) {
    stream_probe_kernel<R, R16, W, W16><<<grid, dim3(kProbeLanes), 0, s>>>(args);
}

typedef void (*ProbeLauncher)(dim3, hipStream_t, const ProbeArgs &);

struct ProbeMix {
    int reads, reads16, writes, writes16;
    ProbeLauncher launch;
};

// fp32 mixes, then the C4 pass's mix (fp32 master + three bf16 streams each
// way) and the C3/C5 pass's mix (three fp32 streams + one 16-bit stream
// each way).
static const ProbeMix kMixes[] = {
    {0, 0, 1, 0, launch_probe<0, 0, 1, 0>}, {0, 0, 3, 0, launch_probe<0, 0, 3, 0>},
    {1, 0, 0, 0, launch_probe<1, 0, 0, 0>}, {1, 0, 1, 0, launch_probe<1, 0, 1, 0>},
    {2, 0, 2, 0, launch_probe<2, 0, 2, 0>}, {4, 0, 0, 0, launch_probe<4, 0, 0, 0>},
    {4, 0, 3, 0, launch_probe<4, 0, 3, 0>}, {5, 0, 4, 0, launch_probe<5, 0, 4, 0>},
    {4, 3, 4, 3, launch_probe<4, 3, 4, 3>}, {4, 1, 4, 1, launch_probe<4, 1, 4, 1>},
};

static ProbeLauncher probe_launcher(int reads, int reads16, int writes, int writes16) {
    for (const ProbeMix &m : kMixes)
        if (m.reads == reads && m.reads16 == reads16 && m.writes == writes && m.writes16 == writes16) return m.launch;
    return nullptr;
}

}  // namespace nt

using namespace nt;

extern "C" {

int32_t nt_stream_probe(const void *const *reads, int32_t nreads, int32_t nreads16, void *const *writes,
                        int32_t nwrites, int32_t nwrites16, uint64_t count, void *stream) {
    clear_error();
    ProbeLauncher launcher = probe_launcher(nreads, nreads16, nwrites, nwrites16);
    if (launcher == nullptr)
        return fail(NT_ERR_VALUE, "nt_stream_probe: supported (reads, 16-bit reads, writes, 16-bit writes): "
                                  "(0,0,1,0) (0,0,3,0) (1,0,0,0) (1,0,1,0) (2,0,2,0) (4,0,0,0) (4,0,3,0) "
                                  "(5,0,4,0) (4,3,4,3) (4,1,4,1)");
    if (count == 0 || count % kProbeQuantum != 0)
        return fail(NT_ERR_VALUE, "nt_stream_probe: count must be a positive multiple of 4096");
    if (count / (uint64_t)kProbeSlice > 0x7fffffffull) return fail(NT_ERR_VALUE, "nt_stream_probe: count too large");
    if ((nreads > 0 && reads == nullptr) || writes == nullptr)
        return fail(NT_ERR_VALUE, "nt_stream_probe: NULL stream table");
    if (nwrites == 0 && (writes[0] == nullptr || (uintptr_t)writes[0] % 16 != 0))
        return fail(NT_ERR_VALUE, "nt_stream_probe: a read-only probe needs one 16-byte aligned fp32 write stream");
    ProbeArgs args{};
    for (int32_t r = 0; r < nreads; ++r) {
        if (reads[r] == nullptr || (uintptr_t)reads[r] % 16 != 0)
            return fail(NT_ERR_VALUE, "nt_stream_probe: read streams must be 16-byte aligned");
        args.reads[r] = reads[r];
    }
    for (int32_t w = 0; w < nwrites; ++w) {
        if (writes[w] == nullptr || (uintptr_t)writes[w] % 16 != 0)
            return fail(NT_ERR_VALUE, "nt_stream_probe: write streams must be 16-byte aligned");
        args.writes[w] = writes[w];
    }
    if (nwrites == 0) args.writes[kProbeMax - 1] = writes[0];
    launcher(dim3((unsigned)(count / (uint64_t)kProbeSlice)), (hipStream_t)stream, args);
    NT_LAUNCH_CHECK("stream_probe_kernel launch");
    return NT_OK;
}

}  // extern "C"
