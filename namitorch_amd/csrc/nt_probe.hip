// nt_probe.hip — streaming probe: the memory access pattern of the
// multi-tensor AdamW pass with the arithmetic reduced to one add per stream,
// so that a benchmark can report the bandwidth this access mix reaches on the
// device next to what the pass reaches.
//
// Each workgroup covers 4096 consecutive fp32 elements of every stream
// (like a pass task), each lane four groups of four elements with
// nontemporal 16-byte accesses: all reads first, then the writes grouped by
// stream.  Stream w (write) receives read stream w plus read stream R-1, so
// every read is used and nothing is optimised away.
#include <hip/hip_runtime.h>

#include "nt_internal.hpp"

namespace nt {

constexpr int kProbeMax = 8;
constexpr int kProbeChunk = kBlock * kVec * kPass2Unroll;   // 4096 elements

struct ProbeArgs {
    const float *reads[kProbeMax];
    float *writes[kProbeMax];
};

template <int R, int W>
__global__ __launch_bounds__(kBlock) void stream_probe_kernel(ProbeArgs args) {
    const uint64_t start = (uint64_t)blockIdx.x * kProbeChunk + (uint64_t)threadIdx.x * kVec;
    f32x4 in[R > 0 ? R : 1][kPass2Unroll];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < kPass2Unroll; ++u)
            in[r][u] = gload<true, f32x4, gf32x4>(args.reads[r] + start + (uint64_t)u * kBlock * kVec);
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
        for (int u = 0; u < kPass2Unroll; ++u) {
            f32x4 value = {1.0f, 1.0f, 1.0f, 1.0f};
            if constexpr (R > 0) value = in[w % R][u] + in[R - 1][u];
            gstore<true, f32x4, gf32x4>(args.writes[w] + start + (uint64_t)u * kBlock * kVec, value);
        }
    if constexpr (W == 0 && R > 0) {
        // Read-only probe: keep the loads alive with a store nobody reads
        // unless the sum has an impossible bit pattern.
        f32x4 sum = in[0][0];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int u = 0; u < kPass2Unroll; ++u) sum += in[r][u];
        if (__builtin_bit_cast(uint32_t, sum.x) == 0x7fbadbadu) args.writes[kProbeMax - 1][start] = sum.y;
    }
}

template <int R, int W>
static void launch_probe(dim3 grid, hipStream_t s, const ProbeArgs &args) {
    stream_probe_kernel<R, W><<<grid, dim3(kBlock), 0, s>>>(args);
}

typedef void (*ProbeLauncher)(dim3, hipStream_t, const ProbeArgs &);

static ProbeLauncher probe_launcher(int reads, int writes) {
    switch (reads * 16 + writes) {
        case 0 * 16 + 1: return launch_probe<0, 1>;
        case 0 * 16 + 3: return launch_probe<0, 3>;
        case 1 * 16 + 0: return launch_probe<1, 0>;
        case 1 * 16 + 1: return launch_probe<1, 1>;
        case 2 * 16 + 2: return launch_probe<2, 2>;
        case 4 * 16 + 0: return launch_probe<4, 0>;
        case 4 * 16 + 3: return launch_probe<4, 3>;
        case 5 * 16 + 4: return launch_probe<5, 4>;
        default: return nullptr;
    }
}

}  // namespace nt

using namespace nt;

extern "C" {

int32_t nt_stream_probe(const float *const *reads, int32_t nreads, float *const *writes, int32_t nwrites,
                        uint64_t count, void *stream) {
    clear_error();
    const bool in_range = nreads >= 0 && nreads < kProbeMax && nwrites >= 0 && nwrites < kProbeMax;
    ProbeLauncher launcher = in_range ? probe_launcher(nreads, nwrites) : nullptr;
    if (launcher == nullptr)
        return fail(NT_ERR_VALUE, "nt_stream_probe: supported (reads, writes): (0,1) (0,3) (1,0) (1,1) (2,2) (4,0) (4,3) (5,4)");
    if (count == 0 || count % (uint64_t)kProbeChunk != 0)
        return fail(NT_ERR_VALUE, "nt_stream_probe: count must be a positive multiple of 4096");
    if (count / (uint64_t)kProbeChunk > 0x7fffffffull) return fail(NT_ERR_VALUE, "nt_stream_probe: count too large");
    if ((nreads > 0 && reads == nullptr) || writes == nullptr)
        return fail(NT_ERR_VALUE, "nt_stream_probe: NULL stream table");
    if (nwrites == 0 && (writes[0] == nullptr || (uintptr_t)writes[0] % 16 != 0))
        return fail(NT_ERR_VALUE, "nt_stream_probe: a read-only probe needs one 16-byte aligned write stream");
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
    launcher(dim3((unsigned)(count / (uint64_t)kProbeChunk)), (hipStream_t)stream, args);
    NT_LAUNCH_CHECK("stream_probe_kernel launch");
    return NT_OK;
}

}  // extern "C"
