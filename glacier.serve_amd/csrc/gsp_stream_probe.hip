// Streaming-read probe: the HBM read rate that a plain kernel reaches on the
// GPU it runs on.  bench.py times it over the same bytes as a decode step, so a
// decode kernel's rate can be read against what this GPU streams at all.  It
// is measurement support, built into its own library (libglacier_probe.so),
// and no part of the attention path.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;

// Workgroup b reads the contiguous share [b * per, (b + 1) * per) of the
// buffer, 16 bytes per lane and load, IN_FLIGHT loads in flight per lane, with
// the non-temporal hint that the decode kernel's page loads carry.  The XOR of
// everything read is stored only when it equals `never`, so the loads stay
// live and nothing else is written.
template <int IN_FLIGHT>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u4* __restrict__ src, int64_t n16,
                                                                     uint32_t never, uint32_t* sink) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b = (int64_t)blockIdx.x * per;
    const int64_t e = b + per < n16 ? b + per : n16;
    u4 acc = {0u, 0u, 0u, 0u};
    for (int64_t i = b + threadIdx.x; i < e; i += (int64_t)kProbeThreads * IN_FLIGHT) {
        u4 v[IN_FLIGHT];
#pragma unroll
        for (int u = 0; u < IN_FLIGHT; ++u) {
            const int64_t j = i + (int64_t)u * kProbeThreads;
            v[u] = j < e ? __builtin_nontemporal_load(&src[j]) : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < IN_FLIGHT; ++u) acc ^= v[u];
    }
    const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (x == never) sink[blockIdx.x] = x;
}

}  // namespace

// Reads `bytes` (a positive multiple of 16) at `src` with `grid` workgroups of
// 256 threads and `in_flight` (2, 4 or 8) loads in flight per lane, on `stream`
// (a hipStream_t; NULL is the null stream).  `sink` holds at least `grid`
// uint32 values; it is written only in the unlikely case that the data's XOR
// equals 0x9E3779B9.  Returns 0, 1 for a bad argument, or 2 when the launch
// fails.
extern "C" __attribute__((visibility("default"))) int gsp_probe_stream_read(const void* src, int64_t bytes, int grid,
                                                                           int in_flight, void* sink, void* stream) {
    if (!src || !sink || bytes < 16 || bytes % 16 != 0 || grid < 1 || grid > 65535) return 1;
    const dim3 g((unsigned)grid), b(kProbeThreads);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const u4* p = static_cast<const u4*>(src);
    uint32_t* out = static_cast<uint32_t*>(sink);
    switch (in_flight) {
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, g, b, 0, s, p, bytes / 16, 0x9E3779B9u, out); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, g, b, 0, s, p, bytes / 16, 0x9E3779B9u, out); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, g, b, 0, s, p, bytes / 16, 0x9E3779B9u, out); break;
        default: return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
