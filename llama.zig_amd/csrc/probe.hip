// probe.hip -- the memory floor the decode GEMV is measured against: a plain
// streaming read of a device buffer with the access shape that reads HBM
// fastest here (each thread 8 x 16-byte loads, every load instruction
// coalesced over the workgroup, 256 threads), XOR-folded so the loads are
// not removed, one word written per wave.  A measurement aid for the
// benchmark; it has no counterpart in the reference.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

namespace {

constexpr int PROBE_THREADS = 256;
constexpr int PROBE_LOADS = 8;  // 16-byte loads in flight per thread

__global__ __launch_bounds__(PROBE_THREADS) void stream_read(const uint4 *__restrict__ p, int64_t n16,
                                                             uint32_t *__restrict__ sink) {
    const int64_t base = (int64_t)blockIdx.x * PROBE_THREADS * PROBE_LOADS + threadIdx.x;
    uint4 a[PROBE_LOADS];
#pragma unroll
    for (int u = 0; u < PROBE_LOADS; ++u) {
        const int64_t i = base + (int64_t)PROBE_THREADS * u;
        a[u] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
    }
    uint32_t v = 0;
#pragma unroll
    for (int u = 0; u < PROBE_LOADS; ++u) v ^= a[u].x ^ a[u].y ^ a[u].z ^ a[u].w;
    for (int o = 32; o > 0; o >>= 1) v ^= __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) sink[(int64_t)blockIdx.x * (PROBE_THREADS / 64) + (threadIdx.x >> 6)] = v;
}

}  // namespace

extern "C" size_t hip_qmm_probe_sink_words(size_t bytes) {
    const size_t per_wg = (size_t)PROBE_THREADS * PROBE_LOADS * 16;
    return (bytes + per_wg - 1) / per_wg * (PROBE_THREADS / 64);
}

extern "C" int hip_qmm_probe_stream_read(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (!src || !sink || bytes % 16 != 0 || (uintptr_t)src % 16 != 0) return (int)hipErrorInvalidValue;
    if (bytes == 0) return 0;
    const size_t per_wg = (size_t)PROBE_THREADS * PROBE_LOADS * 16;
    const size_t nblocks = (bytes + per_wg - 1) / per_wg;
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read, dim3((unsigned)nblocks), dim3(PROBE_THREADS), 0, (hipStream_t)stream,
                       (const uint4 *)src, (int64_t)(bytes / 16), sink);
    return (int)hipGetLastError();
}
