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

// Whether MFMA and VALU work overlap on a SIMD, the fact the MMQ's ceiling
// rests on.  Each wave runs `iters` steps; per step it issues (mode 1) one
// v_mfma_f32_32x32x16_f16 on each of 4 independent accumulator chains, (mode
// 2) 16 fp32 FMAs on each of 4 steps' register sets, (mode 3) both, or (mode
// 4) the MFMAs in even waves and the FMAs in odd waves.  256 threads, two
// workgroups per CU.  sink[t] gets the thread's MFMA sums and sink[n + t] its
// FMA sums (n = threads of the grid), so the work cannot be removed and each
// mode's parts can be checked against the single-kind modes.
namespace {

typedef _Float16 pv8h __attribute__((ext_vector_type(8)));
typedef float pv16f __attribute__((ext_vector_type(16)));

template <int MODE>
__global__ __launch_bounds__(256, 2) void mfma_valu_probe(float *__restrict__ sink, int iters, float m0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    pv8h a, b;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        a[k] = (_Float16)(lane * 0.001f + k);
        b[k] = (_Float16)(k * 0.01f);
    }
    pv16f c[4], acc[2];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) c[j][v] = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = (float)(v + lane);
    float m = m0 + lane * 1e-6f;
    asm volatile("" : "+v"(m));
    const bool do_mfma = MODE == 1 || MODE == 3 || (MODE == 4 && (wave & 1) == 0);
    const bool do_fma = MODE == 2 || MODE == 3 || (MODE == 4 && (wave & 1) == 1);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (do_mfma) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
            if (do_fma) {
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[j & 1][v] = __builtin_fmaf(acc[j & 1][v], m, 1.0f);
                asm volatile("" : "+v"(acc[j & 1]));
            }
        }
    }
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) s0 += c[j][v];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) s1 += acc[j][v];
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    sink[t] = s0;
    sink[(int64_t)gridDim.x * 256 + t] = s1;
}

}  // namespace

extern "C" int hip_qmm_probe_mfma_valu(int mode, int iters, int nblocks, float *sink, void *stream) {
    if (!sink || mode < 1 || mode > 4 || iters < 0 || nblocks < 1 || nblocks > 65536) return (int)hipErrorInvalidValue;
    const dim3 g((unsigned)nblocks), t(256);
    hipStream_t s = (hipStream_t)stream;
    switch (mode) {
    case 1: hipLaunchKernelGGL(mfma_valu_probe<1>, g, t, 0, s, sink, iters, 0.999f); break;
    case 2: hipLaunchKernelGGL(mfma_valu_probe<2>, g, t, 0, s, sink, iters, 0.999f); break;
    case 3: hipLaunchKernelGGL(mfma_valu_probe<3>, g, t, 0, s, sink, iters, 0.999f); break;
    default: hipLaunchKernelGGL(mfma_valu_probe<4>, g, t, 0, s, sink, iters, 0.999f); break;
    }
    return (int)hipGetLastError();
}
