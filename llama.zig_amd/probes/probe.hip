// probe.hip -- measurement aids for bench.py, built into libqmm_probe.so
// (not into the backend library).  Neither has a counterpart in the
// reference.
//
// 1. stream_read: the memory floor the decode GEMV is measured against: a
//    plain streaming read of a device buffer with the access shape that reads
//    HBM fastest here (each thread 8 x 16-byte loads, every load instruction
//    coalesced over the workgroup, 256 threads), XOR-folded so the loads are
//    not removed, one word written per wave.
// 2. mfma_valu_probe: whether MFMA and VALU work overlap on a SIMD, the fact
//    the MMQ's ceiling rests on.
// 3. empty_launch: a launch that does nothing, in the headline GEMV's grid
//    shape (the fixed cost a launch's duration carries), and q4k_gemv_pattern:
//    the headline GEMV's own loads of a Q4_K matrix (14 waves per workgroup,
//    two rows per wave, each lane the 16-byte header and 32 bytes of nibbles
//    of its 64-weight slice) with no arithmetic, XOR-folded.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// ---------------------------------------------------------------- launch cost and the GEMV's access pattern

constexpr int GP_WAVES = 14, GP_ROWS = 2;  // the headline GEMV's workgroup shape

__global__ __launch_bounds__(64 * GP_WAVES) void empty_launch(uint32_t *sink) {
    if (threadIdx.x == 0 && blockIdx.x == 0xFFFFFFFFu) sink[0] = 1;  // never taken
}

__global__ __launch_bounds__(64 * GP_WAVES) void q4k_gemv_pattern(const uint8_t *__restrict__ w, int64_t nrows,
                                                                  int64_t row_stride, uint32_t *__restrict__ sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = ((int64_t)blockIdx.x * GP_WAVES + wave) * GP_ROWS;
    uint4 a[GP_ROWS][3];
#pragma unroll
    for (int r = 0; r < GP_ROWS; ++r) {
        const int64_t row = row0 + r < nrows ? row0 + r : nrows - 1;
        const uint8_t *blk = w + row * row_stride + (lane >> 2) * 144;  // lane's super-block (K = 4096: 16 per row)
        const int c = lane & 3;                                      // its 64-weight slice of the block
        a[r][0] = *reinterpret_cast<const uint4 *>(blk);
        a[r][1] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * c);
        a[r][2] = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * c);
    }
    uint32_t v = 0;
#pragma unroll
    for (int r = 0; r < GP_ROWS; ++r)
#pragma unroll
        for (int u = 0; u < 3; ++u) v ^= a[r][u].x ^ a[r][u].y ^ a[r][u].z ^ a[r][u].w;
    for (int o = 32; o > 0; o >>= 1) v ^= __shfl_xor(v, o);
    if (lane == 0) sink[(int64_t)blockIdx.x * GP_WAVES + wave] = v;
}

// ---------------------------------------------------------------- MFMA / VALU overlap
//
// 512-thread workgroups, one per CU (launch bounds), so each SIMD holds two
// of the workgroup's eight waves.  Per step a wave runs four substeps; the
// work per SIMD and substep is the same in modes 3-6: two
// v_mfma_f32_32x32x16_f16 and 32 wave64 fp32 FMAs.
//   mode 1: every wave 1 MFMA per substep (4 independent accumulator chains)
//   mode 2: every wave 16 FMAs per substep
//   mode 3: every wave both, interleaved
//   mode 4: waves 0-3 two MFMAs per substep, waves 4-7 32 FMAs per substep.
//           The role is a wave-uniform scalar (readfirstlane) and the two
//           roles run separate loops behind a scalar branch, so no wave
//           issues the other role's instructions.
//   mode 5: mode 3 with the MFMA accumulators in AGPRs
//   mode 6: mode 4 with the MFMA accumulators in AGPRs
// sink[t] = the thread's MFMA sums, sink[n + t] its FMA sums (n = threads of
// the grid); hwid[8 * block + wave] = the wave's HW_ID register (SIMD in bits
// 5:4, CU in 11:8, shader engine in 15:13), so the host can see which waves
// shared a SIMD.

typedef _Float16 pv8h __attribute__((ext_vector_type(8)));
typedef float pv16f __attribute__((ext_vector_type(16)));

constexpr int OV_THREADS = 512;

// The AGPR form is inline assembly, which the compiler neither reorders nor
// guards, so its callers keep three other MFMAs between two on one
// accumulator, as the builtin form's schedule does, and start each chain
// with C = 0 instead of copying zeros into the AGPRs.
template <bool AGPR>
__device__ __forceinline__ void ov_mfma(pv16f &c, const pv8h &a, const pv8h &b) {
    if constexpr (AGPR) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    } else {
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
}

// (with wait states first: the compiler may have written a or b just before)
__device__ __forceinline__ void ov_mfma_first(pv16f &c, const pv8h &a, const pv8h &b) {
    asm volatile("s_nop 7\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
}

__device__ __forceinline__ void ov_fma16(pv16f &acc, float m) {
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = __builtin_fmaf(acc[v], m, 1.0f);
    asm volatile("" : "+v"(acc));
}

// Wait states after a wave's last MFMA, issued while its operands are still
// live: the MFMA reads its A / B registers over its passes, and the code
// after the loop may reuse them (the compiler does not guard this write after
// read for v_mfma_f32_32x32x16_f16 here), so no register is rewritten before
// every MFMA in flight has finished reading.
#define OV_DRAIN_NOPS "s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"

template <bool AGPR>
__device__ __forceinline__ void ov_drain(pv16f (&c)[4], const pv8h &a, const pv8h &b) {
    if constexpr (AGPR)  // the AGPR results are read only after the wait
        asm volatile(OV_DRAIN_NOPS : "+a"(c[0]), "+a"(c[1]), "+a"(c[2]), "+a"(c[3]) : "v"(a), "v"(b));
    else
        asm volatile(OV_DRAIN_NOPS :: "v"(a), "v"(b));
}

template <int MODE>
__global__ __launch_bounds__(OV_THREADS, 1) void mfma_valu_probe(float *__restrict__ sink,
                                                                 uint32_t *__restrict__ hwid, int iters, float m0) {
    constexpr bool AGPR = MODE == 5 || MODE == 6;
    constexpr bool SPLIT = MODE == 4 || MODE == 6;
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

    if constexpr (SPLIT) {
        const int role = __builtin_amdgcn_readfirstlane(wave >> 2);
        if (role == 0) {
            int it = 0;
            if constexpr (AGPR) {
                if (iters > 0) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) ov_mfma_first(c[j], a, b);
#pragma unroll
                    for (int j = 0; j < 4; ++j) ov_mfma<AGPR>(c[j], a, b);
                    it = 1;
                }
            }
            for (; it < iters; ++it) {
#pragma unroll
                for (int j = 0; j < 4; ++j) ov_mfma<AGPR>(c[j], a, b);
#pragma unroll
                for (int j = 0; j < 4; ++j) ov_mfma<AGPR>(c[j], a, b);
            }
            ov_drain<AGPR>(c, a, b);
        } else {
            for (int it = 0; it < iters; ++it) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ov_fma16(acc[j & 1], m);
                    ov_fma16(acc[j & 1], m);
                }
            }
        }
    } else {
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (MODE != 2) {
                    if (AGPR && it == 0) ov_mfma_first(c[j], a, b);
                    else ov_mfma<AGPR>(c[j], a, b);
                }
                if constexpr (MODE != 1) ov_fma16(acc[j & 1], m);
            }
        }
        if constexpr (MODE != 2) ov_drain<AGPR>(c, a, b);
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
    const int64_t t = (int64_t)blockIdx.x * OV_THREADS + threadIdx.x;
    sink[t] = s0;
    sink[(int64_t)gridDim.x * OV_THREADS + t] = s1;
    if (lane == 0) {
        uint32_t id;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(id));
        hwid[(int64_t)blockIdx.x * (OV_THREADS / 64) + wave] = id;
    }
}

}  // namespace

extern "C" size_t qmm_probe_sink_words(size_t bytes) {
    const size_t per_wg = (size_t)PROBE_THREADS * PROBE_LOADS * 16;
    return (bytes + per_wg - 1) / per_wg * (PROBE_THREADS / 64);
}

extern "C" int qmm_probe_stream_read(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (!src || !sink || bytes % 16 != 0 || (uintptr_t)src % 16 != 0) return (int)hipErrorInvalidValue;
    if (bytes == 0) return 0;
    const size_t per_wg = (size_t)PROBE_THREADS * PROBE_LOADS * 16;
    const size_t nblocks = (bytes + per_wg - 1) / per_wg;
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read, dim3((unsigned)nblocks), dim3(PROBE_THREADS), 0, (hipStream_t)stream,
                       (const uint4 *)src, (int64_t)(bytes / 16), sink);
    return (int)hipGetLastError();
}

// A launch of nblocks empty workgroups of the headline GEMV's shape (896 threads).
extern "C" int qmm_probe_empty_launch(int nblocks, uint32_t *sink, void *stream) {
    if (!sink || nblocks < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_launch, dim3((unsigned)nblocks), dim3(64 * GP_WAVES), 0, (hipStream_t)stream, sink);
    return (int)hipGetLastError();
}

// The headline GEMV's loads over a Q4_K matrix of K = 4096 (2304-byte rows);
// sink: one word per wave, ceil(nrows / 28) * 14 words.
extern "C" int qmm_probe_q4k_gemv_pattern(const void *w, int64_t nrows, int64_t row_stride, uint32_t *sink,
                                          void *stream) {
    if (!w || !sink || nrows < 1 || row_stride < 2304 || (uintptr_t)w % 16 || row_stride % 16)
        return (int)hipErrorInvalidValue;
    const int64_t nblocks = (nrows + GP_WAVES * GP_ROWS - 1) / (GP_WAVES * GP_ROWS);
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(q4k_gemv_pattern, dim3((unsigned)nblocks), dim3(64 * GP_WAVES), 0, (hipStream_t)stream,
                       (const uint8_t *)w, nrows, row_stride, sink);
    return (int)hipGetLastError();
}

// sink: 2 * nblocks * 512 floats; hwid: nblocks * 8 words.
extern "C" int qmm_probe_mfma_valu(int mode, int iters, int nblocks, float *sink, uint32_t *hwid, void *stream) {
    if (!sink || !hwid || mode < 1 || mode > 6 || iters < 0 || nblocks < 1 || nblocks > 65536)
        return (int)hipErrorInvalidValue;
    const dim3 g((unsigned)nblocks), t(OV_THREADS);
    hipStream_t s = (hipStream_t)stream;
    switch (mode) {
    case 1: hipLaunchKernelGGL(mfma_valu_probe<1>, g, t, 0, s, sink, hwid, iters, 0.999f); break;
    case 2: hipLaunchKernelGGL(mfma_valu_probe<2>, g, t, 0, s, sink, hwid, iters, 0.999f); break;
    case 3: hipLaunchKernelGGL(mfma_valu_probe<3>, g, t, 0, s, sink, hwid, iters, 0.999f); break;
    case 4: hipLaunchKernelGGL(mfma_valu_probe<4>, g, t, 0, s, sink, hwid, iters, 0.999f); break;
    case 5: hipLaunchKernelGGL(mfma_valu_probe<5>, g, t, 0, s, sink, hwid, iters, 0.999f); break;
    default: hipLaunchKernelGGL(mfma_valu_probe<6>, g, t, 0, s, sink, hwid, iters, 0.999f); break;
    }
    return (int)hipGetLastError();
}
