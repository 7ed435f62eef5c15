// quantize_q8_1.hip -- f32 activations -> Q8_1, bit-exact with the
// reference's quantize_row_q8_1_ref (src/ggml/quants/legacy.zig:451-484):
//   amax over 32 values; d = amax / 127 (IEEE division); id = d ? 1/d : 0
//   (IEEE division, not v_rcp); q = trunc-to-int8(roundf(x * id)) with
//   roundf = half away from zero; d and s = fp16(sum(q) * d) rounded to
//   nearest-even (q8_1_code / q8_1_pack_ds in qmm_device.h).  Built without
//   fast-math so '/' stays correctly rounded.
//
// One 32-lane half-wave per Q8_1 block: lane i owns element i of the block;
// amax and sum(q) are butterfly reductions inside the half-wave.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

namespace {

struct Q8_1Val {
    int8_t q;
    float d;
    int sum;
};

__device__ __forceinline__ Q8_1Val quantize_lane32(float x) {
    float amax = fabsf(x);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int8_t q = q8_1_code(x, id);
    int sum = q;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 32);
    return {q, d, sum};
}

// Reference-layout output: one block_q8_1 {d, s, qs[32]} per 32 values.
__global__ __launch_bounds__(256) void quantize_q8_1_aos(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                         int64_t ne00, int64_t s01, int64_t s02, int64_t s03,
                                                         int64_t ne0_padded, int64_t ne1, int64_t ne2) {
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t i1 = blockIdx.y;
    const int64_t i23 = blockIdx.z;
    const int64_t i2 = i23 % ne2, i3 = i23 / ne2;
    if (i0 >= ne0_padded) return;  // whole half-waves: ne0_padded % 32 == 0
    const float xv = i0 < ne00 ? x[i3 * s03 + i2 * s02 + i1 * s01 + i0] : 0.0f;
    const Q8_1Val v = quantize_lane32(xv);
    const int64_t row = (i23 * ne1 + i1);
    uint8_t *blk = y + (row * (ne0_padded / QK8) + i0 / QK8) * 36;
    blk[4 + (i0 & 31)] = (uint8_t)v.q;
    if ((i0 & 31) == 0) *reinterpret_cast<uint32_t *>(blk) = q8_1_pack_ds(v.d, v.sum);
}

// Planar output: qs[c*Kp + k], ds[c*Kp/32 + k/32].
__global__ __launch_bounds__(256) void quantize_q8_1_planar(const float *__restrict__ x, int64_t K,
                                                            int64_t x_col_stride, int64_t Kp,
                                                            int8_t *__restrict__ qs, uint32_t *__restrict__ ds) {
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t c = blockIdx.y;
    if (k >= Kp) return;
    const float xv = k < K ? x[c * x_col_stride + k] : 0.0f;
    const Q8_1Val v = quantize_lane32(xv);
    qs[c * Kp + k] = v.q;
    if ((k & 31) == 0) ds[c * (Kp / QK8) + k / QK8] = q8_1_pack_ds(v.d, v.sum);
}

// Planar output, 8 consecutive values per lane: a 32-block is the 4 lanes of
// one quad, so amax and sum(q) take two DPP exchanges instead of five
// shuffles, and x is read with 16-byte loads.  The max and the integer sum do
// not depend on the order, so the bytes equal the one-value-per-lane
// kernel's.  Needs x 16-byte aligned and x_col_stride a multiple of 4.
__global__ __launch_bounds__(256) void quantize_q8_1_planar8(const float *__restrict__ x, int64_t K,
                                                             int64_t x_col_stride, int64_t Kp,
                                                             int8_t *__restrict__ qs, uint32_t *__restrict__ ds) {
    const int64_t k = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const int64_t c = blockIdx.y;
    // whole quads stay active: Kp is a multiple of 512, so k < Kp for all 4 lanes or none
    if (k >= Kp) return;
    float v[8];
    if (k < K) {  // K % 32 == 0: a 32-block is wholly inside or wholly past K
        const float4 a = *reinterpret_cast<const float4 *>(x + c * x_col_stride + k);
        const float4 b = *reinterpret_cast<const float4 *>(x + c * x_col_stride + k + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    const Q8Quad r = q8_1_quantize_quad(v);
    *reinterpret_cast<uint2 *>(qs + c * Kp + k) = make_uint2(r.lo, r.hi);
    if ((threadIdx.x & 3) == 0) ds[c * (Kp / QK8) + k / QK8] = r.ds;
}

}  // namespace

extern "C" int hip_qmm_quantize_q8_1(const float *x, void *y_q8_1, int64_t ne00, int64_t s01, int64_t s02,
                                     int64_t s03, int64_t ne0_padded, int64_t ne1, int64_t ne2, int64_t ne3,
                                     void *stream) {
    if (!x || !y_q8_1 || ne00 < 0 || ne0_padded < ne00 || ne0_padded % QK8 != 0 || ne1 < 0 || ne2 < 1 ||
        ne3 < 1 || ne1 > 65535 || ne2 * ne3 > 65535)
        return (int)hipErrorInvalidValue;
    if (ne0_padded == 0 || ne1 == 0) return 0;
    const dim3 grid((unsigned)((ne0_padded + 255) / 256), (unsigned)ne1, (unsigned)(ne2 * ne3));
    hipLaunchKernelGGL(quantize_q8_1_aos, grid, dim3(256), 0, (hipStream_t)stream, x, (uint8_t *)y_q8_1, ne00,
                       s01, s02, s03, ne0_padded, ne1, ne2);
    return (int)hipGetLastError();
}

extern "C" int hip_qmm_quantize_q8_1_planar(const float *x, int64_t K, int64_t ncols, int64_t x_col_stride,
                                            int8_t *qs, void *ds, void *stream) {
    if (!x || !qs || !ds || K <= 0 || K % QK8 != 0 || ncols < 0 || ncols > 65535 || x_col_stride < K)
        return (int)hipErrorInvalidValue;
    if (ncols == 0) return 0;
    const int64_t Kp = pad_k(K);
    if ((uintptr_t)x % 16 == 0 && x_col_stride % 4 == 0 && (uintptr_t)qs % 8 == 0) {
        const dim3 grid((unsigned)((Kp / 8 + 255) / 256), (unsigned)ncols);
        hipLaunchKernelGGL(quantize_q8_1_planar8, grid, dim3(256), 0, (hipStream_t)stream, x, K, x_col_stride, Kp, qs,
                           (uint32_t *)ds);
    } else {
        const dim3 grid((unsigned)((Kp + 255) / 256), (unsigned)ncols);
        hipLaunchKernelGGL(quantize_q8_1_planar, grid, dim3(256), 0, (hipStream_t)stream, x, K, x_col_stride, Kp, qs,
                           (uint32_t *)ds);
    }
    return (int)hipGetLastError();
}
