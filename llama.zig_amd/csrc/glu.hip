// glu.hip -- the elementwise ops around the quantized matmul that the HIP
// backend runs when they are not fused into the GEMV epilogue: GLU
// (ggml_compute_forward_glu, src/ggml/cpu/ops/activation.zig:594-608, the
// split form with separate gate and value rows) and the same-shape f32 ADD
// (the bias add of src/ggml/cuda/fusion.zig:1482-1520).
//
// Memory-bound streams: one float per thread per grid-stride step, rows
// addressed through their own strides; glu_apply is the function the fused
// GEMV epilogue calls, so fused and unfused results agree bit for bit.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

namespace {

constexpr int EW_THREADS = 256;

template <bool GLU>
__global__ __launch_bounds__(EW_THREADS) void rows_kernel(int op, float alpha, float limit, int64_t nc, int64_t total,
                                                          const float *__restrict__ a, int64_t a_stride,
                                                          const float *__restrict__ b, int64_t b_stride,
                                                          float *__restrict__ d, int64_t d_stride) {
    const int64_t step = (int64_t)gridDim.x * EW_THREADS;
    for (int64_t i = (int64_t)blockIdx.x * EW_THREADS + threadIdx.x; i < total; i += step) {
        const int64_t r = i / nc, c = i - r * nc;
        const float va = a[r * a_stride + c], vb = b[r * b_stride + c];
        d[r * d_stride + c] = GLU ? glu_apply(op, va, vb, alpha, limit) : va + vb;
    }
}

int launch_rows(bool glu, int op, float alpha, float limit, int64_t nc, int64_t nrows, const float *a,
                int64_t a_stride, const float *b, int64_t b_stride, float *d, int64_t d_stride, void *stream) {
    if (nc < 0 || nrows < 0 || !a || !b || !d) return (int)hipErrorInvalidValue;
    if (a_stride < nc || b_stride < nc || d_stride < nc) return (int)hipErrorInvalidValue;
    if (nc == 0 || nrows == 0) return 0;
    if (nc > ((int64_t)1 << 40) / nrows) return (int)hipErrorInvalidValue;
    const int64_t total = nc * nrows;
    int64_t blocks = (total + EW_THREADS - 1) / EW_THREADS;
    if (blocks > 8192) blocks = 8192;  // grid-stride beyond 32 workgroups per CU
    hipStream_t s = (hipStream_t)stream;
    if (glu)
        hipLaunchKernelGGL(rows_kernel<true>, dim3((unsigned)blocks), dim3(EW_THREADS), 0, s, op, alpha, limit, nc,
                           total, a, a_stride, b, b_stride, d, d_stride);
    else
        hipLaunchKernelGGL(rows_kernel<false>, dim3((unsigned)blocks), dim3(EW_THREADS), 0, s, op, alpha, limit, nc,
                           total, a, a_stride, b, b_stride, d, d_stride);
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int hip_qmm_glu_f32(int glu_op, float alpha, float limit, int64_t nc, int64_t nrows, const float *gate,
                               int64_t gate_stride, const float *up, int64_t up_stride, float *dst,
                               int64_t dst_stride, void *stream) {
    if (glu_op != GLU_REGLU && glu_op != GLU_GEGLU && glu_op != GLU_SWIGLU && glu_op != GLU_SWIGLU_OAI &&
        glu_op != GLU_SWIGLU_CLAMP)
        return (int)hipErrorInvalidValue;
    return launch_rows(true, glu_op, alpha, limit, nc, nrows, gate, gate_stride, up, up_stride, dst, dst_stride,
                       stream);
}

extern "C" int hip_qmm_add_f32(int64_t nc, int64_t nrows, const float *a, int64_t a_stride, const float *b,
                               int64_t b_stride, float *dst, int64_t dst_stride, void *stream) {
    return launch_rows(false, 0, 0.0f, 0.0f, nc, nrows, a, a_stride, b, b_stride, dst, dst_stride, stream);
}
