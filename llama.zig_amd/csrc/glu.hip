// glu.hip -- the elementwise ops around the quantized matmul that the HIP
// backend runs when they are not fused into the GEMV epilogue: GLU
// (ggml_compute_forward_glu, src/ggml/cpu/ops/activation.zig:594-608, the
// split form with separate gate and value rows), the same-shape f32 ADD
// (the bias add of src/ggml/cuda/fusion.zig:1482-1520) and ADD_ID, the
// per-expert bias of MUL_MAT_ID outputs (ggml_compute_forward_add_id_f32,
// src/ggml/cpu/ops/arith.zig:155-213).
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

// ADD_ID over rows (slot s, token t): dst row = a row + b row ids[t][s]; an id
// of -1 (or outside [0, n_b)) copies the a row.
__global__ __launch_bounds__(EW_THREADS) void add_id_kernel(int64_t nc, int64_t n_slots, int64_t total,
                                                            const float *__restrict__ a, int64_t a_slot,
                                                            int64_t a_tok, const float *__restrict__ b,
                                                            int64_t b_row, int64_t n_b, const int32_t *__restrict__ ids,
                                                            int64_t ids_stride, float *__restrict__ d, int64_t d_slot,
                                                            int64_t d_tok) {
    const int64_t step = (int64_t)gridDim.x * EW_THREADS;
    for (int64_t i = (int64_t)blockIdx.x * EW_THREADS + threadIdx.x; i < total; i += step) {
        const int64_t r = i / nc, c = i - r * nc;
        const int64_t t = r / n_slots, sl = r - t * n_slots;
        const int e = ids[t * ids_stride + sl];
        const float va = a[t * a_tok + sl * a_slot + c];
        d[t * d_tok + sl * d_slot + c] = e >= 0 && e < n_b ? va + b[(int64_t)e * b_row + c] : va;
    }
}

}  // namespace

extern "C" int hip_qmm_add_id_f32(int64_t nc, int64_t n_slots, int64_t n_tokens, const float *a, int64_t a_slot_stride,
                                  int64_t a_token_stride, const float *b, int64_t b_row_stride, int64_t n_b,
                                  const int32_t *ids, int64_t ids_stride, float *dst, int64_t dst_slot_stride,
                                  int64_t dst_token_stride, void *stream) {
    if (nc < 0 || n_slots < 0 || n_tokens < 0 || n_b < 0 || !a || !b || !ids || !dst || ids_stride < n_slots ||
        a_slot_stride < nc || dst_slot_stride < nc || b_row_stride < nc || a_token_stride < n_slots * a_slot_stride ||
        dst_token_stride < n_slots * dst_slot_stride)
        return (int)hipErrorInvalidValue;
    if (nc == 0 || n_slots == 0 || n_tokens == 0) return 0;
    if (nc > ((int64_t)1 << 40) / (n_slots * n_tokens)) return (int)hipErrorInvalidValue;
    const int64_t total = nc * n_slots * n_tokens;
    int64_t blocks = (total + EW_THREADS - 1) / EW_THREADS;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(add_id_kernel, dim3((unsigned)blocks), dim3(EW_THREADS), 0, (hipStream_t)stream, nc, n_slots,
                       total, a, a_slot_stride, a_token_stride, b, b_row_stride, n_b, ids, ids_stride, dst,
                       dst_slot_stride, dst_token_stride);
    return (int)hipGetLastError();
}

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
