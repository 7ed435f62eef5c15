// api.hip -- op-level entry points of libggml_hip_qmm.so: workspace sizing and
// the MUL_MAT dispatch (GEMV for <= 8 columns, MMQ above, and the few-column
// Q4_K GEMM for 5-8 columns of large matrices), mirroring
// ggml_cuda_mul_mat's choice between MMVQ and MMQ
// (src/ggml/cuda/mulmat.zig:576-639; mmvq.zig:128-173; mmq.zig:865-917).
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

#include <atomic>
#include <mutex>

using namespace qmm;

extern "C" int hip_qmm_mmq(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                           const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                           int64_t dst_col_stride, void *workspace, size_t workspace_size, void *stream);
extern "C" size_t hip_qmm_mmq_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols);

// mmq.hip: whether the few-column kernel takes this shape (given aligned operands)
bool few_cols_type(int type, int64_t K, int64_t nrows, int64_t ncols);
// mmq_few.hip: whether it takes these weight rows
bool mmq_few_takes(int type, int64_t K, const void *w, int64_t row_stride);

// gemv.hip: 2-4 f32 columns (or twice the kernel's columns as two grid rows)
// through the quantize-in-GEMV kernel, or hipErrorNotSupported for shapes it
// does not take.
int qmm_mul_mat_fx_cols(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x,
                        int64_t ncols, int64_t x_col_stride, float *dst, int64_t dst_col_stride, void *stream);
// gemv.hip: 2-8 f32 columns of a small matrix through the one-column kernel
// (grid y = column), or hipErrorNotSupported where it does not win.
int qmm_mul_mat_fx_percol(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x,
                          int64_t ncols, int64_t x_col_stride, float *dst, int64_t dst_col_stride, void *stream);

namespace {
size_t q8_1_bytes(int64_t K, int64_t ncols) {
    const int64_t Kp = pad_k(K);
    return (size_t)(ncols * Kp) + (size_t)(ncols * (Kp / QK8)) * 4u;  // qs plane, then ds plane
}
size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Whether 2-8 columns go to the MMQ dispatch (the few-column kernel,
// mmq_few.hip) rather than the GEMV.  The GEMV's time grows with the columns
// (each wave re-reads every column's activation slice), the few-column
// kernel's hardly does; the few-column kernel is at its best on long rows (K
// >= 8192, where the GEMV's per-wave activation slices are longest) and on
// >= 12288 rows (an unsplit grid, two K halves per workgroup), while on
// 6144-8192 rows of K = 4096 its split grid loses to the GEMV.  Crossovers
// measured on the op (hip_qmm_mul_mat, us, GEMV path against few-column):
//   - Q4_K: from 5 columns at K >= 8192 on >= 4096 rows (4096x14336: 19.6
//     against 16.4) and on >= 12288 rows (14336x4096 at 5: 14.8 against 14.0;
//     12288x4096 13.9 against 13.4), from 6 at K >= 8192 on >= 2048 rows, from
//     7 on >= 6144 rows; the GEMV stays ahead on smaller matrices (4096x4096 at
//     8 columns: 9.7 against 11.1);
//   - Q5_K: from 4 columns on >= 24M weights of long rows or >= 12288 rows
//     (14336x4096 at 4: 18.0 against 16.0), from 6 on other >= 24M weights
//     (6144x4096 at 4 / 5 / 6: 10.5 / 12.9 / 13.9 against 13.5 / 13.5 / 13.6),
//     8 columns from 12M (4096x4096 11.8 against 11.5);
//   - Q8_0: from 4 columns on >= 24M weights of long rows or >= 12288 rows
//     (4096x14336 at 4: 24.0 against 21.1), 8 columns from 12M on long rows;
//     6144x4096 keeps the GEMV (12.4-14.4 against 14.8-15.1 at 4-8 columns);
//   - Q4_0: on >= 24M weights, from 4 columns on >= 12288 rows (14336x4096:
//     17.9 against 16.5) and on long rows of <= 2048 (2048x14336: 15.2 against
//     14.9), from 5 on other long rows (4096x14336 at 4 / 5: 17.3 / 19.9
//     against 17.9 / 17.9); 6144x4096 keeps the GEMV (9.7-13.2 against
//     13.4-13.7); 8 columns from 12M on long rows;
//   - IQ4_XS: from 5 columns on >= 24M weights of long rows or >= 12288 rows
//     (14336x4096: 18.5 against 18.0; 2048x14336: 16.6 against 15.3), 8
//     columns from 12M on long rows;
//   - Q6_K (two 16-deep sub-blocks per MFMA up to 8 columns): on >= 24M
//     weights from 4 columns on long rows or >= 12288 rows (4096x14336 at 4 /
//     8: 24.7 / 27.9 against 22.4 / 22.3; 14336x4096 at 4: 24.3 against 21.1;
//     2048x14336 at 4: 20.5 against 17.6), from 5 on >= 8192 rows (8192x4096
//     at 4 / 5: 15.4 / 17.4 against 16.7 / 16.7), from 6 on the rest
//     (6144x4096 at 5 / 6: 14.7 / 16.6 against 16.1 / 16.2); 7 columns from
//     12M (4096x4096 13.0 against 12.7), 8 columns on rows of K >= 8192 at <=
//     2048 rows; the GEMV stays ahead on 4096x4096 at 5, 6 and 8 columns (10.7
//     / 12.3 / 11.3 against 12.7 / 12.8 / 12.9) and on 1024x4096.
//   At 3 columns the one-launch GEMV with the quantization fused in stays
//   (Q5_K 14336x4096 16.5 against 15.9; Q8_0 4096x14336 22.4 against 20.9).
bool few_cols_wins(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (K % 256 != 0 || ncols > 8 || !few_cols_type(type, K, nrows, ncols)) return false;
    const int64_t elems = nrows * K;
    const bool large = elems >= ((int64_t)24 << 20), mid = elems >= ((int64_t)12 << 20), long_rows = K >= 8192;
    const bool strong = large && (long_rows || nrows >= 12288);  // the few-column kernel's best grids
    switch (type) {
    case TYPE_Q4_K:
        if (long_rows && nrows >= 4096) return ncols >= 5;
        if (nrows >= 12288) return ncols >= 5;
        if (long_rows && nrows >= 2048) return ncols >= 6;
        if (nrows >= 6144) return ncols >= 7;
        return false;
    case TYPE_Q5_K: return (strong && ncols >= 4) || (large && ncols >= 6) || (mid && ncols == 8);
    case TYPE_Q8_0: return (strong && ncols >= 4) || (mid && long_rows && ncols == 8);
    case TYPE_Q4_0:
        return (strong && ncols >= (long_rows && nrows > 2048 && nrows < 12288 ? 5 : 4)) ||
               (mid && long_rows && ncols == 8);
    case TYPE_IQ4_XS: return (strong && ncols >= 5) || (mid && long_rows && ncols == 8);
    case TYPE_Q6_K:
        return (strong && ncols >= 4) || (large && nrows >= 8192 && ncols >= 5) || (large && ncols >= 6) ||
               (mid && ncols == 7) || (mid && long_rows && nrows <= 2048 && ncols == 8);
    default: return false;
    }
}

// Shape-only (the workspace sizing): the MMQ dispatch takes these columns.
bool use_mmq(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return K % 256 == 0 && (ncols > 8 || few_cols_wins(type, K, nrows, ncols));
}

// At the call: up to 8 columns go to the few-column kernel only where it takes
// the rows (16-byte-aligned rows for the 2- and 8-byte-aligned types); the
// MMQ tile would be slower than the GEMV there.
bool use_mmq_rows(int type, int64_t K, int64_t nrows, int64_t ncols, const void *w, int64_t row_stride) {
    return use_mmq(type, K, nrows, ncols) && (ncols > 8 || mmq_few_takes(type, K, w, row_stride));
}

// Whether gate/up/GLU over ncols columns runs the fused MMQ: where each
// product alone would run the MMQ tile kernel (not the GEMV and not the
// few-column kernel; the reference's shouldFuseMulMatQ likewise leaves the
// matmuls its few-row MMQ and MMVQ take, src/ggml/cuda/mulmat.zig:560-567).
bool glu_fuses_mmq(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return ncols >= 2 && use_mmq(type, K, nrows, ncols) && !few_cols_type(type, K, nrows, ncols);
}

// The unfused gate/up/GLU's workspace: the gate and up products, then
// hip_qmm_mul_mat's own workspace.
size_t glu_unfused_bytes(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return align256((size_t)2 * (size_t)nrows * (size_t)ncols * sizeof(float)) +
           hip_qmm_mul_mat_workspace_size(type, K, nrows, ncols);
}
}  // namespace

extern "C" int hip_qmm_version(void) { return (0 << 16) | 1; }

extern "C" int64_t hip_qmm_row_padding(void) { return ROW_PAD; }

extern "C" size_t hip_qmm_mul_mat_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (K <= 0 || ncols <= 0) return 0;
    size_t n = q8_1_bytes(K, ncols);
    if (nrows > 0 && use_mmq(type, K, nrows, ncols)) n = align256(n) + hip_qmm_mmq_workspace_size(type, K, nrows, ncols);
    return n;
}

extern "C" int hip_qmm_mul_mat_uses_mmq(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return K > 0 && nrows > 0 && ncols > 1 && use_mmq(type, K, nrows, ncols) ? 1 : 0;
}

extern "C" int hip_qmm_mul_mat(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                               const float *x, int64_t ncols, int64_t x_col_stride, float *dst,
                               int64_t dst_col_stride, void *workspace, size_t workspace_size, void *stream) {
    if (ncols <= 0 || !workspace || !x || !dst) return (int)hipErrorInvalidValue;
    // columns must not overlap, whichever kernel the shape picks
    if (ncols > 1 && (dst_col_stride < nrows || x_col_stride < K)) return (int)hipErrorInvalidValue;
    if (workspace_size < hip_qmm_mul_mat_workspace_size(type, K, nrows, ncols)) return (int)hipErrorInvalidValue;
    if ((uintptr_t)workspace % 16) return (int)hipErrorInvalidValue;
    // One column: the quantization runs inside the GEMV (one launch), which
    // measured faster than quantizer + GEMV on every decode shape (e.g. Q4_K
    // 1024x4096 3.3 vs 5.1 us, 14336x4096 8.5 vs 9.6 us, Q6_K 4096x14336 with
    // K shares 14.9 vs 15.6 us).
    if (ncols == 1 && K <= 32768 && K % QK8 == 0 && (uintptr_t)x % 16 == 0)
        return hip_qmm_mul_mat_vec_f32(type, w, K, nrows, row_stride, x, dst, stream);
    if (ncols >= 2 && ncols <= 8 && !use_mmq_rows(type, K, nrows, ncols, w, row_stride)) {
        const int e = qmm_mul_mat_fx_percol(type, w, K, nrows, row_stride, x, ncols, x_col_stride, dst,
                                            dst_col_stride, stream);
        if (e != (int)hipErrorNotSupported) return e;
    }
    if (ncols >= 2 && ncols <= 8 && !use_mmq_rows(type, K, nrows, ncols, w, row_stride)) {
        const int e = qmm_mul_mat_fx_cols(type, w, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride,
                                          stream);
        if (e != (int)hipErrorNotSupported) return e;
    }
    const int64_t Kp = pad_k(K);
    int8_t *qs = (int8_t *)workspace;
    void *ds = (uint8_t *)workspace + ncols * Kp;
    if (int e = hip_qmm_quantize_q8_1_planar(x, K, ncols, x_col_stride, qs, ds, stream)) return e;
    if (ncols <= 8 && !use_mmq_rows(type, K, nrows, ncols, w, row_stride))
        return hip_qmm_mul_mat_vec(type, w, K, nrows, row_stride, qs, ds, ncols, dst, dst_col_stride, stream);
    if (K % 256 == 0) {
        const size_t off = align256(q8_1_bytes(K, ncols));
        return hip_qmm_mmq(type, w, K, nrows, row_stride, qs, ds, ncols, dst, dst_col_stride, (uint8_t *)workspace + off,
                           workspace_size - off, stream);
    }
    // Q8_0 / Q4_0 rows whose length is not a multiple of 256 (the MMQ K-step):
    // GEMV over column groups of 8.
    for (int64_t c0 = 0; c0 < ncols; c0 += 8) {
        const int64_t nc = ncols - c0 < 8 ? ncols - c0 : 8;
        const uint8_t *dsb = (const uint8_t *)ds + c0 * (Kp / QK8) * 4;
        if (int e = hip_qmm_mul_mat_vec(type, w, K, nrows, row_stride, qs + c0 * Kp, dsb, nc,
                                        dst + c0 * dst_col_stride, dst_col_stride, stream))
            return e;
    }
    return 0;
}

extern "C" int hip_qmm_mul_mat_glu_fused(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return K > 0 && nrows > 0 && glu_fuses_mmq(type, K, nrows, ncols) ? 1 : 0;
}

extern "C" size_t hip_qmm_mul_mat_glu_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (K <= 0 || nrows <= 0 || ncols <= 0) return 0;
    if (glu_fuses_mmq(type, K, nrows, ncols)) return q8_1_bytes(K, ncols);
    return glu_unfused_bytes(type, K, nrows, ncols);  // one column: only used when the fused GEMV cannot run
}

extern "C" int hip_qmm_mul_mat_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                   int64_t row_stride, const float *x, int64_t ncols, int64_t x_col_stride,
                                   int glu_op, float glu_alpha, float glu_limit, float *dst, int64_t dst_col_stride,
                                   void *workspace, size_t workspace_size, void *stream) {
    if (ncols <= 0 || nrows <= 0 || K <= 0 || !w || !w_gate || !x || !dst || !glu_op_valid(glu_op))
        return (int)hipErrorInvalidValue;
    if (ncols > 1 && (dst_col_stride < nrows || x_col_stride < K)) return (int)hipErrorInvalidValue;
    if (ncols == 1 && K <= 32768 && K % QK8 == 0 && (uintptr_t)x % 16 == 0)
        return hip_qmm_mul_mat_vec_fused(type, w, w_gate, K, nrows, row_stride, x, nullptr, nullptr, glu_op,
                                         glu_alpha, glu_limit, dst, stream);
    if (!workspace || (uintptr_t)workspace % 256 ||
        workspace_size < hip_qmm_mul_mat_glu_workspace_size(type, K, nrows, ncols))
        return (int)hipErrorInvalidValue;
    if (glu_fuses_mmq(type, K, nrows, ncols)) {
        const int64_t Kp = pad_k(K);
        int8_t *qs = (int8_t *)workspace;
        void *ds = (uint8_t *)workspace + ncols * Kp;
        if (int e = hip_qmm_quantize_q8_1_planar(x, K, ncols, x_col_stride, qs, ds, stream)) return e;
        return hip_qmm_mmq_glu(type, w, w_gate, K, nrows, row_stride, qs, ds, ncols, glu_op, glu_alpha, glu_limit,
                               dst, dst_col_stride, stream);
    }
    float *g = (float *)workspace, *u = g + nrows * ncols;
    const size_t off = align256((size_t)2 * (size_t)nrows * (size_t)ncols * sizeof(float));
    void *rest = (uint8_t *)workspace + off;
    if (int e = hip_qmm_mul_mat(type, w_gate, K, nrows, row_stride, x, ncols, x_col_stride, g, nrows, rest,
                                workspace_size - off, stream))
        return e;
    if (int e = hip_qmm_mul_mat(type, w, K, nrows, row_stride, x, ncols, x_col_stride, u, nrows, rest,
                                workspace_size - off, stream))
        return e;
    return hip_qmm_glu_f32(glu_op, glu_alpha, glu_limit, nrows, ncols, g, nrows, u, nrows, dst, dst_col_stride,
                           stream);
}

// ---------------------------------------------------------------- allocation-free MUL_MAT
//
// For callers that cannot allocate (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc): hip_qmm_mul_mat with its workspace
// taken from a fixed device array instead of an argument.  Each device holds
// its own copy of the array for the life of the process.  Its device address
// is looked up once per device, with that device current, and kept; host
// code never passes the array's name (a host-side stand-in) to a kernel.
// Every call on one device shares its array: calls that overlap on one GPU
// race, and a call leaves its scratch contents behind (nothing in the op
// reads scratch before writing it, so no clearing is needed).

static __device__ __align__(256) uint8_t scratch[HIP_QMM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::atomic<void *> scratch_addr[MAX_DEVICES];
std::mutex scratch_mu;

int current_device_scratch(void **out) {
    int dev = -1;
    if (hipError_t e = hipGetDevice(&dev)) return (int)e;
    if (dev < 0 || dev >= MAX_DEVICES) return (int)hipErrorInvalidDevice;
    void *p = scratch_addr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(scratch_mu);
        p = scratch_addr[dev].load(std::memory_order_relaxed);
        if (!p) {
            if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return (int)e;
            if (!p) return (int)hipErrorInvalidSymbol;
            scratch_addr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return 0;
}
}  // namespace

extern "C" int hip_qmm_mul_mat_noalloc(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                       const float *x, int64_t ncols, int64_t x_col_stride, float *dst,
                                       int64_t dst_col_stride, void *stream) {
    if (ncols <= 0 || K <= 0) return (int)hipErrorInvalidValue;
    if (hip_qmm_mul_mat_workspace_size(type, K, nrows, ncols) > (size_t)HIP_QMM_NOALLOC_SCRATCH_BYTES)
        return (int)hipErrorInvalidValue;
    void *ws = nullptr;
    if (int e = current_device_scratch(&ws)) return e;
    return hip_qmm_mul_mat(type, w, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, ws,
                           (size_t)HIP_QMM_NOALLOC_SCRATCH_BYTES, stream);
}
