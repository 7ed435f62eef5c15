/*
 * ggml_hip_qmm.h -- kernel-level C ABI of the MI355X (gfx950) quantized
 * matmul library, libggml_hip_qmm.so.
 *
 * These are the entry points a ggml HIP backend host layer (e.g. a Zig
 * src/ggml/hip/ next to the reference's src/ggml/cuda/) calls where the
 * reference's CUDA host layer launches its kernels.  Each declaration names
 * the reference call site whose launch arguments it mirrors (paths relative
 * to the mlavergn/llama.zig root).
 *
 * Conventions:
 *  - every pointer except `stream` and host-side scalars is a device pointer;
 *  - `type` is the ggml type id: GGML_TYPE_Q4_0 = 2, Q8_0 = 8, Q4_K = 12,
 *    Q5_K = 13, Q6_K = 14, IQ4_XS = 23;
 *  - weights are ggml rows: `nrows` rows of `K` elements, each row
 *    `row_stride` bytes (ggml nb01); blocks in the reference layout
 *    (block_q4_K 144 B, block_q5_K 176 B, block_q6_K 210 B, block_q8_0 34 B,
 *    block_q4_0 18 B, block_iq4_xs 136 B);
 *  - activations / outputs are column-major f32 (ggml ne0 contiguous);
 *  - calls are asynchronous on `stream` (a hipStream_t; NULL = default
 *    stream), allocate nothing, and return 0 (hipSuccess) or a hipError_t
 *    (hipErrorInvalidValue = 1 for rejected shapes);
 *  - scratch is caller-owned (`workspace`), sized by the *_workspace_size
 *    functions, as the reference's host pool provides it (mmvq.zig:633-643).
 */
#ifndef GGML_HIP_QMM_H
#define GGML_HIP_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_HIP_QMM_TYPE_Q4_0 2
#define GGML_HIP_QMM_TYPE_IQ4_XS 23
#define GGML_HIP_QMM_TYPE_Q8_0 8
#define GGML_HIP_QMM_TYPE_Q4_K 12
#define GGML_HIP_QMM_TYPE_Q5_K 13
#define GGML_HIP_QMM_TYPE_Q6_K 14

/* Library version: (major << 16) | minor. */
int hip_qmm_version(void);

/* Row padding of quantized activations, in elements (cuda/common.zig:50-53,
 * MATRIX_ROW_PADDING = 512). */
int64_t hip_qmm_row_padding(void);

/*
 * f32 -> block_q8_1, bit-exact with quantize_row_q8_1_ref
 * (src/ggml/quants/legacy.zig:451-484).  Replaces quantize_row_q8_1_cuda
 * (src/ggml/cuda/quantize.zig:43-54), same arguments: x is [ne00, ne1, ne2,
 * ne3] with element strides s01/s02/s03; y receives ne1*ne2*ne3 rows of
 * ne0_padded/32 blocks (36 B each); elements ne00..ne0_padded-1 are
 * quantized as zeros.  ne0_padded must be a multiple of 32 and >= ne00.
 */
int hip_qmm_quantize_q8_1(const float *x, void *y_q8_1, int64_t ne00, int64_t s01, int64_t s02,
                          int64_t s03, int64_t ne0_padded, int64_t ne1, int64_t ne2, int64_t ne3,
                          void *stream);

/*
 * The same quantization written in the library's planar activation layout,
 * used between its kernels: for column c (of ncols), int8 values at
 * qs[c*Kp + k] and the block header (d, s) as two halves at
 * ((uint32_t*)ds)[c*Kp/32 + k/32], Kp = K rounded up to 512.  Per 32-block
 * the bytes equal quantize_row_q8_1_ref's.  x[c*x_col_stride + k].
 * Replaces the per-layout quantize_mmq_q8_1 variants (quantize.zig:61-118).
 */
int hip_qmm_quantize_q8_1_planar(const float *x, int64_t K, int64_t ncols, int64_t x_col_stride,
                                 int8_t *qs, void *ds, void *stream);

/* Bytes of workspace hip_qmm_mul_mat needs for an nrows x K weight and ncols
 * activation columns: the planar Q8_1 copy, plus split-K partials when the
 * MMQ spreads K over several workgroups. */
size_t hip_qmm_mul_mat_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols);

/* 1 if hip_qmm_mul_mat runs an MMQ kernel (the few-column GEMM or the tile)
 * rather than the GEMV for this shape on 16-byte-aligned rows, else 0 (the
 * shape rules that hip_qmm_mul_mat_workspace_size applies).  No counterpart
 * in the reference: a query for measurement and tests that time or check the
 * kernel the op takes. */
int hip_qmm_mul_mat_uses_mmq(int type, int64_t K, int64_t nrows, int64_t ncols);

/* 1 if hip_qmm_mul_mat runs these 2-8 f32 columns as rows of the one-column
 * fused kernel's grid (each column quantized in the kernel and equal bit for
 * bit to hip_qmm_mul_mat_vec_f32 on it; 16-byte-aligned x with a column
 * stride of a multiple of 4 floats), else 0.  No counterpart in the reference:
 * a query for measurement and tests, like hip_qmm_mul_mat_uses_mmq. */
int hip_qmm_mul_mat_per_column(int type, int64_t K, int64_t nrows, int64_t ncols);

/*
 * Decode GEMV against planar Q8_1 activations, 1..8 columns: dst[c*dst_col_stride + r]
 * = sum_k W[r,k] * y[c,k].  Replaces mul_mat_vec_q_switch_type
 * (src/ggml/cuda/mmvq.zig:275-300, 349-493; the MMVQ path chosen for
 * ncols_dst <= 8 at mmvq.zig:128-173).
 */
int hip_qmm_mul_mat_vec(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                        const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                        int64_t dst_col_stride, void *stream);

/*
 * The reference's mul_mat_vec_q launch, argument for argument: the parameter
 * list of mul_mat_vec_q_switch_type (src/ggml/cuda/mmvq.zig:496), which fills
 * the kernel's Common struct (:260-280) at :349-420 from the strides
 * mulMatVecQ computes (:531-696).  vy is AoS block_q8_1 as
 * hip_qmm_quantize_q8_1 writes it; units as there: stride_*_x in weight
 * blocks, stride_*_y in Q8_1 blocks, stride_*_dst in floats; ncols_x = K,
 * nrows_x = M, ncols_dst 1..8.
 *  - ids == NULL (MUL_MAT): for channel ch < nchannels_dst, sample s <
 *    nsamples_dst and column c < ncols_dst, the rows
 *    dst[c*stride_col_dst + ch*stride_channel_dst + s*stride_sample_dst + r]
 *    = W[ch / (nchannels_dst/nchannels_x), s / (nsamples_dst/nsamples_x)]
 *      . y[c*stride_col_y + ch*stride_channel_y + s*stride_sample_y];
 *    nchannels_y == nchannels_dst, the ratios whole numbers.
 *  - ids != NULL (MUL_MAT_ID): ncols_dst tokens, nchannels_dst slots; slot
 *    ch of token c reads expert e = ids[c*ids_stride + ch] (weights at
 *    e*stride_channel_x) and the activation row
 *    y[c*stride_col_y + (ch % nchannels_y)*stride_channel_y], and writes the
 *    row at dst[c*stride_col_dst + ch*stride_channel_dst]; an id outside
 *    [0, nchannels_x) writes a zero row.  nsamples_x = nsamples_dst = 1.
 * One launch (grid: rows x channels x samples or tokens), no workspace.
 * Weight rows and strides at the blocks' natural alignment (16 B for Q4_K /
 * Q5_K, 8 for IQ4_XS, 2 otherwise), vy 4-byte aligned.
 */
int hip_qmm_mul_mat_vec_q(int type, const void *vx, const void *vy, const int32_t *ids, float *dst,
                          int64_t ncols_x, int64_t nrows_x, int64_t ncols_dst, int64_t stride_row_x,
                          int64_t stride_col_y, int64_t stride_col_dst, int64_t nchannels_x, int64_t nchannels_y,
                          int64_t nchannels_dst, int64_t stride_channel_x, int64_t stride_channel_y,
                          int64_t stride_channel_dst, int64_t nsamples_x, int64_t nsamples_dst,
                          int64_t stride_sample_x, int64_t stride_sample_y, int64_t stride_sample_dst,
                          int64_t ids_stride, void *stream);

/*
 * Decode GEMV of one f32 activation column with the Q8_1 quantization fused
 * in: dst[r] = sum_k W[r,k] * q8_1(x)[k], bit-identical to
 * hip_qmm_quantize_q8_1_planar followed by hip_qmm_mul_mat_vec on one column
 * (two-rows-per-wave kernel).  x 16-byte aligned, K a multiple of the block
 * size and at most 32768; hip_qmm_mul_mat_vec_fused without a gate or a
 * bias.  The MMVQ path of mmvq.zig:275-300 with the
 * quantizer launch of mmvq.zig:633-643 folded in (the quantize-in-GEMV
 * prologue of the fusion arguments, mmvq.zig:552-622).
 */
int hip_qmm_mul_mat_vec_f32(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                            const float *x, float *dst, void *stream);

/* ggml_glu_op values (positions in GGML_GLU_OP_NAME, src/ggml/types.zig:103-106)
 * the fused and standalone GLU entry points accept. */
#define HIP_QMM_GLU_REGLU 0
#define HIP_QMM_GLU_GEGLU 1
#define HIP_QMM_GLU_SWIGLU 2
#define HIP_QMM_GLU_SWIGLU_OAI 3
#define HIP_QMM_GLU_SWIGLU_CLAMP 6

/*
 * One f32 activation column through the Q8_1-quantizing GEMV with the
 * reference's mul_mat_vec fusion epilogue (ggml_cuda_mm_fusion_args_device,
 * src/ggml/cuda/common.zig:1448-1459, applied by mulMatVecQ at
 * src/ggml/cuda/mmvq.zig:571-622; the graph patterns that reach it are
 * src/ggml/cuda/fusion.zig:1308-1390 and 1482-1520):
 *   u[r] = sum_k W[r,k] * q8_1(x)[k]  (+ bias[r] when bias != NULL)
 *   w_gate == NULL:  dst[r] = u[r]
 *   otherwise:       g[r] = sum_k Wg[r,k] * q8_1(x)[k] (+ gate_bias[r]),
 *                    dst[r] = glu(glu_op, g[r], u[r])
 * glu is the CPU op (src/ggml/cpu/ops/activation.zig:434-556): REGLU, GEGLU
 * (f16-table gelu), SWIGLU, SWIGLU_OAI (alpha = op param 2, limit = op param
 * 3) or SWIGLU_CLAMP (limit).  W and Wg share type, shape and row stride.
 * u and g equal hip_qmm_mul_mat_vec_f32's output bit for bit.  K a multiple
 * of the block size and of 32, at most 32768; x 16-byte aligned.  No
 * workspace.  hipErrorInvalidValue for anything else.
 */
int hip_qmm_mul_mat_vec_fused(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                              int64_t row_stride, const float *x, const float *bias, const float *gate_bias,
                              int glu_op, float glu_alpha, float glu_limit, float *dst, void *stream);

/*
 * hip_qmm_mul_mat_vec_fused over the (token, slot) pairs of a MUL_MAT_ID
 * with few tokens: the reference's MMVQ with ids and its fusion arguments
 * (src/ggml/cuda/mmvq.zig:531-622; MUL_MAT_ID gate/up/GLU fusion,
 * src/ggml/cuda/fusion.zig:1153-1306, 1308-1390).  For pair (t, s) with
 * expert e = ids[t*ids_stride + s] and column x + (t*ne11 + s % ne11)*x_row_stride:
 *   u = W_e . q8_1(x);  w_gate == NULL: row = u;  else row = glu(glu_op, Wg_e . q8_1(x), u)
 * written at dst + (t*n_ids + s)*dst_row_stride; an id outside [0, n_as) writes
 * a zero row.  W_e = w + e*expert_stride (Wg_e likewise).  n_tokens*n_ids at most
 * 65535; x 16-byte aligned with x_row_stride a multiple of 4; the limits of
 * hip_qmm_mul_mat_vec_fused otherwise.  No workspace.
 */
int hip_qmm_mul_mat_id_vec_fused(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                 int64_t row_stride, int64_t expert_stride, int64_t n_as, const float *x,
                                 int64_t ne11, int64_t n_tokens, int64_t x_row_stride, const int32_t *ids,
                                 int64_t n_ids, int64_t ids_stride, int glu_op, float glu_alpha, float glu_limit,
                                 float *dst, int64_t dst_row_stride, void *stream);

/*
 * hip_qmm_mul_mat_id_vec_fused with per-expert biases (the MUL_MAT_ID bias
 * lanes, ADD_ID nodes, of src/ggml/cuda/fusion.zig:1308-1360, 1482-1520;
 * the x_bias / gate_bias fusion arguments of mmvq.zig:591-610): the row of
 * pair (t, s) with expert e adds bias + e*bias_expert_stride (u, before the
 * GLU) and gate_bias + e*bias_expert_stride (g); either may be NULL, gate_bias
 * only with w_gate.  bias_expert_stride >= nrows (floats).
 */
int hip_qmm_mul_mat_id_vec_fused_bias(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                      int64_t row_stride, int64_t expert_stride, int64_t n_as, const float *x,
                                      int64_t ne11, int64_t n_tokens, int64_t x_row_stride, const int32_t *ids,
                                      int64_t n_ids, int64_t ids_stride, const float *bias, const float *gate_bias,
                                      int64_t bias_expert_stride, int glu_op, float glu_alpha, float glu_limit,
                                      float *dst, int64_t dst_row_stride, void *stream);

/*
 * hip_qmm_mul_mat_id_vec_fused (gated, one activation row per token, ne11 = 1)
 * with a shared expert in the same launch: the reference's shared_up /
 * shared_gate / shared_dst fusion arguments (src/ggml/cuda/common.zig:1448-1459,
 * mmvq.zig:300-320, 574-590; the graph pattern of fusion.zig:930-955).
 * Besides the routed rows, token t's column x + t*x_row_stride goes through
 * the shared expert: shared_dst + t*shared_dst_row_stride =
 * glu(glu_op, shared_gate . q8_1(x_t), shared_up . q8_1(x_t)).  The shared
 * weights have the experts' type, row count, K and row_stride (block-aligned);
 * n_tokens*(n_ids + 1) at most 65535.
 */
int hip_qmm_mul_mat_id_vec_fused_shared(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                        int64_t row_stride, int64_t expert_stride, int64_t n_as, const float *x,
                                        int64_t n_tokens, int64_t x_row_stride, const int32_t *ids, int64_t n_ids,
                                        int64_t ids_stride, int glu_op, float glu_alpha, float glu_limit, float *dst,
                                        int64_t dst_row_stride, const void *shared_up, const void *shared_gate,
                                        float *shared_dst, int64_t shared_dst_row_stride, void *stream);

/*
 * Standalone ADD_ID (ggml_compute_forward_add_id_f32,
 * src/ggml/cpu/ops/arith.zig:155-213) over n_tokens x n_slots rows of nc floats:
 * dst[t*dst_token_stride + s*dst_slot_stride + i] = a[...] + b[ids[t*ids_stride + s]*b_row_stride + i],
 * or a[...] alone where the id is -1 (or outside [0, n_b), which the reference
 * asserts against).  Strides in floats (ids: int32 elements).
 */
int hip_qmm_add_id_f32(int64_t nc, int64_t n_slots, int64_t n_tokens, const float *a, int64_t a_slot_stride,
                       int64_t a_token_stride, const float *b, int64_t b_row_stride, int64_t n_b, const int32_t *ids,
                       int64_t ids_stride, float *dst, int64_t dst_slot_stride, int64_t dst_token_stride,
                       void *stream);

/*
 * Standalone GLU over rows of f32 (ggml_compute_forward_glu,
 * src/ggml/cpu/ops/activation.zig:594-608, per element as above):
 * dst[r*dst_stride + i] = glu(op, gate[r*gate_stride + i], up[r*up_stride + i])
 * for i < nc, r < nrows; strides in floats.
 */
int hip_qmm_glu_f32(int glu_op, float alpha, float limit, int64_t nc, int64_t nrows, const float *gate,
                    int64_t gate_stride, const float *up, int64_t up_stride, float *dst, int64_t dst_stride,
                    void *stream);

/*
 * Elementwise f32 add of two same-shape row sets (ggml_add without
 * broadcasting, the bias add the fused GEMV epilogue replaces):
 * dst[r*dst_stride + i] = a[r*a_stride + i] + b[r*b_stride + i].
 */
int hip_qmm_add_f32(int64_t nc, int64_t nrows, const float *a, int64_t a_stride, const float *b, int64_t b_stride,
                    float *dst, int64_t dst_stride, void *stream);

/*
 * Small-batch GEMV on int8 MFMA, 1..16 columns, K a multiple of 256: 16 rows
 * per workgroup contracted against all columns at once (v_mfma_i32_16x16x32_i8),
 * same arguments and result as hip_qmm_mul_mat_vec.  The MMVQ path of
 * mmvq.zig:275-300 for 2..8 columns and the small-column MMQ tiles of
 * mmq.zig:865-917 for 9..16.
 */
int hip_qmm_gemv_mfma(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *y_qs,
                      const void *y_ds, int64_t ncols, float *dst, int64_t dst_col_stride, void *stream);

/*
 * Op-level MUL_MAT: quantizes x to Q8_1 into `workspace` and runs one of
 * three kernels, as the dispatch in ggml_cuda_mul_mat picks between MMVQ, its
 * few-row MMQ and MMQ (src/ggml/cuda/mulmat.zig:576-639):
 *  - the GEMV for up to 8 columns.  One column, and 2-4 columns of rows with
 *    K <= 4096 (below 8192 rows, except for K <= 2048 and Q8_0 at 3-4
 *    columns), skip the separate quantizer: the GEMV quantizes the columns in
 *    its prologue, as it does for 4 columns of the K-quants, 6 of IQ4_XS and 8
 *    of Q8_0 on at most 4096 rows (two rows of its grid).  2-8 columns of
 *    small matrices (at most 2048 rows of K <= 4096; Q8_0 / Q4_0 at most 1024
 *    rows, and 4 columns unless K <= 2048) run as rows of the one-column
 *    kernel's grid, each column quantized in the kernel
 *    (hip_qmm_mul_mat_per_column), with no workspace;
 *  - the few-column GEMM (16x16 int8 MFMA tiles) for 9-32 columns (9-16 for
 *    Q6_K; Q8_0 / Q4_0 at 17-32 columns of 8 MiB of weights and more take the
 *    tile), and also for 4-8 columns of large matrices, where it measured
 *    faster than the GEMV (the shape rules are hip_qmm_mul_mat_workspace_size's
 *    and hip_qmm_mul_mat_uses_mmq's: e.g. Q4_K from 5 columns at K >= 8192 on
 *    >= 4096 rows and on >= 12288 rows, from 7 columns on >= 6144 rows; Q6_K
 *    from 4 columns on >= 24M weights of long rows or >= 12288 rows).  On
 *    those 4-8 column shapes the workspace grows by the
 *    few-column kernel's split-K partials, and the results differ from
 *    hip_qmm_mul_mat_vec's in fp32 rounding (another summation order; both
 *    pass the f64 and CPU gates);
 *  - the int8-MFMA MMQ tile for the rest.
 * x[c*x_col_stride + k] f32, dst[c*dst_col_stride + r] f32.
 */
int hip_qmm_mul_mat(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                    const float *x, int64_t ncols, int64_t x_col_stride, float *dst,
                    int64_t dst_col_stride, void *workspace, size_t workspace_size, void *stream);

/* Scratch bytes behind hip_qmm_mul_mat_noalloc, per device (32 MiB). */
#define HIP_QMM_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * hip_qmm_mul_mat without the workspace arguments: the same dispatch, the
 * same kernels and the same results, with its scratch (the Q8_1 copy of x and
 * any split-K partials) in a fixed device array of
 * HIP_QMM_NOALLOC_SCRATCH_BYTES that each device holds for the life of the
 * process.  It calls no hipMalloc / hipFree or anything that allocates; the
 * array's address is looked up once per device on the first call with that
 * device current.  Uses the current device's array: `stream` must belong to
 * the current device.  Shapes whose workspace
 * (hip_qmm_mul_mat_workspace_size) exceeds the array are rejected with
 * hipErrorInvalidValue before any launch.  All calls on one device share the
 * array, so calls that may overlap on one GPU (different streams, threads)
 * race; calls in one stream's order do not.
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid allocation).
 */
int hip_qmm_mul_mat_noalloc(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                            const float *x, int64_t ncols, int64_t x_col_stride, float *dst,
                            int64_t dst_col_stride, void *stream);

/*
 * int8-MFMA GEMM against planar Q8_1 activations for any column count
 * (K a multiple of 256).  Replaces launch_mul_mat_q (src/ggml/cuda/mmq.zig:282-408).
 * When the output tiles alone would leave the GPU under-filled, K is split
 * over several workgroups (the reference's stream-k fixup, mmq.zig:359-407)
 * and the partials, kept in `workspace`, are summed in a fixed order; with
 * no or too small a workspace the GEMM runs unsplit.
 */
int hip_qmm_mmq(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *y_qs,
                const void *y_ds, int64_t ncols, float *dst, int64_t dst_col_stride, void *workspace,
                size_t workspace_size, void *stream);

/* Bytes of split-K workspace hip_qmm_mmq uses for this shape (0: no split). */
size_t hip_qmm_mmq_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols);

/* Column-tile width (32 or 64) for ncols columns: 32 up to 32 columns, 64
 * above.  hip_qmm_mmq also takes 32 for Q4_K, Q5_K, Q8_0 and Q4_0 on rows of
 * at most 16 K-steps where 64-column tiles would number at most 256 and
 * 32-column ones at most 512; hip_qmm_mmq_glu does the same over its tiles of
 * 64 output rows, except for Q8_0.  hip_qmm_mmq_split_k: the K-split factor
 * hip_qmm_mmq picks (1: no split; otherwise a divisor of K / 256). */
int hip_qmm_mmq_tile_n(int64_t ncols);
int hip_qmm_mmq_split_k(int type, int64_t K, int64_t nrows, int64_t ncols);

/*
 * Expert-grouped MMQ over device-side tile tables (see hip_qmm_mul_mat_id):
 * tiles[4*i .. 4*i+3] = {expert, col_low, col_high, unused}, the layout of
 * the reference's ggml_cuda_mm_id_tile_spec (src/ggml/cuda/mmid.zig:18-27):
 * routed columns col_low .. col_high-1 (at most bn of them) of that expert;
 * *n_tiles live entries, at most max_tiles; col_src / col_dst map a routed
 * column to its activation row and its dst row.  Mirrors mul_mat_q's ids
 * path (src/ggml/cuda/mmq.zig:750-855).  tiles 16-byte aligned.
 */
int hip_qmm_mmq_grouped(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                        int64_t expert_stride, const int8_t *y_qs, const void *y_ds, float *dst,
                        int64_t dst_row_stride, int bn, int64_t max_tiles, const int32_t *tiles,
                        const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst, void *stream);

/*
 * Gate/up/GLU fused MMQ: dst[c*dst_col_stride + r] = glu(glu_op, (Wg . y_c)[r], (W . y_c)[r]) over
 * planar Q8_1 columns y, glu as in hip_qmm_mul_mat_vec_fused.  The reference's mul_mat_q with
 * a gate (src/ggml/cuda/mmq.zig:568-640, called from its gate/up/GLU fusion,
 * src/ggml/cuda/fusion.zig:1226-1298, 1391).  W and Wg share type, shape and row stride; the
 * limits of hip_qmm_mmq otherwise.  One tile kernel reads both weights (64 output rows per
 * 128-row tile), with no K split, so each gate and up sum equals hip_qmm_mmq's without a
 * workspace bit for bit.  No workspace.
 */
int hip_qmm_mmq_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows, int64_t row_stride,
                    const int8_t *y_qs, const void *y_ds, int64_t ncols, int glu_op, float glu_alpha,
                    float glu_limit, float *dst, int64_t dst_col_stride, void *stream);

/* hip_qmm_mmq_grouped with a gate: the routed columns of each expert through
 * W_e and Wg_e = w_gate + e*expert_stride, writing glu(gate, up) rows
 * (the reference's mul_mat_q with ids and a gate, src/ggml/cuda/mmq.zig:568-640). */
int hip_qmm_mmq_grouped_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                            int64_t row_stride, int64_t expert_stride, const int8_t *y_qs, const void *y_ds,
                            float *dst, int64_t dst_row_stride, int bn, int64_t max_tiles, const int32_t *tiles,
                            const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst, int glu_op,
                            float glu_alpha, float glu_limit, void *stream);

/* Bytes of workspace hip_qmm_mul_mat_glu needs (none for one column when the fused GEMV takes it). */
size_t hip_qmm_mul_mat_glu_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols);

/* 1 if hip_qmm_mul_mat_glu runs the fused MMQ for this shape (the products
 * would each run the MMQ tile kernel), else 0: the reference's
 * shouldFuseMulMatQ (src/ggml/cuda/mulmat.zig:548-571) for this backend. */
int hip_qmm_mul_mat_glu_fused(int type, int64_t K, int64_t nrows, int64_t ncols);

/*
 * Op-level gate/up/GLU, the {MUL_MAT gate, MUL_MAT up, GLU} subgraph the
 * reference fuses (src/ggml/cuda/fusion.zig:1391-1440; shouldFuseMulMatQ,
 * src/ggml/cuda/mulmat.zig:548-571): dst[c][r] = glu(glu_op, (Wg . x_c)[r], (W . x_c)[r])
 * for ncols f32 columns x[c*x_col_stride + k].  One column:
 * hip_qmm_mul_mat_vec_fused.  Where the unfused products would run the MMQ
 * tile kernel: one Q8_1 quantization and hip_qmm_mmq_glu.  Between (the
 * GEMV's and the few-column kernel's column counts, which the reference does
 * not fuse either): the two hip_qmm_mul_mat products into the workspace and
 * hip_qmm_glu_f32, as the unfused graph runs.  Limits of hip_qmm_mul_mat.
 */
int hip_qmm_mul_mat_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows, int64_t row_stride,
                        const float *x, int64_t ncols, int64_t x_col_stride, int glu_op, float glu_alpha,
                        float glu_limit, float *dst, int64_t dst_col_stride, void *workspace, size_t workspace_size,
                        void *stream);

/* Bytes of workspace hip_qmm_mul_mat_id needs. */
size_t hip_qmm_mul_mat_id_workspace_size(int type, int64_t K, int64_t n_as, int64_t ne11, int64_t n_tokens,
                                         int64_t n_ids);

/*
 * Op-level MUL_MAT_ID (ggml_mul_mat_id, src/ggml/ops.zig:1104-1125; CPU
 * semantics src/ggml/cpu/mulmat.zig:555-777): n_as experts of nrows x K
 * weights, expert e at w + e*expert_stride; activations x row (t, i11) at
 * x + (t*ne11 + i11)*x_row_stride (ne11 = 1 broadcasts one row per token,
 * ne11 = n_ids gives one per slot); ids[t*ids_stride + s] selects the expert
 * of slot s of token t; dst row (t, s) at dst + (t*n_ids + s)*dst_row_stride.
 * An id of -1 (or any id outside [0, n_as)) yields a zero row.  Up to 8
 * tokens (the reference's MMVQ-with-ids batch limit on AMD,
 * src/ggml/cuda/mmvq.zig:116-125) it runs hip_qmm_mul_mat_id_vec_fused
 * without a gate: one launch, no workspace touched.  Above that, expert
 * grouping runs on the device (no host synchronisation) and feeds the
 * grouped MMQ; replaces ggml_cuda_mul_mat_id
 * (src/ggml/cuda/mulmat.zig:669-800) and mm_ids_helper
 * (src/ggml/cuda/mmid.zig:32-90).  K a multiple of 256; at most 1024
 * experts.
 */
int hip_qmm_mul_mat_id(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                       int64_t expert_stride, int64_t n_as, const float *x, int64_t ne11, int64_t n_tokens,
                       int64_t x_row_stride, const int32_t *ids, int64_t n_ids, int64_t ids_stride, float *dst,
                       int64_t dst_row_stride, void *workspace, size_t workspace_size, void *stream);

/*
 * hip_qmm_mul_mat_id with a gate: dst row (t, s) = glu(glu_op, Wg_e . x, W_e . x)
 * for expert e = ids[t*ids_stride + s] (a zero row for an id outside
 * [0, n_as)), Wg_e = w_gate + e*expert_stride; the reference's MUL_MAT_ID
 * gate/up/GLU fusion (src/ggml/cuda/fusion.zig:1153-1306, into mmvq or
 * mul_mat_q with ids).  Up to 8 tokens: hip_qmm_mul_mat_id_vec_fused; above,
 * one grouping and Q8_1 copy feed hip_qmm_mmq_grouped_glu.  Workspace and
 * limits of hip_qmm_mul_mat_id.
 */
int hip_qmm_mul_mat_id_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                           int64_t row_stride, int64_t expert_stride, int64_t n_as, const float *x, int64_t ne11,
                           int64_t n_tokens, int64_t x_row_stride, const int32_t *ids, int64_t n_ids,
                           int64_t ids_stride, int glu_op, float glu_alpha, float glu_limit, float *dst,
                           int64_t dst_row_stride, void *workspace, size_t workspace_size, void *stream);

/*
 * Test hook: the integer block dot products the GEMV forms, written out
 * instead of scaled.  out[c][r][i] int32 with i over K/32 sub-blocks (Q4_K,
 * Q8_0) or K/16 (Q6_K).  Shares the device code of hip_qmm_mul_mat_vec.
 */
int hip_qmm_block_dots(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                       const int8_t *y_qs, int64_t ncols, int32_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
