/*
 * qmm_oracle.h -- CPU restatement of the reference's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * backend, the Python host mirror) may link, load or call this.  Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker / CPU baseline.
 *
 * Every function restates, in plain C, the algorithm of the reference file
 * named in its comment (paths relative to the mlavergn/llama.zig root).  The
 * reference is Zig-only and its C headers come from an empty submodule, so it
 * cannot be built here; the restatement is pinned instead against the golden
 * vectors the reference's own tests hold (src/ggml/quants/golden.zig and
 * src/ggml/cpu/quants/golden.zig), reproduced bit-for-bit by tests/.
 */
#ifndef QMM_ORACLE_H
#define QMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids used on this path (values as the reference's goldens record
 * them: quants/golden.zig:74-133 `.type = ...`). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_Q4_0 = 2,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q8_1 = 9,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q5_K = 13,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
    ORC_TYPE_IQ4_XS = 23,
};

/* Implementation selector for the dot-product drivers. */
enum {
    ORC_IMPL_GENERIC = 0, /* ggml_vec_dot_*_generic + reference row quantizers */
    ORC_IMPL_AVX2    = 1, /* the reference's x86 AVX2 kernels (arch/x86)       */
};

size_t   orc_type_size(int type);   /* bytes per block */
int64_t  orc_blck_size(int type);   /* elements per block */
size_t   orc_row_size(int type, int64_t ne);

uint16_t orc_fp32_to_fp16(float f);
float    orc_fp16_to_fp32(uint16_t h);
int      orc_nearest_int(float f);
uint64_t orc_fnv1a(const void *p, size_t n);

/* reference quantizers / dequantizers */
void orc_quantize_row_q4_0_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q4_K_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q5_K_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q6_K_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_0_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_1_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_q8_K_ref(const float *x, void *y, int64_t k);
void orc_quantize_row_iq4_xs_ref(const float *x, void *y, int64_t k);
void orc_dequantize_row_q4_0(const void *x, float *y, int64_t k);
void orc_dequantize_row_q4_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q5_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q6_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q8_0(const void *x, float *y, int64_t k);
void orc_dequantize_row_q8_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_iq4_xs(const void *x, float *y, int64_t k);
size_t orc_quantize_chunk(int type, const float *src, void *dst, int64_t start,
                          int64_t nrows, int64_t n_per_row, const float *imatrix);

/* x86 row quantizer (round-half-even, id = 127/max) */
void orc_quantize_row_q8_0_avx2(const float *x, void *y, int64_t k);

/* dot products, reference signature without the nrc/stride arguments */
float orc_vec_dot(int type, int impl, int n, const void *vx, const void *vy);

/* GPU-semantics block dot: the integer sums the device kernels form against
 * Q8_1 activations.  Q4_K: one int per 32-sub-block (K/32 per row); Q6_K: one
 * per 16-sub-block (K/16 per row); Q8_0: one per 32-block. */
void orc_block_dots_q8_1(int type, const void *w, int64_t nrows, int64_t K,
                         const void *y_q8_1, int32_t *out);
/* f64 evaluation of out = sum_b d*sc*d8*S - dmin*m*s8 (Q4_K), d*sc*d8*T (Q6_K),
 * d*d8*S (Q8_0) against Q8_1 activations (AoS block_q8_1, ncols columns of K). */
void orc_mul_mat_q8_1_f64(int type, const void *w, int64_t nrows, int64_t K,
                          const void *y_q8_1, int64_t ncols, double *dst);

/* ggml_compute_forward_mul_mat restated: W [K x nrows] quantized, X [K x ncols]
 * f32 column-major (x[c*K + k]), dst[c*nrows + r]. */
void orc_mul_mat(int type, int impl, const void *w, int64_t nrows, int64_t K,
                 const float *x, int64_t ncols, float *dst, int nth);

/* ggml_compute_forward_mul_mat_id restated.  w: n_as experts, each nrows rows;
 * x[(t*ne11 + i11)*K + k]; ids[t*n_ids + s]; dst[(t*n_ids + s)*nrows + r]. */
void orc_mul_mat_id(int type, int impl, const void *w, int64_t n_as, int64_t nrows,
                    int64_t K, const float *x, int64_t ne11, int64_t n_tokens,
                    const int32_t *ids, int64_t n_ids, float *dst, int nth);

/* The reference's x86 tiled K-quant GEMM (the CPU mul_mat for src1 with 8 or
 * more columns on AVX2 hosts, src/ggml/cpu/tiled.zig:1262-1268), for Q4_K,
 * Q5_K, Q6_K and IQ4_XS; same layouts as orc_mul_mat.  Returns 0 (and writes
 * nothing) when the type is not tiled or the host lacks AVX2. */
int orc_mul_mat_tiled(int type, const void *w, int64_t nrows, int64_t K, const float *x, int64_t ncols, float *dst,
                      int nth);

/* The reference's x86 Q8_0 / Q4_0 GEMM (llamafile_sgemm's tinyBLAS_Q0_AVX,
 * src/ggml/cpu/ops/sgemm.zig:578-880, reached from mul_mat for 2 or more
 * columns, src/ggml/cpu/mulmat.zig:336-367).  orc_tinyblas_q0 takes the
 * columns already as Q8_0 (ncols x K/32 blocks); orc_mul_mat_tinyblas
 * quantizes f32 columns with the x86 quantize_row_q8_0 first.  Layouts as
 * orc_mul_mat.  Return 0 (writing nothing) for other types, and
 * orc_mul_mat_tinyblas also below 2 columns or without AVX2. */
int orc_tinyblas_q0(int type, const void *w, int64_t nrows, int64_t K, const void *y_q8_0, int64_t ncols,
                    float *dst, int nth);
int orc_tinyblas_q0_per_output(int type, const void *w, int64_t nrows, int64_t K, const void *y_q8_0, int64_t ncols,
                               float *dst, int nth);
int orc_mul_mat_tinyblas(int type, const void *w, int64_t nrows, int64_t K, const float *x, int64_t ncols,
                         float *dst, int nth);

/* GLU ops (ggml_glu_op: positions in GGML_GLU_OP_NAME, src/ggml/types.zig:103-106) */
#define ORC_GLU_REGLU 0
#define ORC_GLU_GEGLU 1
#define ORC_GLU_SWIGLU 2
#define ORC_GLU_SWIGLU_OAI 3
#define ORC_GLU_SWIGLU_CLAMP 6

/* ggml_gelu_f32 as the CPU's f16 gelu table is built from it
 * (src/ggml/cpu/convert.zig:250-260): 0.5x(1 + tanh(sqrt(2/pi) x (1 + a x^2)))
 * with the inner 1 + a*x*x as one fused multiply-add. */
float orc_gelu_f32(float x);
/* ggml_compute_forward_glu, split form, one row of n:
 * out[i] = glu(gate[i], up[i]); alpha / limit are op params 2 / 3. */
void orc_glu_f32(int op, int64_t n, const float *gate, const float *up, float alpha, float limit, float *out);
/* The op over nrows contiguous rows of nc, with SWIGLU's 8-lane vector arm
 * (ggml_vec_swiglu_f32 on an AVX2 host) and its scalar tail. */
void orc_glu_f32_rows(int op, int64_t nrows, int64_t nc, const float *gate, const float *up, float alpha, float limit,
                      float *out);
/* ggml_v_expf and ggml_v_silu, one lane. */
float orc_v_expf(float x);
void orc_v_expf_n(int64_t n, const float *x, float *out);
float orc_v_silu(float x);

/* synthetic inputs: SplitMix64 -> Box-Muller (double) -> f32 */
void orc_fill_normal(uint64_t seed, int64_t n, float mean, float stddev, float *out);
/* the same values from nth threads */
void orc_fill_normal_mt(uint64_t seed, int64_t n, float mean, float stddev, float *out, int nth);
/* nrows rows of quantize_row_<type>_ref (orc_quantize_chunk, no imatrix) from nth threads */
void orc_quantize_rows_mt(int type, const float *src, void *dst, int64_t nrows, int64_t n_per_row, int nth);

int orc_has_avx2(void);

#ifdef __cplusplus
}
#endif
#endif
