/*
 * qmm_oracle.c -- CPU restatement of the reference's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU
 * baseline bench.py times.  The product never links or calls this file.
 *
 * Built with -ffp-contract=off: the reference's goldens were captured from C
 * compiled that way (src/ggml/quants/helpers.zig:27-59), and its Zig port is
 * strict (no contraction) -- every float expression below is evaluated in the
 * order written, one rounding per operation, exactly as the Zig does.  The
 * AVX2 kernels use explicit FMA intrinsics where the reference does.
 *
 * Parity status of each part (pinned = reproduced bit-for-bit against a
 * golden the reference's tests hold; see tests/test_oracle_golden.py):
 *   fp16 <-> fp32 ................. pinned through every quant/dequant golden
 *   quantize_row_q4_K/q6_K/q8_0/q8_1/q8_K_ref, dequantize_* . pinned
 *   quantize_q4_K / q6_K (imatrix impls) ......... pinned (chunk_imatrix goldens)
 *   vec_dot q4_K/q6_K/q8_0 generic ............... pinned (cpu/quants/golden.zig)
 *   vec_dot AVX2 + quantize_row_q8_0 AVX2 ........ the tree holds no x86
 *       goldens: pinned by constructed cases on which the specification and
 *       a plausible mistake differ (tie rule, 127/amax multiplier, lane
 *       accumulation, hsum_float_8 order, min-lane fold, fused block scale;
 *       tests/test_oracle_x86_pins.py), and held to the generic kernels.
 *   v_expf / v_silu (SWIGLU's vector arm) ........ pinned to the routine's
 *       published error bound, exact points, range limits and the row split
 *       (tests/test_oracle_glu.py).
 *   mul_mat / mul_mat_id drivers .................. pinned by construction
 *       (each output is one vec_dot call) + thread-count invariance tests.
 *   block_dots_q8_1 / mul_mat_q8_1_f64 ........... GPU-semantics restatement;
 *       pinned against brute force on tiny inputs and the dequantised f64 dot.
 */
#include "qmm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define ORC_X86 1
#else
#define ORC_X86 0
#endif

#define QK_K 256
#define QK8_0 32
#define QK8_1 32
#define K_SCALE_SIZE 12

/* Block layouts: src/ggml/quants/blocks.zig:67-222 (ggml-common.h). */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;                     /* 18 B */
typedef struct { uint16_t d; int8_t qs[QK8_0]; } blk_q8_0;                  /* 34 B */
typedef struct { uint16_t d; uint16_t s; int8_t qs[QK8_1]; } blk_q8_1;      /* 36 B */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[K_SCALE_SIZE]; uint8_t qs[QK_K / 2]; } blk_q4_K; /* 144 B */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[K_SCALE_SIZE]; uint8_t qh[QK_K / 8]; uint8_t qs[QK_K / 2]; } blk_q5_K; /* 176 B */
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; } blk_q6_K;  /* 210 B */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } blk_q8_K;                               /* 292 B */
typedef struct { uint16_t d; uint16_t scales_h; uint8_t scales_l[QK_K / 64]; uint8_t qs[QK_K / 2]; } blk_iq4_xs; /* 136 B */

_Static_assert(sizeof(blk_q4_0) == 18, "q4_0");
_Static_assert(sizeof(blk_q8_0) == 34, "q8_0");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K");
_Static_assert(sizeof(blk_q5_K) == 176, "q5_K");
_Static_assert(sizeof(blk_q6_K) == 210, "q6_K");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K");
_Static_assert(sizeof(blk_iq4_xs) == 136, "iq4_xs");

size_t orc_type_size(int type) {
    switch (type) {
    case ORC_TYPE_F32: return 4;
    case ORC_TYPE_Q4_0: return sizeof(blk_q4_0);
    case ORC_TYPE_Q8_0: return sizeof(blk_q8_0);
    case ORC_TYPE_Q8_1: return sizeof(blk_q8_1);
    case ORC_TYPE_Q4_K: return sizeof(blk_q4_K);
    case ORC_TYPE_Q5_K: return sizeof(blk_q5_K);
    case ORC_TYPE_Q6_K: return sizeof(blk_q6_K);
    case ORC_TYPE_Q8_K: return sizeof(blk_q8_K);
    case ORC_TYPE_IQ4_XS: return sizeof(blk_iq4_xs);
    default: return 0;
    }
}

int64_t orc_blck_size(int type) {
    switch (type) {
    case ORC_TYPE_F32: return 1;
    case ORC_TYPE_Q4_0: case ORC_TYPE_Q8_0: case ORC_TYPE_Q8_1: return 32;
    case ORC_TYPE_Q4_K: case ORC_TYPE_Q5_K: case ORC_TYPE_Q6_K: case ORC_TYPE_Q8_K: case ORC_TYPE_IQ4_XS: return QK_K;
    default: return 0;
    }
}

size_t orc_row_size(int type, int64_t ne) {
    return orc_type_size(type) * (size_t)(ne / orc_blck_size(type));
}

/* ------------------------------------------------------------------------ */
/* fp16 conversions: src/ggml/impl.zig:770-830 (ggml-impl.h:403, 426).  The
 * bit-manipulation method is the public FP16 library's (M. Dukhan), which the
 * reference uses; restated here from that published algorithm. */

static inline float f_from_bits(uint32_t w) { float f; memcpy(&f, &w, 4); return f; }
static inline uint32_t f_to_bits(float f) { uint32_t w; memcpy(&w, &f, 4); return w; }

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t w = (uint32_t)h << 16;
    const uint32_t sign = w & 0x80000000u;
    const uint32_t two_w = w + w;
    const uint32_t exp_offset = 0xE0u << 23;
    const float exp_scale = f_from_bits(0x7800000u);
    const float normalized_value = f_from_bits((two_w >> 4) + exp_offset) * exp_scale;
    const uint32_t magic_mask = 126u << 23;
    const float magic_bias = 0.5f;
    const float denormalized_value = f_from_bits((two_w >> 17) | magic_mask) - magic_bias;
    const uint32_t denormalized_cutoff = 1u << 27;
    const uint32_t result = sign | (two_w < denormalized_cutoff ? f_to_bits(denormalized_value)
                                                                : f_to_bits(normalized_value));
    return f_from_bits(result);
}

uint16_t orc_fp32_to_fp16(float f) {
    const float scale_to_inf = f_from_bits(0x77800000u);
    const float scale_to_zero = f_from_bits(0x08800000u);
    float base = (fabsf(f) * scale_to_inf) * scale_to_zero;
    const uint32_t w = f_to_bits(f);
    const uint32_t shl1_w = w + w;
    const uint32_t sign = w & 0x80000000u;
    uint32_t bias = shl1_w & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base = f_from_bits((bias >> 1) + 0x07800000u) + base;
    const uint32_t bits = f_to_bits(base);
    const uint32_t exp_bits = (bits >> 13) & 0x00007C00u;
    const uint32_t mantissa_bits = bits & 0x00000FFFu;
    const uint32_t nonsign = exp_bits + mantissa_bits;
    return (uint16_t)((sign >> 16) | (shl1_w > 0xFF000000u ? 0x7E00u : nonsign));
}

#define FP16(x) orc_fp32_to_fp16(x)
#define F32(h) orc_fp16_to_fp32(h)

uint64_t orc_fnv1a(const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; ++i) { h ^= b[i]; h *= 0x100000001b3ull; }
    return h;
}

/* ------------------------------------------------------------------------ */
/* Scale fitting: src/ggml/quants/helpers.zig */

/* nearestInt, helpers.zig:99-104: round half to even via the 1.5*2^23 trick. */
int orc_nearest_int(float fval) {
    const float val = fval + 12582912.0f;
    int32_t i; memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}
#define nearest_int orc_nearest_int

static const float GROUP_MAX_EPS = 1e-15f; /* helpers.zig:79 */

/* C float -> integer cast with the reference's clamp (impl.zig:744-752). */
static inline int8_t trunc_i8(float f) {
    const float t = truncf(f);
    if (isnan(t)) return 0;
    if (t <= -128.0f) return -128;
    if (t >= 127.0f) return 127;
    return (int8_t)t;
}

/* makeQxQuants, helpers.zig:125-203 (rmse_type 1 or imatrix weights). */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *L, int rmse_type,
                            const float *qw) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            L[i] = (int8_t)(nmax + l);
        }
        return 1 / iscale;
    }
    int return_early = 0;
    if (rmse_type < 0) { rmse_type = -rmse_type; return_early = 1; }
#define QX_W(i) (qw ? qw[i] : (rmse_type == 1 ? x[i] * x[i] : rmse_type == 2 ? 1.0f : rmse_type == 3 ? fabsf(x[i]) : sqrtf(fabsf(x[i]))))
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float w = QX_W(i);
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0 ? sumlx / suml2 : 0.0f;
    if (return_early) return suml2 > 0 ? 0.5f * (scale + 1 / iscale) : 1 / iscale;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = QX_W(i);
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
#undef QX_W
    return scale;
}

/* makeQkx2Quants, helpers.zig:307-405. */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L,
                              float *the_min, uint8_t *Laux, float rmin, float rdelta, int nstep,
                              int use_mad) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = (float)nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : (l > nmax ? nmax : l));
        float diff = scale * (float)L[i] + min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) { *the_min = -min; return scale; }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            const float v = iscale * (x[i] - min);
            const float nmax_f = (float)nmax;
            const int l = v > 0 ? nearest_int(v < nmax_f ? v : nmax_f) : 0;
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            const float lf = (float)l;
            sum_l += w * lf;
            sum_l2 += w * lf * lf;
            sum_xl += w * lf * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) { this_min = 0; this_scale = sum_xl / sum_l2; }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = use_mad ? fabsf(diff) : diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* makeQkx3Quants, helpers.zig:420-510 (weights always given on this path). */
static float make_qkx3_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L,
                              float *the_min, uint8_t *Laux, float rmin, float rdelta, int nstep,
                              int use_mad) {
#define X3_W(i) (weights ? weights[i] : x[i] * x[i])
    float min = x[0], max = x[0];
    float sum_w = X3_W(0);
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = X3_W(i);
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max <= min) {
        memset(L, 0, (size_t)n);
        *the_min = -min;
        return 0.0f;
    }
    float iscale = (float)nmax / (max - min);
    float scale = 1 / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : (l > nmax ? nmax : l));
        float diff = scale * (float)L[i] + min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best_mad += X3_W(i) * diff;
    }
    if (nstep < 1) { *the_min = -min; return scale; }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            const float w = X3_W(i);
            const float lf = (float)l;
            sum_l += w * lf;
            sum_l2 += w * lf * lf;
            sum_xl += w * lf * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) { this_min = 0; this_scale = sum_xl / sum_l2; }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = use_mad ? fabsf(diff) : diff * diff;
                mad += X3_W(i) * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
#undef X3_W
    *the_min = -min;
    return scale;
}

/* makeQpQuants, helpers.zig:525-610. */
static float make_qp_quants(int n, int nmax, const float *x, uint8_t *L, const float *quant_weights) {
    float max = 0;
    for (int i = 0; i < n; ++i) max = x[i] > max ? x[i] : max;
    if (max < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = (float)nmax / max;
    for (int i = 0; i < n; ++i) L[i] = (uint8_t)(uint32_t)nearest_int(iscale * x[i]);
    const float scale = 1 / iscale;
    float best_mse = 0;
    for (int i = 0; i < n; ++i) {
        const float diff = x[i] - scale * (float)L[i];
        best_mse += quant_weights[i] * diff * diff;
    }
    for (int is = -4; is <= 4; ++is) {
        if (is == 0) continue;
        const float iscale_is = (0.1f * (float)is + (float)nmax) / max;
        const float scale_is = 1 / iscale_is;
        float mse = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale_is * x[i]);
            l = l < nmax ? l : nmax;
            const float diff = x[i] - scale_is * (float)l;
            mse += quant_weights[i] * diff * diff;
        }
        if (mse < best_mse) { best_mse = mse; iscale = iscale_is; }
    }
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < nmax ? l : nmax;
        L[i] = (uint8_t)(uint32_t)l;
        const float w = quant_weights[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    for (int itry = 0; itry < 5; ++itry) {
        int n_changed = 0;
        for (int i = 0; i < n; ++i) {
            const float w = quant_weights[i];
            float slx = sumlx - w * x[i] * (float)L[i];
            float sl2 = suml2 - w * (float)L[i] * (float)L[i];
            if (slx > 0 && sl2 > 0) {
                int new_l = nearest_int(x[i] * sl2 / slx);
                new_l = new_l < nmax ? new_l : nmax;
                if (new_l != (int)L[i]) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = (uint8_t)(uint32_t)new_l;
                        sumlx = slx;
                        suml2 = sl2;
                        ++n_changed;
                    }
                }
            }
        }
        if (!n_changed) break;
    }
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

/* getScaleMinK4, helpers.zig:621-629. */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* Q4_K: src/ggml/quants/k.zig:330-470 */

/* packScalesK / packScalePair, k.zig:372-390, chunks.zig:614-624. */
static inline void pack_scale_pair(uint8_t *s, int j, uint8_t ls, uint8_t lm) {
    if (j < 4) {
        s[j] = ls;
        s[j + 4] = lm;
    } else {
        s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        s[j - 4] |= (uint8_t)((ls >> 4) << 6);
        s[j - 0] |= (uint8_t)((lm >> 4) << 6);
    }
}

/* The body quantize_row_q4_K_ref and quantize_row_q5_K_ref share
 * (k.zig:331-390 fitScalesK + packScalesK, then the levels against the
 * rounded scales, :393-434 and :472-535): nmax 15, rmin -1, 20 steps for
 * q4_K; nmax 31, rmin -0.5, 15 steps for q5_K.  Leaves d, dmin, the packed
 * scales and the per-weight levels L. */
static void k45_ref_levels(const float *x, int nmax, float rmin, int nstep, uint16_t *d_out, uint16_t *dmin_out,
                           uint8_t *scales_out, uint8_t L[QK_K]) {
    uint8_t Laux[32];
    float mins[QK_K / 32], scales[QK_K / 32], weights[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < QK_K / 32; ++j) {           /* fitScalesK, k.zig:338-363 */
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, rmin, 0.1f, nstep, 0);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    memset(scales_out, 0, K_SCALE_SIZE);
    const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < QK_K / 32; ++j) {
        uint8_t ls = (uint8_t)(uint32_t)nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)(uint32_t)nearest_int(inv_min * mins[j]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        pack_scale_pair(scales_out, j, ls, lm);
    }
    *d_out = FP16(max_scale / 63.0f);
    *dmin_out = FP16(max_min / 63.0f);
    for (int j = 0; j < QK_K / 32; ++j) {
        uint8_t sc, m;
        get_scale_min_k4(j, scales_out, &sc, &m);
        const float d = F32(*d_out) * (float)sc;
        if (d == 0) continue;
        const float dm = F32(*dmin_out) * (float)m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            L[32 * j + ii] = (uint8_t)l;
        }
    }
}

/* q4_K: level j and j+32 of each 64-weight span share a byte (k.zig:426-431). */
static void pack_q4_levels(const uint8_t L[QK_K], uint8_t *q) {
    for (int j = 0; j < QK_K; j += 64) {
        for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
        q += 32;
    }
}

/* q5_K: the low four bits as q4_K, the fifth in qh, two bits per 64-weight
 * span (k.zig:508-532; chunks.zig:586-609). */
static void pack_q5_levels(const uint8_t L[QK_K], uint8_t *qh, uint8_t *ql) {
    memset(qh, 0, QK_K / 8);
    uint8_t m1 = 1, m2 = 2;
    for (int n = 0; n < QK_K; n += 64) {
        for (int j = 0; j < 32; ++j) {
            int l1 = L[n + j];
            if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
            int l2 = L[n + j + 32];
            if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
            ql[j] = (uint8_t)(l1 | (l2 << 4));
        }
        m1 = (uint8_t)(m1 << 2);
        m2 = (uint8_t)(m2 << 2);
        ql += 32;
    }
}

void orc_quantize_row_q4_K_ref(const float *x, void *vy, int64_t k) {
    blk_q4_K *y = (blk_q4_K *)vy;
    uint8_t L[QK_K];
    for (int64_t i = 0; i < k / QK_K; ++i) {
        k45_ref_levels(x, 15, -1.0f, 20, &y[i].d, &y[i].dmin, y[i].scales, L);
        pack_q4_levels(L, y[i].qs);
        x += QK_K;
    }
}

/* quantize_row_q5_K_ref, k.zig:472-535. */
void orc_quantize_row_q5_K_ref(const float *x, void *vy, int64_t k) {
    blk_q5_K *y = (blk_q5_K *)vy;
    uint8_t L[QK_K];
    for (int64_t i = 0; i < k / QK_K; ++i) {
        k45_ref_levels(x, 31, -0.5f, 15, &y[i].d, &y[i].dmin, y[i].scales, L);
        pack_q5_levels(L, y[i].qh, y[i].qs);
        x += QK_K;
    }
}

void orc_dequantize_row_q4_K(const void *vx, float *y, int64_t k) {
    const blk_q4_K *x = (const blk_q4_K *)vx;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t *q = x[i].qs;
        const float d = F32(x[i].d);
        const float min = F32(x[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = min * (float)m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = min * (float)m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* dequantize_row_q5_K, k.zig:538-575. */
void orc_dequantize_row_q5_K(const void *vx, float *y, int64_t k) {
    const blk_q5_K *x = (const blk_q5_K *)vx;
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const uint8_t *ql = x[i].qs, *qh = x[i].qh;
        const float d = F32(x[i].d), min = F32(x[i].dmin);
        int is = 0;
        uint8_t sc, m, u1 = 1, u2 = 2;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = min * (float)m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = min * (float)m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (float)((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (float)((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
            ql += 32;
            is += 2;
            u1 = (uint8_t)(u1 << 2);
            u2 = (uint8_t)(u2 << 2);
        }
    }
}

/* quantize_row_q{4,5}_K_impl with imatrix: chunks.zig:478-626
 * (fitScalesKImpl, q4_KImpl / q5_KImpl, requantizeK).  q5_K clamps the packed
 * levels to 63 where q4_K does not (chunks.zig:535-538 vs 572-575). */
static void k45_impl_levels(const float *x, int64_t i, const float *qw_all, int nmax, int clamp63,
                            uint16_t *d_out, uint16_t *dmin_out, uint8_t *scales_out, uint8_t L[QK_K]) {
    uint8_t Laux[32], ls[QK_K / 32], lm[QK_K / 32];
    float sw[QK_K / 32], mins[QK_K / 32], scales[QK_K / 32], weights[32];
    float sum_x2 = 0;
    for (int l = 0; l < QK_K; ++l) sum_x2 += x[l] * x[l];
    const float sigma2 = 2 * sum_x2 / QK_K;
    const float av_x = sqrtf(sigma2);
    for (int j = 0; j < QK_K / 32; ++j) {
        if (qw_all) {
            const float *qw = qw_all + QK_K * i + 32 * j;
            for (int l = 0; l < 32; ++l) weights[l] = qw[l] * sqrtf(sigma2 + x[32 * j + l] * x[32 * j + l]);
        } else {
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        }
        float sumw = 0;
        for (int l = 0; l < 32; ++l) sumw += weights[l];
        sw[j] = sumw;
        scales[j] = make_qkx3_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.9f, 0.05f, 36, 0);
    }
    const float d_block = make_qp_quants(QK_K / 32, 63, scales, ls, sw);
    const float m_block = make_qp_quants(QK_K / 32, 63, mins, lm, sw);
    memset(scales_out, 0, K_SCALE_SIZE);
    for (int j = 0; j < QK_K / 32; ++j) {
        const uint8_t a = clamp63 && ls[j] > 63 ? 63 : ls[j], b = clamp63 && lm[j] > 63 ? 63 : lm[j];
        pack_scale_pair(scales_out, j, a, b);
    }
    *d_out = FP16(d_block);
    *dmin_out = FP16(m_block);
    const float d_all = F32(*d_out), dmin_all = F32(*dmin_out);
    for (int j = 0; j < QK_K / 32; ++j) {            /* requantizeK */
        uint8_t sc, m;
        get_scale_min_k4(j, scales_out, &sc, &m);
        const float d = d_all * (float)sc;
        if (d == 0) continue;
        const float dm = dmin_all * (float)m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            L[32 * j + ii] = (uint8_t)l;
        }
    }
}

static void q4_K_impl(const float *x, blk_q4_K *y, int64_t n_per_row, const float *qw_all) {
    uint8_t L[QK_K];
    for (int64_t i = 0; i < n_per_row / QK_K; ++i) {
        k45_impl_levels(x, i, qw_all, 15, 0, &y[i].d, &y[i].dmin, y[i].scales, L);
        pack_q4_levels(L, y[i].qs);
        x += QK_K;
    }
}

static void q5_K_impl(const float *x, blk_q5_K *y, int64_t n_per_row, const float *qw_all) {
    uint8_t L[QK_K];
    for (int64_t i = 0; i < n_per_row / QK_K; ++i) {
        k45_impl_levels(x, i, qw_all, 31, 1, &y[i].d, &y[i].dmin, y[i].scales, L);
        pack_q5_levels(L, y[i].qh, y[i].qs);
        x += QK_K;
    }
}

/* ------------------------------------------------------------------------ */
/* Q6_K: k.zig:585-696, chunks.zig:642-712 */

static void q6_K_common(const float *x, blk_q6_K *y, int64_t k, const float *qw_all) {
    const int64_t nb = k / QK_K;
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < nb; ++i) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, 1,
                                               qw_all ? qw_all + QK_K * i + 16 * ib : NULL);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) { max_abs_scale = abs_scale; max_scale = scale; }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            memset(&y[i], 0, sizeof(blk_q6_K));
            y[i].d = FP16(0.0f);
            x += QK_K;
            continue;
        }
        const float iscale = -128.0f / max_scale;
        y[i].d = FP16(1 / iscale);
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const int v = nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            const float d = F32(y[i].d) * (float)y[i].scales[j];
            if (d == 0) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = y[i].ql, *qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = (uint8_t)L[j + l + 0] & 0xF;
                const uint8_t q2 = (uint8_t)L[j + l + 32] & 0xF;
                const uint8_t q3 = (uint8_t)L[j + l + 64] & 0xF;
                const uint8_t q4 = (uint8_t)L[j + l + 96] & 0xF;
                ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)(((uint8_t)L[j + l] >> 4) | (((uint8_t)L[j + l + 32] >> 4) << 2) |
                                  (((uint8_t)L[j + l + 64] >> 4) << 4) | (((uint8_t)L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += QK_K;
    }
}

void orc_quantize_row_q6_K_ref(const float *x, void *y, int64_t k) { q6_K_common(x, (blk_q6_K *)y, k, NULL); }

void orc_dequantize_row_q6_K(const void *vx, float *y, int64_t k) {
    const blk_q6_K *x = (const blk_q6_K *)vx;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = F32(x[i].d);
        const uint8_t *ql = x[i].ql, *qh = x[i].qh;
        const int8_t *sc = x[i].scales;
        for (int n = 0; n < QK_K; n += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * (float)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_0 / Q8_1: src/ggml/quants/legacy.zig:407-484 */

/* quantize_row_q4_0_ref, legacy.zig:151-184: d = max / -8 (max the element of
 * largest magnitude, with its sign), q = min(15, trunc-narrow(x / d + 8.5));
 * element j and j + 16 share byte j. */
void orc_quantize_row_q4_0_ref(const float *x, void *vy, int64_t k) {
    blk_q4_0 *y = (blk_q4_0 *)vy;
    for (int64_t i = 0; i < k / 32; ++i) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = x[i * 32 + j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = FP16(d);
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[i * 32 + j] * id, x1 = x[i * 32 + 16 + j] * id;
            int xi0 = trunc_i8(x0 + 8.5f), xi1 = trunc_i8(x1 + 8.5f);
            xi0 = xi0 < 15 ? xi0 : 15;
            xi1 = xi1 < 15 ? xi1 : 15;
            y[i].qs[j] = (uint8_t)((uint8_t)xi0 | ((uint8_t)xi1 << 4));
        }
    }
}

/* dequantize_row_q4_0, legacy.zig:187-202. */
void orc_dequantize_row_q4_0(const void *vx, float *y, int64_t k) {
    const blk_q4_0 *x = (const blk_q4_0 *)vx;
    for (int64_t i = 0; i < k / 32; ++i) {
        const float d = F32(x[i].d);
        for (int j = 0; j < 16; ++j) {
            y[i * 32 + j] = (float)((x[i].qs[j] & 0x0F) - 8) * d;
            y[i * 32 + j + 16] = (float)((x[i].qs[j] >> 4) - 8) * d;
        }
    }
}

/* quantize_row_q4_0_impl with an imatrix, chunks.zig:164-186: weights
 * qw * sqrt(sigma2 + x^2) with sigma2 = mean x^2 over the row, levels from
 * makeQxQuants(32, 8, ..., rmse_type 1). */
static void q4_0_impl(const float *x, blk_q4_0 *y, int64_t n_per_row, const float *qw_all) {
    float weight[32];
    int8_t L[32];
    float sum_x2 = 0;
    for (int64_t j = 0; j < n_per_row; ++j) sum_x2 += x[j] * x[j];
    const float sigma2 = sum_x2 / (float)n_per_row;
    for (int64_t ib = 0; ib < n_per_row / 32; ++ib) {
        const float *xb = x + 32 * ib, *qw = qw_all + 32 * ib;
        for (int j = 0; j < 32; ++j) weight[j] = qw[j] * sqrtf(sigma2 + xb[j] * xb[j]);
        const float d = make_qx_quants(32, 8, xb, L, 1, weight);
        y[ib].d = FP16(d);
        for (int j = 0; j < 16; ++j) y[ib].qs[j] = (uint8_t)((uint8_t)L[j] | ((uint8_t)L[j + 16] << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* IQ4_XS: src/ggml/quants/iq4.zig, iq_dequant.zig:360-381. */

/* The format's 16 non-linear levels (kvalues_iq4nl, ggml-common.h, which the
 * reference reaches through @cImport, iq4.zig:12-14); dense near zero. */
static const int8_t KV_IQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* best_index_iq4nl, iq4.zig:31-40: 15 minus the midpoints x lies below, so a
 * tie goes to the higher level. */
static inline int best_index_iq4nl(const float *mid, float x) {
    int l = 15;
    for (int k = 0; k < 15; ++k) l -= x < mid[k];
    return l;
}

/* quantize_row_iq4_nl_impl for IQ4_XS (iq4.zig:60-194): super-block 256,
 * sub-blocks of 32, ntry 7.  Per sub-block: weights x^2 (or qw * sqrt(sigma2 +
 * x^2)), a least-squares scale over 16 candidate inverse scales, then a 6-bit
 * scale l = nearest(scale / d) in [-32, 31] against d = -max_scale / 32 and
 * the levels requantized with the rounded scale; stored as l + 32, four bits
 * in scales_l and two in scales_h. */
static void iq4_xs_block(const float *x, blk_iq4_xs *y, const float *qw_all) {
    const int ntry = 7, nt = 2 * ntry + 2;
    float sigma2 = 0;
    for (int j = 0; j < QK_K; ++j) sigma2 += x[j] * x[j];
    sigma2 *= 2.0f / (float)QK_K;
    memset(y->qs, 0, sizeof y->qs);
    float mid[15], fval[16];
    for (int k = 0; k < 15; ++k) mid[k] = 0.5f * (float)((int)KV_IQ4NL[k] + KV_IQ4NL[k + 1]);
    for (int k = 0; k < 16; ++k) fval[k] = (float)KV_IQ4NL[k];
    float scales[QK_K / 32], weight[32];
    uint8_t L[QK_K];
    memset(L, 0, sizeof L);
    float max_scale = 0, amax_scale = 0;
    for (int ib = 0; ib < QK_K / 32; ++ib) {
        const float *xb = x + 32 * ib;
        if (qw_all) {
            const float *qw = qw_all + 32 * ib;
            for (int j = 0; j < 32; ++j) weight[j] = qw[j] * sqrtf(sigma2 + xb[j] * xb[j]);
        } else {
            for (int j = 0; j < 32; ++j) weight[j] = xb[j] * xb[j];
        }
        float amax = 0, max = 0;
        for (int j = 0; j < 32; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (amax < GROUP_MAX_EPS) {
            scales[ib] = 0;
            continue;
        }
        float d = -max / (float)KV_IQ4NL[0];
        float idt[16], sqx[16], sq2[16];
        idt[0] = 1 / d;
        for (int lane = 1; lane < nt; ++lane) idt[lane] = (float)(lane - 1 - ntry + KV_IQ4NL[0]) / max;
        for (int lane = 0; lane < nt; ++lane) sqx[lane] = sq2[lane] = 0;
        for (int j = 0; j < 32; ++j) {
            const float w = weight[j];
            for (int lane = 0; lane < nt; ++lane) {
                const float q = fval[best_index_iq4nl(mid, idt[lane] * xb[j])];
                sqx[lane] += w * q * xb[j];
                sq2[lane] += w * q * q;
            }
        }
        d = sq2[0] > 0 ? sqx[0] / sq2[0] : 0.0f;
        float best = d * sqx[0];
        for (int lane = 1; lane < nt; ++lane)
            if (sq2[lane] > 0 && sqx[lane] * sqx[lane] > best * sq2[lane]) {
                d = sqx[lane] / sq2[lane];
                best = d * sqx[lane];
            }
        scales[ib] = d;
        if (fabsf(d) > amax_scale) {
            amax_scale = fabsf(d);
            max_scale = d;
        }
    }
    y->scales_h = 0;
    const float d = -max_scale / 32;
    y->d = FP16(d);
    const float id = d != 0 ? 1 / d : 0.0f;
    for (int ib = 0; ib < QK_K / 32; ++ib) {
        int l = nearest_int(id * scales[ib]);
        l = l < -32 ? -32 : (l > 31 ? 31 : l);
        const float dl = d * (float)l;
        const float idl = dl != 0 ? 1 / dl : 0.0f;
        for (int j = 0; j < 32; ++j) L[32 * ib + j] = (uint8_t)best_index_iq4nl(mid, idl * x[32 * ib + j]);
        l += 32;
        const uint8_t l_l = (uint8_t)(l & 0xf), l_h = (uint8_t)(l >> 4);
        if (ib % 2 == 0) y->scales_l[ib / 2] = l_l;
        else y->scales_l[ib / 2] |= (uint8_t)(l_l << 4);
        y->scales_h |= (uint16_t)(l_h << (2 * (ib % 8)));
    }
    for (int i = 0; i < QK_K / 32; ++i)
        for (int j = 0; j < 16; ++j) y->qs[16 * i + j] = (uint8_t)(L[32 * i + j] | (L[32 * i + 16 + j] << 4));
}

/* quantize_iq4_xs (iq4.zig:283-325) row by row; quantize_row_iq4_xs_ref is
 * the same without an imatrix (iq4.zig:327-330). */
static void iq4_xs_rows(const float *x, uint8_t *y, int64_t nrows, int64_t n_per_row, const float *qw) {
    const int64_t nb = n_per_row / QK_K;
    for (int64_t r = 0; r < nrows; ++r) {
        blk_iq4_xs *row = (blk_iq4_xs *)(y + (size_t)r * (size_t)nb * sizeof(blk_iq4_xs));
        for (int64_t i = 0; i < nb; ++i)
            iq4_xs_block(x + r * n_per_row + i * QK_K, &row[i], qw ? qw + i * QK_K : NULL);
    }
}

void orc_quantize_row_iq4_xs_ref(const float *x, void *vy, int64_t k) { iq4_xs_rows(x, (uint8_t *)vy, 1, k, NULL); }

/* dequantize_row_iq4_xs, iq_dequant.zig:360-381: w = d * (ls - 32) * level. */
void orc_dequantize_row_iq4_xs(const void *vx, float *y, int64_t k) {
    const blk_iq4_xs *x = (const blk_iq4_xs *)vx;
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const float d = F32(x[i].d);
        for (int ib = 0; ib < QK_K / 32; ++ib) {
            const int ls = ((x[i].scales_l[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((x[i].scales_h >> (2 * ib)) & 3) << 4);
            const float dl = d * (float)(ls - 32);
            const uint8_t *qs = x[i].qs + 16 * ib;
            for (int j = 0; j < 16; ++j) {
                y[j] = dl * (float)KV_IQ4NL[qs[j] & 0xf];
                y[j + 16] = dl * (float)KV_IQ4NL[qs[j] >> 4];
            }
            y += 32;
        }
    }
}

/* the 6-bit scale of sub-block ib, l + 32 */
static inline int iq4_xs_ls(const blk_iq4_xs *x, int ib) {
    return ((x->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((x->scales_h >> (2 * ib)) & 3) << 4);
}

void orc_quantize_row_q8_0_ref(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; ++j) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / (float)((1 << 7) - 1);
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = FP16(d);
        for (int j = 0; j < QK8_0; ++j) y[i].qs[j] = trunc_i8(roundf(x[i * QK8_0 + j] * id));
    }
}

void orc_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
    const blk_q8_0 *x = (const blk_q8_0 *)vx;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = F32(x[i].d);
        for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = (float)x[i].qs[j] * d;
    }
}

void orc_quantize_row_q8_1_ref(const float *x, void *vy, int64_t k) {
    blk_q8_1 *y = (blk_q8_1 *)vy;
    const int64_t nb = k / QK8_1;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_1; ++j) amax = fmaxf(amax, fabsf(x[i * QK8_1 + j]));
        const float d = amax / (float)((1 << 7) - 1);
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = FP16(d);
        int sum = 0;
        for (int j = 0; j < QK8_1 / 2; ++j) {
            const float v0 = x[i * QK8_1 + j] * id;
            const float v1 = x[i * QK8_1 + QK8_1 / 2 + j] * id;
            y[i].qs[j] = trunc_i8(roundf(v0));
            y[i].qs[QK8_1 / 2 + j] = trunc_i8(roundf(v1));
            sum += y[i].qs[j];
            sum += y[i].qs[QK8_1 / 2 + j];
        }
        y[i].s = FP16((float)sum * d);
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_K: k.zig:710-760 */

void orc_quantize_row_q8_K_ref(const float *x, void *vy, int64_t k) {
    blk_q8_K *y = (blk_q8_K *)vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        if (amax == 0) {
            /* bsums left untouched, as the reference does (k.zig:727-733) */
            y[i].d = 0;
            memset(y[i].qs, 0, QK_K);
            x += QK_K;
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; ++j) {
            const int v = nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1 / iscale;
        x += QK_K;
    }
}

void orc_dequantize_row_q8_K(const void *vx, float *y, int64_t k) {
    const blk_q8_K *x = (const blk_q8_K *)vx;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i)
        for (int j = 0; j < QK_K; ++j) *y++ = x[i].d * (float)x[i].qs[j];
}

/* ggml_quantize_chunk for the three weight types (chunks.zig:99-128, 289-305,
 * 716-724): without an imatrix the whole buffer goes through the reference
 * quantizer; with one, q4_K / q6_K run their impls row by row.  q8_0 ignores it. */
size_t orc_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows,
                          int64_t n_per_row, const float *imatrix) {
    const size_t row_size = orc_row_size(type, n_per_row);
    const int64_t start_row = start / n_per_row;
    uint8_t *out = (uint8_t *)dst + (size_t)start_row * row_size;
    src += start;
    switch (type) {
    case ORC_TYPE_Q4_0:
        if (!imatrix) orc_quantize_row_q4_0_ref(src, out, nrows * n_per_row);
        else for (int64_t r = 0; r < nrows; ++r)
            q4_0_impl(src + r * n_per_row, (blk_q4_0 *)(out + (size_t)r * row_size), n_per_row, imatrix);
        break;
    case ORC_TYPE_Q8_0:
        orc_quantize_row_q8_0_ref(src, out, nrows * n_per_row);
        break;
    case ORC_TYPE_IQ4_XS:
        iq4_xs_rows(src, out, nrows, n_per_row, imatrix);
        break;
    case ORC_TYPE_Q4_K:
        if (!imatrix) orc_quantize_row_q4_K_ref(src, out, nrows * n_per_row);
        else for (int64_t r = 0; r < nrows; ++r)
            q4_K_impl(src + r * n_per_row, (blk_q4_K *)(out + (size_t)r * row_size), n_per_row, imatrix);
        break;
    case ORC_TYPE_Q5_K:
        if (!imatrix) orc_quantize_row_q5_K_ref(src, out, nrows * n_per_row);
        else for (int64_t r = 0; r < nrows; ++r)
            q5_K_impl(src + r * n_per_row, (blk_q5_K *)(out + (size_t)r * row_size), n_per_row, imatrix);
        break;
    case ORC_TYPE_Q6_K:
        if (!imatrix) orc_quantize_row_q6_K_ref(src, out, nrows * n_per_row);
        else for (int64_t r = 0; r < nrows; ++r)
            q6_K_common(src + r * n_per_row, (blk_q6_K *)(out + (size_t)r * row_size), n_per_row, imatrix);
        break;
    default:
        return 0;
    }
    return (size_t)nrows * row_size;
}

/* ------------------------------------------------------------------------ */
/* Generic dot products: src/ggml/cpu/quants/k.zig:146-177, 269-353, 377-438;
 * cpu/quants/legacy.zig:563-599. */

typedef struct {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    int32_t aux32[8];
    float sums[8]; /* not reset between super-blocks */
} dot_scratch;

static inline void scratch_accumulate(dot_scratch *s, int32_t scale, const int8_t *q8, const int8_t *a) {
    for (int l = 0; l < 8; ++l) s->aux16[l] = (int16_t)(q8[l] * a[l]);
    for (int l = 0; l < 8; ++l) s->aux32[l] += scale * s->aux16[l];
}

/* The body ggml_vec_dot_q4_K_q8_K_generic and _q5_K_ share (k.zig:262-353):
 * q5_K adds 16 to a level whose qh bit is set.  `x` walks blocks of `bsize`
 * bytes laid out as {d, dmin, scales[12], [qh[32]], qs[128]}. */
static float vec_dot_q45_K_q8_K_generic(int n, const uint8_t *x, size_t bsize, int q5, const void *vy) {
    const blk_q8_K *y = (const blk_q8_K *)vy;
    const int nb = n / QK_K;
    dot_scratch sc;
    memset(&sc, 0, sizeof sc);
    float sumf = 0;
    for (int i = 0; i < nb; ++i, x += bsize) {
        uint16_t xd, xdmin;
        memcpy(&xd, x, 2);
        memcpy(&xdmin, x + 2, 2);
        const uint8_t *scales_p = x + 4;
        const uint8_t *qh = q5 ? x + 16 : NULL;
        const uint8_t *qs = x + (q5 ? 48 : 16);
        memset(sc.aux32, 0, sizeof sc.aux32);
        int a = 0, q4 = 0;
        uint8_t m = 1;
        for (int c = 0; c < QK_K / 64; ++c) {
            for (int l = 0; l < 32; ++l) sc.aux8[a + l] = (int8_t)(qs[q4 + l] & 0xF);
            if (q5) {
                for (int l = 0; l < 32; ++l) sc.aux8[a + l] = (int8_t)(sc.aux8[a + l] + (qh[l] & m ? 16 : 0));
                m = (uint8_t)(m << 1);
            }
            a += 32;
            for (int l = 0; l < 32; ++l) sc.aux8[a + l] = (int8_t)(qs[q4 + l] >> 4);
            if (q5) {
                for (int l = 0; l < 32; ++l) sc.aux8[a + l] = (int8_t)(sc.aux8[a + l] + (qh[l] & m ? 16 : 0));
                m = (uint8_t)(m << 1);
            }
            a += 32;
            q4 += 32;
        }
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4(j, scales_p, &scales[j], &mins[j]);
        int32_t sumi = 0;
        for (int j = 0; j < QK_K / 16; ++j) sumi += (int32_t)y[i].bsums[j] * mins[j / 2];
        a = 0;
        int q8 = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            const int32_t scale = scales[j];
            for (int l = 0; l < 4; ++l) { scratch_accumulate(&sc, scale, y[i].qs + q8, sc.aux8 + a); q8 += 8; a += 8; }
        }
        const float d = F32(xd) * y[i].d;
        for (int l = 0; l < 8; ++l) sc.sums[l] += d * (float)sc.aux32[l];
        const float dmin = F32(xdmin) * y[i].d;
        sumf -= dmin * (float)sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sc.sums[l];
    return sumf;
}

static float vec_dot_q4_K_q8_K_generic(int n, const void *vx, const void *vy) {
    return vec_dot_q45_K_q8_K_generic(n, (const uint8_t *)vx, sizeof(blk_q4_K), 0, vy);
}

/* ggml_vec_dot_q5_K_q8_K_generic, k.zig:355-375. */
static float vec_dot_q5_K_q8_K_generic(int n, const void *vx, const void *vy) {
    return vec_dot_q45_K_q8_K_generic(n, (const uint8_t *)vx, sizeof(blk_q5_K), 1, vy);
}

static float vec_dot_q6_K_q8_K_generic(int n, const void *vx, const void *vy) {
    const blk_q6_K *x = (const blk_q6_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    const int nb = n / QK_K;
    dot_scratch sc;
    memset(&sc, 0, sizeof sc);
    for (int i = 0; i < nb; ++i) {
        memset(sc.aux32, 0, sizeof sc.aux32);
        int a = 0, q4 = 0, qh = 0;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t h = x[i].qh[qh + l];
                sc.aux8[a + l + 0] = (int8_t)((x[i].ql[q4 + l + 0] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
                sc.aux8[a + l + 32] = (int8_t)((x[i].ql[q4 + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
                sc.aux8[a + l + 64] = (int8_t)((x[i].ql[q4 + l + 0] >> 4) | (((h >> 4) & 3) << 4)) - 32;
                sc.aux8[a + l + 96] = (int8_t)((x[i].ql[q4 + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
            }
            a += 128;
            q4 += 64;
            qh += 32;
        }
        a = 0;
        int q8 = 0;
        for (int is = 0; is < QK_K / 16; ++is) {
            const int32_t scale = x[i].scales[is];
            scratch_accumulate(&sc, scale, y[i].qs + q8, sc.aux8 + a); q8 += 8; a += 8;
            scratch_accumulate(&sc, scale, y[i].qs + q8, sc.aux8 + a); q8 += 8; a += 8;
        }
        const float d = F32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sc.sums[l] += d * (float)sc.aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sc.sums[l];
    return sumf;
}

/* ggml_vec_dot_q4_0_q8_0_generic, cpu/quants/legacy.zig:174-212. */
static float vec_dot_q4_0_q8_0_generic(int n, const void *vx, const void *vy) {
    const blk_q4_0 *x = (const blk_q4_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float sumf = 0;
    for (int ib = 0; ib < n / 32; ++ib) {
        int32_t sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < 16; ++j) {
            const int32_t v0 = (int32_t)(x[ib].qs[j] & 0x0F) - 8, v1 = (int32_t)(x[ib].qs[j] >> 4) - 8;
            sumi0 += v0 * y[ib].qs[j];
            sumi1 += v1 * y[ib].qs[j + 16];
        }
        const int32_t sumi = sumi0 + sumi1;
        sumf += (float)sumi * F32(x[ib].d) * F32(y[ib].d);
    }
    return sumf;
}

/* ggml_vec_dot_iq4_xs_q8_K_generic, cpu/quants/iq.zig:526-578: sub-blocks in
 * pairs, scales from scales_l and two bits of scales_h each. */
static float vec_dot_iq4_xs_q8_K_generic(int n, const void *vx, const void *vy) {
    const blk_iq4_xs *x = (const blk_iq4_xs *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float sumf = 0;
    for (int ibl = 0; ibl < n / QK_K; ++ibl) {
        const float d4d8 = F32(x[ibl].d) * y[ibl].d;
        uint16_t h = x[ibl].scales_h;
        int qs = 0, q8 = 0;
        for (int ib = 0; ib < QK_K / 32; ib += 2) {
            const uint8_t sl = x[ibl].scales_l[ib / 2];
            const uint8_t ls1 = (uint8_t)((sl & 0xf) | ((h << 4) & 0x30));
            const uint8_t ls2 = (uint8_t)((sl >> 4) | ((h << 2) & 0x30));
            h >>= 4;
            const float d1 = d4d8 * (float)((int)ls1 - 32);
            const float d2 = d4d8 * (float)((int)ls2 - 32);
            for (int pass = 0; pass < 2; ++pass) {
                int32_t sumi1 = 0, sumi2 = 0;
                for (int j = 0; j < 16; ++j) {
                    sumi1 += (int32_t)y[ibl].qs[q8 + j] * KV_IQ4NL[x[ibl].qs[qs + j] & 0xf];
                    sumi2 += (int32_t)y[ibl].qs[q8 + j + 16] * KV_IQ4NL[x[ibl].qs[qs + j] >> 4];
                }
                sumf += (pass == 0 ? d1 : d2) * (float)(sumi1 + sumi2);
                qs += 16;
                q8 += 32;
            }
        }
    }
    return sumf;
}

static float vec_dot_q8_0_q8_0_generic(int n, const void *vx, const void *vy) {
    const blk_q8_0 *x = (const blk_q8_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    const int nb = n / QK8_0;
    float sumf = 0;
    for (int ib = 0; ib < nb; ++ib) {
        int32_t sumi = 0;
        for (int j = 0; j < QK8_0; ++j) sumi += (int32_t)x[ib].qs[j] * y[ib].qs[j];
        sumf += (float)sumi * (F32(x[ib].d) * F32(y[ib].d));
    }
    return sumf;
}

/* ------------------------------------------------------------------------ */
/* x86 AVX2 kernels: src/ggml/cpu/quants/x86/{k,legacy,rows,common}.zig.
 * Compiled with target attributes so the file still builds for hosts without
 * AVX2; orc_has_avx2() gates their use. */
#if ORC_X86
#define AVX2_FN __attribute__((target("avx2,fma,f16c")))

/* hsum_float_8, x86/common.zig:36-42 */
AVX2_FN static inline float hsum_float_8(__m256 x) {
    __m128 res = _mm256_extractf128_ps(x, 1);
    res = _mm_add_ps(res, _mm256_castps256_ps128(x));
    res = _mm_add_ps(res, _mm_movehl_ps(res, res));
    res = _mm_add_ss(res, _mm_movehdup_ps(res));
    return _mm_cvtss_f32(res);
}

/* get_scale_shuffle_k4 (x86/common.zig:64-77): control bytes 2i,2i+1 repeated. */
AVX2_FN static inline __m256i scale_shuffle_k4(int i) {
    return _mm256_set1_epi16((short)((2 * i) | ((2 * i + 1) << 8)));
}

/* get_scale_shuffle (x86/common.zig:153-163): byte i repeated 8 times, twice (i=2r, 2r+1). */
AVX2_FN static inline __m128i scale_shuffle_q6(int i) {
    return _mm_set_epi8((char)(2 * i + 1), (char)(2 * i + 1), (char)(2 * i + 1), (char)(2 * i + 1),
                        (char)(2 * i + 1), (char)(2 * i + 1), (char)(2 * i + 1), (char)(2 * i + 1),
                        (char)(2 * i), (char)(2 * i), (char)(2 * i), (char)(2 * i),
                        (char)(2 * i), (char)(2 * i), (char)(2 * i), (char)(2 * i));
}

/* unpackScales, x86/common.zig:168-182 */
static inline void unpack_scales_k4(const uint8_t *packed, uint32_t utmp[4]) {
    const uint32_t kmask1 = 0x3f3f3f3f, kmask2 = 0x0f0f0f0f, kmask3 = 0x03030303;
    memcpy(utmp, packed, 12);
    utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
    const uint32_t uaux = utmp[1] & kmask1;
    utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
    utmp[2] = uaux;
    utmp[0] &= kmask1;
}

/* ggml_vec_dot_q4_K_q8_K AVX2 arm, x86/k.zig:256-343 */
AVX2_FN static float vec_dot_q4_K_q8_K_avx2(int n, const void *vx, const void *vy) {
    const blk_q4_K *x = (const blk_q4_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    const int nb = n / QK_K;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (int i = 0; i < nb; ++i) {
        const float d = y[i].d * F32(x[i].d);
        const float dmin = -y[i].d * F32(x[i].dmin);
        uint32_t utmp[4];
        unpack_scales_k4(x[i].scales, utmp);
        const uint8_t *q4 = x[i].qs;
        const int8_t *q8 = y[i].qs;
        const __m256i mins_and_scales = _mm256_cvtepu8_epi16(
            _mm_set_epi32((int)utmp[3], (int)utmp[2], (int)utmp[1], (int)utmp[0]));
        const __m256i q8sums = _mm256_loadu_si256((const __m256i *)y[i].bsums);
        const __m128i q8s = _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0), _mm256_extracti128_si256(q8sums, 1));
        const __m128i prod = _mm_madd_epi16(_mm256_extracti128_si256(mins_and_scales, 1), q8s);
        acc_m = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), acc_m);
        const __m128i sc128 = _mm256_extracti128_si256(mins_and_scales, 0);
        const __m256i scales = _mm256_set_m128i(sc128, sc128);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < QK_K / 64; ++j) {
            const __m256i scale_l = _mm256_shuffle_epi8(scales, scale_shuffle_k4(2 * j + 0));
            const __m256i scale_h = _mm256_shuffle_epi8(scales, scale_shuffle_k4(2 * j + 1));
            const __m256i q4bits = _mm256_loadu_si256((const __m256i *)q4); q4 += 32;
            const __m256i q4l = _mm256_and_si256(q4bits, m4);
            const __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            const __m256i q8l = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            __m256i p16l = _mm256_maddubs_epi16(q4l, q8l);
            p16l = _mm256_madd_epi16(scale_l, p16l);
            const __m256i q8h = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            __m256i p16h = _mm256_maddubs_epi16(q4h, q8h);
            p16h = _mm256_madd_epi16(scale_h, p16h);
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16l, p16h));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    acc_m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    acc_m = _mm_add_ss(acc_m, _mm_movehdup_ps(acc_m));
    return hsum_float_8(acc) + _mm_cvtss_f32(acc_m);
}

/* ggml_vec_dot_q6_K_q8_K AVX2 arm, x86/k.zig:454-552 */
AVX2_FN static float vec_dot_q6_K_q8_K_avx2(int n, const void *vx, const void *vy) {
    const blk_q6_K *x = (const blk_q6_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    const int nb = n / QK_K;
    const __m256i m3 = _mm256_set1_epi8(3);
    const __m256i m15 = _mm256_set1_epi8(15);
    __m256 acc = _mm256_setzero_ps();
    for (int i = 0; i < nb; ++i) {
        const float d = y[i].d * F32(x[i].d);
        const uint8_t *q4 = x[i].ql, *qh = x[i].qh;
        const int8_t *q8 = y[i].qs;
        const __m256i q8sums = _mm256_loadu_si256((const __m256i *)y[i].bsums);
        const __m128i scales = _mm_loadu_si128((const __m128i *)x[i].scales);
        const __m256i scales_16 = _mm256_cvtepi8_epi16(scales);
        const __m256i q8sclsub = _mm256_slli_epi32(_mm256_madd_epi16(q8sums, scales_16), 5);
        __m256i sumi = _mm256_setzero_si256();
        int is = 0;
        for (int j = 0; j < QK_K / 128; ++j) {
            const __m256i q4bits1 = _mm256_loadu_si256((const __m256i *)q4); q4 += 32;
            const __m256i q4bits2 = _mm256_loadu_si256((const __m256i *)q4); q4 += 32;
            const __m256i q4bitsH = _mm256_loadu_si256((const __m256i *)qh); qh += 32;
            const __m256i q4h_0 = _mm256_slli_epi16(_mm256_and_si256(q4bitsH, m3), 4);
            const __m256i q4h_1 = _mm256_slli_epi16(_mm256_and_si256(q4bitsH, _mm256_set1_epi8(12)), 2);
            const __m256i q4h_2 = _mm256_and_si256(q4bitsH, _mm256_set1_epi8(48));
            const __m256i q4h_3 = _mm256_srli_epi16(_mm256_and_si256(q4bitsH, _mm256_set1_epi8(-64)), 2);
            const __m256i q4_0 = _mm256_or_si256(_mm256_and_si256(q4bits1, m15), q4h_0);
            const __m256i q4_1 = _mm256_or_si256(_mm256_and_si256(q4bits2, m15), q4h_1);
            const __m256i q4_2 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits1, 4), m15), q4h_2);
            const __m256i q4_3 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits2, 4), m15), q4h_3);
            const __m256i q8_0 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            const __m256i q8_1 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            const __m256i q8_2 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            const __m256i q8_3 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            __m256i p16_0 = _mm256_maddubs_epi16(q4_0, q8_0);
            __m256i p16_1 = _mm256_maddubs_epi16(q4_1, q8_1);
            __m256i p16_2 = _mm256_maddubs_epi16(q4_2, q8_2);
            __m256i p16_3 = _mm256_maddubs_epi16(q4_3, q8_3);
            const __m128i scale_0 = _mm_shuffle_epi8(scales, scale_shuffle_q6(is + 0));
            const __m128i scale_1 = _mm_shuffle_epi8(scales, scale_shuffle_q6(is + 1));
            const __m128i scale_2 = _mm_shuffle_epi8(scales, scale_shuffle_q6(is + 2));
            const __m128i scale_3 = _mm_shuffle_epi8(scales, scale_shuffle_q6(is + 3));
            is += 4;
            p16_0 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(scale_0), p16_0);
            p16_1 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(scale_1), p16_1);
            p16_2 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(scale_2), p16_2);
            p16_3 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(scale_3), p16_3);
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16_0, p16_1));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16_2, p16_3));
        }
        sumi = _mm256_sub_epi32(sumi, q8sclsub);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum_float_8(acc);
}

/* ggml_vec_dot_q8_0_q8_0 AVX2 arm, x86/legacy.zig:537-572 with
 * mul_sum_i8_pairs_float (x86/common.zig:120-150, non-VNNI arm). */
AVX2_FN static float vec_dot_q8_0_q8_0_avx2(int n, const void *vx, const void *vy) {
    const blk_q8_0 *x = (const blk_q8_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    const int nb = n / QK8_0;
    __m256 acc = _mm256_setzero_ps();
    for (int ib = 0; ib < nb; ++ib) {
        const __m256 d = _mm256_set1_ps(F32(x[ib].d) * F32(y[ib].d));
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i dot = _mm256_maddubs_epi16(ax, sy);
        const __m256 q = _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_set1_epi16(1), dot));
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum_float_8(acc);
}

/* mul_sum_i8_pairs_float (x86/common.zig:120-150, non-VNNI arm): lane i is
 * the exact sum of the products 4i..4i+3, as a float. */
AVX2_FN static inline __m256 mul_sum_i8_pairs_float(__m256i x, __m256i y) {
    const __m256i ax = _mm256_sign_epi8(x, x);
    const __m256i sy = _mm256_sign_epi8(y, x);
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_set1_epi16(1), _mm256_maddubs_epi16(ax, sy)));
}

/* bytes_from_nibbles_32 (x86/common.zig:111-116): 16 bytes to 32 nibbles, low first. */
AVX2_FN static inline __m256i bytes_from_nibbles_32(const uint8_t *rsi) {
    const __m128i tmp = _mm_loadu_si128((const __m128i *)rsi);
    return _mm256_and_si256(_mm256_set1_epi8(0xF), _mm256_set_m128i(_mm_srli_epi16(tmp, 4), tmp));
}

/* ggml_vec_dot_q4_0_q8_0 AVX2 arm, x86/legacy.zig:189-226: nibbles - 8,
 * the q8_0 arm's lane sums, one fused multiply-add per block, hsum_float_8. */
AVX2_FN static float vec_dot_q4_0_q8_0_avx2(int n, const void *vx, const void *vy) {
    const blk_q4_0 *x = (const blk_q4_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    const int nb = n / QK8_0;
    __m256 acc = _mm256_setzero_ps();
    for (int ib = 0; ib < nb; ++ib) {
        const __m256 d = _mm256_set1_ps(F32(x[ib].d) * F32(y[ib].d));
        const __m256i qx = _mm256_sub_epi8(bytes_from_nibbles_32(x[ib].qs), _mm256_set1_epi8(8));
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        acc = _mm256_fmadd_ps(d, mul_sum_i8_pairs_float(qx, qy), acc);
    }
    return hsum_float_8(acc);
}

/* ggml_vec_dot_q5_K_q8_K AVX2 arm, x86/k.zig:355-451: q4_K's lanes with the
 * fifth bit added from qh one bit plane per 32 weights; the mins fold to a
 * scalar per super-block (hadd twice) and accumulate as summs = fma(dmin,
 * hsum, summs), added after hsum_float_8 of the lanes. */
AVX2_FN static float vec_dot_q5_K_q8_K_avx2(int n, const void *vx, const void *vy) {
    const blk_q5_K *x = (const blk_q5_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    const int nb = n / QK_K;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    const __m128i mzero = _mm_setzero_si128();
    const __m256i mone = _mm256_set1_epi8(1);
    __m256 acc = _mm256_setzero_ps();
    float summs = 0.0f;
    for (int i = 0; i < nb; ++i) {
        const uint8_t *q5 = x[i].qs;
        const int8_t *q8 = y[i].qs;
        const float d = y[i].d * F32(x[i].d);
        const float dmin = -y[i].d * F32(x[i].dmin);
        uint32_t utmp[4];
        unpack_scales_k4(x[i].scales, utmp);
        const __m256i mins_and_scales = _mm256_cvtepu8_epi16(
            _mm_set_epi32((int)utmp[3], (int)utmp[2], (int)utmp[1], (int)utmp[0]));
        const __m256i q8sums = _mm256_loadu_si256((const __m256i *)y[i].bsums);
        const __m128i q8s = _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0), _mm256_extracti128_si256(q8sums, 1));
        const __m128i prod = _mm_madd_epi16(_mm256_extracti128_si256(mins_and_scales, 1), q8s);
        const __m128i hsum = _mm_hadd_epi32(_mm_hadd_epi32(prod, mzero), mzero);
        summs = fmaf(dmin, (float)_mm_extract_epi32(hsum, 0), summs);
        const __m128i sc128 = _mm256_extracti128_si256(mins_and_scales, 0);
        const __m256i scales = _mm256_set_m128i(sc128, sc128);
        const __m256i hbits = _mm256_loadu_si256((const __m256i *)x[i].qh);
        __m256i hmask = mone;
        __m256i sumi = _mm256_setzero_si256();
        int bit = 0;
        for (int j = 0; j < QK_K / 64; ++j) {
            const __m256i scale_0 = _mm256_shuffle_epi8(scales, scale_shuffle_k4(2 * j + 0));
            const __m256i scale_1 = _mm256_shuffle_epi8(scales, scale_shuffle_k4(2 * j + 1));
            const __m256i q5bits = _mm256_loadu_si256((const __m256i *)q5); q5 += 32;
            const __m256i q5l_0 = _mm256_and_si256(q5bits, m4);
            const __m256i q5h_0 = _mm256_slli_epi16(
                _mm256_srl_epi16(_mm256_and_si256(hbits, hmask), _mm_cvtsi32_si128(bit)), 4);
            ++bit;
            const __m256i q5_0 = _mm256_add_epi8(q5l_0, q5h_0);
            hmask = _mm256_slli_epi16(hmask, 1);
            const __m256i q5l_1 = _mm256_and_si256(_mm256_srli_epi16(q5bits, 4), m4);
            const __m256i q5h_1 = _mm256_slli_epi16(
                _mm256_srl_epi16(_mm256_and_si256(hbits, hmask), _mm_cvtsi32_si128(bit)), 4);
            ++bit;
            const __m256i q5_1 = _mm256_add_epi8(q5l_1, q5h_1);
            hmask = _mm256_slli_epi16(hmask, 1);
            const __m256i q8_0 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            const __m256i q8_1 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            __m256i p16_0 = _mm256_maddubs_epi16(q5_0, q8_0);
            __m256i p16_1 = _mm256_maddubs_epi16(q5_1, q8_1);
            p16_0 = _mm256_madd_epi16(scale_0, p16_0);
            p16_1 = _mm256_madd_epi16(scale_1, p16_1);
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16_0, p16_1));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum_float_8(acc) + summs;
}

/* ggml_vec_dot_iq4_xs_q8_K AVX2 arm, x86/iq.zig:731-790: the codebook by
 * pshufb, 32 weights per madd with the group scale ls - 32; two lane
 * accumulators per super-block (even and odd groups) added before the one
 * fused multiply-add with f32(d) * y.d. */
AVX2_FN static float vec_dot_iq4_xs_q8_K_avx2(int n, const void *vx, const void *vy) {
    const blk_iq4_xs *x = (const blk_iq4_xs *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    const int nb = n / QK_K;
    const __m128i values128 = _mm_loadu_si128((const __m128i *)KV_IQ4NL);
    const __m128i m4b = _mm_set1_epi8(0x0f);
    __m256 accum = _mm256_setzero_ps();
    for (int ibl = 0; ibl < nb; ++ibl) {
        const uint8_t *qs = x[ibl].qs;
        const int8_t *q8 = y[ibl].qs;
        uint16_t sh = x[ibl].scales_h;
        __m256i sumi1 = _mm256_setzero_si256(), sumi2 = _mm256_setzero_si256();
        for (int ib = 0; ib < QK_K / 32; ib += 2) {
            const __m128i q4bits_1 = _mm_loadu_si128((const __m128i *)qs); qs += 16;
            const __m128i q4bits_2 = _mm_loadu_si128((const __m128i *)qs); qs += 16;
            const __m256i q8b_1 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            const __m256i q8b_2 = _mm256_loadu_si256((const __m256i *)q8); q8 += 32;
            const __m256i q4b_1 = _mm256_set_m128i(
                _mm_shuffle_epi8(values128, _mm_and_si128(_mm_srli_epi16(q4bits_1, 4), m4b)),
                _mm_shuffle_epi8(values128, _mm_and_si128(q4bits_1, m4b)));
            const __m256i q4b_2 = _mm256_set_m128i(
                _mm_shuffle_epi8(values128, _mm_and_si128(_mm_srli_epi16(q4bits_2, 4), m4b)),
                _mm_shuffle_epi8(values128, _mm_and_si128(q4bits_2, m4b)));
            const __m256i p16_1 = _mm256_maddubs_epi16(_mm256_sign_epi8(q4b_1, q4b_1), _mm256_sign_epi8(q8b_1, q4b_1));
            const __m256i p16_2 = _mm256_maddubs_epi16(_mm256_sign_epi8(q4b_2, q4b_2), _mm256_sign_epi8(q8b_2, q4b_2));
            const int sl = x[ibl].scales_l[ib / 2];
            const int16_t ls1 = (int16_t)(((sl & 0xf) | (((int)sh << 4) & 0x30)) - 32);
            const int16_t ls2 = (int16_t)(((sl >> 4) | (((int)sh << 2) & 0x30)) - 32);
            sh >>= 4;
            sumi1 = _mm256_add_epi32(_mm256_madd_epi16(p16_1, _mm256_set1_epi16(ls1)), sumi1);
            sumi2 = _mm256_add_epi32(_mm256_madd_epi16(p16_2, _mm256_set1_epi16(ls2)), sumi2);
        }
        accum = _mm256_fmadd_ps(_mm256_set1_ps(F32(x[ibl].d) * y[ibl].d),
                                _mm256_cvtepi32_ps(_mm256_add_epi32(sumi1, sumi2)), accum);
    }
    return hsum_float_8(accum);
}

/* quantize_row_q8_0 AVX2 arm, x86/rows.zig:27-105: id = 127/max and
 * round-half-even, saturating packs. */
AVX2_FN static void quantize_row_q8_0_avx2_impl(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        __m256 v0 = _mm256_loadu_ps(x), v1 = _mm256_loadu_ps(x + 8);
        __m256 v2 = _mm256_loadu_ps(x + 16), v3 = _mm256_loadu_ps(x + 24);
        x += 32;
        const __m256 signBit = _mm256_set1_ps(-0.0f);
        __m256 maxAbs = _mm256_andnot_ps(signBit, v0);
        maxAbs = _mm256_max_ps(maxAbs, _mm256_andnot_ps(signBit, v1));
        maxAbs = _mm256_max_ps(maxAbs, _mm256_andnot_ps(signBit, v2));
        maxAbs = _mm256_max_ps(maxAbs, _mm256_andnot_ps(signBit, v3));
        __m128 max4 = _mm_max_ps(_mm256_extractf128_ps(maxAbs, 1), _mm256_castps256_ps128(maxAbs));
        max4 = _mm_max_ps(max4, _mm_movehl_ps(max4, max4));
        max4 = _mm_max_ss(max4, _mm_movehdup_ps(max4));
        const float max_scalar = _mm_cvtss_f32(max4);
        const float d = max_scalar / 127.f;
        y[i].d = FP16(d);
        const float id = (max_scalar != 0.0f) ? 127.f / max_scalar : 0.0f;
        const __m256 mul = _mm256_set1_ps(id);
        v0 = _mm256_round_ps(_mm256_mul_ps(v0, mul), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        v1 = _mm256_round_ps(_mm256_mul_ps(v1, mul), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        v2 = _mm256_round_ps(_mm256_mul_ps(v2, mul), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        v3 = _mm256_round_ps(_mm256_mul_ps(v3, mul), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        __m256i i0 = _mm256_cvtps_epi32(v0);
        const __m256i i1 = _mm256_cvtps_epi32(v1);
        __m256i i2 = _mm256_cvtps_epi32(v2);
        const __m256i i3 = _mm256_cvtps_epi32(v3);
        i0 = _mm256_packs_epi32(i0, i1);
        i2 = _mm256_packs_epi32(i2, i3);
        i0 = _mm256_packs_epi16(i0, i2);
        const __m256i perm = _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7);
        i0 = _mm256_permutevar8x32_epi32(i0, perm);
        _mm256_storeu_si256((__m256i *)y[i].qs, i0);
    }
}
#endif /* ORC_X86 */

int orc_has_avx2(void) {
#if ORC_X86
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
#else
    return 0;
#endif
}

void orc_quantize_row_q8_0_avx2(const float *x, void *y, int64_t k) {
#if ORC_X86
    if (orc_has_avx2()) { quantize_row_q8_0_avx2_impl(x, y, k); return; }
#endif
    orc_quantize_row_q8_0_ref(x, y, k);
}

typedef float (*dot_fn)(int, const void *, const void *);
typedef void (*from_float_fn)(const float *, void *, int64_t);

static dot_fn pick_dot(int type, int impl) {
#if ORC_X86
    if (impl == ORC_IMPL_AVX2 && orc_has_avx2()) {
        switch (type) {
        case ORC_TYPE_Q4_0: return vec_dot_q4_0_q8_0_avx2;
        case ORC_TYPE_Q4_K: return vec_dot_q4_K_q8_K_avx2;
        case ORC_TYPE_Q5_K: return vec_dot_q5_K_q8_K_avx2;
        case ORC_TYPE_Q6_K: return vec_dot_q6_K_q8_K_avx2;
        case ORC_TYPE_Q8_0: return vec_dot_q8_0_q8_0_avx2;
        case ORC_TYPE_IQ4_XS: return vec_dot_iq4_xs_q8_K_avx2;
        }
    }
#endif
    (void)impl;
    switch (type) {
    case ORC_TYPE_Q4_0: return vec_dot_q4_0_q8_0_generic;
    case ORC_TYPE_Q4_K: return vec_dot_q4_K_q8_K_generic;
    case ORC_TYPE_Q5_K: return vec_dot_q5_K_q8_K_generic;
    case ORC_TYPE_Q6_K: return vec_dot_q6_K_q8_K_generic;
    case ORC_TYPE_Q8_0: return vec_dot_q8_0_q8_0_generic;
    case ORC_TYPE_IQ4_XS: return vec_dot_iq4_xs_q8_K_generic;
    }
    return NULL;
}

/* vec_dot_type and from_float per cpu/traits.zig:158-201 and x86/rows.zig:
 * K-quants take Q8_K (scalar ref on x86 too); Q8_0 takes Q8_0 (AVX2 row
 * quantizer on x86, the reference quantizer in the generic build). */
static int vec_dot_type(int type) {
    return type == ORC_TYPE_Q8_0 || type == ORC_TYPE_Q4_0 ? ORC_TYPE_Q8_0 : ORC_TYPE_Q8_K;
}
static from_float_fn pick_from_float(int type, int impl) {
    if (vec_dot_type(type) == ORC_TYPE_Q8_0)
        return impl == ORC_IMPL_AVX2 ? orc_quantize_row_q8_0_avx2 : orc_quantize_row_q8_0_ref;
    return orc_quantize_row_q8_K_ref;
}

float orc_vec_dot(int type, int impl, int n, const void *vx, const void *vy) {
    dot_fn f = pick_dot(type, impl);
    return f ? f(n, vx, vy) : NAN;
}

/* ------------------------------------------------------------------------ */
/* GPU semantics against Q8_1 activations (the device kernels' contract). */

void orc_block_dots_q8_1(int type, const void *w, int64_t nrows, int64_t K, const void *vy, int32_t *out) {
    const blk_q8_1 *y = (const blk_q8_1 *)vy;
    const size_t rs = orc_row_size(type, K);
    for (int64_t r = 0; r < nrows; ++r) {
        const uint8_t *row = (const uint8_t *)w + (size_t)r * rs;
        if (type == ORC_TYPE_Q4_K) {
            const blk_q4_K *x = (const blk_q4_K *)row;
            for (int64_t b = 0; b < K / QK_K; ++b)
                for (int j = 0; j < 8; ++j) {
                    const blk_q8_1 *yb = &y[b * 8 + j];
                    int32_t s = 0;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t byte = x[b].qs[32 * (j / 2) + l];
                        const int q = (j & 1) ? (byte >> 4) : (byte & 0xF);
                        s += q * yb->qs[l];
                    }
                    *out++ = s;
                }
        } else if (type == ORC_TYPE_Q5_K) {
            const blk_q5_K *x = (const blk_q5_K *)row;
            for (int64_t b = 0; b < K / QK_K; ++b)
                for (int j = 0; j < 8; ++j) {
                    const blk_q8_1 *yb = &y[b * 8 + j];
                    int32_t s = 0;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t byte = x[b].qs[32 * (j / 2) + l];
                        const int q = ((j & 1) ? (byte >> 4) : (byte & 0xF)) + ((x[b].qh[l] >> j) & 1) * 16;
                        s += q * yb->qs[l];
                    }
                    *out++ = s;
                }
        } else if (type == ORC_TYPE_Q6_K) {
            const blk_q6_K *x = (const blk_q6_K *)row;
            for (int64_t b = 0; b < K / QK_K; ++b) {
                int8_t q6[QK_K];
                for (int n = 0; n < 2; ++n)
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t *ql = x[b].ql + 64 * n, *qh = x[b].qh + 32 * n;
                        q6[128 * n + l + 0] = (int8_t)(((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
                        q6[128 * n + l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                        q6[128 * n + l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                        q6[128 * n + l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                    }
                for (int k = 0; k < 16; ++k) {
                    const blk_q8_1 *yb = &y[b * 8 + k / 2];
                    int32_t s = 0;
                    for (int l = 0; l < 16; ++l) s += q6[16 * k + l] * yb->qs[16 * (k & 1) + l];
                    *out++ = s;
                }
            }
        } else if (type == ORC_TYPE_Q8_0) {
            const blk_q8_0 *x = (const blk_q8_0 *)row;
            for (int64_t b = 0; b < K / 32; ++b) {
                int32_t s = 0;
                for (int l = 0; l < 32; ++l) s += x[b].qs[l] * y[b].qs[l];
                *out++ = s;
            }
        } else if (type == ORC_TYPE_IQ4_XS) {
            /* S = sum level[q] * q8 over each 32-value sub-block */
            const blk_iq4_xs *x = (const blk_iq4_xs *)row;
            for (int64_t b = 0; b < K / QK_K; ++b)
                for (int ib = 0; ib < 8; ++ib) {
                    const blk_q8_1 *yb = &y[b * 8 + ib];
                    const uint8_t *qs = x[b].qs + 16 * ib;
                    int32_t s = 0;
                    for (int l = 0; l < 16; ++l) {
                        s += KV_IQ4NL[qs[l] & 0xf] * yb->qs[l];
                        s += KV_IQ4NL[qs[l] >> 4] * yb->qs[l + 16];
                    }
                    *out++ = s;
                }
        } else if (type == ORC_TYPE_Q4_0) {
            /* S = sum (q - 8) * q8 over the block: the offset applied in integers */
            const blk_q4_0 *x = (const blk_q4_0 *)row;
            for (int64_t b = 0; b < K / 32; ++b) {
                int32_t s = 0;
                for (int l = 0; l < 16; ++l) {
                    s += ((x[b].qs[l] & 0x0F) - 8) * y[b].qs[l];
                    s += ((x[b].qs[l] >> 4) - 8) * y[b].qs[l + 16];
                }
                *out++ = s;
            }
        }
    }
}

void orc_mul_mat_q8_1_f64(int type, const void *w, int64_t nrows, int64_t K, const void *vy,
                          int64_t ncols, double *dst) {
    const size_t rs = orc_row_size(type, K);
    const int64_t nsub = type == ORC_TYPE_Q6_K ? K / 16 : K / 32;
    int32_t *S = (int32_t *)malloc(sizeof(int32_t) * (size_t)nsub);
    for (int64_t c = 0; c < ncols; ++c) {
        const blk_q8_1 *y = (const blk_q8_1 *)vy + c * (K / 32);
        for (int64_t r = 0; r < nrows; ++r) {
            const uint8_t *row = (const uint8_t *)w + (size_t)r * rs;
            orc_block_dots_q8_1(type, row, 1, K, y, S);
            double acc = 0.0;
            if (type == ORC_TYPE_Q4_K) {
                const blk_q4_K *x = (const blk_q4_K *)row;
                for (int64_t b = 0; b < K / QK_K; ++b)
                    for (int j = 0; j < 8; ++j) {
                        uint8_t sc, m;
                        get_scale_min_k4(j, x[b].scales, &sc, &m);
                        const blk_q8_1 *yb = &y[b * 8 + j];
                        acc += (double)F32(x[b].d) * sc * F32(yb->d) * S[b * 8 + j] -
                               (double)F32(x[b].dmin) * m * F32(yb->s);
                    }
            } else if (type == ORC_TYPE_Q5_K) {
                const blk_q5_K *x = (const blk_q5_K *)row;
                for (int64_t b = 0; b < K / QK_K; ++b)
                    for (int j = 0; j < 8; ++j) {
                        uint8_t sc, m;
                        get_scale_min_k4(j, x[b].scales, &sc, &m);
                        const blk_q8_1 *yb = &y[b * 8 + j];
                        acc += (double)F32(x[b].d) * sc * F32(yb->d) * S[b * 8 + j] -
                               (double)F32(x[b].dmin) * m * F32(yb->s);
                    }
            } else if (type == ORC_TYPE_Q6_K) {
                const blk_q6_K *x = (const blk_q6_K *)row;
                for (int64_t b = 0; b < K / QK_K; ++b)
                    for (int k = 0; k < 16; ++k)
                        acc += (double)F32(x[b].d) * x[b].scales[k] * F32(y[b * 8 + k / 2].d) * S[b * 16 + k];
            } else if (type == ORC_TYPE_Q4_0) {
                const blk_q4_0 *x = (const blk_q4_0 *)row;
                for (int64_t b = 0; b < K / 32; ++b) acc += (double)F32(x[b].d) * F32(y[b].d) * S[b];
            } else if (type == ORC_TYPE_IQ4_XS) {
                const blk_iq4_xs *x = (const blk_iq4_xs *)row;
                for (int64_t b = 0; b < K / QK_K; ++b)
                    for (int ib = 0; ib < 8; ++ib)
                        acc += (double)F32(x[b].d) * (iq4_xs_ls(&x[b], ib) - 32) * F32(y[b * 8 + ib].d) * S[b * 8 + ib];
            } else {
                const blk_q8_0 *x = (const blk_q8_0 *)row;
                for (int64_t b = 0; b < K / 32; ++b) acc += (double)F32(x[b].d) * F32(y[b].d) * S[b];
            }
            dst[c * nrows + r] = acc;
        }
    }
    free(S);
}

/* ------------------------------------------------------------------------ */
/* mul_mat driver: src/ggml/cpu/mulmat.zig:92-423 (oneChunk + chunking). */

typedef struct {
    int type, impl, nth;
    const uint8_t *w;
    int64_t nrows, K, ncols;
    const float *x;
    float *dst;
    uint8_t *wdata;
    size_t wrow; /* bytes per staged src1 row */
    atomic_long current_chunk;
    int64_t nchunk0, nchunk1, dr0, dr1;
} mm_ctx;

typedef struct { mm_ctx *ctx; int ith; } mm_thread;

static void one_chunk(mm_ctx *c, int64_t ir0_start, int64_t ir0_end, int64_t ir1_start, int64_t ir1_end) {
    if (ir0_start >= ir0_end || ir1_start >= ir1_end) return;
    dot_fn dot = pick_dot(c->type, c->impl);
    const size_t rs = orc_row_size(c->type, c->K);
    const int64_t blck_0 = 16, blck_1 = 16;
    float tmp[32];
    for (int64_t iir1 = ir1_start; iir1 < ir1_end; iir1 += blck_1)
        for (int64_t iir0 = ir0_start; iir0 < ir0_end; iir0 += blck_0)
            for (int64_t ir1 = iir1; ir1 < iir1 + blck_1 && ir1 < ir1_end; ++ir1) {
                const uint8_t *src1_col = c->wdata + (size_t)ir1 * c->wrow;
                float *dst_col = c->dst + ir1 * c->nrows;
                for (int64_t ir0 = iir0; ir0 < iir0 + blck_0 && ir0 < ir0_end; ++ir0)
                    tmp[ir0 - iir0] = dot((int)c->K, c->w + (size_t)ir0 * rs, src1_col);
                const int64_t end = iir0 + blck_0 < ir0_end ? iir0 + blck_0 : ir0_end;
                memcpy(dst_col + iir0, tmp, sizeof(float) * (size_t)(end - iir0));
            }
}

static void *mm_stage_worker(void *arg) {
    mm_thread *t = (mm_thread *)arg;
    mm_ctx *c = t->ctx;
    const int vdt = vec_dot_type(c->type);
    from_float_fn ff = pick_from_float(c->type, c->impl);
    const int64_t bs = orc_blck_size(vdt);
    const size_t nbw0 = orc_type_size(vdt);
    const int64_t block_start = (int64_t)t->ith * (c->K / bs) / c->nth;
    const int64_t block_end = ((int64_t)t->ith + 1) * (c->K / bs) / c->nth;
    for (int64_t j11 = 0; j11 < c->ncols; ++j11)
        ff(c->x + j11 * c->K + block_start * bs, c->wdata + (size_t)j11 * c->wrow + (size_t)block_start * nbw0,
           (block_end - block_start) * bs);
    return NULL;
}

static void *mm_compute_worker(void *arg) {
    mm_thread *t = (mm_thread *)arg;
    mm_ctx *c = t->ctx;
    long current_chunk = t->ith;
    const int64_t nr0 = c->nrows, nr1 = c->ncols;
    while (current_chunk < c->nchunk0 * c->nchunk1) {
        const int64_t ith0 = current_chunk % c->nchunk0, ith1 = current_chunk / c->nchunk0;
        const int64_t ir0_start = c->dr0 * ith0, ir1_start = c->dr1 * ith1;
        const int64_t ir0_end = ir0_start + c->dr0 < nr0 ? ir0_start + c->dr0 : nr0;
        const int64_t ir1_end = ir1_start + c->dr1 < nr1 ? ir1_start + c->dr1 : nr1;
        one_chunk(c, ir0_start, ir0_end, ir1_start, ir1_end);
        if (c->nth >= c->nchunk0 * c->nchunk1) break;
        current_chunk = atomic_fetch_add(&c->current_chunk, 1);
    }
    return NULL;
}

/* Thread k of a parallel region runs fn(ts + k * stride); the caller is
 * thread 0.  The other threads come from a persistent pool, as ggml's CPU
 * backend keeps its threadpool alive across ops, so a call costs a wake-up, not
 * thread creation: this matters only for timing (the CPU baseline), not for
 * the results, which depend on the work split alone.  Workers spin briefly on
 * the job counter before sleeping on a condition variable; callers are
 * serialized. */
typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t start, done;
    atomic_long gen;   /* job number, bumped (under mu) when a job is posted */
    atomic_int pending; /* pool threads still running the current job */
    int nworkers;      /* pool threads created so far (thread indices 1..nworkers) */
    int active;        /* threads of the current job (indices < active run it) */
    void *(*fn)(void *);
    char *ts;
    size_t stride;
} orc_pool;
static orc_pool pool = {.mu = PTHREAD_MUTEX_INITIALIZER, .start = PTHREAD_COND_INITIALIZER,
                        .done = PTHREAD_COND_INITIALIZER};
static pthread_mutex_t pool_call = PTHREAD_MUTEX_INITIALIZER;
#define ORC_POOL_MAX 256
/* the job number current when pool thread k was created (under pool.mu):
 * the thread waits for the next one, whenever it gets to run */
static long pool_born[ORC_POOL_MAX + 1];

static void *pool_worker(void *arg) {
    const int idx = (int)(intptr_t)arg;
    long seen = pool_born[idx];
    for (;;) {
        for (long spin = 0; spin < (1L << 16) && atomic_load_explicit(&pool.gen, memory_order_acquire) == seen; ++spin) {
#if defined(__x86_64__)
            _mm_pause();
#endif
        }
        pthread_mutex_lock(&pool.mu);
        while (atomic_load_explicit(&pool.gen, memory_order_relaxed) == seen) pthread_cond_wait(&pool.start, &pool.mu);
        seen = atomic_load_explicit(&pool.gen, memory_order_relaxed);
        const int run = idx < pool.active;
        void *(*fn)(void *) = pool.fn;
        char *arg_k = pool.ts + (size_t)idx * pool.stride;
        pthread_mutex_unlock(&pool.mu);
        if (!run) continue;
        fn(arg_k);
        if (atomic_fetch_sub_explicit(&pool.pending, 1, memory_order_acq_rel) == 1) {
            pthread_mutex_lock(&pool.mu);
            pthread_cond_signal(&pool.done);
            pthread_mutex_unlock(&pool.mu);
        }
    }
    return NULL;
}

/* A child forked from a process that has pool threads inherits none of them:
 * it starts an empty pool (fresh locks, no threads). */
static void pool_after_fork_child(void) {
    pthread_mutex_init(&pool.mu, NULL);
    pthread_cond_init(&pool.start, NULL);
    pthread_cond_init(&pool.done, NULL);
    pthread_mutex_init(&pool_call, NULL);
    pool.nworkers = 0;
    atomic_store_explicit(&pool.pending, 0, memory_order_relaxed);
}
static pthread_once_t pool_once = PTHREAD_ONCE_INIT;
static void pool_register_fork_handler(void) { pthread_atfork(NULL, NULL, pool_after_fork_child); }

static void run_threads(int nth, void *ts, size_t stride, void *(*fn)(void *)) {
    if (nth <= 1) {
        fn(ts);
        return;
    }
    pthread_once(&pool_once, pool_register_fork_handler);
    pthread_mutex_lock(&pool_call);
    pthread_mutex_lock(&pool.mu);
    while (pool.nworkers < nth - 1 && pool.nworkers < ORC_POOL_MAX) {
        pthread_t th;
        pool_born[pool.nworkers + 1] = atomic_load_explicit(&pool.gen, memory_order_relaxed);
        if (pthread_create(&th, NULL, pool_worker, (void *)(intptr_t)(pool.nworkers + 1)) != 0) break;
        pthread_detach(th);
        ++pool.nworkers;
    }
    const int helpers = pool.nworkers < nth - 1 ? pool.nworkers : nth - 1;
    pool.fn = fn;
    pool.ts = (char *)ts;
    pool.stride = stride;
    pool.active = helpers + 1;
    atomic_store_explicit(&pool.pending, helpers, memory_order_relaxed);
    atomic_fetch_add_explicit(&pool.gen, 1, memory_order_release);
    pthread_cond_broadcast(&pool.start);
    pthread_mutex_unlock(&pool.mu);
    fn(ts);
    /* threads the pool could not provide: the caller runs their shares */
    for (int k = helpers + 1; k < nth; ++k) fn((char *)ts + (size_t)k * stride);
    pthread_mutex_lock(&pool.mu);
    while (atomic_load_explicit(&pool.pending, memory_order_acquire) > 0) pthread_cond_wait(&pool.done, &pool.mu);
    pthread_mutex_unlock(&pool.mu);
    pthread_mutex_unlock(&pool_call);
}

void orc_mul_mat(int type, int impl, const void *w, int64_t nrows, int64_t K, const float *x,
                 int64_t ncols, float *dst, int nth) {
    if (nth < 1) nth = 1;
    mm_ctx c;
    memset(&c, 0, sizeof c);
    c.type = type; c.impl = impl; c.nth = nth; c.w = (const uint8_t *)w;
    c.nrows = nrows; c.K = K; c.ncols = ncols; c.x = x; c.dst = dst;
    c.wrow = orc_row_size(vec_dot_type(type), K);
    c.wdata = (uint8_t *)calloc((size_t)ncols, c.wrow);
    mm_thread *ts = (mm_thread *)malloc(sizeof(mm_thread) * (size_t)nth);
    for (int i = 0; i < nth; ++i) { ts[i].ctx = &c; ts[i].ith = i; }
    run_threads(nth, ts, sizeof *ts, mm_stage_worker);
    const int64_t nr0 = nrows, nr1 = ncols;
    int64_t chunk_size = (nr0 == 1 || nr1 == 1) ? 64 : 16;
    int64_t nchunk0 = (nr0 + chunk_size - 1) / chunk_size;
    int64_t nchunk1 = (nr1 + chunk_size - 1) / chunk_size;
    if (nchunk0 * nchunk1 < (int64_t)nth * 4) {
        nchunk0 = nr0 > nr1 ? nth : 1;
        nchunk1 = nr0 > nr1 ? 1 : nth;
    }
    c.nchunk0 = nchunk0; c.nchunk1 = nchunk1;
    c.dr0 = (nr0 + nchunk0 - 1) / nchunk0;
    c.dr1 = (nr1 + nchunk1 - 1) / nchunk1;
    atomic_store(&c.current_chunk, nth);
    run_threads(nth, ts, sizeof *ts, mm_compute_worker);
    free(ts);
    free(c.wdata);
}

/* mul_mat_id driver: mulmat.zig:429-777 (grouping by expert, -1 -> zero row). */

typedef struct { int32_t i1, i2; } row_mapping;

typedef struct {
    int type, impl, nth;
    const uint8_t *w;
    int64_t n_as, nrows, K, ne11, n_tokens, n_ids;
    const float *x;
    const int32_t *ids;
    float *dst;
    uint8_t *wdata;
    size_t wrow;
    int64_t *counts;
    row_mapping *rows;
    atomic_long *chunk;
} mmid_ctx;

typedef struct { mmid_ctx *ctx; int ith; } mmid_thread;

static void *mmid_stage_worker(void *arg) {
    mmid_thread *t = (mmid_thread *)arg;
    mmid_ctx *c = t->ctx;
    const int vdt = vec_dot_type(c->type);
    from_float_fn ff = pick_from_float(c->type, c->impl);
    const int64_t bs = orc_blck_size(vdt);
    const size_t nbw0 = orc_type_size(vdt);
    const int64_t block_start = (int64_t)t->ith * (c->K / bs) / c->nth;
    const int64_t block_end = ((int64_t)t->ith + 1) * (c->K / bs) / c->nth;
    for (int64_t r = 0; r < c->ne11 * c->n_tokens; ++r)
        ff(c->x + r * c->K + block_start * bs, c->wdata + (size_t)r * c->wrow + (size_t)block_start * nbw0,
           (block_end - block_start) * bs);
    return NULL;
}

static void *mmid_compute_worker(void *arg) {
    mmid_thread *t = (mmid_thread *)arg;
    mmid_ctx *c = t->ctx;
    dot_fn dot = pick_dot(c->type, c->impl);
    const size_t rs = orc_row_size(c->type, c->K);
    const int nth = c->nth;
    for (int64_t cur_a = 0; cur_a < c->n_as; ++cur_a) {
        const int64_t cne1 = c->counts[cur_a];
        if (cne1 == 0) continue;
        const uint8_t *src0_cur = c->w + (size_t)cur_a * (size_t)c->nrows * rs;
        const int64_t nr0 = c->nrows, nr1 = cne1;
        int64_t chunk_size = (nr0 == 1 || nr1 == 1) ? 64 : 16;
        int64_t nchunk0 = (nr0 + chunk_size - 1) / chunk_size;
        int64_t nchunk1 = (nr1 + chunk_size - 1) / chunk_size;
        if (nchunk0 * nchunk1 < (int64_t)nth * 4) {
            nchunk0 = nr0 > nr1 ? nth : 1;
            nchunk1 = nr0 > nr1 ? 1 : nth;
        }
        const int64_t dr0 = (nr0 + nchunk0 - 1) / nchunk0, dr1 = (nr1 + nchunk1 - 1) / nchunk1;
        long current_chunk = t->ith;
        while (current_chunk < nchunk0 * nchunk1) {
            const int64_t ith0 = current_chunk % nchunk0, ith1 = current_chunk / nchunk0;
            const int64_t ir0_start = dr0 * ith0, ir1_start = dr1 * ith1;
            const int64_t ir0_end = ir0_start + dr0 < nr0 ? ir0_start + dr0 : nr0;
            const int64_t ir1_end = ir1_start + dr1 < nr1 ? ir1_start + dr1 : nr1;
            for (int64_t ir1 = ir1_start; ir1 < ir1_end; ++ir1) {
                const row_mapping rm = c->rows[cur_a * c->n_ids * c->n_tokens + ir1];
                const int64_t j11 = rm.i1 % c->ne11, j12 = rm.i2;
                const uint8_t *src1_col = c->wdata + (size_t)(j11 + j12 * c->ne11) * c->wrow;
                float *dst_col = c->dst + ((int64_t)rm.i2 * c->n_ids + rm.i1) * c->nrows;
                for (int64_t ir0 = ir0_start; ir0 < ir0_end; ++ir0)
                    dst_col[ir0] = dot((int)c->K, src0_cur + (size_t)ir0 * rs, src1_col);
            }
            if (nth >= nchunk0 * nchunk1) break;
            current_chunk = atomic_fetch_add(&c->chunk[cur_a], 1);
        }
    }
    return NULL;
}

void orc_mul_mat_id(int type, int impl, const void *w, int64_t n_as, int64_t nrows, int64_t K,
                    const float *x, int64_t ne11, int64_t n_tokens, const int32_t *ids, int64_t n_ids,
                    float *dst, int nth) {
    if (nth < 1) nth = 1;
    mmid_ctx c;
    memset(&c, 0, sizeof c);
    c.type = type; c.impl = impl; c.nth = nth; c.w = (const uint8_t *)w;
    c.n_as = n_as; c.nrows = nrows; c.K = K; c.ne11 = ne11; c.n_tokens = n_tokens; c.n_ids = n_ids;
    c.x = x; c.ids = ids; c.dst = dst;
    c.wrow = orc_row_size(vec_dot_type(type), K);
    c.wdata = (uint8_t *)calloc((size_t)(ne11 * n_tokens), c.wrow);
    c.counts = (int64_t *)calloc((size_t)n_as, sizeof(int64_t));
    c.rows = (row_mapping *)calloc((size_t)(n_as * n_ids * n_tokens), sizeof(row_mapping));
    c.chunk = (atomic_long *)calloc((size_t)n_as, sizeof(atomic_long));
    mmid_thread *ts = (mmid_thread *)malloc(sizeof(mmid_thread) * (size_t)nth);
    for (int i = 0; i < nth; ++i) { ts[i].ctx = &c; ts[i].ith = i; }
    run_threads(nth, ts, sizeof *ts, mmid_stage_worker);
    for (int64_t t = 0; t < n_tokens; ++t)
        for (int64_t s = 0; s < n_ids; ++s) {
            const int32_t e = ids[t * n_ids + s];
            if (e == -1) {
                memset(dst + (t * n_ids + s) * nrows, 0, sizeof(float) * (size_t)nrows);
                continue;
            }
            c.rows[e * n_ids * n_tokens + c.counts[e]] = (row_mapping){(int32_t)s, (int32_t)t};
            c.counts[e] += 1;
        }
    for (int64_t a = 0; a < n_as; ++a) atomic_store(&c.chunk[a], nth);
    run_threads(nth, ts, sizeof *ts, mmid_compute_worker);
    free(ts);
    free(c.chunk);
    free(c.rows);
    free(c.counts);
    free(c.wdata);
}

/* ------------------------------------------------------------------------ */
/* Synthetic inputs: SplitMix64 (public-domain generator by S. Vigna) feeding
 * Box-Muller in double precision, rounded to f32. */

/* ---------------------------------------------------------------- GLU
 * The CPU GLU ops on f32 rows (ggml_compute_forward_glu,
 * src/ggml/cpu/ops/activation.zig:594-608), split form (gate and value in
 * separate rows, gluRows / GluRows.halves at :365-376, :391-403):
 *   REGLU        ggml_vec_reglu_f32        (vecinline.zig:507-511)
 *   GEGLU        ggml_vec_geglu_f32, the GGML_GELU_FP16 arm (vecinline.zig:522-536):
 *                0 at x <= -10, x*g at x >= 10, else table[f16(x)] * g with
 *                table[t] = f16(gelu(f32(t))) (cpu/convert.zig:224-228)
 *   SWIGLU       ggml_vec_swiglu_f32's scalar arm: silu(x)*g, silu = x/(1+exp(-x))
 *                (vec.zig:658-668, vecinline.zig:617-620).  The vector arm
 *                evaluates exp with its own polynomial; the two agree to a few
 *                ulp, which the tests allow.
 *   SWIGLU_OAI   swigluOaiRows f32 (activation.zig:475-503)
 *   SWIGLU_CLAMP swigluClampRows f32 (activation.zig:523-548)
 * std::min(a, b) = b < a ? b : a and std::clamp(v, lo, hi) =
 * v < lo ? lo : (hi < v ? hi : v) (activation.zig:458-463). */
float orc_gelu_f32(float x) {
    const float a = 0.044715f;                          /* GELU_COEF_A, convert.zig:242 */
    const float s = 0.79788456080286535587989211986876f; /* SQRT_2_OVER_PI, convert.zig:248 */
    return 0.5f * x * (1.0f + tanhf(s * x * fmaf(a * x, x, 1.0f)));
}

static float glu_one(int op, float x, float g, float alpha, float limit) {
    switch (op) {
    case ORC_GLU_REGLU: return x > 0.0f ? x * g : 0.0f;
    case ORC_GLU_GEGLU:
        if (x <= -10.0f) return 0.0f;
        if (x >= 10.0f) return x * g;
        return orc_fp16_to_fp32(orc_fp32_to_fp16(orc_gelu_f32(orc_fp16_to_fp32(orc_fp32_to_fp16(x))))) * g;
    case ORC_GLU_SWIGLU: return (x / (1.0f + expf(-x))) * g;
    case ORC_GLU_SWIGLU_OAI: {
        const float xm = limit < x ? limit : x;
        const float y = g < -limit ? -limit : (limit < g ? limit : g);
        const float out_glu = xm / (1.0f + expf(alpha * (-xm)));
        return out_glu * (y + 1.0f);
    }
    default: { /* ORC_GLU_SWIGLU_CLAMP */
        const float gate = limit < x ? limit : x;
        const float up = g < -limit ? -limit : (limit < g ? limit : g);
        return gate / (1.0f + expf(-gate)) * up;
    }
    }
}

void orc_glu_f32(int op, int64_t n, const float *gate, const float *up, float alpha, float limit, float *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = glu_one(op, gate[i], up[i], alpha, limit);
}

/* ggml_v_expf, the AVX2 / NEON arm (src/ggml/cpu/vec.zig:537-588): ARM's
 * optimised expf, maximum error 1.45358 + 0.5 ulp.  fma_f32(a, b, c) there is
 * a + b * c fused and fms_f32(a, b, c) is a - b * c fused; every fusion is
 * written as fmaf here in the same place.  The vector code takes a fast path
 * when no lane has |n| > 126, giving k + j * k, which is also what its slow
 * path gives a lane with |n| <= 126, so evaluating one lane at a time gives
 * the vector's bits. */
float orc_v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    uint32_t zb, kb;
    memcpy(&zb, &z, 4);
    const uint32_t e = zb << 23;
    kb = e + 0x3f800000u; /* bits of 1.0f */
    float k;
    memcpy(&k, &kb, 4);
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u, fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)), u,
                         0x1.ffffecp-1f * b);
    if (!(fabsf(n) > 126.0f)) return fmaf(j, k, k);
    const uint32_t d = n <= 0.0f ? 0x82000000u : 0u;
    const uint32_t s1b = d + 0x7f000000u, s2b = e - d;
    float s1, s2;
    memcpy(&s1, &s1b, 4);
    memcpy(&s2, &s2b, 4);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

void orc_v_expf_n(int64_t n, const float *x, float *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_v_expf(x[i]);
}

/* ggml_v_silu (vec.zig:592-599): x / (1 + v_expf(0 - x)). */
float orc_v_silu(float x) { return x / (1.0f + orc_v_expf(0.0f - x)); }

/* The CPU GLU op over nrows contiguous rows of nc (gluRows,
 * cpu/ops/activation.zig:379-447).  SWIGLU calls ggml_vec_swiglu_f32
 * (vec.zig:653-665) per row: on an AVX2 host 8-lane steps of
 * v_silu(x) * g, then the scalar (x / (1 + expf(-x))) * g for the last
 * nc % 8.  The other ops are elementwise (glu_one). */
void orc_glu_f32_rows(int op, int64_t nrows, int64_t nc, const float *gate, const float *up, float alpha, float limit,
                      float *out) {
    for (int64_t r = 0; r < nrows; ++r) {
        const float *x = gate + r * nc, *g = up + r * nc;
        float *y = out + r * nc;
        int64_t i = 0;
        if (op == ORC_GLU_SWIGLU)
            for (const int64_t nv = nc - nc % 8; i < nv; ++i) y[i] = orc_v_silu(x[i]) * g[i];
        for (; i < nc; ++i) y[i] = glu_one(op, x[i], g[i], alpha, limit);
    }
}

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* The values from element i0 (even) on: SplitMix64 advances its state by one
 * constant per draw and each pair of outputs takes two draws, so the state
 * before pair i0/2 is seed + i0 * 0x9E3779B97F4A7C15. */
static void fill_normal_from(uint64_t seed, int64_t i0, int64_t n, float mean, float stddev, float *out) {
    uint64_t s = seed + (uint64_t)i0 * 0x9E3779B97F4A7C15ull;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = i0; i < n; i += 2) {
        const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
        const double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);       /* [0,1) */
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stddev * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * r * sin(two_pi * u2));
    }
}

void orc_fill_normal(uint64_t seed, int64_t n, float mean, float stddev, float *out) {
    fill_normal_from(seed, 0, n, mean, stddev, out);
}

/* Threaded forms of the input generators, equal to the serial ones element
 * for element: the normal fill split at even indices (each part starts from
 * the SplitMix64 state of its first pair) and the row quantizer split by rows
 * (quantize_row_*_ref treats rows independently). */
typedef struct {
    int kind; /* 0: fill, 1: quantize rows */
    uint64_t seed; int64_t i0, i1; float mean, stddev; float *out;
    int type; const float *src; uint8_t *dst; int64_t n_per_row;
} gen_job;

static void *gen_worker(void *arg) {
    gen_job *j = (gen_job *)arg;
    if (j->kind == 0) {
        fill_normal_from(j->seed, j->i0, j->i1, j->mean, j->stddev, j->out);
    } else {
        const size_t rs = orc_row_size(j->type, j->n_per_row);
        if (j->i1 > j->i0)
            orc_quantize_chunk(j->type, j->src + j->i0 * j->n_per_row, j->dst + (size_t)j->i0 * rs, 0, j->i1 - j->i0,
                               j->n_per_row, NULL);
    }
    return NULL;
}

void orc_fill_normal_mt(uint64_t seed, int64_t n, float mean, float stddev, float *out, int nth) {
    if (nth < 1) nth = 1;
    gen_job *js = (gen_job *)calloc((size_t)nth, sizeof(gen_job));
    const int64_t pairs = (n + 1) / 2, per = (pairs + nth - 1) / nth;
    for (int i = 0; i < nth; ++i) {
        const int64_t p0 = per * i < pairs ? per * i : pairs, p1 = per * (i + 1) < pairs ? per * (i + 1) : pairs;
        js[i].kind = 0; js[i].seed = seed; js[i].i0 = 2 * p0; js[i].i1 = 2 * p1 < n ? 2 * p1 : n;
        js[i].mean = mean; js[i].stddev = stddev; js[i].out = out;
    }
    run_threads(nth, js, sizeof(gen_job), gen_worker);
    free(js);
}

void orc_quantize_rows_mt(int type, const float *src, void *dst, int64_t nrows, int64_t n_per_row, int nth) {
    if (nth < 1) nth = 1;
    gen_job *js = (gen_job *)calloc((size_t)nth, sizeof(gen_job));
    const int64_t per = (nrows + nth - 1) / nth;
    for (int i = 0; i < nth; ++i) {
        js[i].kind = 1; js[i].type = type; js[i].src = src; js[i].dst = (uint8_t *)dst; js[i].n_per_row = n_per_row;
        js[i].i0 = per * i < nrows ? per * i : nrows; js[i].i1 = per * (i + 1) < nrows ? per * (i + 1) : nrows;
    }
    run_threads(nth, js, sizeof(gen_job), gen_worker);
    free(js);
}

/* ------------------------------------------------------------------------ */
/* The x86 tiled K-quant GEMM: what the reference's CPU mul_mat runs first on
 * x86 when src1 has at least 8 columns (src/ggml/cpu/mulmat.zig:218-220,
 * ggml_compute_forward_mul_mat_tiled at src/ggml/cpu/tiled.zig:1262-1268).
 * Restated from src/ggml/cpu/tiled.zig (unpackers :102-330, src1 staging
 * :565-594, narrow K extent :697-710, window store :714-737, one chunk
 * :982-1112, driver :1114-1223) and src/ggml/cpu/tiled_kernel.zig (tiles
 * :80-117, the AVX2 microtile :505-690 with its column reduction :226-240,
 * the repacks :721-797), the __AVX2__ arm, for the tiled types this path
 * serves: Q4_K, Q5_K, Q6_K and IQ4_XS.  Activations are staged to Q8_K with
 * quantize_row_q8_K_ref, per thread slices, as the reference's driver does. */
#if ORC_X86

#define TL_K 256      /* TILED_TILE_K */
#define TL_ROWS 256   /* TILED_TILE_ROWS */
#define TL_MICRO 16   /* TILED_MICRO */
#define TL_NBMAX 16   /* NB_MAX */

typedef struct {
    uint8_t q[TL_ROWS * TL_K];
    float d[TL_ROWS], dmin[TL_ROWS];
    int32_t scales[TL_ROWS * TL_NBMAX], mins[TL_ROWS * TL_NBMAX];
} tl_src0;

typedef struct {
    int8_t q[TL_ROWS * TL_K];
    int32_t bsums[(TL_K / 16) * TL_ROWS];
    float d[TL_ROWS];
} tl_src1;

typedef struct {
    tl_src0 src0;
    tl_src1 src1;
    float acc[TL_ROWS * TL_ROWS];
} tl_ws;

/* The per-format constants of ggml_tiled_matmul_type_dispatch
 * (tiled.zig:786-803): sub-block width, min term, weight bias, act bias. */
typedef struct { int subblk, has_min, bias, actbias; } tl_fmt;

static int tl_fmt_of(int type, tl_fmt *f) {
    switch (type) {
    case ORC_TYPE_Q6_K: *f = (tl_fmt){16, 0, 32, 1}; return 1;
    case ORC_TYPE_Q5_K: *f = (tl_fmt){32, 1, 0, 0}; return 1;
    case ORC_TYPE_Q4_K: *f = (tl_fmt){32, 1, 0, 0}; return 1;
    case ORC_TYPE_IQ4_XS: *f = (tl_fmt){32, 0, 128, 0}; return 1;
    }
    return 0;
}

/* 32 packed bytes to their low and high nibbles (unpkNib4). */
static void tl_nib4(const uint8_t *src, uint8_t *lo, uint8_t *hi) {
    for (int l = 0; l < 32; ++l) { lo[l] = src[l] & 0x0F; hi[l] = src[l] >> 4; }
}

/* ORs the m-bit field at bit s of src[l] into bit d of dst[l] (unpkOr). */
static void tl_or(int s, int d, int m, uint8_t *dst, const uint8_t *src) {
    for (int l = 0; l < 32; ++l) dst[l] |= (uint8_t)(((src[l] >> s) & m) << d);
}

/* One unpacker per format (tiled.zig:102-330): num_k consecutive blocks of
 * n_rows rows, rows rs blocks apart, into the weight tile. */
static void tl_unpack_src0(int type, const uint8_t *base, size_t bsize, int64_t rs, int n_rows, tl_src0 *t, int num_k) {
    const int nb = type == ORC_TYPE_Q6_K ? 16 : 8;
    const size_t qk_stride = (size_t)num_k * TL_K, nb_stride = (size_t)nb * num_k;
    for (int slab = 0; slab < num_k; ++slab)
        for (int r = 0; r < n_rows; ++r) {
            const size_t d_off = (size_t)slab * TL_MICRO + r;
            uint8_t *q = t->q + r * qk_stride + (size_t)slab * TL_K;
            const size_t s_off = r * nb_stride + (size_t)slab * nb;
            const uint8_t *blk = base + ((size_t)r * rs + slab) * bsize;
            if (type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q5_K) {
                const uint16_t d = type == ORC_TYPE_Q4_K ? ((const blk_q4_K *)blk)->d : ((const blk_q5_K *)blk)->d;
                const uint16_t dm = type == ORC_TYPE_Q4_K ? ((const blk_q4_K *)blk)->dmin : ((const blk_q5_K *)blk)->dmin;
                const uint8_t *sc = type == ORC_TYPE_Q4_K ? ((const blk_q4_K *)blk)->scales : ((const blk_q5_K *)blk)->scales;
                const uint8_t *qs = type == ORC_TYPE_Q4_K ? ((const blk_q4_K *)blk)->qs : ((const blk_q5_K *)blk)->qs;
                t->d[d_off] = F32(d);
                t->dmin[d_off] = F32(dm);
                uint32_t utmp[4];
                unpack_scales_k4(sc, utmp); /* kScaleMins: eight scales then eight mins */
                const uint8_t *sm = (const uint8_t *)utmp;
                for (int s = 0; s < 8; ++s) { t->scales[s_off + s] = sm[s]; t->mins[s_off + s] = sm[8 + s]; }
                for (int c = 0; c < 4; ++c) tl_nib4(qs + 32 * c, q + 64 * c, q + 64 * c + 32);
                if (type == ORC_TYPE_Q5_K) /* 64-element chunk j takes qh bits 2j and 2j+1 */
                    for (int b = 0; b < 8; ++b) tl_or(b, 4, 1, q + 32 * b, ((const blk_q5_K *)blk)->qh);
            } else if (type == ORC_TYPE_Q6_K) {
                const blk_q6_K *x = (const blk_q6_K *)blk;
                t->d[d_off] = F32(x->d);
                for (int h = 0; h < 2; ++h) {
                    uint8_t *out = q + 128 * h;
                    const uint8_t *ql = x->ql + 64 * h, *qh = x->qh + 32 * h;
                    tl_nib4(ql, out, out + 64);
                    tl_nib4(ql + 32, out + 32, out + 96);
                    for (int b = 0; b < 4; ++b) tl_or(2 * b, 4, 3, out + 32 * b, qh);
                }
                for (int s = 0; s < 16; ++s) t->scales[s_off + s] = x->scales[s];
            } else { /* IQ4_XS: codes through kvalues_iq4nl + 128, scales ls - 32 */
                const blk_iq4_xs *x = (const blk_iq4_xs *)blk;
                t->d[d_off] = F32(x->d);
                for (int s = 0; s < 8; ++s) {
                    const int lo = (x->scales_l[s / 2] >> (4 * (s % 2))) & 0xf, hi = (x->scales_h >> (2 * s)) & 3;
                    t->scales[s_off + s] = (lo | (hi << 4)) - 32;
                }
                for (int w = 0; w < 4; ++w) {
                    uint8_t lo[32], hi[32];
                    tl_nib4(x->qs + 32 * w, lo, hi);
                    for (int j = 0; j < 16; ++j) {
                        q[64 * w + j] = (uint8_t)(KV_IQ4NL[lo[j]] + 128);
                        q[64 * w + 16 + j] = (uint8_t)(KV_IQ4NL[hi[j]] + 128);
                        q[64 * w + 32 + j] = (uint8_t)(KV_IQ4NL[lo[16 + j]] + 128);
                        q[64 * w + 48 + j] = (uint8_t)(KV_IQ4NL[hi[16 + j]] + 128);
                    }
                }
            }
        }
}

/* tiled_unpack_src1_q8_K (tiled.zig:565-594): num_k Q8_K blocks of each of
 * n_rows activation rows from block kblk on; the 16-row band's ragged tail
 * zeroed. */
static void tl_unpack_src1(const blk_q8_K *const *rows, int n_rows, tl_src1 *t, int kblk, int num_k) {
    const int n_padded = (n_rows + TL_MICRO - 1) & ~(TL_MICRO - 1);
    const int bs_stride = num_k == 1 ? TL_ROWS : TL_MICRO;
    const int n16 = TL_K / TL_MICRO;
    for (int slab = 0; slab < num_k; ++slab) {
        for (int r = 0; r < n_padded; ++r) {
            int8_t *dst = t->q + (size_t)r * num_k * TL_K + (size_t)slab * TL_K;
            if (r < n_rows) memcpy(dst, rows[r][kblk + slab].qs, TL_K);
            else memset(dst, 0, TL_K);
        }
        for (int r = 0; r < n_padded; ++r) {
            const blk_q8_K *x = r < n_rows ? &rows[r][kblk + slab] : NULL;
            for (int s = 0; s < n16; ++s) t->bsums[(slab * n16 + s) * bs_stride + r] = x ? x->bsums[s] : 0;
            t->d[slab * TL_MICRO + r] = x ? x->d : 0.0f;
        }
    }
}

/* tiled_repack_src1, __AVX2__ arm (tiled_kernel.zig:738-751): with the act
 * bias, each code of the 16-row band as q + 128 (sign bit flipped). */
static void tl_repack_src1(tl_src1 *t, int row0, int num_k, int bias) {
    if (!bias) return;
    const size_t row_stride = (size_t)num_k * TL_K;
    uint8_t *base = (uint8_t *)t->q + (size_t)row0 * row_stride;
    for (int r = 0; r < TL_MICRO; ++r)
        for (size_t o = 0; o < row_stride; ++o) base[r * row_stride + o] ^= 0x80;
}

/* tiled_repack_src0 (tiled_kernel.zig:773-797): for the act-bias formats,
 * each row's correction 128 * sum_s scales[s] * (sum of the sub-block's
 * debiased weights), kept in mins[r][0] (wrapping i32 arithmetic). */
static void tl_repack_src0(const tl_fmt *f, tl_src0 *t, int n_rows, int num_k) {
    if (!f->actbias) return;
    const int nb = TL_K / f->subblk;
    const size_t nb_stride = (size_t)nb * num_k;
    for (int slab = 0; slab < num_k; ++slab)
        for (int r = 0; r < n_rows; ++r) {
            const uint8_t *q = t->q + (size_t)r * num_k * TL_K + (size_t)slab * TL_K;
            const int32_t *sc = t->scales + r * nb_stride + (size_t)slab * nb;
            uint32_t corr = 0;
            for (int s = 0; s < nb; ++s) {
                int32_t qsum = 0;
                for (int k = 0; k < f->subblk; ++k) qsum += q[s * f->subblk + k];
                corr += 128u * (uint32_t)sc[s] * (uint32_t)(qsum - f->subblk * f->bias);
            }
            t->mins[r * nb_stride + (size_t)slab * nb] = (int32_t)corr;
        }
}

/* The column reduction the AVX2 microtile ends each group on
 * (tiled_kernel.zig:226-240): lane t = wrapping sum of acc[t]'s lanes. */
AVX2_FN static inline __m256i tl_column_sums(const __m256i acc[8]) {
    const __m256i ab = _mm256_hadd_epi32(acc[0], acc[1]), cd = _mm256_hadd_epi32(acc[2], acc[3]);
    const __m256i ef = _mm256_hadd_epi32(acc[4], acc[5]), gh = _mm256_hadd_epi32(acc[6], acc[7]);
    const __m256i abcd = _mm256_hadd_epi32(ab, cd), efgh = _mm256_hadd_epi32(ef, gh);
    const __m256i lo = _mm256_permute2x128_si256(abcd, efgh, 0x20), hi = _mm256_permute2x128_si256(abcd, efgh, 0x31);
    return _mm256_add_epi32(lo, hi);
}

/* tiled_run_microtile_avx2 (tiled_kernel.zig:505-690): the 16 x 16
 * microtile at (ri0, j0) over slab `slab` of a num_k-slab tile, added into
 * buf (row-major, buf_stride floats per row).  Per row, 8-column groups:
 * maddubs + madd against the broadcast sub-block scale; the min term from the
 * Q8_K bsums; then d * s1 (- dmin * s2 fused) and buf += res * d8 fused. */
AVX2_FN static void tl_microtile(const tl_fmt *f, const tl_src0 *s0, const tl_src1 *s1, int ri0, int j0, int num_k,
                                 int slab, float *buf, int buf_stride) {
    const int NB = TL_K / f->subblk;
    const size_t qk_stride = (size_t)num_k * TL_K, qk_off = (size_t)slab * TL_K;
    const size_t nb_stride = (size_t)NB * num_k, nb_off = (size_t)slab * NB;
    const size_t bs_stride = num_k == 1 ? TL_ROWS : TL_MICRO, bs_off = (size_t)slab * TL_MICRO;
    const __m256i bias8 = _mm256_set1_epi8((char)(uint8_t)f->bias);
    for (int i = 0; i < TL_MICRO; ++i) {
        const int ar = ri0 + i;
        const size_t d_off = (size_t)slab * TL_MICRO + ar;
        const float d0 = s0->d[d_off], dmin0 = s0->dmin[d_off];
        const uint8_t *q0 = s0->q + ar * qk_stride + qk_off;
        const int32_t *scales_row = s0->scales + ar * nb_stride + nb_off;
        const int32_t *mins_row = s0->mins + ar * nb_stride + nb_off;
        for (int g = 0; g < TL_MICRO; g += 8) {
            const int8_t *q1p[8];
            for (int t = 0; t < 8; ++t) q1p[t] = s1->q + (size_t)(j0 + g + t) * qk_stride + qk_off;
            __m256i s2 = _mm256_setzero_si256();
            __m256i acc[8];
            for (int t = 0; t < 8; ++t) acc[t] = _mm256_setzero_si256();
            if (f->subblk == 32) {
                for (int s = 0; s < NB; ++s) {
                    const __m256i q0v = _mm256_loadu_si256((const __m256i *)(q0 + s * 32));
                    const __m256i sc16 = _mm256_set1_epi16((short)scales_row[s]);
                    if (f->bias) { /* IQ4_XS: the sign trick on the debiased levels */
                        const __m256i w = _mm256_sub_epi8(q0v, bias8);
                        const __m256i ax = _mm256_sign_epi8(w, w);
                        for (int t = 0; t < 8; ++t) {
                            const __m256i q1 = _mm256_loadu_si256((const __m256i *)(q1p[t] + s * 32));
                            acc[t] = _mm256_add_epi32(acc[t],
                                                      _mm256_madd_epi16(sc16, _mm256_maddubs_epi16(ax, _mm256_sign_epi8(q1, w))));
                        }
                    } else {
                        for (int t = 0; t < 8; ++t) {
                            const __m256i q1 = _mm256_loadu_si256((const __m256i *)(q1p[t] + s * 32));
                            acc[t] = _mm256_add_epi32(acc[t], _mm256_madd_epi16(sc16, _mm256_maddubs_epi16(q0v, q1)));
                        }
                    }
                    if (f->has_min) {
                        const __m256i b0 = _mm256_loadu_si256((const __m256i *)(s1->bsums + (bs_off + 2 * s) * bs_stride + j0 + g));
                        const __m256i b1 = _mm256_loadu_si256((const __m256i *)(s1->bsums + (bs_off + 2 * s + 1) * bs_stride + j0 + g));
                        s2 = _mm256_add_epi32(s2, _mm256_mullo_epi32(_mm256_add_epi32(b0, b1), _mm256_set1_epi32(mins_row[s])));
                    }
                }
            } else { /* 16-wide sub-blocks (Q6_K): two per 32-byte load, scale per 128-bit half */
                for (int sp = 0; sp < NB; sp += 2) {
                    const __m256i q0v = _mm256_loadu_si256((const __m256i *)(q0 + sp * 16));
                    const __m256i scv = _mm256_set_m128i(_mm_set1_epi16((short)scales_row[sp + 1]),
                                                         _mm_set1_epi16((short)scales_row[sp]));
                    const __m256i w = _mm256_sub_epi8(q0v, bias8); /* debiased weight; act pre-biased by 128 */
                    for (int t = 0; t < 8; ++t) {
                        const __m256i q1b = _mm256_loadu_si256((const __m256i *)(q1p[t] + sp * 16));
                        acc[t] = _mm256_add_epi32(acc[t], _mm256_madd_epi16(scv, _mm256_maddubs_epi16(q1b, w)));
                    }
                }
            }
            __m256i s1v = tl_column_sums(acc);
            if (f->bias && f->actbias) s1v = _mm256_sub_epi32(s1v, _mm256_set1_epi32(mins_row[0]));
            const __m256 d1 = _mm256_loadu_ps(s1->d + (size_t)slab * TL_MICRO + j0 + g);
            __m256 res = _mm256_mul_ps(_mm256_set1_ps(d0), _mm256_cvtepi32_ps(s1v));
            if (f->has_min) res = _mm256_fnmadd_ps(_mm256_set1_ps(dmin0), _mm256_cvtepi32_ps(s2), res);
            float *bp = buf + (size_t)ar * buf_stride + j0 + g;
            _mm256_storeu_ps(bp, _mm256_fmadd_ps(res, d1, _mm256_loadu_ps(bp)));
        }
    }
}

/* ggml_tiled_narrow_k_extent (tiled.zig:697-710). */
static int tl_narrow_k_extent(int64_t n_rows, int64_t ne00) {
    const int l1 = 31 * 1024;
    int rows = (int)n_rows < TL_MICRO ? TL_MICRO : (int)n_rows;
    int ke = l1 / (TL_MICRO + rows);
    ke &= ~(TL_K - 1);
    const int ke_max = TL_ROWS * TL_K / TL_MICRO;
    if (ke > ke_max) ke = ke_max;
    while (ke >= TL_K && ne00 % ke != 0) ke -= TL_K;
    return ke < TL_K ? 0 : ke;
}

/* tiled_store_window (tiled.zig:714-737): the window back out, column-major. */
static void tl_store_window(const float *buf, int n0, int n1, int bs, float *dst, size_t dst_stride) {
    for (int ri = 0; ri < n0; ++ri)
        for (int j = 0; j < n1; ++j) dst[ri + j * dst_stride] = buf[(size_t)ri * bs + j];
}

typedef struct {
    int type, nth;
    tl_fmt f;
    const uint8_t *w;
    int64_t nrows, K, ncols;
    const float *x;
    float *dst;
    uint8_t *wdata; /* Q8_K rows of x */
    size_t wrow;
    tl_ws *ws;      /* one per thread */
    atomic_long current_chunk;
    int64_t nchunk0, nchunk1, dr0, dr1;
} tl_ctx;

typedef struct { tl_ctx *ctx; int ith; } tl_thread;

/* ggml_compute_forward_mul_mat_tiled_one_chunk (tiled.zig:982-1112), one
 * batch: 256 x 256 windows, the narrow path for windows of at most 16
 * columns, the standard per-slab path otherwise. */
AVX2_FN static void tl_one_chunk(tl_ctx *c, tl_ws *ws, int64_t ir0_start, int64_t ir0_end, int64_t ir1_start,
                                 int64_t ir1_end) {
    if (ir0_start >= ir0_end || ir1_start >= ir1_end) return;
    const size_t bsize = orc_type_size(c->type), rs_bytes = orc_row_size(c->type, c->K);
    const int64_t src0_stride = (int64_t)(rs_bytes / bsize);
    const blk_q8_K *rows[TL_ROWS];
    for (int64_t iir1 = ir1_start; iir1 < ir1_end;) {
        const int64_t iir1_end = iir1 + TL_ROWS < ir1_end ? iir1 + TL_ROWS : ir1_end;
        const int n_src1 = (int)(iir1_end - iir1);
        for (int r = 0; r < n_src1; ++r) rows[r] = (const blk_q8_K *)(c->wdata + (size_t)(iir1 + r) * c->wrow);
        for (int64_t iir0 = ir0_start; iir0 < ir0_end; iir0 += TL_ROWS) {
            const int64_t iir0_end = iir0 + TL_ROWS < ir0_end ? iir0 + TL_ROWS : ir0_end;
            const int n_src0 = (int)(iir0_end - iir0);
            memset(ws->acc, 0, sizeof ws->acc);
            if (n_src1 <= TL_MICRO) {
                const int k_extent = tl_narrow_k_extent(n_src1, c->K);
                const int num_k = k_extent / TL_K;
                for (int64_t k0 = 0; k0 < c->K; k0 += k_extent) {
                    const int kstart = (int)(k0 / TL_K);
                    tl_unpack_src1(rows, n_src1, &ws->src1, kstart, num_k);
                    tl_repack_src1(&ws->src1, 0, num_k, c->f.actbias);
                    for (int64_t ir0 = iir0; ir0 < iir0_end; ir0 += TL_MICRO) {
                        const int n0 = (int)(iir0_end - ir0 < TL_MICRO ? iir0_end - ir0 : TL_MICRO);
                        tl_unpack_src0(c->type, c->w + (size_t)ir0 * rs_bytes + (size_t)kstart * bsize, bsize,
                                       src0_stride, n0, &ws->src0, num_k);
                        tl_repack_src0(&c->f, &ws->src0, n0, num_k);
                        float *buf = ws->acc + (size_t)(ir0 - iir0) * TL_ROWS;
                        for (int slab = 0; slab < num_k; ++slab)
                            tl_microtile(&c->f, &ws->src0, &ws->src1, 0, 0, num_k, slab, buf, TL_ROWS);
                    }
                }
            } else {
                for (int64_t ib = 0; ib < c->K; ib += TL_K) {
                    const int kblk = (int)(ib / TL_K);
                    tl_unpack_src0(c->type, c->w + (size_t)iir0 * rs_bytes + (size_t)kblk * bsize, bsize, src0_stride,
                                   n_src0, &ws->src0, 1);
                    tl_repack_src0(&c->f, &ws->src0, n_src0, 1);
                    tl_unpack_src1(rows, n_src1, &ws->src1, kblk, 1);
                    for (int64_t ir1 = iir1; ir1 < iir1_end; ir1 += TL_MICRO) {
                        tl_repack_src1(&ws->src1, (int)(ir1 - iir1), 1, c->f.actbias);
                        for (int64_t ir0 = iir0; ir0 < iir0_end; ir0 += TL_MICRO)
                            tl_microtile(&c->f, &ws->src0, &ws->src1, (int)(ir0 - iir0), (int)(ir1 - iir1), 1, 0,
                                         ws->acc, TL_ROWS);
                    }
                }
            }
            tl_store_window(ws->acc, n_src0, n_src1, TL_ROWS, c->dst + iir0 + iir1 * c->nrows, (size_t)c->nrows);
        }
        iir1 = iir1_end;
    }
}

static void *tl_stage_worker(void *arg) {
    tl_thread *t = (tl_thread *)arg;
    tl_ctx *c = t->ctx;
    const int64_t nbk = c->K / QK_K;
    const int64_t b0 = (int64_t)t->ith * nbk / c->nth, b1 = ((int64_t)t->ith + 1) * nbk / c->nth;
    for (int64_t j = 0; j < c->ncols; ++j)
        orc_quantize_row_q8_K_ref(c->x + j * c->K + b0 * QK_K, c->wdata + (size_t)j * c->wrow + (size_t)b0 * sizeof(blk_q8_K),
                                  (b1 - b0) * QK_K);
    return NULL;
}

static void *tl_compute_worker(void *arg) {
    tl_thread *t = (tl_thread *)arg;
    tl_ctx *c = t->ctx;
    long chunk = t->ith;
    while (chunk < c->nchunk0 * c->nchunk1) {
        const int64_t i0 = chunk % c->nchunk0, i1 = chunk / c->nchunk0;
        const int64_t r0 = c->dr0 * i0, r1 = c->dr1 * i1;
        tl_one_chunk(c, &c->ws[t->ith], r0, r0 + c->dr0 < c->nrows ? r0 + c->dr0 : c->nrows, r1,
                     r1 + c->dr1 < c->ncols ? r1 + c->dr1 : c->ncols);
        if (c->nth >= c->nchunk0 * c->nchunk1) break;
        chunk = atomic_fetch_add(&c->current_chunk, 1);
    }
    return NULL;
}
#endif /* ORC_X86 */

int orc_mul_mat_tiled(int type, const void *w, int64_t nrows, int64_t K, const float *x, int64_t ncols, float *dst,
                      int nth) {
#if ORC_X86
    tl_fmt f;
    if (!orc_has_avx2() || !tl_fmt_of(type, &f) || K % QK_K != 0 || nrows <= 0 || ncols <= 0) return 0;
    if (nth < 1) nth = 1;
    tl_ctx c;
    memset(&c, 0, sizeof c);
    c.type = type; c.nth = nth; c.f = f; c.w = (const uint8_t *)w;
    c.nrows = nrows; c.K = K; c.ncols = ncols; c.x = x; c.dst = dst;
    c.wrow = (size_t)(K / QK_K) * sizeof(blk_q8_K);
    c.wdata = (uint8_t *)malloc(c.wrow * (size_t)ncols);
    c.ws = (tl_ws *)aligned_alloc(64, sizeof(tl_ws) * (size_t)nth);
    memset(c.ws, 0, sizeof(tl_ws) * (size_t)nth);
    tl_thread *ts = (tl_thread *)malloc(sizeof(tl_thread) * (size_t)nth);
    for (int i = 0; i < nth; ++i) { ts[i].ctx = &c; ts[i].ith = i; }
    run_threads(nth, ts, sizeof(tl_thread), tl_stage_worker);
    /* chunking of mulMatDriver (tiled.zig:1175-1195): 256 halved until four
     * chunks per thread, not below the 16-row microtile */
    int64_t chunk = 256;
    int64_t n0 = (nrows + chunk - 1) / chunk, n1 = (ncols + chunk - 1) / chunk;
    while (n0 * n1 < (int64_t)nth * 4 && chunk > 16) {
        chunk /= 2;
        n0 = (nrows + chunk - 1) / chunk;
        n1 = (ncols + chunk - 1) / chunk;
    }
    c.nchunk0 = n0; c.nchunk1 = n1;
    c.dr0 = (nrows + n0 - 1) / n0; c.dr1 = (ncols + n1 - 1) / n1;
    atomic_store(&c.current_chunk, nth);
    run_threads(nth, ts, sizeof(tl_thread), tl_compute_worker);
    free(ts);
    free(c.ws);
    free(c.wdata);
    return 1;
#else
    (void)type; (void)w; (void)nrows; (void)K; (void)x; (void)ncols; (void)dst; (void)nth;
    return 0;
#endif
}

/* ------------------------------------------------------------------------ */
/* The reference's x86 Q8_0 / Q4_0 GEMM: llamafile_sgemm's tinyBLAS_Q0_AVX
 * (src/ggml/cpu/ops/sgemm.zig:578-880, dispatched at :1067-1070 and reached
 * from mul_mat's second llamafile attempt, src/ggml/cpu/mulmat.zig:336-367,
 * for src1 of 2 or more columns once it is staged as Q8_0).  Every tile
 * kernel (gemm4xN, gemmMx4, gemm; sgemm.zig:771-880) gives an output the same
 * value, so only the per-output arithmetic is restated:
 *   for each block l: s = f32(d_a) * f32(d_b); lane i (0..7) of the block's
 *   dot is the exact int32 sum of elements 4i..4i+3 (dot via maddubs / madd,
 *   sgemm.zig:634-645; no saturation for these operands), converted to f32;
 *   acc[i] = fma(s, lane_i, acc[i]);
 *   out = hsumAvx(acc) = (h0 + h2) + (h1 + h3) with h = acc[4..7] + acc[0..3]
 *   (sgemm.zig:119-124).
 * Q4_0 weights are their nibbles minus 8, low nibbles first (denibble,
 * sgemm.zig:594-600, 618-620). */

static int tb_lane_dots(int type, const uint8_t *a, const blk_q8_0 *b, int32_t lanes[8], float *da) {
    int8_t av[32];
    if (type == ORC_TYPE_Q8_0) {
        const blk_q8_0 *q = (const blk_q8_0 *)a;
        memcpy(av, q->qs, 32);
        *da = orc_fp16_to_fp32(q->d);
    } else {
        const blk_q4_0 *q = (const blk_q4_0 *)a;
        for (int j = 0; j < 16; ++j) {
            av[j] = (int8_t)((q->qs[j] & 0x0F) - 8);
            av[j + 16] = (int8_t)((q->qs[j] >> 4) - 8);
        }
        *da = orc_fp16_to_fp32(q->d);
    }
    for (int i = 0; i < 8; ++i) {
        int32_t s = 0;
        for (int m = 0; m < 4; ++m) s += (int32_t)av[4 * i + m] * (int32_t)b->qs[4 * i + m];
        lanes[i] = s;
    }
    return 0;
}

typedef struct {
    int type;
    const uint8_t *w;
    const blk_q8_0 *y;
    int64_t nrows, nb, ncols, nth;
    size_t wrow;
    float *dst;
} tb_ctx;

typedef struct { tb_ctx *c; int ith; } tb_thread;

/* The per-output restatement above, one output at a time: the values every
 * tile kernel must give (kept as the check of the tile loops below). */
static void *tb_worker_scalar(void *arg) {
    tb_thread *t = (tb_thread *)arg;
    const tb_ctx *c = t->c;
    const size_t ab = c->type == ORC_TYPE_Q8_0 ? sizeof(blk_q8_0) : sizeof(blk_q4_0);
    const int64_t r0 = c->nrows * t->ith / c->nth, r1 = c->nrows * (t->ith + 1) / c->nth;
    for (int64_t col = 0; col < c->ncols; ++col)
        for (int64_t r = r0; r < r1; ++r) {
            float acc[8] = {0};
            for (int64_t l = 0; l < c->nb; ++l) {
                int32_t lanes[8];
                float da;
                const blk_q8_0 *b = c->y + col * c->nb + l;
                tb_lane_dots(c->type, c->w + (size_t)r * c->wrow + (size_t)l * ab, b, lanes, &da);
                const float s = da * orc_fp16_to_fp32(b->d);
                for (int i = 0; i < 8; ++i) acc[i] = fmaf(s, (float)lanes[i], acc[i]);
            }
            float h[4];
            for (int i = 0; i < 4; ++i) h[i] = acc[4 + i] + acc[i];
            c->dst[col * c->nrows + r] = (h[0] + h[2]) + (h[1] + h[3]);
        }
    return NULL;
}

#if ORC_X86
/* tinyBLAS_Q0_AVX's tile loops (sgemm.zig:578-880), the x86-64-v3 arm
 * (VECTOR_REGISTERS 16): mnpack (:667-760) covers the m x n outputs with
 * gemm4xN (4 rows of A, their deltas converted together, against RN
 * columns), gemmMx4 (RM rows against 4 columns) and gemm (RM x RN), each
 * splitting its tiles statically over the threads (duty, :763-769, columns
 * fastest).  Every kernel gives an output the same value: per block l,
 * fma(f32(d_a) * f32(d_b), updot(|a|, b * sign a), acc), then hsumAvx. */
typedef struct {
    int q4;                 /* A is Q4_0 (else Q8_0) */
    const uint8_t *A;
    size_t ab;              /* bytes per A block */
    int64_t lda;            /* A row stride, blocks */
    const blk_q8_0 *B;
    int64_t ldb;            /* B column stride, blocks */
    float *C;
    int64_t ldc, k, ith, nth;
} tbq;

AVX2_FN static inline const uint8_t *tbq_a(const tbq *t, int64_t row, int64_t l) {
    return t->A + (size_t)(t->lda * row + l) * t->ab;
}
AVX2_FN static inline uint16_t tbq_ad(const tbq *t, int64_t row, int64_t l) {
    uint16_t d;
    memcpy(&d, tbq_a(t, row, l), 2);
    return d;
}
/* load (sgemm.zig:620-631): a block's 32 weights as signed bytes */
AVX2_FN static inline __m256i tbq_load_a(const tbq *t, int64_t row, int64_t l) {
    const uint8_t *p = tbq_a(t, row, l) + 2;
    if (!t->q4) return _mm256_loadu_si256((const __m256i *)p);
    const __m128i x = _mm_loadu_si128((const __m128i *)p);
    const __m256i nib = _mm256_and_si256(_mm256_set1_epi8(15), _mm256_set_m128i(_mm_srli_epi16(x, 4), x));
    return _mm256_sub_epi8(nib, _mm256_set1_epi8(8));
}
AVX2_FN static inline __m256i tbq_load_b(const tbq *t, int64_t col, int64_t l) {
    return _mm256_loadu_si256((const __m256i *)t->B[t->ldb * col + l].qs);
}
/* dot (sgemm.zig:645-648): updot(sign(a, a), sign(b, a)) */
AVX2_FN static inline __m256 tbq_dot(__m256i a, __m256i b) {
    const __m256i u = _mm256_maddubs_epi16(_mm256_sign_epi8(a, a), _mm256_sign_epi8(b, a));
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_set1_epi16(1), u));
}
/* hsumAvx (sgemm.zig:119-124) */
AVX2_FN static inline float tbq_hsum(__m256 x) {
    const __m128 h = _mm_add_ps(_mm256_extractf128_ps(x, 1), _mm256_castps256_ps128(x));
    float v[4];
    _mm_storeu_ps(v, h);
    return (v[0] + v[2]) + (v[1] + v[3]);
}
static inline void tbq_duty(const tbq *t, int64_t tiles, int64_t *start, int64_t *end) {
    const int64_t d = (tiles + t->nth - 1) / t->nth;
    *start = d * t->ith;
    *end = *start + d < tiles ? *start + d : tiles;
}

#define TBQ_INLINE __attribute__((always_inline, target("avx2,fma,f16c"))) static inline

TBQ_INLINE void tbq_gemm4xN(const tbq *t, const int RN, int64_t m0, int64_t m, int64_t n0, int64_t n) {
    const int64_t ytiles = (m - m0) / 4, xtiles = (n - n0) / RN;
    int64_t job, end;
    tbq_duty(t, xtiles * ytiles, &job, &end);
    for (; job < end; ++job) {
        const int64_t ii = m0 + job / xtiles * 4, jj = n0 + job % xtiles * RN;
        __m256 Cv[4][4];
        for (int j = 0; j < RN; ++j)
            for (int i = 0; i < 4; ++i) Cv[j][i] = _mm256_setzero_ps();
        for (int64_t l = 0; l < t->k; ++l) {
            const __m128 da = _mm_cvtph_ps(_mm_set_epi16(0, 0, 0, 0, (short)tbq_ad(t, ii + 3, l),
                                                        (short)tbq_ad(t, ii + 2, l), (short)tbq_ad(t, ii + 1, l),
                                                        (short)tbq_ad(t, ii + 0, l)));
            __m256i avec[4];
            for (int i = 0; i < 4; ++i) avec[i] = tbq_load_a(t, ii + i, l);
            for (int j = 0; j < RN; ++j) {
                const blk_q8_0 *b = &t->B[t->ldb * (jj + j) + l];
                float dv[4];
                _mm_storeu_ps(dv, _mm_mul_ps(da, _mm_set1_ps(_cvtsh_ss(b->d))));
                const __m256i bv = _mm256_loadu_si256((const __m256i *)b->qs);
                for (int i = 0; i < 4; ++i) Cv[j][i] = _mm256_fmadd_ps(_mm256_set1_ps(dv[i]), tbq_dot(avec[i], bv), Cv[j][i]);
            }
        }
        for (int j = 0; j < RN; ++j)
            for (int i = 0; i < 4; ++i) t->C[t->ldc * (jj + j) + ii + i] = tbq_hsum(Cv[j][i]);
    }
}

TBQ_INLINE void tbq_gemmMx4(const tbq *t, const int RM, int64_t m0, int64_t m, int64_t n0, int64_t n) {
    const int64_t ytiles = (m - m0) / RM, xtiles = (n - n0) / 4;
    int64_t job, end;
    tbq_duty(t, xtiles * ytiles, &job, &end);
    for (; job < end; ++job) {
        const int64_t ii = m0 + job / xtiles * RM, jj = n0 + job % xtiles * 4;
        __m256 Cv[4][4];
        for (int j = 0; j < 4; ++j)
            for (int i = 0; i < RM; ++i) Cv[j][i] = _mm256_setzero_ps();
        for (int64_t l = 0; l < t->k; ++l) {
            const __m128 db = _mm_cvtph_ps(_mm_set_epi16(0, 0, 0, 0, (short)t->B[t->ldb * (jj + 3) + l].d,
                                                        (short)t->B[t->ldb * (jj + 2) + l].d,
                                                        (short)t->B[t->ldb * (jj + 1) + l].d,
                                                        (short)t->B[t->ldb * (jj + 0) + l].d));
            __m256i bvec[4];
            for (int j = 0; j < 4; ++j) bvec[j] = tbq_load_b(t, jj + j, l);
            for (int i = 0; i < RM; ++i) {
                float dv[4];
                _mm_storeu_ps(dv, _mm_mul_ps(_mm_set1_ps(_cvtsh_ss(tbq_ad(t, ii + i, l))), db));
                const __m256i av = tbq_load_a(t, ii + i, l);
                for (int j = 0; j < 4; ++j) Cv[j][i] = _mm256_fmadd_ps(_mm256_set1_ps(dv[j]), tbq_dot(av, bvec[j]), Cv[j][i]);
            }
        }
        for (int j = 0; j < 4; ++j)
            for (int i = 0; i < RM; ++i) t->C[t->ldc * (jj + j) + ii + i] = tbq_hsum(Cv[j][i]);
    }
}

TBQ_INLINE void tbq_gemm(const tbq *t, const int RM, const int RN, int64_t m0, int64_t m, int64_t n0, int64_t n) {
    const int64_t ytiles = (m - m0) / RM, xtiles = (n - n0) / RN;
    int64_t job, end;
    tbq_duty(t, xtiles * ytiles, &job, &end);
    for (; job < end; ++job) {
        const int64_t ii = m0 + job / xtiles * RM, jj = n0 + job % xtiles * RN;
        __m256 Cv[3][3];
        for (int j = 0; j < RN; ++j)
            for (int i = 0; i < RM; ++i) Cv[j][i] = _mm256_setzero_ps();
        for (int64_t l = 0; l < t->k; ++l)
            for (int j = 0; j < RN; ++j)
                for (int i = 0; i < RM; ++i) {
                    const blk_q8_0 *b = &t->B[t->ldb * (jj + j) + l];
                    const __m256 ud = tbq_dot(tbq_load_a(t, ii + i, l), _mm256_loadu_si256((const __m256i *)b->qs));
                    const float d = _cvtsh_ss(tbq_ad(t, ii + i, l)) * _cvtsh_ss(b->d);
                    Cv[j][i] = _mm256_fmadd_ps(_mm256_set1_ps(d), ud, Cv[j][i]);
                }
        for (int j = 0; j < RN; ++j)
            for (int i = 0; i < RM; ++i) t->C[t->ldc * (jj + j) + ii + i] = tbq_hsum(Cv[j][i]);
    }
}

/* mnpack (sgemm.zig:667-760), VECTOR_REGISTERS 16 */
AVX2_FN static void tbq_mnpack(const tbq *t, int64_t m0, int64_t m, int64_t n0, int64_t n) {
    const int64_t dm = m - m0 < 4 ? m - m0 : 4, dn = n - n0 < 4 ? n - n0 : 4;
    int64_t mc, nc;
    switch ((dm << 4) | dn) {
    case 0x44: case 0x43: case 0x42: tbq_gemm4xN(t, 2, m0, m, n0, n); mc = 4; nc = 2; break;
    case 0x34: case 0x24: tbq_gemmMx4(t, 2, m0, m, n0, n); mc = 2; nc = 4; break;
    case 0x33: case 0x32: tbq_gemm(t, 3, 2, m0, m, n0, n); mc = 3; nc = 2; break;
    case 0x23: tbq_gemm(t, 2, 3, m0, m, n0, n); mc = 2; nc = 3; break;
    case 0x41: tbq_gemm4xN(t, 1, m0, m, n0, n); mc = 4; nc = 1; break;
    case 0x22: tbq_gemm(t, 2, 2, m0, m, n0, n); mc = 2; nc = 2; break;
    case 0x14: tbq_gemmMx4(t, 1, m0, m, n0, n); mc = 1; nc = 4; break;
    case 0x31: tbq_gemm(t, 3, 1, m0, m, n0, n); mc = 3; nc = 1; break;
    case 0x13: tbq_gemm(t, 1, 3, m0, m, n0, n); mc = 1; nc = 3; break;
    case 0x21: tbq_gemm(t, 2, 1, m0, m, n0, n); mc = 2; nc = 1; break;
    case 0x12: tbq_gemm(t, 1, 2, m0, m, n0, n); mc = 1; nc = 2; break;
    case 0x11: tbq_gemm(t, 1, 1, m0, m, n0, n); mc = 1; nc = 1; break;
    default: return;
    }
    const int64_t mp = m0 + (m - m0) / mc * mc, np = n0 + (n - n0) / nc * nc;
    tbq_mnpack(t, mp, m, n0, np);
    tbq_mnpack(t, m0, m, np, n);
}
#endif /* ORC_X86 */

/* One thread's llamafile_sgemm call (mulmat.zig:336-367 calls it from every
 * thread with its ith / nth; tinyBLAS_Q0_AVX's matmul = mnpack(0, m, 0, n)). */
static void *tb_worker(void *arg) {
    tb_thread *t = (tb_thread *)arg;
    const tb_ctx *c = t->c;
#if ORC_X86
    tbq q;
    q.q4 = c->type == ORC_TYPE_Q4_0;
    q.A = c->w;
    q.ab = q.q4 ? sizeof(blk_q4_0) : sizeof(blk_q8_0);
    q.lda = (int64_t)(c->wrow / q.ab);
    q.B = c->y;
    q.ldb = c->nb;
    q.C = c->dst;
    q.ldc = c->nrows;
    q.k = c->nb;
    q.ith = t->ith;
    q.nth = c->nth;
    tbq_mnpack(&q, 0, c->nrows, 0, c->ncols);
    return NULL;
#else
    return tb_worker_scalar(arg);
#endif
}

int orc_tinyblas_q0(int type, const void *w, int64_t nrows, int64_t K, const void *y_q8_0, int64_t ncols,
                    float *dst, int nth) {
    if ((type != ORC_TYPE_Q8_0 && type != ORC_TYPE_Q4_0) || K % QK8_0 != 0 || nrows <= 0 || ncols <= 0) return 0;
    if (nth < 1) nth = 1;
    tb_ctx c;
    c.type = type;
    c.w = (const uint8_t *)w;
    c.y = (const blk_q8_0 *)y_q8_0;
    c.nrows = nrows;
    c.nb = K / QK8_0;
    c.ncols = ncols;
    c.nth = nth;
    c.wrow = orc_row_size(type, K);
    c.dst = dst;
    tb_thread *ts = (tb_thread *)malloc(sizeof(tb_thread) * (size_t)nth);
    for (int i = 0; i < nth; ++i) { ts[i].c = &c; ts[i].ith = i; }
    run_threads(nth, ts, sizeof *ts, tb_worker);
    free(ts);
    return 1;
}

/* The same outputs, one at a time (the per-output restatement: the check of
 * the tile loops). */
int orc_tinyblas_q0_per_output(int type, const void *w, int64_t nrows, int64_t K, const void *y_q8_0, int64_t ncols,
                               float *dst, int nth) {
    if ((type != ORC_TYPE_Q8_0 && type != ORC_TYPE_Q4_0) || K % QK8_0 != 0 || nrows <= 0 || ncols <= 0) return 0;
    if (nth < 1) nth = 1;
    tb_ctx c;
    c.type = type;
    c.w = (const uint8_t *)w;
    c.y = (const blk_q8_0 *)y_q8_0;
    c.nrows = nrows;
    c.nb = K / QK8_0;
    c.ncols = ncols;
    c.nth = nth;
    c.wrow = orc_row_size(type, K);
    c.dst = dst;
    tb_thread *ts = (tb_thread *)malloc(sizeof(tb_thread) * (size_t)nth);
    for (int i = 0; i < nth; ++i) { ts[i].c = &c; ts[i].ith = i; }
    run_threads(nth, ts, sizeof *ts, tb_worker_scalar);
    free(ts);
    return 1;
}

int orc_mul_mat_tinyblas(int type, const void *w, int64_t nrows, int64_t K, const float *x, int64_t ncols,
                         float *dst, int nth) {
    /* llamafile_sgemm returns false below 2 columns (sgemm.zig:898) */
    if ((type != ORC_TYPE_Q8_0 && type != ORC_TYPE_Q4_0) || ncols < 2 || K % QK8_0 != 0 || !orc_has_avx2())
        return 0;
    const size_t yrow = orc_row_size(ORC_TYPE_Q8_0, K);
    uint8_t *y = (uint8_t *)malloc(yrow * (size_t)ncols);
    for (int64_t col = 0; col < ncols; ++col) orc_quantize_row_q8_0_avx2(x + col * K, y + (size_t)col * yrow, K);
    const int ok = orc_tinyblas_q0(type, w, nrows, K, y, ncols, dst, nth);
    free(y);
    return ok;
}
