// mmq.hip -- prefill GEMM (more than 8 activation columns) of Q4_K / Q6_K /
// Q8_0 weights against planar Q8_1 activations on CDNA4 int8 MFMA.
//
// Replaces the reference's MMQ path (mul_mat_q, src/ggml/cuda/mmq.zig:282-408,
// chosen at mmq.zig:865-917).  Integer block dots are formed exactly by
// v_mfma_i32_32x32x32_i8 (one 32-deep Q8_1 block: Q4_K sub-blocks, Q8_0
// blocks) or v_mfma_i32_32x32x16_i8 (Q6_K's 16-deep sub-blocks) and then
// scaled per (row, column, block) in fp32:
//   Q4_K: out = sum_j d*sc_j*d8_j*S_j - sum_j dmin*m_j*s8_j
//   Q6_K: out = sum_k d*sc_k*d8_{k/2}*T_k      (T over q6-32)
//   Q8_0: out = sum_b d_b*d8_b*S_b
// The Q4_K min term is itself a small GEMM over K/32: per super-block the f16
// MFMA (v_mfma_f32_32x32x8_f16, K = its 8 sub-blocks) forms sum_j m_j*s8_j
// exactly (6-bit integers times f16 values), and dmin scales it in fp32.
//
// Tiling: a 256-thread workgroup computes a 128x128 output tile; each wave a
// 64x64 quarter as 2x2 MFMA tiles of 32x32.  K advances one 256-element
// super-block at a time: the workgroup unpacks the 128 weight rows' nibbles
// / 6-bit values to int8 in LDS (with their fp32 sub-block scales) and stages
// the 128 activation columns' int8 values and (d8, s8) beside them.
//
// MFMA operand convention: for a 32x32xK tile, lane l supplies row (l % 32)
// of A and column (l % 32) of B over the K-slice [(l / 32) * K/2, +K/2).  A and
// B use the same slice, so the sum over K is formed whatever order the
// hardware assigns to the slices.  Results use the 32x32 accumulator layout:
// value v of lane l is row 8*(v/4) + 4*(l/32) + v%4, column l%32.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 256;
constexpr int LDA = BK + 16;  // int8 row stride in LDS (pad breaks bank aliasing)
constexpr int NTHREADS = 256;

template <int TYPE>
struct MmqFmt {
    static constexpr int GK = TYPE == TYPE_Q6_K ? 16 : 32;  // depth of one integer block dot
    static constexpr int NG = BK / GK;                      // scale groups per K-step
};

template <int TYPE>
struct Smem {
    int8_t a[BM * LDA];
    int8_t b[BN * LDA];
    float ascale[MmqFmt<TYPE>::NG][BM];  // d * sc per (group, row)
    float bd[8][BN];                      // d8 per (Q8_1 block, column)
    _Float16 amin[BM][8];                 // m_j as f16 (Q4_K)
    float admin[BM];                      // dmin       (Q4_K)
    _Float16 bs8[BN][8];                  // s8          (Q4_K)
};

// ---- staging of one K-step (256 elements) of the 128 weight rows ----------

__device__ __forceinline__ void store16(int8_t *dst, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *reinterpret_cast<uint4 *>(dst) = make_uint4(a, b, c, d);
}

template <int TYPE>
__device__ void stage_a(Smem<TYPE> &sm, const uint8_t *w, int64_t row_stride, int64_t nrows, int64_t row0,
                        int64_t kb) {
    const int t = threadIdx.x;
    if constexpr (TYPE == TYPE_Q4_K) {
        const int r = t >> 1, half = t & 1;
        int8_t *arow = sm.a + r * LDA;
        if (row0 + r < nrows) {
            const uint8_t *blk = w + (row0 + r) * row_stride + kb * Q4K_BYTES;
            const uint4 hdr = ld_u128(blk);
            const float d = h2f(hdr.x);
            if (half == 0) sm.admin[r] = h2f(hdr.x >> 16);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int c = 2 * half + cc;
                const uint4 q0 = ld_u128(blk + 16 + 32 * c);
                const uint4 q1 = ld_u128(blk + 16 + 32 * c + 16);
                const uint32_t m = 0x0F0F0F0Fu;
                store16(arow + 64 * c + 0, q0.x & m, q0.y & m, q0.z & m, q0.w & m);
                store16(arow + 64 * c + 16, q1.x & m, q1.y & m, q1.z & m, q1.w & m);
                store16(arow + 64 * c + 32, (q0.x >> 4) & m, (q0.y >> 4) & m, (q0.z >> 4) & m, (q0.w >> 4) & m);
                store16(arow + 64 * c + 48, (q1.x >> 4) & m, (q1.y >> 4) & m, (q1.z >> 4) & m, (q1.w >> 4) & m);
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int j = 2 * c + jj;
                    uint32_t sc, mn;
                    q4k_scale_min(j, hdr.y, hdr.z, hdr.w, sc, mn);
                    sm.ascale[j][r] = d * (float)sc;
                    sm.amin[r][j] = (_Float16)(float)mn;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) store16(arow + 128 * half + 16 * i, 0, 0, 0, 0);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                sm.ascale[4 * half + jj][r] = 0.0f;
                sm.amin[r][4 * half + jj] = (_Float16)0.0f;
            }
            if (half == 0) sm.admin[r] = 0.0f;
        }
    } else if constexpr (TYPE == TYPE_Q6_K) {
        const int r = t >> 1, n = t & 1;
        int8_t *arow = sm.a + r * LDA + 128 * n;
        if (row0 + r < nrows) {
            const uint8_t *blk = w + (row0 + r) * row_stride + kb * Q6K_BYTES;
            const float d = h2f(ld_u16(blk + 208));
            const uint4 sc = ld16_a2(blk + 192);
#pragma unroll
            for (int i = 0; i < 8; ++i) sm.ascale[8 * n + i][r] = d * (float)(int8_t)byte_of(sc, 8 * n + i);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const uint4 l0 = ld16_a2(blk + 64 * n + 16 * hh);
                const uint4 l1 = ld16_a2(blk + 64 * n + 32 + 16 * hh);
                const uint4 qh = ld16_a2(blk + 128 + 32 * n + 16 * hh);
                const uint32_t L0[4] = {l0.x, l0.y, l0.z, l0.w}, L1[4] = {l1.x, l1.y, l1.z, l1.w};
                const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
                uint32_t v[4][4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = 0x0F0F0F0Fu, hm = 0x30303030u;
                    const uint32_t u0 = (L0[i] & m) | ((H[i] << 4) & hm);
                    const uint32_t u1 = (L1[i] & m) | ((H[i] << 2) & hm);
                    const uint32_t u2 = ((L0[i] >> 4) & m) | (H[i] & hm);
                    const uint32_t u3 = ((L1[i] >> 4) & m) | ((H[i] >> 2) & hm);
                    // bytewise -32 without borrows: (u | 0x80) - 0x20, then flip the top bit back
                    v[0][i] = ((u0 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                    v[1][i] = ((u1 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                    v[2][i] = ((u2 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                    v[3][i] = ((u3 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                }
#pragma unroll
                for (int g = 0; g < 4; ++g) store16(arow + 32 * g + 16 * hh, v[g][0], v[g][1], v[g][2], v[g][3]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) store16(arow + 16 * i, 0, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 8; ++i) sm.ascale[8 * n + i][r] = 0.0f;
        }
    } else {  // Q8_0: 8 blocks of 34 B per row per K-step
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int idx = t + NTHREADS * it;  // 0..1023 = row * 8 + block
            const int r = idx >> 3, b = idx & 7;
            int8_t *dst = sm.a + r * LDA + 32 * b;
            if (row0 + r < nrows) {
                const uint8_t *blk = w + (row0 + r) * row_stride + (kb * 8 + b) * Q80_BYTES;
                const uint4 q0 = ld16_a2(blk + 2), q1 = ld16_a2(blk + 18);
                store16(dst, q0.x, q0.y, q0.z, q0.w);
                store16(dst + 16, q1.x, q1.y, q1.z, q1.w);
                sm.ascale[b][r] = h2f(ld_u16(blk));
            } else {
                store16(dst, 0, 0, 0, 0);
                store16(dst + 16, 0, 0, 0, 0);
                sm.ascale[b][r] = 0.0f;
            }
        }
    }
}

template <int TYPE>
__device__ void stage_b(Smem<TYPE> &sm, const int8_t *yqs, const uint32_t *yds, int64_t Kp, int64_t ncols,
                        int64_t col0, int64_t kb) {
    const int t = threadIdx.x;
    const int c = t >> 1, half = t & 1;
    int8_t *brow = sm.b + c * LDA + 128 * half;
    if (col0 + c < ncols) {
        const uint8_t *src = reinterpret_cast<const uint8_t *>(yqs + (col0 + c) * Kp + kb * BK + 128 * half);
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4 *>(brow + 16 * i) = ld_u128(src + 16 * i);
        const uint4 ds = *reinterpret_cast<const uint4 *>(yds + (col0 + c) * (Kp / QK8) + kb * 8 + 4 * half);
        const uint32_t dv[4] = {ds.x, ds.y, ds.z, ds.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sm.bd[4 * half + i][c] = h2f(dv[i]);
            if constexpr (TYPE == TYPE_Q4_K) sm.bs8[c][4 * half + i] = __builtin_bit_cast(_Float16, (uint16_t)(dv[i] >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4 *>(brow + 16 * i) = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sm.bd[4 * half + i][c] = 0.0f;
            if constexpr (TYPE == TYPE_Q4_K) sm.bs8[c][4 * half + i] = (_Float16)0.0f;
        }
    }
}

template <int TYPE>
__global__ __launch_bounds__(NTHREADS) void mmq_kernel(const uint8_t *__restrict__ w, int64_t K, int64_t nrows,
                                                       int64_t row_stride, const int8_t *__restrict__ yqs,
                                                       const uint32_t *__restrict__ yds, int64_t ncols,
                                                       float *__restrict__ dst, int64_t dst_col_stride) {
    using F = MmqFmt<TYPE>;
    __shared__ Smem<TYPE> sm;
    const int64_t Kp = pad_k(K);
    const int64_t row0 = (int64_t)blockIdx.x * BM;
    const int64_t col0 = (int64_t)blockIdx.y * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;  // wave's sub-tile
    const int li = lane & 31, lh = lane >> 5;

    v16f acc[2][2], accm[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = accm[i][j][v] = 0.0f;

    const int64_t nkb = K / BK;
    for (int64_t kb = 0; kb < nkb; ++kb) {
        stage_a<TYPE>(sm, w, row_stride, nrows, row0, kb);
        stage_b<TYPE>(sm, yqs, yds, Kp, ncols, col0, kb);
        __syncthreads();

#pragma unroll 2
        for (int g = 0; g < F::NG; ++g) {
            v16i S[2][2];
            if constexpr (F::GK == 32) {
                v4i a[2], b[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    a[i] = *reinterpret_cast<const v4i *>(sm.a + (wr + 32 * i + li) * LDA + 32 * g + 16 * lh);
                    b[i] = *reinterpret_cast<const v4i *>(sm.b + (wc + 32 * i + li) * LDA + 32 * g + 16 * lh);
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const v16i z = {0};
                        S[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], z, 0, 0, 0);
                    }
            } else {
                long a[2], b[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    a[i] = *reinterpret_cast<const long *>(sm.a + (wr + 32 * i + li) * LDA + 16 * g + 8 * lh);
                    b[i] = *reinterpret_cast<const long *>(sm.b + (wc + 32 * i + li) * LDA + 16 * g + 8 * lh);
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const v16i z = {0};
                        S[i][j] = __builtin_amdgcn_mfma_i32_32x32x16_i8(a[i], b[j], z, 0, 0, 0);
                    }
            }
            const int qb = F::GK == 32 ? g : g >> 1;  // Q8_1 block of this group
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float d8 = sm.bd[qb][wc + 32 * j + li];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
#pragma unroll
                    for (int v4 = 0; v4 < 4; ++v4) {
                        const int rr = wr + 32 * i + 8 * v4 + 4 * lh;
                        const float4 sc = *reinterpret_cast<const float4 *>(&sm.ascale[g][rr]);
                        const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int v = 4 * v4 + u;
                            acc[i][j][v] += (float)S[i][j][v] * (d8 * scv[u]);
                        }
                    }
                }
            }
        }
        if constexpr (TYPE == TYPE_Q4_K) {
            // min term: dmin[r] * sum_j m_j[r] * s8_j[c] over the 8 sub-blocks (K = 8, f16 MFMA)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const v4h am = *reinterpret_cast<const v4h *>(&sm.amin[wr + 32 * i + li][4 * lh]);
                float dm[16];
#pragma unroll
                for (int v4 = 0; v4 < 4; ++v4) {
                    const float4 t = *reinterpret_cast<const float4 *>(&sm.admin[wr + 32 * i + 8 * v4 + 4 * lh]);
                    dm[4 * v4 + 0] = t.x;
                    dm[4 * v4 + 1] = t.y;
                    dm[4 * v4 + 2] = t.z;
                    dm[4 * v4 + 3] = t.w;
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v4h bm = *reinterpret_cast<const v4h *>(&sm.bs8[wc + 32 * j + li][4 * lh]);
                    const v16f z = {0};
                    const v16f P = __builtin_amdgcn_mfma_f32_32x32x8f16(am, bm, z, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; ++v) accm[i][j][v] += dm[v] * P[v];
                }
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t c = col0 + wc + 32 * j + li;
            if (c >= ncols) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t r = row0 + wr + 32 * i + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (r < nrows) dst[c * dst_col_stride + r] = acc[i][j][v] - accm[i][j][v];
            }
        }
}

template <int TYPE>
int launch(const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs, const void *yds,
           int64_t ncols, float *dst, int64_t dst_col_stride, hipStream_t s) {
    const int64_t gx = (nrows + BM - 1) / BM, gy = (ncols + BN - 1) / BN;
    if (gx > 0x7FFFFFFF || gy > 65535) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(mmq_kernel<TYPE>, dim3((unsigned)gx, (unsigned)gy), dim3(NTHREADS), 0, s,
                       (const uint8_t *)w, K, nrows, row_stride, yqs, (const uint32_t *)yds, ncols, dst,
                       dst_col_stride);
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int hip_qmm_mmq(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                           const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                           int64_t dst_col_stride, void *stream) {
    if (!w || !y_qs || !y_ds || !dst || K <= 0 || nrows <= 0 || ncols <= 0 || dst_col_stride < nrows)
        return (int)hipErrorInvalidValue;
    if (K % BK != 0) return (int)hipErrorInvalidValue;  // Q8_0 rows of K % 256 != 0: not supported here
    hipStream_t s = (hipStream_t)stream;
    switch (type) {
    case TYPE_Q4_K:
        if (row_stride < K / QK_K * Q4K_BYTES || row_stride % 16 || (uintptr_t)w % 16) return (int)hipErrorInvalidValue;
        return launch<TYPE_Q4_K>(w, K, nrows, row_stride, y_qs, y_ds, ncols, dst, dst_col_stride, s);
    case TYPE_Q6_K:
        if (row_stride < K / QK_K * Q6K_BYTES || row_stride % 2 || (uintptr_t)w % 2) return (int)hipErrorInvalidValue;
        return launch<TYPE_Q6_K>(w, K, nrows, row_stride, y_qs, y_ds, ncols, dst, dst_col_stride, s);
    case TYPE_Q8_0:
        if (row_stride < K / QK8 * Q80_BYTES || row_stride % 2 || (uintptr_t)w % 2) return (int)hipErrorInvalidValue;
        return launch<TYPE_Q8_0>(w, K, nrows, row_stride, y_qs, y_ds, ncols, dst, dst_col_stride, s);
    default:
        return (int)hipErrorInvalidValue;
    }
}
