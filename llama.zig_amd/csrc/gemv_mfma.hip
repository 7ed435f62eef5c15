// gemv_mfma.hip -- decode GEMV for 2..16 activation columns on int8 MFMA.
//
// The v_dot4 GEMV (gemv.hip) gives each wave 2 rows, so every wave re-reads
// all activation columns of its K-slice: at 4-8 columns that activation
// traffic and its registers, not the weights, set the time.  Here a wave
// owns 16 rows and contracts them against up to 16 columns at once with
// v_mfma_i32_16x16x32_i8, one 32-deep scale group per MFMA, so the
// activations are read once per 16 rows.  The 8 waves of a workgroup split
// K eight ways over the same 16 rows and add their partial sums through LDS
// in a fixed order.
//
// Where it pays: each lane reads 8-byte pieces of 16 different rows, which
// the memory pipeline serves less efficiently than the v_dot4 GEMV's
// row-contiguous loads, so at 1-4 columns the v_dot4 GEMV is faster.  From 8
// columns on, the v_dot4 GEMV's per-wave activation traffic dominates and
// this kernel wins for the K-quants on large matrices (hip_qmm_mul_mat_vec
// picks it there; measured in the decode suite of bench.py).
//
// Semantics are those of gemv.hip (the reference's MMVQ path,
// src/ggml/cuda/mmvq.zig:275-300): exact integer block dots, scaled in fp32
// per (row, column, block):
//   Q4_K: out = sum_b d_b * sum_j (sc_bj*d8_j) * S_bj - dmin_b * sum_j m_bj*s8_j
//   Q6_K: out = sum_b d_b * sum_k (sc_bk*d8_{k/2}) * T_bk
//   Q8_0: out = sum_b (d_b*d8_b) * S_b
// The per-(row, column) factor in parentheses is an outer product of exact
// f16 values, formed exactly in fp32 by v_mfma_f32_16x16x16_f16 with one live
// K slot (lanes 0-15 hold the row scale and the column d8 in slot 0, every
// other slot is zero).  d_b, dmin_b (read back in the result layout from a
// per-wave LDS row table) and the Q4_K min term (a K=8 f16 MFMA of m_j x s8_j)
// are applied once per super-block.
//
// 16x16 MFMA operand convention: lane l supplies row (l % 16) of A and column
// (l % 16) of B over the K-slice [(l / 16) * K/4, +K/4); the result value i
// of lane l is row 4*(l/16) + i, column l % 16.  A and B use the same slice,
// so the sum over K does not depend on how the hardware orders the slices.
// Q6_K's 16-deep sub-blocks are two lane groups of a 32-deep window; the
// window is contracted twice with the other sub-block's lanes zeroed.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// K-split ways per workgroup: 8 measured best (4 leaves each wave several
// super-blocks with exposed load latency, 16 costs a larger reduction)
constexpr int WAVES = 8;
constexpr int ROWS = 16;  // rows per workgroup (one MFMA tile)
constexpr int MAXCOLS = 16; // columns per MFMA tile

// 8 bytes at a 2-byte-aligned address: one global_load_dwordx2 (see ld16_u).
__device__ __forceinline__ uint2 ld8_a2(const uint8_t *p) {
    uint2 r;
    __builtin_memcpy(&r, __builtin_assume_aligned(p, 2), 8);
    return r;
}

__device__ __forceinline__ long as_long(uint2 v) { return (long)(((uint64_t)v.y << 32) | v.x); }

__device__ __forceinline__ uint32_t f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// slot-0 f16 operand: {h, 0, 0, 0} for the lanes that carry it, zero elsewhere
__device__ __forceinline__ v4h slot0(uint32_t h16, bool live) {
    const uint2 u = make_uint2(live ? (h16 & 0xFFFFu) : 0u, 0u);
    return __builtin_bit_cast(v4h, u);
}

// Activation operands of one super-block (256 K) for this lane's column:
// qs[j] = 8 int8 of K-slice [256sb + 32j + 8g, +8), ds[j] = (d8 | s8 << 16)
// of Q8_1 block 8sb + j.  Columns past ncols read as zero.
struct ActSB {
    uint2 qs[8];
    uint32_t ds[8];
    __device__ __forceinline__ void load(const int8_t *qcol, const uint32_t *dcol, int sb, int g, bool live) {
        if (live) {
            const uint8_t *p = reinterpret_cast<const uint8_t *>(qcol) + QK_K * sb + 8 * g;
#pragma unroll
            for (int j = 0; j < 8; ++j) qs[j] = *reinterpret_cast<const uint2 *>(p + 32 * j);
            const uint4 a = *reinterpret_cast<const uint4 *>(dcol + 8 * sb);
            const uint4 b = *reinterpret_cast<const uint4 *>(dcol + 8 * sb + 4);
            ds[0] = a.x; ds[1] = a.y; ds[2] = a.z; ds[3] = a.w;
            ds[4] = b.x; ds[5] = b.y; ds[6] = b.z; ds[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                qs[j] = make_uint2(0, 0);
                ds[j] = 0;
            }
        }
    }
};

// Weight operands of one super-block for this lane's row.
template <int TYPE>
struct WtSB;

// Q4_K: q[c] = qs[32c + 8g, +8): low nibbles are sub-block 2c, high 2c+1.
template <>
struct WtSB<TYPE_Q4_K> {
    uint4 hdr;
    uint2 q[4];
    __device__ __forceinline__ void load(const uint8_t *row, int sb, int g) {
        const uint8_t *blk = row + (int64_t)sb * Q4K_BYTES;
        hdr = ld_u128(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * c + 8 * g);
    }
};

// Q6_K window (n, qd) covers K 128n + 32qd + [0, 32); lane group g takes
// l in [8g, 8g+8): ql[64n + 32(qd&1) + l] (nibble qd>>1) and qh[32n + l]
// (bits 2qd..2qd+1).  l0[n] / l1[n]: ql at 64n + 8g and 64n + 32 + 8g;
// h[n]: qh at 32n + 8g.
template <>
struct WtSB<TYPE_Q6_K> {
    uint2 l0[2], l1[2], h[2];
    uint4 sc;
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *row, int sb, int g) {
        const uint8_t *blk = row + (int64_t)sb * Q6K_BYTES;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            l0[n] = ld8_a2(blk + 64 * n + 8 * g);
            l1[n] = ld8_a2(blk + 64 * n + 32 + 8 * g);
            h[n] = ld8_a2(blk + 128 + 32 * n + 8 * g);
        }
        sc = ld16_a2(blk + 192);
        d = ld_u16(blk + 208);
    }
};

// Q8_0: the super-block is 8 blocks of 34 bytes; q[j] = qs[2 + 8g, +8) of block j.
template <>
struct WtSB<TYPE_Q8_0> {
    uint2 q[8];
    uint32_t d[8];
    __device__ __forceinline__ void load(const uint8_t *row, int sb, int g) {
        const uint8_t *b0 = row + (int64_t)sb * 8 * Q80_BYTES;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            d[j] = ld_u16(b0 + j * Q80_BYTES);
            q[j] = ld8_a2(b0 + j * Q80_BYTES + 2 + 8 * g);
        }
    }
};

// Materialise an accumulator at this point of the program: the block's
// epilogue then cannot be sunk below later blocks' MFMAs, which would keep
// every MFMA result of the super-block live at once.
__device__ __forceinline__ void pin(v4f &v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ uint32_t minus32(uint32_t u) {
    // bytewise u - 32 for bytes in [0, 63], without borrows between bytes
    return ((u | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

template <int TYPE>
__global__ __launch_bounds__(64 * WAVES) void gemv_mfma_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t Kp, int ncols, float *__restrict__ dst, int64_t dst_col_stride) {
    __shared__ alignas(16) float rowd[WAVES][2][ROWS];       // d, dmin of the 16 rows, per wave
    __shared__ alignas(16) float red[WAVES][64][4];          // per-wave partial results
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, g = lane >> 4;
    const int64_t row0 = (int64_t)blockIdx.x * ROWS;
    const int64_t my_row = row0 + li < nrows ? row0 + li : nrows - 1;  // clamped for loading
    const uint8_t *rowp = w + my_row * row_stride;
    const bool col_live = li < ncols;
    const int8_t *qcol = yqs + (int64_t)(col_live ? li : 0) * Kp;
    const uint32_t *dcol = yds + (int64_t)(col_live ? li : 0) * (Kp / QK8);

    // this wave's share of the super-blocks (Q8_0: groups of 8 blocks)
    const int nsb = (int)(K / QK_K);
    const int sb0 = nsb * wave / WAVES, sb1 = nsb * (wave + 1) / WAVES;

    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const v4i zi = {0, 0, 0, 0};
    const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool g0 = g == 0;

    // one super-block: MFMAs, the fp32 epilogue, the per-row d / dmin and the
    // Q4_K min term; branch-free so that no scaling work is sunk below a
    // branch (which would keep every MFMA result of the super-block live)
    auto process = [&](const WtSB<TYPE> &wc, const ActSB &a) {
            if constexpr (TYPE == TYPE_Q8_0) {
    #pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(wc.q[j]), as_long(a.qs[j]), zi, 0, 0, 0);
                    const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(slot0(wc.d[j], g0), slot0(a.ds[j], g0), zf, 0, 0, 0);
    #pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = fmaf((float)S[i], SC[i], acc[i]);
                    pin(acc);
                }
            } else {
                v4f accb = zf;
                if constexpr (TYPE == TYPE_Q4_K) {
                    const uint32_t m4 = 0x0F0F0F0Fu;
    #pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint2 q = wc.q[j >> 1];
                        const uint2 v = (j & 1) ? make_uint2((q.x >> 4) & m4, (q.y >> 4) & m4)
                                                : make_uint2(q.x & m4, q.y & m4);
                        uint32_t sc, mn;
                        q4k_scale_min(j, wc.hdr.y, wc.hdr.z, wc.hdr.w, sc, mn);
                        const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(v), as_long(a.qs[j]), zi, 0, 0, 0);
                        const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(slot0(f16_bits((float)sc), g0),
                                                                             slot0(a.ds[j], g0), zf, 0, 0, 0);
    #pragma unroll
                        for (int i = 0; i < 4; ++i) accb[i] = fmaf((float)S[i], SC[i], accb[i]);
                        pin(accb);
                    }
                } else {  // Q6_K: window (n, qd) = sub-blocks 8n + 2qd (lane groups 0,1) and +1 (groups 2,3)
    #pragma unroll
                    for (int n = 0; n < 2; ++n) {
    #pragma unroll
                        for (int qd = 0; qd < 4; ++qd) {
                            const uint2 lq = (qd & 1) ? wc.l1[n] : wc.l0[n];
                            const int ls = 4 * (qd >> 1), hs = 2 * qd;
                            const uint32_t vx = minus32(((lq.x >> ls) & 0x0F0F0F0Fu) | (((wc.h[n].x >> hs) & 0x03030303u) << 4));
                            const uint32_t vy = minus32(((lq.y >> ls) & 0x0F0F0F0Fu) | (((wc.h[n].y >> hs) & 0x03030303u) << 4));
                            const int j = 4 * n + qd;  // Q8_1 block of this window
                            const bool lo = g < 2;
                            const uint2 va = lo ? make_uint2(vx, vy) : make_uint2(0u, 0u);
                            const uint2 vb = lo ? make_uint2(0u, 0u) : make_uint2(vx, vy);
                            const int k0 = 8 * n + 2 * qd;
                            const float s0 = (float)(int8_t)byte_of(wc.sc, k0), s1 = (float)(int8_t)byte_of(wc.sc, k0 + 1);
                            const v4i Sa = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(va), as_long(a.qs[j]), zi, 0, 0, 0);
                            const v4i Sb = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(vb), as_long(a.qs[j]), zi, 0, 0, 0);
                            const v4f Ca = __builtin_amdgcn_mfma_f32_16x16x16f16(slot0(f16_bits(s0), g0),
                                                                                 slot0(a.ds[j], g0), zf, 0, 0, 0);
                            const v4f Cb = __builtin_amdgcn_mfma_f32_16x16x16f16(slot0(f16_bits(s1), g0),
                                                                                 slot0(a.ds[j], g0), zf, 0, 0, 0);
    #pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                accb[i] = fmaf((float)Sa[i], Ca[i], accb[i]);
                                accb[i] = fmaf((float)Sb[i], Cb[i], accb[i]);
                            }
                            pin(accb);
                        }
                    }
                }
                // per-row d (and dmin) in the result layout, through this wave's LDS row table
                float dr, dm = 0.0f;
                if constexpr (TYPE == TYPE_Q4_K) {
                    dr = h2f(wc.hdr.x);
                    dm = h2f(wc.hdr.x >> 16);
                } else {
                    dr = h2f(wc.d);
                }
                // the 4 lanes of a row store the same values: no branch needed
                rowd[wave][0][li] = dr;
                rowd[wave][1][li] = dm;
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the table is written
                const float4 D = *reinterpret_cast<const float4 *>(&rowd[wave][0][4 * g]);
                const float dd[4] = {D.x, D.y, D.z, D.w};
                if constexpr (TYPE == TYPE_Q4_K) {
                    // min term: sum_j m_j * s8_j as a K=8 f16 MFMA (slots 4g..4g+3 for g < 2)
                    uint32_t mlo = 0, mhi = 0;
    #pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        // m of sub-block t (lane groups 0, 2) or 4 + t (groups 1, 3), selected
                        uint32_t sc, m_lo, m_hi;
                        q4k_scale_min(t, wc.hdr.y, wc.hdr.z, wc.hdr.w, sc, m_lo);
                        q4k_scale_min(4 + t, wc.hdr.y, wc.hdr.z, wc.hdr.w, sc, m_hi);
                        const uint32_t mn = (g & 1) ? m_hi : m_lo;
                        const uint32_t hb = f16_bits((float)mn);
                        if (t < 2) mlo |= hb << (16 * t);
                        else mhi |= hb << (16 * (t - 2));
                    }
                    uint32_t slo = 0, shi = 0;
    #pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t sv = ((g & 1) ? a.ds[4 + t] : a.ds[t]) >> 16;  // no dynamic index
                        if (t < 2) slo |= sv << (16 * t);
                        else shi |= sv << (16 * (t - 2));
                    }
                    const bool live = g < 2;
                    const v4h am = __builtin_bit_cast(v4h, live ? make_uint2(mlo, mhi) : make_uint2(0u, 0u));
                    const v4h bs = __builtin_bit_cast(v4h, live ? make_uint2(slo, shi) : make_uint2(0u, 0u));
                    const v4f P = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bs, zf, 0, 0, 0);
                    const float4 M = *reinterpret_cast<const float4 *>(&rowd[wave][1][4 * g]);
                    const float dmv[4] = {M.x, M.y, M.z, M.w};
    #pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = fmaf(dd[i], accb[i], fmaf(-dmv[i], P[i], acc[i]));
                } else {
    #pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = fmaf(dd[i], accb[i], acc[i]);
                }
                __builtin_amdgcn_wave_barrier();
            }

    };

    // No software prefetch: a wave's loads are exposed, and the other waves
    // resident on the SIMD (few registers each) cover that latency.
    for (int sb = sb0; sb < sb1; ++sb) {
        WtSB<TYPE> wt;
        ActSB ac;
        wt.load(rowp, sb, g);
        ac.load(qcol, dcol, sb, g, col_live);
        process(wt, ac);
    }

    // fixed-order sum of the 4 waves' partial tiles
    *reinterpret_cast<float4 *>(&red[wave][lane][0]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (wave == 0) {
        float4 s = *reinterpret_cast<const float4 *>(&red[0][lane][0]);
#pragma unroll
        for (int v = 1; v < WAVES; ++v) {
            const float4 t = *reinterpret_cast<const float4 *>(&red[v][lane][0]);
            s.x += t.x;
            s.y += t.y;
            s.z += t.z;
            s.w += t.w;
        }
        if (col_live) {
            const float o[4] = {s.x, s.y, s.z, s.w};
            float *out = dst + (int64_t)li * dst_col_stride;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t r = row0 + 4 * g + i;
                if (r < nrows) out[r] = o[i];
            }
        }
    }
}

}  // namespace

// Small-N GEMV on int8 MFMA: 1..16 columns, K a multiple of 256, Q4_K rows
// 16-byte aligned.  Called by hip_qmm_mul_mat_vec / hip_qmm_mul_mat.
extern "C" int hip_qmm_gemv_mfma(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                 const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                                 int64_t dst_col_stride, void *stream) {
    if (!w || !y_qs || !y_ds || !dst || K <= 0 || nrows <= 0 || ncols < 1 || ncols > MAXCOLS ||
        dst_col_stride < nrows)
        return (int)hipErrorInvalidValue;
    if (K % QK_K != 0 || K > (1 << 30)) return (int)hipErrorInvalidValue;
    const int64_t bb = type == TYPE_Q4_K ? Q4K_BYTES : type == TYPE_Q6_K ? Q6K_BYTES : type == TYPE_Q8_0 ? Q80_BYTES : 0;
    if (!bb) return (int)hipErrorInvalidValue;
    const int64_t bs = type == TYPE_Q8_0 ? QK8 : QK_K;
    if (row_stride < K / bs * bb) return (int)hipErrorInvalidValue;
    if (type == TYPE_Q4_K ? (row_stride % 16 || (uintptr_t)w % 16) : (row_stride % 2 || (uintptr_t)w % 2))
        return (int)hipErrorInvalidValue;
    const int64_t Kp = pad_k(K);
    const int64_t nblocks = (nrows + ROWS - 1) / ROWS;
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)y_ds;
    const dim3 grid((unsigned)nblocks), block(64 * WAVES);
    switch (type) {
    case TYPE_Q4_K:
        hipLaunchKernelGGL(gemv_mfma_kernel<TYPE_Q4_K>, grid, block, 0, s, wb, K, nrows, row_stride, y_qs, ds, Kp,
                           (int)ncols, dst, dst_col_stride);
        break;
    case TYPE_Q6_K:
        hipLaunchKernelGGL(gemv_mfma_kernel<TYPE_Q6_K>, grid, block, 0, s, wb, K, nrows, row_stride, y_qs, ds, Kp,
                           (int)ncols, dst, dst_col_stride);
        break;
    default:
        hipLaunchKernelGGL(gemv_mfma_kernel<TYPE_Q8_0>, grid, block, 0, s, wb, K, nrows, row_stride, y_qs, ds, Kp,
                           (int)ncols, dst, dst_col_stride);
        break;
    }
    return (int)hipGetLastError();
}
