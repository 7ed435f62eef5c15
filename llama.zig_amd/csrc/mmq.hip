// mmq.hip -- prefill GEMM (more than 8 activation columns) and the
// expert-grouped MoE GEMM of Q4_K / Q6_K / Q8_0 weights against planar Q8_1
// activations, on CDNA4 int8 MFMA.
//
// Replaces the reference's MMQ path (mul_mat_q, src/ggml/cuda/mmq.zig:282-408,
// chosen at mmq.zig:865-917) and its mul_mat_id form (mmq.zig:750-855 with the
// mm_ids_helper tile specs, src/ggml/cuda/mmid.zig:32-90).
//
// Arithmetic.  Integer block dots are formed exactly on the MFMA:
// v_mfma_i32_32x32x32_i8 for one 32-deep Q8_1 block (Q4_K sub-blocks, Q8_0
// blocks), v_mfma_i32_32x32x16_i8 for Q6_K's 16-deep sub-blocks.  Each dot is
// then scaled per (row, column, block):
//   Q4_K: out = sum_b d_b * sum_j (sc_bj*d8_j) * S_bj  -  sum_b dmin_b * sum_j m_bj*s8_j
//   Q6_K: out = sum_b d_b * sum_k (sc_bk*d8_{k/2}) * T_bk
//   Q8_0: out = sum_b (d_b*d8_b) * S_b
// The per-(row, column) factor in parentheses is an outer product of exactly
// representable f16 values (6-bit / int8 scales, f16 d8 and d), formed exactly
// in fp32 by one v_mfma_f32_32x32x8_f16 with a single live K slot.  The VALU
// then spends one convert and one FMA per output and block; d_b and the Q4_K
// min term (a K=8 f16 MFMA of m_j x s8_j) are applied once per super-block.
//
// Tiling: a 256-thread workgroup computes a BM=128 x BN output tile (BN = 32
// or 64); the four waves split it into 32x32 MFMA tiles.  K advances one
// 256-element super-block at a time.  While the MFMAs of step kb run, the
// workgroup's global loads for step kb+1 are already in flight into
// registers; they are unpacked into LDS (weights as int8, scales as f16)
// after the step.
//
// MFMA operand convention: for a 32x32xK tile, lane l supplies row (l % 32)
// of A and column (l % 32) of B over the K-slice [(l / 32) * K/2, +K/2).  A and
// B use the same slice, so the sum over K is formed whatever order the
// hardware gives the slices.  Results: value v of lane l is row
// 8*(v/4) + 4*(l/32) + v%4, column l%32.
#include <type_traits>

#include "../../include/ggml_hip_qmm.h"
#include "mmq_dma.h"
#include "qmm_device.h"

using namespace qmm;

// mmq_q4k_dma.hip: the Q4_K kernel fed by direct global->LDS loads
int mmq_q4k_dma_launch(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride,
                       const int8_t *yqs, const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride,
                       dim3 grid, const int32_t *tiles, const int32_t *n_tiles, const int32_t *col_src,
                       const int32_t *col_dst, float *partial, const MmqGlu &glu, hipStream_t s);
// mmq_legacy_dma.hip: the Q8_0 / Q4_0 kernel fed by direct global->LDS loads (dense or expert-grouped)
int mmq_legacy_dma_launch(int type, int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                          const int8_t *yqs, const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride,
                          dim3 grid, float *partial, const qmm_dma::MmqGroups *grp, const MmqGlu &glu,
                          hipStream_t s);
// mmq_iq4xs_dma.hip: the IQ4_XS kernel fed by direct global->LDS loads (dense or expert-grouped)
int mmq_iq4xs_dma_launch(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                         const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, dim3 grid, float *partial,
                         const qmm_dma::MmqGroups *grp, const MmqGlu &glu, hipStream_t s);
// mmq_q5k_dma.hip: the Q5_K kernel fed by direct global->LDS loads (dense or expert-grouped)
int mmq_q5k_dma_launch(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                       const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, dim3 grid, float *partial,
                       const qmm_dma::MmqGroups *grp, const MmqGlu &glu, hipStream_t s);
// mmq_few.hip: the Q4_K / Q8_0 / Q6_K kernel for at most 32 columns
int mmq_few_split_k(int64_t K, int64_t nrows);
bool mmq_few_takes(int type, int64_t K, const void *w, int64_t row_stride);
int mmq_few_launch(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                   const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int split, float *partial,
                   hipStream_t s);

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int BK = 256;
constexpr int LDA = BK + 16;  // int8 row stride in LDS (the pad staggers banks)
constexpr int NTHREADS = 256;

template <int TYPE>
struct MmqFmt {
    static constexpr int GK = TYPE == TYPE_Q6_K ? 16 : 32;  // depth of one integer block dot
    static constexpr int NG = BK / GK;                      // scale groups per K-step
};

// Every member is 16-byte aligned so the compiler can prove it and read the
// MFMA operands with ds_read_b128 (conflict-free with the 272-byte row
// stride); unproven alignment degrades them to ds_read2_b32 pairs, whose
// rows r and r+16 share banks.
template <int TYPE, int BN>
struct Smem {
    alignas(16) int8_t a[BM * LDA];
    alignas(16) int8_t b[BN * LDA];
    // Scale operands of the f16 outer-product MFMA, stored as the 8-byte
    // (4 x f16) operand each lane hands the MFMA, so reading one is a single
    // ds_read_b64 with no VALU work.  asc holds {s, 0, 0, 0}; bd8[h] holds
    // the column's d8 in K slot h: lanes 0-31 (K slots 0-3) read bd8[0],
    // lanes 32-63 (slots 4-7) read bd8[1], so only slot 0 pairs two nonzero
    // values and the MFMA returns exactly s_r * d8_c.
    alignas(16) uint2 asc[MmqFmt<TYPE>::NG][BM];  // sc_j (Q4_K, Q5_K), sc_k (Q6_K), ls_j - 32 (IQ4_XS) or d_b (Q8_0, Q4_0), exact in f16
    alignas(16) uint2 bd8[2][8][BN];              // d8 per (Q8_1 block, column)
    alignas(16) float ad[BM];                        // d per row (Q4_K, Q5_K, Q6_K, IQ4_XS)
    alignas(16) float admin[BM];                     // dmin per row (Q4_K)
    alignas(16) _Float16 am[BM][8];                  // m_j per row (Q4_K)
    alignas(16) _Float16 bs8[BN][8];                 // s8 per column (Q4_K)
};

// Global data of one K-step, held in registers between the load and the LDS
// write.  Each thread owns one (row, half) of the A tile.
template <int TYPE>
struct AReg;

template <>
struct AReg<TYPE_Q4_K> {
    uint4 hdr, q[4];  // block header and this half's 64 qs bytes
    __device__ __forceinline__ void load(const uint8_t *blk, int half) {
        hdr = ld_u128(blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ld_u128(blk + 16 + 64 * half + 16 * i);
    }
    __device__ __forceinline__ void zero() {
        hdr = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = make_uint4(0, 0, 0, 0);
    }
};

// Q5_K: the Q4_K registers plus the block's 32 qh bytes, whose bits 4h..4h+3
// are the fifth bits of the half's four sub-blocks.
template <>
struct AReg<TYPE_Q5_K> {
    uint4 hdr, q[4], h[2];
    __device__ __forceinline__ void load(const uint8_t *blk, int half) {
        hdr = ld_u128(blk);
        h[0] = ld_u128(blk + 16);
        h[1] = ld_u128(blk + 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ld_u128(blk + 48 + 64 * half + 16 * i);
    }
    __device__ __forceinline__ void zero() {
        hdr = h[0] = h[1] = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = make_uint4(0, 0, 0, 0);
    }
};

template <>
struct AReg<TYPE_Q6_K> {
    uint4 l0[2], l1[2], qh[2], sc;
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *blk, int n) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            l0[hh] = ld16_u(blk + 64 * n + 16 * hh);
            l1[hh] = ld16_u(blk + 64 * n + 32 + 16 * hh);
            qh[hh] = ld16_u(blk + 128 + 32 * n + 16 * hh);
        }
        sc = ld16_u(blk + 192);
        d = ld_u16(blk + 208);
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) l0[hh] = l1[hh] = qh[hh] = make_uint4(0, 0, 0, 0);
        sc = make_uint4(0, 0, 0, 0);
        d = 0;
    }
};

// Q8_0: thread t owns blocks (row t/2, blocks 4*(t%2) .. +4) of the step
template <>
struct AReg<TYPE_Q8_0> {
    uint4 q[4][2];
    uint32_t d[4];
    __device__ __forceinline__ void load(const uint8_t *blk0, int) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint8_t *blk = blk0 + b * Q80_BYTES;
            d[b] = ld_u16(blk);
            q[b][0] = ld16_u(blk + 2);
            q[b][1] = ld16_u(blk + 18);
        }
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            d[b] = 0;
            q[b][0] = q[b][1] = make_uint4(0, 0, 0, 0);
        }
    }
};

// Q4_0: as Q8_0, thread t owns blocks 4*(t%2) .. +4 of row t/2 in the step
template <>
struct AReg<TYPE_Q4_0> {
    uint4 q[4];
    uint32_t d[4];
    __device__ __forceinline__ void load(const uint8_t *blk0, int) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint8_t *blk = blk0 + b * Q40_BYTES;
            d[b] = ld_u16(blk);
            q[b] = ld16_u(blk + 2);
        }
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            d[b] = 0;
            q[b] = make_uint4(0, 0, 0, 0);
        }
    }
};

// IQ4_XS: the 8-byte header (d, scales_h, scales_l) and this half's 64 qs
// bytes (sub-blocks 4*half .. +3), at 8-byte alignment.
template <>
struct AReg<TYPE_IQ4_XS> {
    uint2 hdr;
    uint4 q[4];
    __device__ __forceinline__ void load(const uint8_t *blk, int half) {
        hdr = *reinterpret_cast<const uint2 *>(blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ld16_u(blk + 8 + 64 * half + 16 * i);
    }
    __device__ __forceinline__ void zero() {
        hdr = make_uint2(0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = make_uint4(0, 0, 0, 0);
    }
};

__device__ __forceinline__ uint32_t f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

__device__ __forceinline__ void st16(int8_t *dst, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *reinterpret_cast<uint4 *>(dst) = make_uint4(a, b, c, d);
}

__device__ __forceinline__ uint32_t minus32(uint32_t u) {
    // bytewise u - 32 for bytes in [0, 63], without borrows between bytes
    return ((u | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

__device__ __forceinline__ uint32_t minus8(uint32_t u) {
    // bytewise u - 8 for bytes in [0, 15], without borrows between bytes
    return ((u | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

template <int TYPE, int BN>
__device__ __forceinline__ void store_a(Smem<TYPE, BN> &sm, const AReg<TYPE> &ar) {
    const int t = threadIdx.x;
    const int r = t >> 1, half = t & 1;
    if constexpr (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) {
        int8_t *arow = sm.a + r * LDA;
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int c = 2 * half + cc;
            const uint4 q0 = ar.q[2 * cc], q1 = ar.q[2 * cc + 1];
            // Q5_K: bit j of qh[l] is the fifth bit of sub-block j's element l
            uint4 f0 = make_uint4(0, 0, 0, 0), f1 = f0, g0 = f0, g1 = f0;
            if constexpr (TYPE == TYPE_Q5_K) {
                const uint32_t one = 0x01010101u;
                const uint4 h0 = ar.h[0], h1 = ar.h[1];
                const int j0 = 2 * c, j1 = 2 * c + 1;
                f0 = make_uint4(((h0.x >> j0) & one) << 4, ((h0.y >> j0) & one) << 4, ((h0.z >> j0) & one) << 4,
                                ((h0.w >> j0) & one) << 4);
                f1 = make_uint4(((h1.x >> j0) & one) << 4, ((h1.y >> j0) & one) << 4, ((h1.z >> j0) & one) << 4,
                                ((h1.w >> j0) & one) << 4);
                g0 = make_uint4(((h0.x >> j1) & one) << 4, ((h0.y >> j1) & one) << 4, ((h0.z >> j1) & one) << 4,
                                ((h0.w >> j1) & one) << 4);
                g1 = make_uint4(((h1.x >> j1) & one) << 4, ((h1.y >> j1) & one) << 4, ((h1.z >> j1) & one) << 4,
                                ((h1.w >> j1) & one) << 4);
            }
            st16(arow + 64 * c + 0, (q0.x & m) | f0.x, (q0.y & m) | f0.y, (q0.z & m) | f0.z, (q0.w & m) | f0.w);
            st16(arow + 64 * c + 16, (q1.x & m) | f1.x, (q1.y & m) | f1.y, (q1.z & m) | f1.z, (q1.w & m) | f1.w);
            st16(arow + 64 * c + 32, ((q0.x >> 4) & m) | g0.x, ((q0.y >> 4) & m) | g0.y, ((q0.z >> 4) & m) | g0.z,
                 ((q0.w >> 4) & m) | g0.w);
            st16(arow + 64 * c + 48, ((q1.x >> 4) & m) | g1.x, ((q1.y >> 4) & m) | g1.y, ((q1.z >> 4) & m) | g1.z,
                 ((q1.w >> 4) & m) | g1.w);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * c + jj;
                uint32_t sc, mn;
                q4k_scale_min(j, ar.hdr.y, ar.hdr.z, ar.hdr.w, sc, mn);
                sm.asc[j][r] = make_uint2(f16_bits((float)sc), 0u);
                sm.am[r][j] = (_Float16)(float)mn;
            }
        }
        if (half == 0) {
            sm.ad[r] = h2f(ar.hdr.x);
            sm.admin[r] = h2f(ar.hdr.x >> 16);
        }
    } else if constexpr (TYPE == TYPE_Q6_K) {
        const int n = half;
        int8_t *arow = sm.a + r * LDA + 128 * n;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const uint32_t L0[4] = {ar.l0[hh].x, ar.l0[hh].y, ar.l0[hh].z, ar.l0[hh].w};
            const uint32_t L1[4] = {ar.l1[hh].x, ar.l1[hh].y, ar.l1[hh].z, ar.l1[hh].w};
            const uint32_t H[4] = {ar.qh[hh].x, ar.qh[hh].y, ar.qh[hh].z, ar.qh[hh].w};
            uint32_t v[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 0x0F0F0F0Fu, hm = 0x30303030u;
                v[0][i] = minus32((L0[i] & m) | ((H[i] << 4) & hm));
                v[1][i] = minus32((L1[i] & m) | ((H[i] << 2) & hm));
                v[2][i] = minus32(((L0[i] >> 4) & m) | (H[i] & hm));
                v[3][i] = minus32(((L1[i] >> 4) & m) | ((H[i] >> 2) & hm));
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) st16(arow + 32 * g + 16 * hh, v[g][0], v[g][1], v[g][2], v[g][3]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) sm.asc[8 * n + i][r] = make_uint2(f16_bits((float)(int8_t)byte_of(ar.sc, 8 * n + i)), 0u);
        if (half == 0) sm.ad[r] = h2f(ar.d);
    } else if constexpr (TYPE == TYPE_IQ4_XS) {
        // levels as int8: low nibbles are elements 0..15 of a sub-block, high
        // nibbles 16..31; scale ls - 32 per sub-block, d per row
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * half + i;
            int8_t *dst = sm.a + r * LDA + 32 * j;
            const uint4 q = ar.q[i];
            st16(dst, iq4nl_levels(q.x & m), iq4nl_levels(q.y & m), iq4nl_levels(q.z & m), iq4nl_levels(q.w & m));
            st16(dst + 16, iq4nl_levels((q.x >> 4) & m), iq4nl_levels((q.y >> 4) & m), iq4nl_levels((q.z >> 4) & m),
                 iq4nl_levels((q.w >> 4) & m));
            const uint32_t ls = ((ar.hdr.y >> (4 * j)) & 0xFu) | (((ar.hdr.x >> (16 + 2 * j)) & 3u) << 4);
            sm.asc[j][r] = make_uint2(f16_bits((float)((int)ls - 32)), 0u);
        }
        if (half == 0) sm.ad[r] = h2f(ar.hdr.x);
    } else if constexpr (TYPE == TYPE_Q4_0) {
        // q - 8 as int8: low nibbles are elements 0..15, high nibbles 16..31
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int blk = 4 * half + b;
            int8_t *dst = sm.a + r * LDA + 32 * blk;
            const uint4 q = ar.q[b];
            st16(dst, minus8(q.x & m), minus8(q.y & m), minus8(q.z & m), minus8(q.w & m));
            st16(dst + 16, minus8((q.x >> 4) & m), minus8((q.y >> 4) & m), minus8((q.z >> 4) & m),
                 minus8((q.w >> 4) & m));
            sm.asc[blk][r] = make_uint2(ar.d[b] & 0xFFFFu, 0u);
        }
    } else {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int blk = 4 * half + b;
            int8_t *dst = sm.a + r * LDA + 32 * blk;
            st16(dst, ar.q[b][0].x, ar.q[b][0].y, ar.q[b][0].z, ar.q[b][0].w);
            st16(dst + 16, ar.q[b][1].x, ar.q[b][1].y, ar.q[b][1].z, ar.q[b][1].w);
            sm.asc[blk][r] = make_uint2(ar.d[b] & 0xFFFFu, 0u);
        }
    }
}

// B: BN columns x (256 int8 + 8 (d, s)) per step, split into PARTS pieces of
// BYTES bytes per thread.
template <int BN>
struct BReg {
    static constexpr int BYTES = BN >= 128 ? 128 : BN * 256 / NTHREADS;  // bytes per part
    static constexpr int PARTS = BN * 256 / (NTHREADS * BYTES);           // parts per thread
    uint4 q[PARTS][BYTES / 16];
    uint32_t ds[PARTS][BYTES / 32];
};

template <int BN>
__device__ __forceinline__ void bpart(int p, int &c, int &off) {
    constexpr int BYTES = BReg<BN>::BYTES;
    constexpr int PER_COL = 256 / BYTES;
    const int idx = threadIdx.x + NTHREADS * p;
    c = idx / PER_COL;
    off = (idx % PER_COL) * BYTES;
}

template <int TYPE, int BN>
__global__ __launch_bounds__(NTHREADS, 2) void mmq_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride,
    const int8_t *__restrict__ yqs, const uint32_t *__restrict__ yds, int64_t ncols, float *__restrict__ dst,
    int64_t dst_col_stride,
    // expert-grouped mode (tiles != nullptr): column tile table and gather/scatter maps
    const int32_t *__restrict__ tiles, const int32_t *__restrict__ n_tiles, const int32_t *__restrict__ col_src,
    const int32_t *__restrict__ col_dst,
    // split-K (gridDim.z > 1): this workgroup's share of the K-steps goes to
    // partial[z][col][row] instead of dst
    float *__restrict__ partial,
    // gate/up/GLU fusion (glu.gate != nullptr): 64 output rows per tile, no split-K
    MmqGlu glu) {
    using F = MmqFmt<TYPE>;
    constexpr bool KMIN = TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K;  // scales with a min term
    constexpr bool LEGACY = TYPE == TYPE_Q8_0 || TYPE == TYPE_Q4_0;  // one scale per 32-block, no super-block
    __shared__ Smem<TYPE, BN> sm;
    const int64_t Kp = pad_k(K);
    const bool fused = glu.gate != nullptr;  // uniform
    // dense tiles in the XCD-aware banded order (one K part); grouped tiles as launched
    int bx = (int)blockIdx.x, by = (int)blockIdx.y;
    if (!tiles && gridDim.z == 1) mmq_tile_order(bx + (int)gridDim.x * by, (int)gridDim.x, (int)gridDim.y, bx, by);
    const int64_t row0 = (int64_t)bx * (fused ? BM / 2 : BM);  // first output row
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 31, lh = lane >> 5;

    // column tile: dense (col0 .. col0+BN of ncols) or one expert's routed columns
    int64_t col0 = (int64_t)by * BN, col_end = ncols;
    const uint8_t *wexp = w, *wgexp = glu.gate;
    if (tiles) {
        if ((int)blockIdx.y >= *n_tiles) return;  // uniform per workgroup
        const int4 t = *reinterpret_cast<const int4 *>(tiles + 4 * blockIdx.y);  // {expert, col_low, col_high, -}
        wexp = w + (int64_t)t.x * expert_stride;
        wgexp = fused ? glu.gate + (int64_t)t.x * expert_stride : nullptr;
        col0 = t.y;
        col_end = t.z;
    }

    // wave -> sub-tile: TI x TJ MFMA tiles of 32x32 at (wr, wc)
    constexpr int TI = BN == 128 ? 2 : 1;
    constexpr int TJ = BN == 32 ? 1 : 2;
    const int wr = BN == 128 ? (wave >> 1) * 64 : wave * 32;
    const int wc = BN == 128 ? (wave & 1) * 64 : 0;

    v16f acc[TI][TJ], accb[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // ---- register staging of one K-step ----
    const int ar_row = threadIdx.x >> 1, ar_half = threadIdx.x & 1;
    const int64_t a_orow = row0 + (fused ? mmq_glu_tile_row(ar_row) : ar_row);
    const bool a_ok = a_orow < nrows;
    const uint8_t *a_row = (fused && (ar_row & 2) == 0 ? wgexp : wexp) + (a_ok ? a_orow : 0) * row_stride;
    AReg<TYPE> areg;
    BReg<BN> breg;
    auto gload = [&](int64_t kb) {
        if (a_ok) {
            if constexpr (TYPE == TYPE_Q4_K) areg.load(a_row + kb * Q4K_BYTES, ar_half);
            else if constexpr (TYPE == TYPE_Q5_K) areg.load(a_row + kb * Q5K_BYTES, ar_half);
            else if constexpr (TYPE == TYPE_Q6_K) areg.load(a_row + kb * Q6K_BYTES, ar_half);
            else if constexpr (TYPE == TYPE_IQ4_XS) areg.load(a_row + kb * IQ4XS_BYTES, ar_half);
            else if constexpr (TYPE == TYPE_Q4_0) areg.load(a_row + (kb * 8 + 4 * ar_half) * Q40_BYTES, 0);
            else areg.load(a_row + (kb * 8 + 4 * ar_half) * Q80_BYTES, 0);
        } else {
            areg.zero();
        }
#pragma unroll
        for (int p = 0; p < BReg<BN>::PARTS; ++p) {
            int c, off;
            bpart<BN>(p, c, off);
            const int64_t cc = col0 + c;
            if (cc < col_end) {
                const int64_t src = tiles ? (int64_t)col_src[cc] : cc;
                const uint8_t *q = reinterpret_cast<const uint8_t *>(yqs + src * Kp + kb * BK + off);
#pragma unroll
                for (int i = 0; i < BReg<BN>::BYTES / 16; ++i) breg.q[p][i] = ld_u128(q + 16 * i);
                const uint32_t *d = yds + src * (Kp / QK8) + kb * 8 + off / 32;
#pragma unroll
                for (int i = 0; i < BReg<BN>::BYTES / 32; ++i) breg.ds[p][i] = d[i];
            } else {
#pragma unroll
                for (int i = 0; i < BReg<BN>::BYTES / 16; ++i) breg.q[p][i] = make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < BReg<BN>::BYTES / 32; ++i) breg.ds[p][i] = 0;
            }
        }
    };
    auto lstore = [&]() {
        store_a<TYPE, BN>(sm, areg);
#pragma unroll
        for (int p = 0; p < BReg<BN>::PARTS; ++p) {
            int c, off;
            bpart<BN>(p, c, off);
            int8_t *brow = sm.b + c * LDA + off;
#pragma unroll
            for (int i = 0; i < BReg<BN>::BYTES / 16; ++i) *reinterpret_cast<uint4 *>(brow + 16 * i) = breg.q[p][i];
#pragma unroll
            for (int i = 0; i < BReg<BN>::BYTES / 32; ++i) {
                const uint32_t v = breg.ds[p][i];
                sm.bd8[0][off / 32 + i][c] = make_uint2(v & 0xFFFFu, 0u);
                sm.bd8[1][off / 32 + i][c] = make_uint2(v << 16, 0u);
                if constexpr (KMIN) sm.bs8[c][off / 32 + i] = __builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
            }
        }
    };

    const int64_t nkb_all = K / BK;
    const int64_t kb_begin = nkb_all * blockIdx.z / gridDim.z;
    const int64_t nkb = nkb_all * (blockIdx.z + 1) / gridDim.z;
    gload(kb_begin);
    for (int64_t kb = kb_begin; kb < nkb; ++kb) {
        lstore();
        __syncthreads();
        if (kb + 1 < nkb) gload(kb + 1);  // in flight during this step's MFMAs

        // One step is NG x (TI*TJ) (scale group, tile) pairs.  Each pair is an
        // int8 MFMA (the exact block dots) plus an f16 MFMA (the exact scale
        // outer product); its VALU epilogue is one convert and one FMA per
        // output.  The pairs are software-pipelined one deep: pair p+1's MFMAs
        // are issued before pair p's epilogue so the matrix core runs under the
        // VALU work.  The first pair of a super-block writes accb instead of
        // accumulating into it.
        constexpr int NT = TI * TJ;
        constexpr int NP = F::NG * NT;
        using SType = typename std::conditional<F::GK == 32, v4i, long>::type;
        // The A-side operands (weights and the row scale) depend on the scale
        // group only: they are read once per group and shared by the TJ
        // column tiles (2 buffers, by group parity).
        static_assert(TI == 1, "one 32-row strip per wave");
        struct AOps {
            SType a;
            v4h sa;
        };
        struct BOps {
            SType b;
            v4h sb;
        };
        AOps aops[2];
        auto load_ops = [&](int p, BOps &o) {
            const int g = p / NT, j = p % NT;
            const int qb = F::GK == 32 ? g : g >> 1;  // Q8_1 block of this group
            if (j == 0) {
                aops[g & 1].sa = __builtin_bit_cast(v4h, sm.asc[g][wr + li]);
                aops[g & 1].a = *reinterpret_cast<const SType *>(sm.a + (wr + li) * LDA + F::GK * g + (F::GK / 2) * lh);
            }
            o.sb = __builtin_bit_cast(v4h, sm.bd8[lh][qb][wc + 32 * j + li]);
            o.b = *reinterpret_cast<const SType *>(sm.b + (wc + 32 * j + li) * LDA + F::GK * g + (F::GK / 2) * lh);
        };
        auto issue = [&](int p, const BOps &o, v16i &S, v16f &SC) {
            const AOps &ao = aops[(p / NT) & 1];
            const v16i z = {0};
            const v16f zf = {0};
            if constexpr (F::GK == 32) S = __builtin_amdgcn_mfma_i32_32x32x32_i8(ao.a, o.b, z, 0, 0, 0);
            else S = __builtin_amdgcn_mfma_i32_32x32x16_i8(ao.a, o.b, z, 0, 0, 0);
            SC = __builtin_amdgcn_mfma_f32_32x32x8f16(ao.sa, o.sb, zf, 0, 0, 0);
        };
        auto consume = [&](int p, const v16i &S, const v16f &SC) {
            const int g = p / NT, t = p % NT, i = t / TJ, j = t % TJ;
            if constexpr (LEGACY) {
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf((float)S[v], SC[v], acc[i][j][v]);
            } else if (g == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) accb[i][j][v] = (float)S[v] * SC[v];
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v) accb[i][j][v] = fmaf((float)S[v], SC[v], accb[i][j][v]);
            }
        };
        // Software pipeline over the NP (scale group, tile) pairs: while the
        // VALU scales pair p, the matrix core runs pair p+1 and the LDS
        // delivers the operands of pair p+2.  The scheduling fences pin that
        // order; left alone the scheduler consumes each MFMA result right
        // after issuing it and stalls on the MFMA latency.
        BOps ops[2];
        v16i Sb[2];
        v16f SCb[2];
        load_ops(0, ops[0]);
        if (NP > 1) load_ops(1, ops[1]);
        issue(0, ops[0], Sb[0], SCb[0]);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            __builtin_amdgcn_sched_barrier(0);
            if (p + 1 < NP) issue(p + 1, ops[(p + 1) & 1], Sb[(p + 1) & 1], SCb[(p + 1) & 1]);
            if (p + 2 < NP) load_ops(p + 2, ops[p & 1]);
            __builtin_amdgcn_sched_barrier(0);
            consume(p, Sb[p & 1], SCb[p & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);

        if constexpr (!LEGACY) {
            // acc += d[r] * accb; Q4_K / Q5_K also subtract dmin[r] * sum_j m_j[r] * s8_j[c]
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                float dr[16], dm[16];
#pragma unroll
                for (int v4 = 0; v4 < 4; ++v4) {
                    const int rr = wr + 32 * i + 8 * v4 + 4 * lh;
                    const float4 t = *reinterpret_cast<const float4 *>(&sm.ad[rr]);
                    dr[4 * v4 + 0] = t.x;
                    dr[4 * v4 + 1] = t.y;
                    dr[4 * v4 + 2] = t.z;
                    dr[4 * v4 + 3] = t.w;
                    if constexpr (KMIN) {
                        const float4 u = *reinterpret_cast<const float4 *>(&sm.admin[rr]);
                        dm[4 * v4 + 0] = u.x;
                        dm[4 * v4 + 1] = u.y;
                        dm[4 * v4 + 2] = u.z;
                        dm[4 * v4 + 3] = u.w;
                    }
                }
                v4h am;
                if constexpr (KMIN) am = *reinterpret_cast<const v4h *>(&sm.am[wr + 32 * i + li][4 * lh]);
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    if constexpr (KMIN) {
                        const v4h bm = *reinterpret_cast<const v4h *>(&sm.bs8[wc + 32 * j + li][4 * lh]);
                        const v16f zf = {0};
                        const v16f P = __builtin_amdgcn_mfma_f32_32x32x8f16(am, bm, zf, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 16; ++v)
                            acc[i][j][v] = fmaf(dr[v], accb[i][j][v], fmaf(-dm[v], P[v], acc[i][j][v]));
                    } else {
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(dr[v], accb[i][j][v], acc[i][j][v]);
                    }
                }
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int64_t c = col0 + wc + 32 * j + li;
            if (c >= col_end) continue;
            const int64_t drow = tiles ? (int64_t)col_dst[c] : c;
            float *o = partial ? partial + ((int64_t)blockIdx.z * ncols + c) * nrows : dst + drow * dst_col_stride;
            if (fused) {
                store_glu_column(o, row0 + wr / 2 + 2 * lh, nrows, acc[i][j], glu);
                continue;
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t r = row0 + wr + 32 * i + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (r < nrows) o[r] = acc[i][j][v];
            }
        }
}

// dst[c][r] = sum over z of partial[z][c][r], in z order (deterministic).
// Each thread sums 4 consecutive partial values with 16-byte loads (the
// planes are 16-byte aligned when nrows * ncols % 4 == 0; the workspace is)
// and keeps 4 planes' loads in flight.
constexpr int RED_V = 4;
__global__ __launch_bounds__(256) void splitk_reduce(const float *__restrict__ partial, int split, int64_t nrows,
                                                     int64_t ncols, float *__restrict__ dst, int64_t dst_col_stride) {
    const int64_t n = nrows * ncols;
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * RED_V;
    if (i0 >= n) return;
    float a[RED_V] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (n % RED_V == 0) {
        const float *p = partial + i0;
        int z = 0;
        for (; z + 4 <= split; z += 4) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4 *>(p + (int64_t)(z + u) * n);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[0] += v[u].x;
                a[1] += v[u].y;
                a[2] += v[u].z;
                a[3] += v[u].w;
            }
        }
        for (; z < split; ++z) {
            const float4 v = *reinterpret_cast<const float4 *>(p + (int64_t)z * n);
            a[0] += v.x;
            a[1] += v.y;
            a[2] += v.z;
            a[3] += v.w;
        }
    } else {
        for (int z = 0; z < split; ++z)
#pragma unroll
            for (int e = 0; e < RED_V; ++e)
                if (i0 + e < n) a[e] += partial[(int64_t)z * n + i0 + e];
    }
#pragma unroll
    for (int e = 0; e < RED_V; ++e) {
        const int64_t i = i0 + e;
        if (i < n) dst[(i / nrows) * dst_col_stride + i % nrows] = a[e];
    }
}

int launch_reduce(const float *partial, int split, int64_t nrows, int64_t ncols, float *dst, int64_t dst_col_stride,
                  hipStream_t s) {
    const int64_t n = nrows * ncols;
    const int64_t nthr = (n + RED_V - 1) / RED_V;
    hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s, partial, split, nrows,
                       ncols, dst, dst_col_stride);
    return (int)hipGetLastError();
}

template <int TYPE, int BN>
int launch(const void *w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride, const int8_t *yqs,
           const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int64_t gy, const int32_t *tiles,
           const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst, int split, float *partial,
           const MmqGlu &glu, hipStream_t s) {
    const int64_t tile_rows = glu.gate ? BM / 2 : BM;  // output rows per tile
    const int64_t gx = (nrows + tile_rows - 1) / tile_rows;
    if (gx > 0x7FFFFFFF || gy > 65535 || gy < 1 || split < 1 || split > 64 || (glu.gate && split != 1))
        return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)split);
    const qmm_dma::MmqGroups grp{tiles, n_tiles, col_src, col_dst, expert_stride};
    // the direct-transfer kernels move 16-byte chunks of the weight rows
    // (both weights' when fused) and of the activation planes
    const bool dma_rows = (uintptr_t)w % 16 == 0 && (!glu.gate || (uintptr_t)glu.gate % 16 == 0) &&
                          row_stride % 16 == 0 && expert_stride % 16 == 0 && (uintptr_t)yqs % 16 == 0 &&
                          (uintptr_t)yds % 16 == 0;
    // Q4_K with 16-byte aligned operands (the transfer unit of the direct
    // global->LDS loads; the weight rows are checked by check_weights)
    if (TYPE == TYPE_Q4_K && (uintptr_t)yqs % 16 == 0 && (uintptr_t)yds % 16 == 0) {
        if (int e = mmq_q4k_dma_launch(BN, w, K, nrows, row_stride, expert_stride, yqs, yds, ncols, dst,
                                       dst_col_stride, grid, tiles, n_tiles, col_src, col_dst,
                                       split > 1 ? partial : nullptr, glu, s))
            return e;
    } else if ((TYPE == TYPE_Q8_0 || TYPE == TYPE_Q4_0) && dma_rows) {
        // Q8_0 / Q4_0 on 16-byte aligned rows, dense or expert-grouped, plain
        // or gate/up-fused: direct global->LDS steps
        if (int e = mmq_legacy_dma_launch(TYPE, BN, w, K, nrows, row_stride, yqs, yds, ncols, dst, dst_col_stride,
                                          grid, split > 1 ? partial : nullptr, tiles ? &grp : nullptr, glu, s))
            return e;
    } else if (TYPE == TYPE_Q5_K && dma_rows) {
        // Q5_K (176-byte blocks, 16-byte aligned in aligned rows), dense or
        // expert-grouped, plain or gate/up-fused: direct global->LDS steps
        if (int e = mmq_q5k_dma_launch(BN, w, K, nrows, row_stride, yqs, yds, ncols, dst, dst_col_stride, grid,
                                       split > 1 ? partial : nullptr, tiles ? &grp : nullptr, glu, s))
            return e;
    } else if (TYPE == TYPE_IQ4_XS && K % 512 == 0 && (K / QK_K) % (2 * split) == 0 && dma_rows) {
        // IQ4_XS on 16-byte aligned rows of K % 512 == 0 (super-blocks in
        // 16-byte aligned pairs), dense or expert-grouped, plain or
        // gate/up-fused: direct global->LDS steps
        if (int e = mmq_iq4xs_dma_launch(BN, w, K, nrows, row_stride, yqs, yds, ncols, dst, dst_col_stride, grid,
                                         split > 1 ? partial : nullptr, tiles ? &grp : nullptr, glu, s))
            return e;
    } else {
        hipLaunchKernelGGL((mmq_kernel<TYPE, BN>), grid, dim3(NTHREADS), 0, s, (const uint8_t *)w, K, nrows,
                           row_stride, expert_stride, yqs, (const uint32_t *)yds, ncols, dst, dst_col_stride, tiles,
                           n_tiles, col_src, col_dst, split > 1 ? partial : nullptr, glu);
        if (int e = (int)hipGetLastError()) return e;
    }
    return split > 1 ? launch_reduce(partial, split, nrows, ncols, dst, dst_col_stride, s) : 0;
}

template <int TYPE>
int launch_bn(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride,
              const int8_t *yqs, const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int64_t gy,
              const int32_t *tiles, const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst,
              int split, float *partial, const MmqGlu &glu, hipStream_t s) {
    // A 128-column tile needs more than the 256 registers per lane that two
    // workgroups per CU leave (its two accumulator sets alone take 128), so
    // tiles stop at 64 columns.
    if (bn == 32)
        return launch<TYPE, 32>(w, K, nrows, row_stride, expert_stride, yqs, yds, ncols, dst, dst_col_stride, gy, tiles, n_tiles, col_src, col_dst, split, partial, glu, s);
    return launch<TYPE, 64>(w, K, nrows, row_stride, expert_stride, yqs, yds, ncols, dst, dst_col_stride, gy, tiles, n_tiles, col_src, col_dst, split, partial, glu, s);
}

int launch_type(int type, int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride,
                const int8_t *yqs, const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int64_t gy,
                const int32_t *tiles, const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst,
                int split, float *partial, const MmqGlu &glu, hipStream_t s) {
#define MMQ_TYPE_CASE(T)                                                                                              \
    case T:                                                                                                          \
        return launch_bn<T>(bn, w, K, nrows, row_stride, expert_stride, yqs, yds, ncols, dst, dst_col_stride, gy,    \
                            tiles, n_tiles, col_src, col_dst, split, partial, glu, s)
    switch (type) {
        MMQ_TYPE_CASE(TYPE_Q4_K);
        MMQ_TYPE_CASE(TYPE_Q5_K);
        MMQ_TYPE_CASE(TYPE_Q6_K);
        MMQ_TYPE_CASE(TYPE_Q4_0);
        MMQ_TYPE_CASE(TYPE_IQ4_XS);
        MMQ_TYPE_CASE(TYPE_Q8_0);
    default: return (int)hipErrorInvalidValue;
    }
#undef MMQ_TYPE_CASE
}

int check_weights(int type, const void *w, int64_t K, int64_t row_stride) {
    switch (type) {
    case TYPE_Q4_K:
        return (row_stride < K / QK_K * Q4K_BYTES || row_stride % 16 || (uintptr_t)w % 16) ? (int)hipErrorInvalidValue : 0;
    case TYPE_Q5_K:
        return (row_stride < K / QK_K * Q5K_BYTES || row_stride % 16 || (uintptr_t)w % 16) ? (int)hipErrorInvalidValue : 0;
    case TYPE_Q6_K:
        return (row_stride < K / QK_K * Q6K_BYTES || row_stride % 2 || (uintptr_t)w % 2) ? (int)hipErrorInvalidValue : 0;
    case TYPE_Q8_0:
        return (row_stride < K / QK8 * Q80_BYTES || row_stride % 2 || (uintptr_t)w % 2) ? (int)hipErrorInvalidValue : 0;
    case TYPE_Q4_0:
        return (row_stride < K / QK8 * Q40_BYTES || row_stride % 2 || (uintptr_t)w % 2) ? (int)hipErrorInvalidValue : 0;
    case TYPE_IQ4_XS:
        return (row_stride < K / QK_K * IQ4XS_BYTES || row_stride % 8 || (uintptr_t)w % 8) ? (int)hipErrorInvalidValue : 0;
    default:
        return (int)hipErrorInvalidValue;
    }
}

}  // namespace

// Column-tile width for a dense problem with `ncols` columns: the widest tile
// that does not leave most of a tile empty.
extern "C" int hip_qmm_mmq_tile_n(int64_t ncols) { return ncols <= 32 ? 32 : 64; }

// Column-tile width of the plain MMQ: hip_qmm_mmq_tile_n's, except that the
// Q4_K, Q5_K, Q8_0 and Q4_0 direct-transfer kernels take 32-column tiles on
// rows of at most 16 K-steps whenever 64-column tiles would leave the chip at
// one workgroup per CU or fewer (at most 256 tiles) and 32-column tiles fit
// one round of two per CU (at most 512): twice the tiles fill the grid with
// fewer K shares and two workgroups per CU.  Graph-timed against 64 columns
// (A/B of both libraries, same box): Q4_K 14336x4096 at 48 / 64 / 96 / 128
// columns 28.4-28.5 / 29.5-29.9 / 39.0 / 41.2 -> 25.9-26.2 / 27.0-27.1 /
// 35.0-35.1 / 38.6-38.8 us; 4096x4096 at 128 / 256 / 512 20.8 / 29.7 / 39.9
// -> 18.7-18.8 / 23.8 / 33.8-33.9; 8192x4096 at 256 40.3-40.4 -> 34.1-34.4;
// 2048x4096 at 512 29.7 -> 23.4; 1024x4096 at 128 13.5 -> 11.2; Q5_K / Q4_0 /
// Q8_0 4096x4096 at 512 42.1-42.2 / 40.7-40.8 / 39.1-39.2 -> 39.2-39.3 /
// 37.8-38.1 / 38.5.  Where 64-column tiles already fill the chip they keep it
// (Q4_K 14336x4096 at 256: 52.8-53.2 against 60.6-61.2; 4096x4096 at 1024:
// 53.8-54.1 against 61.6-62.2), and so do longer rows (Q4_K 4096x14336 at 512:
// 98.5-98.7 against 105.2-105.6), IQ4_XS (14336x4096 at 128: 44.8-46.4
// against 47.6-48.0; 4096x4096 at 512: 44.7 against 46.0-46.1) and the staged
// kernel (Q6_K 14336x4096 at 128: 70.5-71.8 against 77.7-80.0; 4096x4096 at
// 512: 70.1-70.2 against 76.8-77.2).
int mmq_bn(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (ncols <= 32) return 32;
    const bool narrow = type == TYPE_Q4_K || type == TYPE_Q8_0 || type == TYPE_Q5_K || type == TYPE_Q4_0;
    const int64_t rt = (nrows + BM - 1) / BM;
    return narrow && K / BK <= 16 && rt * ((ncols + 63) / 64) <= 256 && rt * ((ncols + 31) / 32) <= 512 ? 32 : 64;
}

// Column-tile width of the gate/up-fused MMQ: mmq_bn's rule over its tiles of
// 64 output rows (each tile reads 64 rows of both weights, the work of one
// 128-row tile of the plain kernel), except for Q8_0.  The fused kernel splits
// no K, so twice the column tiles are its only way to fill the chip.  The
// whole call graph-timed, 64- against 32-column tiles (A/B of both libraries,
// same box, us): Q4_K 14336x4096 at 33 / 48 / 64 columns 47.0-47.1 / 46.6-46.8
// / 46.8-47.0 -> 37.9-38.1 / 38.2-38.5 / 38.6-38.9; 4096x4096 at 64 / 128 /
// 256 44.4-44.5 / 44.7-44.8 / 45.8-45.9 -> 27.5 / 27.8 / 38.9-39.2; 8192x4096
// at 128 46.0-46.1 -> 39.1-39.4; 2048x4096 at 512 47.1 -> 40.1-40.4; Q5_K /
// Q4_0 14336x4096 at 48 52.2-52.4 / 48.3-48.4 -> 45.2-45.4 / 41.9-42.0, and
// 4096x4096 at 256 51.7-51.8 / 47.3-47.4 -> 44.2-44.3 / 41.7-41.8.  Q8_0 loses
// on the large weights (14336x4096 at 48 / 64: 49.4-49.5 / 49.8-49.9 against
// 53.7-53.8 / 56.0-56.1) for 2 us won at 4096x4096 (256 columns 46.0-46.2
// against 43.9-44.2), and keeps 64 columns.  Where 64-column tiles already
// fill the chip nothing changes (Q4_K 14336x4096 at 96 / 128: 59.0-59.4 /
// 59.7-60.2 either way).
int mmq_glu_bn(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return type == TYPE_Q8_0 ? hip_qmm_mmq_tile_n(ncols) : mmq_bn(type, K, 2 * nrows, ncols);
}

// K-split factor: spread the K-steps over more workgroups until the grid
// holds about one workgroup per CU (256 CUs on MI355X) for the Q4_K
// direct-to-LDS kernel on rows of at most 16 K-steps, about two otherwise;
// at least 2 K-steps per share and equal shares.  Chosen by a sweep of every
// split on 1024-14336 rows, K 4096 / 14336 and 9-512 columns: the one-per-CU
// target won at short K (e.g. Q4_K 4096x4096 at 24 columns 13.5 us against
// 16.9 us for two per CU), two per CU at K = 14336 (Q4_K 4096 rows at 512
// columns: 108 us against 135 us unsplit), and unequal shares lost to the
// next smaller equal split (14336 rows at 24 columns: 3 shares 21.9 us, 2
// shares 19.3 us).  A split never takes the grid past two workgroups per CU
// (512): the second round of workgroups costs more than the split hides
// (14336x4096 at 256 columns, 448 tiles, graph-timed unsplit against 2
// shares: Q8_0 65.2 against 80.3 us, Q4_0 59.6 / 74.3, Q5_K 62.9 / 77.6,
// IQ4_XS 66.2 / 80.4, Q6_K 113.9 / 131.7).  Q8_0's direct-transfer kernel
// takes the one-per-CU target too (graph-timed against two per CU: 4096x2048
// at 256 / 512 columns 21.0 / 23.3 us against 24.0 / 30.9, 2048x4096 at 256
// 20.7 against 23.2; 2048x4096 at 512 29.1 against 27.0).
int split_std(int type, int64_t K, int64_t nrows, int64_t ncols) {
    const int64_t bn = mmq_bn(type, K, nrows, ncols);
    const int64_t wgs = ((nrows + BM - 1) / BM) * ((ncols + bn - 1) / bn);
    const int64_t nkb = K / BK;
    const int64_t target = ((type == TYPE_Q4_K || type == TYPE_Q8_0) && nkb <= 16) ? 256 : 512;
    int64_t split = (target + wgs - 1) / wgs;
    while (split > 1 && wgs * split > 512) --split;
    const int64_t cap = nkb / 2 < 16 ? nkb / 2 : 16;
    if (split > cap) split = cap;
    if (split < 1) split = 1;
    while (nkb % split) --split;
    return (int)split;
}

// The few-column kernel (mmq_few.hip) takes Q4_K, Q5_K, Q8_0, Q4_0 and IQ4_XS
// up to 32 columns and Q6_K up to 16 (K % 2048 == 0; Q8_0 / Q4_0 / Q6_K /
// IQ4_XS on 16-byte-aligned rows), when the activation planes are 16-byte
// aligned, except Q8_0 and Q4_0 at 17-32 columns of 8 MiB of weights and
// more: their 128-row tile moves the weights by direct global->LDS transfers
// and is faster there.  Measured, the whole call in HIP graphs, few-column
// against the tile (us): Q4_0 14336x4096 at 24 / 32 columns 23.3 / 23.7
// against 19.0 / 19.5, Q8_0 14336x4096 23.1 / 23.4 against 21.5 / 22.4, Q8_0
// 6144x4096 15.9 / 16.8 against 15.1 / 15.8, Q4_0 4096x4096 12.1 / 13.0
// against 11.6 / 12.1; on 1024x4096 (4.5 MB of Q8_0) the few-column kernel
// stays ahead (9.4 / 9.7 against 10.6 / 10.7).  Up to 16 columns, and for the
// K-quants and IQ4_XS up to 32, the few-column kernel is as fast or faster on
// every shape measured (Q4_K 1024x4096 at 9: 7.3 against 9.5; 4096x14336 at
// 32: 20.3 against 21.4).  Earlier, against the staged tile: Q8_0 4096x14336
// at 9 / 32 columns 18.6 / 23.2 against 33.2 / 39.1; Q6_K 9 / 16 columns 22.6
// / 23.2 against 28.3 / 29.3, but 48.3 / 48.8 against 31.3 / 33.4 at 24 / 32
// (two column tiles), so those keep the tile.  few_cols_type is the part that
// depends on the shape alone (the split and workspace queries); the dispatch
// also checks the rows (mmq_few_takes).
bool few_cols_type(int type, int64_t K, int64_t nrows, int64_t ncols) {
    const bool takes = (ncols <= 32 && (type == TYPE_Q4_K || type == TYPE_Q8_0 || type == TYPE_Q5_K ||
                                        type == TYPE_Q4_0)) ||
                       (ncols <= 32 && type == TYPE_IQ4_XS && K % 512 == 0) ||
                       (ncols <= 16 && type == TYPE_Q6_K && K % 2048 == 0);
    if (!takes) return false;
    if ((type == TYPE_Q8_0 || type == TYPE_Q4_0) && ncols > 16) {
        const int64_t wbytes = nrows * (K / QK8) * (type == TYPE_Q8_0 ? Q80_BYTES : Q40_BYTES);
        return wbytes < ((int64_t)8 << 20);
    }
    return true;
}

extern "C" int hip_qmm_mmq_split_k(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (K <= 0 || nrows <= 0 || ncols <= 0) return 1;
    return few_cols_type(type, K, nrows, ncols) ? mmq_few_split_k(K, nrows) : split_std(type, K, nrows, ncols);
}

extern "C" size_t hip_qmm_mmq_workspace_size(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (K <= 0 || nrows <= 0 || ncols <= 0) return 0;
    int split = split_std(type, K, nrows, ncols);
    if (few_cols_type(type, K, nrows, ncols) && mmq_few_split_k(K, nrows) > split) split = mmq_few_split_k(K, nrows);
    return split > 1 ? (size_t)split * (size_t)nrows * (size_t)ncols * sizeof(float) : 0;
}

extern "C" int hip_qmm_mmq(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                           const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                           int64_t dst_col_stride, void *workspace, size_t workspace_size, void *stream) {
    if (!w || !y_qs || !y_ds || !dst || K <= 0 || nrows <= 0 || ncols <= 0 || dst_col_stride < nrows)
        return (int)hipErrorInvalidValue;
    if (K % BK != 0 || K > (1 << 30)) return (int)hipErrorInvalidValue;
    if (int e = check_weights(type, w, K, row_stride)) return e;
    const int bn = mmq_bn(type, K, nrows, ncols);
    const int64_t gy = (ncols + bn - 1) / bn;
    const bool few = few_cols_type(type, K, nrows, ncols) && mmq_few_takes(type, K, w, row_stride) &&
                     (uintptr_t)y_qs % 16 == 0 && (uintptr_t)y_ds % 16 == 0;
    // split K only when the caller's workspace holds the partials
    int split = few ? mmq_few_split_k(K, nrows) : split_std(type, K, nrows, ncols);
    if (split > 1 && (!workspace || workspace_size < (size_t)split * (size_t)nrows * (size_t)ncols * sizeof(float) ||
                      (uintptr_t)workspace % 16))
        split = 1;
    float *partial = (float *)workspace;
    hipStream_t s = (hipStream_t)stream;
    if (few) {
        if (int e = mmq_few_launch(type, w, K, nrows, row_stride, y_qs, y_ds, ncols, dst, dst_col_stride, split,
                                   partial, s))
            return e;
        return split > 1 ? launch_reduce(partial, split, nrows, ncols, dst, dst_col_stride, s) : 0;
    }
    return launch_type(type, bn, w, K, nrows, row_stride, 0, y_qs, y_ds, ncols, dst, dst_col_stride, gy, nullptr, nullptr,
                       nullptr, nullptr, split, partial, MmqGlu{}, s);
}

// Expert-grouped form used by hip_qmm_mul_mat_id: column tiles come from the
// device tile table written by the grouping kernel; `max_tiles` bounds the
// grid (workgroups past the table's count exit at once).
extern "C" int hip_qmm_mmq_grouped(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                   int64_t expert_stride, const int8_t *y_qs, const void *y_ds, float *dst,
                                   int64_t dst_row_stride, int bn, int64_t max_tiles, const int32_t *tiles,
                                   const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst,
                                   void *stream) {
    if (!w || !y_qs || !y_ds || !dst || !tiles || !n_tiles || !col_src || !col_dst || K <= 0 ||
        nrows <= 0 || dst_row_stride < nrows || max_tiles < 1 || (uintptr_t)tiles % 16 != 0)
        return (int)hipErrorInvalidValue;
    if (K % BK != 0 || K > (1 << 30) || (bn != 32 && bn != 64)) return (int)hipErrorInvalidValue;
    if (int e = check_weights(type, w, K, row_stride)) return e;
    hipStream_t s = (hipStream_t)stream;
    return launch_type(type, bn, w, K, nrows, row_stride, expert_stride, y_qs, y_ds, 0, dst, dst_row_stride, max_tiles,
                       tiles, n_tiles, col_src, col_dst, 1, nullptr, MmqGlu{}, s);
}

// Gate/up/GLU fused forms (the reference's mul_mat_q with a gate, its
// gate/up/GLU fusion, src/ggml/cuda/mmq.zig:568-640 and fusion.zig:1391,
// 1226-1298): both weights' rows go through one tile kernel, 64 output rows
// per tile, and the tile writes glu(gate, up).  No K split (the reference's
// fused kernel also runs one block per tile).  Each gate and up sum is the
// unfused kernel's at the same K order, so the output equals the GLU of two
// unsplit MMQs bit for bit.
extern "C" int hip_qmm_mmq_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                               int64_t row_stride, const int8_t *y_qs, const void *y_ds, int64_t ncols, int glu_op,
                               float glu_alpha, float glu_limit, float *dst, int64_t dst_col_stride, void *stream) {
    if (!w || !w_gate || !y_qs || !y_ds || !dst || K <= 0 || nrows <= 0 || ncols <= 0 || dst_col_stride < nrows ||
        !glu_op_valid(glu_op))
        return (int)hipErrorInvalidValue;
    if (K % BK != 0 || K > (1 << 30)) return (int)hipErrorInvalidValue;
    if (int e = check_weights(type, w, K, row_stride)) return e;
    if (int e = check_weights(type, w_gate, K, row_stride)) return e;
    const int bn = mmq_glu_bn(type, K, nrows, ncols);
    const int64_t gy = (ncols + bn - 1) / bn;
    const MmqGlu glu{(const uint8_t *)w_gate, glu_op, glu_alpha, glu_limit};
    return launch_type(type, bn, w, K, nrows, row_stride, 0, y_qs, y_ds, ncols, dst, dst_col_stride, gy, nullptr,
                       nullptr, nullptr, nullptr, 1, nullptr, glu, (hipStream_t)stream);
}

extern "C" int hip_qmm_mmq_grouped_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                       int64_t row_stride, int64_t expert_stride, const int8_t *y_qs,
                                       const void *y_ds, float *dst, int64_t dst_row_stride, int bn,
                                       int64_t max_tiles, const int32_t *tiles, const int32_t *n_tiles,
                                       const int32_t *col_src, const int32_t *col_dst, int glu_op, float glu_alpha,
                                       float glu_limit, void *stream) {
    if (!w || !w_gate || !y_qs || !y_ds || !dst || !tiles || !n_tiles || !col_src || !col_dst || K <= 0 ||
        nrows <= 0 || dst_row_stride < nrows || max_tiles < 1 || (uintptr_t)tiles % 16 != 0 || !glu_op_valid(glu_op))
        return (int)hipErrorInvalidValue;
    if (K % BK != 0 || K > (1 << 30) || (bn != 32 && bn != 64)) return (int)hipErrorInvalidValue;
    if (int e = check_weights(type, w, K, row_stride)) return e;
    if (int e = check_weights(type, w_gate, K, row_stride)) return e;
    const MmqGlu glu{(const uint8_t *)w_gate, glu_op, glu_alpha, glu_limit};
    return launch_type(type, bn, w, K, nrows, row_stride, expert_stride, y_qs, y_ds, 0, dst, dst_row_stride, max_tiles,
                       tiles, n_tiles, col_src, col_dst, 1, nullptr, glu, (hipStream_t)stream);
}
