// gemv.hip -- decode GEMV (1..8 activation columns) of Q4_K / Q6_K / Q8_0
// weights against planar Q8_1 activations, for gfx950.
//
// Replaces the reference's MMVQ path (src/ggml/cuda/mmvq.zig:275-300, chosen
// for ncols_dst <= 8 at mmvq.zig:128-173).  Semantics (integer block dots and
// their float combination) follow the formats' definitions:
//   Q4_K x Q8_1: S_bj = sum_{l<32} q4 * q8 per 32-sub-block j of super-block b,
//                out += d_b*sc_bj*d8 * S_bj - dmin_b*m_bj * s8
//   Q6_K x Q8_1: T_bk = sum_{l<16} (q6 - 32) * q8 per 16-sub-block k,
//                out += d_b*sc_bk*d8 * T_bk
//   Q8_0 x Q8_1: S_b = sum_{l<32} q * q8, out += d_b*d8 * S_b
//
//   Q5_K x Q8_1: as Q4_K with q5 = nibble + 16 * (qh bit j of the element)
//   Q4_0 x Q8_1: S_b = sum_{l<32} (q - 8) * q8, out += d_b*d8 * S_b
//
// Mapping: one 64-lane wavefront owns RPW consecutive weight rows and walks K
// in steps of 64 lanes x W weights (W = 64 for the K-quants, 32 for Q8_0).
// Within a step every lane owns a fixed K-slice: it loads that slice of the
// NC activation columns once (registers) and reuses it for all RPW rows,
// whose weight slices are loaded back to back before any arithmetic so the
// wave keeps RPW x 48 B per lane in flight.  Integer dots use v_dot4_i32_i8;
// each lane's partial sums are exactly the sub-block dots defined above.  One
// DPP reduction per (row, column) at the end.  Weights are read with plain
// loads: the nontemporal variant measured ~30% slower on gfx950.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

namespace {

template <int TYPE>
struct Fmt;

template <>
struct Fmt<TYPE_Q4_K> {
    static constexpr int W = 64;  // weights per lane per step
    static constexpr int NSUB = 2;  // integer block dots per lane per step
};
template <>
struct Fmt<TYPE_Q5_K> {
    static constexpr int W = 64;
    static constexpr int NSUB = 2;
};
template <>
struct Fmt<TYPE_Q6_K> {
    static constexpr int W = 64;
    static constexpr int NSUB = 4;
};
template <>
struct Fmt<TYPE_Q8_0> {
    static constexpr int W = 32;
    static constexpr int NSUB = 1;
};
template <>
struct Fmt<TYPE_IQ4_XS> {
    static constexpr int W = 64;
    static constexpr int NSUB = 2;
};
template <>
struct Fmt<TYPE_Q4_0> {
    static constexpr int W = 32;
    static constexpr int NSUB = 1;
};

// Activation slice of one column for one lane and step.
template <int TYPE>
struct Act;

template <>
struct Act<TYPE_Q4_K> {
    uint4 q[4];      // 64 int8: weights kl..kl+63
    uint32_t ds[2];  // (d, s) of the two Q8_1 blocks
    __device__ __forceinline__ void load(const int8_t *qs, const uint32_t *dsp, int kl) {
        const uint8_t *p = reinterpret_cast<const uint8_t *>(qs + kl);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ld_u128(p + 16 * i);
        const uint2 t = *reinterpret_cast<const uint2 *>(dsp + kl / QK8);
        ds[0] = t.x;
        ds[1] = t.y;
    }
    // The same slice from AoS block_q8_1 (36 B: d, s, qs[32]) of one column.
    __device__ __forceinline__ void load_aos(const uint8_t *col, int kl) {
        const uint8_t *b0 = col + (kl / QK8) * Q81_BYTES, *b1 = b0 + Q81_BYTES;
        ds[0] = ld_u32(b0);
        ds[1] = ld_u32(b1);
        q[0] = ld16_u(b0 + 4);
        q[1] = ld16_u(b0 + 20);
        q[2] = ld16_u(b1 + 4);
        q[3] = ld16_u(b1 + 20);
    }
};

// Q5_K and IQ4_XS take the activation slice as Q4_K does (64 values, two
// Q8_1 blocks).
template <>
struct Act<TYPE_Q5_K> : Act<TYPE_Q4_K> {};
template <>
struct Act<TYPE_IQ4_XS> : Act<TYPE_Q4_K> {};

// Q6_K lane (sb, n, h) covers weights 256sb + 128n + 32g + 16h + [0,16), g=0..3.
template <>
struct Act<TYPE_Q6_K> {
    uint4 q[4];
    uint32_t ds[4];
    uint32_t asum[4];  // sum of the 16 int8 activations of group g (for the -32 bias)
    __device__ __forceinline__ void load(const int8_t *qs, const uint32_t *dsp, int kl) {
        // kl = 256sb + 64q (q = lane % 4) -> n = q / 2, h = q % 2
        const int sb = kl / QK_K;
        const int qq = (kl % QK_K) / 64;
        const int n = qq >> 1, h = qq & 1;
        const uint8_t *p = reinterpret_cast<const uint8_t *>(qs + sb * QK_K + 128 * n + 16 * h);
#pragma unroll
        for (int g = 0; g < 4; ++g) q[g] = ld_u128(p + 32 * g);
        const uint4 t = *reinterpret_cast<const uint4 *>(dsp + sb * 8 + 4 * n);
        ds[0] = t.x;
        ds[1] = t.y;
        ds[2] = t.z;
        ds[3] = t.w;
        sums();
    }
    // The same slice from AoS block_q8_1: group g is half h of block 8sb + 4n + g.
    __device__ __forceinline__ void load_aos(const uint8_t *col, int kl) {
        const int sb = kl / QK_K;
        const int qq = (kl % QK_K) / 64;
        const int n = qq >> 1, h = qq & 1;
        const uint8_t *b = col + (int64_t)(sb * 8 + 4 * n) * Q81_BYTES;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            ds[g] = ld_u32(b + g * Q81_BYTES);
            q[g] = ld16_u(b + g * Q81_BYTES + 4 + 16 * h);
        }
        sums();
    }
    __device__ __forceinline__ void sums() {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            int s = dot4(q[g].x, 0x01010101u, 0);
            s = dot4(q[g].y, 0x01010101u, s);
            s = dot4(q[g].z, 0x01010101u, s);
            s = dot4(q[g].w, 0x01010101u, s);
            asum[g] = (uint32_t)s;
        }
    }
};

template <>
struct Act<TYPE_Q8_0> {
    uint4 q[2];
    uint32_t ds;
    __device__ __forceinline__ void load(const int8_t *qs, const uint32_t *dsp, int kl) {
        const uint8_t *p = reinterpret_cast<const uint8_t *>(qs + kl);
        q[0] = ld_u128(p);
        q[1] = ld_u128(p + 16);
        ds = dsp[kl / QK8];
    }
    __device__ __forceinline__ void load_aos(const uint8_t *col, int kl) {
        const uint8_t *b = col + (kl / QK8) * Q81_BYTES;
        ds = ld_u32(b);
        q[0] = ld16_u(b + 4);
        q[1] = ld16_u(b + 20);
    }
};

// Q4_0: the Q8_0 slice plus its integer sum, which turns the dot of the raw
// nibbles into the dot of q - 8 (computed once, shared by the wave's rows).
template <>
struct Act<TYPE_Q4_0> : Act<TYPE_Q8_0> {
    int asum;
    __device__ __forceinline__ void load_aos(const uint8_t *col, int kl) {
        Act<TYPE_Q8_0>::load_aos(col, kl);
        sum();
    }
    __device__ __forceinline__ void load(const int8_t *qs, const uint32_t *dsp, int kl) {
        Act<TYPE_Q8_0>::load(qs, dsp, kl);
        sum();
    }
    __device__ __forceinline__ void sum() {
        int s = dot4(q[0].x, 0x01010101u, 0);
        s = dot4(q[0].y, 0x01010101u, s);
        s = dot4(q[0].z, 0x01010101u, s);
        s = dot4(q[0].w, 0x01010101u, s);
        s = dot4(q[1].x, 0x01010101u, s);
        s = dot4(q[1].y, 0x01010101u, s);
        s = dot4(q[1].z, 0x01010101u, s);
        asum = dot4(q[1].w, 0x01010101u, s);
    }
};

// Weight slice of one row for one lane and step.
template <int TYPE>
struct Wt;

template <>
struct Wt<TYPE_Q4_K> {
    uint4 hdr;   // d, dmin, scales[12]
    uint4 q[2];  // qs[32c .. 32c+32)
    __device__ __forceinline__ void load(const uint8_t *row, int kl) {
        const uint8_t *blk = row + (kl / QK_K) * Q4K_BYTES;
        const int c = (kl % QK_K) / 64;
        hdr = ld_u128(blk);
        q[0] = ld_u128(blk + 16 + 32 * c);
        q[1] = ld_u128(blk + 16 + 32 * c + 16);
    }
    // Integer dots of the two 32-sub-blocks (j = 2c low nibbles, 2c+1 high).
    __device__ __forceinline__ void dots(const Act<TYPE_Q4_K> &a, int S[2], int = 0) const {
        const uint32_t w[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
        const uint32_t av[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s0 = dot4(w[i] & 0x0F0F0F0Fu, av[i], s0);
            s1 = dot4((w[i] >> 4) & 0x0F0F0F0Fu, av[8 + i], s1);
        }
        S[0] = s0;
        S[1] = s1;
    }
    __device__ __forceinline__ float combine(const Act<TYPE_Q4_K> &a, const int S[2], int kl) const {
        const int c = (kl % QK_K) / 64;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
        q4k_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
        const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
        const float d80 = h2f(a.ds[0]), s80 = h2f(a.ds[0] >> 16);
        const float d81 = h2f(a.ds[1]), s81 = h2f(a.ds[1] >> 16);
        const float t = (float)S[0] * d80 * (float)sc0 + (float)S[1] * d81 * (float)sc1;
        const float u = (float)m0 * s80 + (float)m1 * s81;
        return d * t - dmin * u;
    }
};

// Q5_K (block_q5_K {d, dmin, scales[12], qh[32], qs[128]}, 176 B): the lane's
// 64-weight slice c reads the 16-byte header, its 32 qs bytes and all 32 qh
// bytes, whose bits 2c and 2c+1 are the fifth bits of sub-blocks 2c and 2c+1
// (quantize_row_q5_K_ref's packing, src/ggml/quants/k.zig:508-532).
template <>
struct Wt<TYPE_Q5_K> {
    uint4 hdr, q[2], h[2];
    __device__ __forceinline__ void load(const uint8_t *row, int kl) {
        const uint8_t *blk = row + (kl / QK_K) * Q5K_BYTES;
        const int c = (kl % QK_K) / 64;
        hdr = ld_u128(blk);
        h[0] = ld_u128(blk + 16);
        h[1] = ld_u128(blk + 32);
        q[0] = ld_u128(blk + 48 + 32 * c);
        q[1] = ld_u128(blk + 48 + 32 * c + 16);
    }
    __device__ __forceinline__ void dots(const Act<TYPE_Q5_K> &a, int S[2], int kl) const {
        const int c = (kl % QK_K) / 64;
        const uint32_t w[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
        const uint32_t hb[8] = {h[0].x, h[0].y, h[0].z, h[0].w, h[1].x, h[1].y, h[1].z, h[1].w};
        const uint32_t av[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = (w[i] & 0x0F0F0F0Fu) | (((hb[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((w[i] >> 4) & 0x0F0F0F0Fu) | (((hb[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            s0 = dot4(lo, av[i], s0);
            s1 = dot4(hi, av[8 + i], s1);
        }
        S[0] = s0;
        S[1] = s1;
    }
    __device__ __forceinline__ float combine(const Act<TYPE_Q5_K> &a, const int S[2], int kl) const {
        const int c = (kl % QK_K) / 64;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
        q4k_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
        const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
        const float d80 = h2f(a.ds[0]), s80 = h2f(a.ds[0] >> 16);
        const float d81 = h2f(a.ds[1]), s81 = h2f(a.ds[1] >> 16);
        const float t = (float)S[0] * d80 * (float)sc0 + (float)S[1] * d81 * (float)sc1;
        const float u = (float)m0 * s80 + (float)m1 * s81;
        return d * t - dmin * u;
    }
};

template <>
struct Wt<TYPE_Q6_K> {
    uint4 ql0, ql1, qh, sc;  // ql[64n+16h..], ql[64n+32+16h..], qh[32n+16h..], scales[16]
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *row, int kl) {
        const uint8_t *blk = row + (kl / QK_K) * Q6K_BYTES;
        const int qq = (kl % QK_K) / 64;
        const int n = qq >> 1, h = qq & 1;
        ql0 = ld16_u(blk + 64 * n + 16 * h);
        ql1 = ld16_u(blk + 64 * n + 32 + 16 * h);
        qh = ld16_u(blk + 128 + 32 * n + 16 * h);
        sc = ld16_u(blk + 192);
        d = ld_u16(blk + 208);
    }
    __device__ __forceinline__ void dots(const Act<TYPE_Q6_K> &a, int T[4], int = 0) const {
        const uint32_t l0[4] = {ql0.x, ql0.y, ql0.z, ql0.w};
        const uint32_t l1[4] = {ql1.x, ql1.y, ql1.z, ql1.w};
        const uint32_t hh[4] = {qh.x, qh.y, qh.z, qh.w};
        int t0 = 0, t1 = 0, t2 = 0, t3 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a0 = i == 0 ? a.q[0].x : i == 1 ? a.q[0].y : i == 2 ? a.q[0].z : a.q[0].w;
            const uint32_t a1 = i == 0 ? a.q[1].x : i == 1 ? a.q[1].y : i == 2 ? a.q[1].z : a.q[1].w;
            const uint32_t a2 = i == 0 ? a.q[2].x : i == 1 ? a.q[2].y : i == 2 ? a.q[2].z : a.q[2].w;
            const uint32_t a3 = i == 0 ? a.q[3].x : i == 1 ? a.q[3].y : i == 2 ? a.q[3].z : a.q[3].w;
            // unbiased 6-bit values 0..63, the -32 is applied through asum
            const uint32_t v0 = (l0[i] & 0x0F0F0F0Fu) | ((hh[i] << 4) & 0x30303030u);
            const uint32_t v1 = (l1[i] & 0x0F0F0F0Fu) | ((hh[i] << 2) & 0x30303030u);
            const uint32_t v2 = ((l0[i] >> 4) & 0x0F0F0F0Fu) | (hh[i] & 0x30303030u);
            const uint32_t v3 = ((l1[i] >> 4) & 0x0F0F0F0Fu) | ((hh[i] >> 2) & 0x30303030u);
            t0 = dot4(v0, a0, t0);
            t1 = dot4(v1, a1, t1);
            t2 = dot4(v2, a2, t2);
            t3 = dot4(v3, a3, t3);
        }
        T[0] = t0 - 32 * (int)a.asum[0];
        T[1] = t1 - 32 * (int)a.asum[1];
        T[2] = t2 - 32 * (int)a.asum[2];
        T[3] = t3 - 32 * (int)a.asum[3];
    }
    __device__ __forceinline__ float combine(const Act<TYPE_Q6_K> &a, const int T[4], int kl) const {
        const int qq = (kl % QK_K) / 64;
        const int n = qq >> 1, h = qq & 1;
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int idx = 8 * n + h + 2 * g;  // scales[8n + l/16 + 2g], l/16 = h
            const float s = (float)(int8_t)byte_of(sc, idx);
            t += (float)T[g] * h2f(a.ds[g]) * s;
        }
        return h2f(d) * t;
    }
};

// IQ4_XS (block_iq4_xs {d, scales_h, scales_l[4], qs[128]}, 136 B, at 8-byte
// alignment): the lane's 64-weight slice c is sub-blocks 2c and 2c+1, the
// 8-byte header and qs[32c .. 32c+32).  Byte j of a sub-block's 16 holds the
// level indices of its elements j (low nibble) and j + 16 (high nibble); the
// 6-bit scale of sub-block i is scales_l nibble i | scales_h bits 2i..2i+1 << 4,
// biased by 32 (quantize_row_iq4_nl_impl, src/ggml/quants/iq4.zig:165-193).
template <>
struct Wt<TYPE_IQ4_XS> {
    uint2 hdr;   // d | scales_h << 16, scales_l[4]
    uint2 q[4];  // qs[32c .. 32c+32)
    __device__ __forceinline__ void load(const uint8_t *row, int kl) {
        const uint8_t *blk = row + (kl / QK_K) * IQ4XS_BYTES;
        const int c = (kl % QK_K) / 64;
        hdr = *reinterpret_cast<const uint2 *>(blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = *reinterpret_cast<const uint2 *>(blk + 8 + 32 * c + 8 * i);
    }
    __device__ __forceinline__ void dots(const Act<TYPE_IQ4_XS> &a, int S[2], int = 0) const {
        const uint32_t w[8] = {q[0].x, q[0].y, q[1].x, q[1].y, q[2].x, q[2].y, q[3].x, q[3].y};
        const uint32_t av[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        const uint32_t m = 0x0F0F0F0Fu;
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s0 = dot4(iq4nl_levels(w[t] & m), av[t], s0);
            s0 = dot4(iq4nl_levels((w[t] >> 4) & m), av[4 + t], s0);
            s1 = dot4(iq4nl_levels(w[4 + t] & m), av[8 + t], s1);
            s1 = dot4(iq4nl_levels((w[4 + t] >> 4) & m), av[12 + t], s1);
        }
        S[0] = s0;
        S[1] = s1;
    }
    __device__ __forceinline__ float combine(const Act<TYPE_IQ4_XS> &a, const int S[2], int kl) const {
        const int c = (kl % QK_K) / 64;
        const uint32_t sl = (hdr.y >> (8 * c)) & 0xFFu, sh = (hdr.x >> (16 + 4 * c)) & 0xFu;
        const int ls0 = (int)((sl & 0xFu) | ((sh & 3u) << 4)) - 32, ls1 = (int)((sl >> 4) | ((sh >> 2) << 4)) - 32;
        const float t = (float)S[0] * h2f(a.ds[0]) * (float)ls0 + (float)S[1] * h2f(a.ds[1]) * (float)ls1;
        return h2f(hdr.x) * t;
    }
};

// Q4_0 (block_q4_0 {d, qs[16]}, 18 B): byte j holds element j (low nibble)
// and element j + 16 (high nibble) (quantize_row_q4_0_ref,
// src/ggml/quants/legacy.zig:151-184).
template <>
struct Wt<TYPE_Q4_0> {
    uint4 q;
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *row, int kl) {
        const uint8_t *blk = row + (kl / QK8) * Q40_BYTES;
        d = ld_u16(blk);
        q = ld16_a2(blk + 2);
    }
    __device__ __forceinline__ void dots(const Act<TYPE_Q4_0> &a, int S[1], int = 0) const {
        const uint32_t m = 0x0F0F0F0Fu;
        int s = 0;
        s = dot4(q.x & m, a.q[0].x, s);
        s = dot4(q.y & m, a.q[0].y, s);
        s = dot4(q.z & m, a.q[0].z, s);
        s = dot4(q.w & m, a.q[0].w, s);
        s = dot4((q.x >> 4) & m, a.q[1].x, s);
        s = dot4((q.y >> 4) & m, a.q[1].y, s);
        s = dot4((q.z >> 4) & m, a.q[1].z, s);
        s = dot4((q.w >> 4) & m, a.q[1].w, s);
        S[0] = s - 8 * a.asum;
    }
    __device__ __forceinline__ float combine(const Act<TYPE_Q4_0> &a, const int S[1], int) const {
        return h2f(d) * h2f(a.ds) * (float)S[0];
    }
};

template <>
struct Wt<TYPE_Q8_0> {
    uint4 q0, q1;
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *row, int kl) {
        const uint8_t *blk = row + (kl / QK8) * Q80_BYTES;
        d = ld_u16(blk);
        q0 = ld16_a2(blk + 2);
        q1 = ld16_a2(blk + 18);
    }
    __device__ __forceinline__ void dots(const Act<TYPE_Q8_0> &a, int S[1], int = 0) const {
        int s = 0;
        s = dot4(q0.x, a.q[0].x, s);
        s = dot4(q0.y, a.q[0].y, s);
        s = dot4(q0.z, a.q[0].z, s);
        s = dot4(q0.w, a.q[0].w, s);
        s = dot4(q1.x, a.q[1].x, s);
        s = dot4(q1.y, a.q[1].y, s);
        s = dot4(q1.z, a.q[1].z, s);
        s = dot4(q1.w, a.q[1].w, s);
        S[0] = s;
    }
    __device__ __forceinline__ float combine(const Act<TYPE_Q8_0> &a, const int S[1], int) const {
        return h2f(d) * h2f(a.ds) * (float)S[0];
    }
};

constexpr int WAVES_PER_BLOCK = 4;

// MODE 0: scaled GEMV into dst; MODE 1: write the integer block dots.
// Rows past nrows are clamped to the last row for loading (branch-free) and
// masked at the store.  K < 2^31 (checked on the host), so in-row offsets are
// 32-bit.
// Occupancy target: one column of Q4_K / Q8_0 fits in 64 VGPRs without
// spilling, which keeps 8 waves per SIMD so a 14336-row grid (7168 waves) is
// resident in one round.  Q5_K, Q6_K and wider GEMVs would spill at that bound.
template <int TYPE, int NC>
constexpr int gemv_min_waves() { return NC == 1 && TYPE != TYPE_Q6_K && TYPE != TYPE_Q5_K ? 8 : 1; }

template <int TYPE, int NC, int RPW, int MODE>
__global__ __launch_bounds__(64 * WAVES_PER_BLOCK, (gemv_min_waves<TYPE, NC>())) void gemv_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t Kp, float *__restrict__ dst, int64_t dst_col_stride,
    int32_t *__restrict__ dots_out) {
    using F = Fmt<TYPE>;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: row math in SGPRs
    const int64_t row0 = ((int64_t)blockIdx.x * WAVES_PER_BLOCK + wave) * RPW;
    if (row0 >= nrows) return;

    const uint8_t *rowp[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rowp[r] = w + (row0 + r < nrows ? row0 + r : nrows - 1) * row_stride;

    float acc[RPW][NC];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;

    constexpr int STEP = 64 * F::W;
    const int K32 = (int)K;
    for (int k0 = 0; k0 < K32; k0 += STEP) {
        const int kl = k0 + lane * F::W;
        if (kl < K32) {
            Wt<TYPE> wt[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) wt[r].load(rowp[r], kl);
            Act<TYPE> a[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) a[c].load(yqs + c * Kp, yds + c * (Kp / QK8), kl);
            // Keep every load of this step above the arithmetic: left alone, the
            // scheduler sinks row r+1's loads below row r's dots, which costs a
            // second memory round trip per wave.
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    int S[F::NSUB];
                    wt[r].dots(a[c], S, kl);
                    if constexpr (MODE == 0) {
                        acc[r][c] += wt[r].combine(a[c], S, kl);
                    } else {
                        if (row0 + r >= nrows) continue;
                        const int64_t nsub_row = TYPE == TYPE_Q6_K ? K / 16 : K / 32;
                        int32_t *o = dots_out + ((int64_t)c * nrows + row0 + r) * nsub_row;
                        if constexpr (TYPE == TYPE_Q6_K) {
                            const int sb = kl / QK_K;
                            const int qq = (kl % QK_K) / 64;
                            const int n = qq >> 1, h = qq & 1;
#pragma unroll
                            for (int g = 0; g < 4; ++g) o[sb * 16 + 8 * n + 2 * g + h] = S[g];
                        } else {
#pragma unroll
                            for (int s = 0; s < F::NSUB; ++s) o[kl / 32 + s] = S[s];
                        }
                    }
                }
            }
        }
    }
    if constexpr (MODE == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float v = wave_sum(acc[r][c]);
                if (lane == r * NC + c && row0 + r < nrows) dst[(int64_t)c * dst_col_stride + row0 + r] = v;
            }
    }
}

// Row-streaming GEMV (2..8 columns on large Q4_K matrices).  The v_dot4
// GEMV above re-loads every column's activation slice for each pair of rows,
// and at 4-8 columns those loads, not the weights, occupy the texture
// addresser.  Here a wave owns R rows: per K-step it loads the activation
// slice once, streams the R rows' weight slices through a queue of D loads in
// flight, and keeps per-lane partial sums of all R x NC outputs.  The sums
// across the 64 lanes go through LDS, 64 outputs at a time: lane o adds
// output o of every lane in lane order.
template <int TYPE, int NC, int R, int D>
__global__ __launch_bounds__(256) void gemv_rows_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t Kp, float *__restrict__ dst, int64_t dst_col_stride) {
    using F = Fmt<TYPE>;
    constexpr int NO = R * NC;  // outputs per wave
    constexpr int LD = 65;      // padded LDS row of one lane's 64 partial sums
    __shared__ float red[WAVES_PER_BLOCK][64 * LD];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t r0 = ((int64_t)blockIdx.x * WAVES_PER_BLOCK + wave) * R;
    if (r0 >= nrows) return;  // uniform per wave; no workgroup barrier follows
    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowp[r] = w + (r0 + r < nrows ? r0 + r : nrows - 1) * row_stride;
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    constexpr int STEP = 64 * F::W;
    const int K32 = (int)K;
    for (int k0 = 0; k0 < K32; k0 += STEP) {
        const int kl = k0 + lane * F::W;
        const bool live = kl < K32;
        const int klc = live ? kl : k0;  // lanes past K load a valid slice and add nothing
        Act<TYPE> a[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) a[c].load(yqs + c * Kp, yds + c * (Kp / QK8), klc);
        Wt<TYPE> q[D];
#pragma unroll
        for (int i = 0; i < D && i < R; ++i) q[i].load(rowp[i], klc);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const Wt<TYPE> cur = q[r % D];
            if (r + D < R) q[r % D].load(rowp[r + D], klc);
            // the next row's loads stay above this row's arithmetic
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                int S[F::NSUB];
                cur.dots(a[c], S, klc);
                const float v = cur.combine(a[c], S, klc);
                acc[r][c] += live ? v : 0.0f;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float *buf = red[wave];
#pragma unroll
    for (int o0 = 0; o0 < NO; o0 += 64) {
#pragma unroll
        for (int o = o0; o < o0 + 64 && o < NO; ++o) buf[lane * LD + (o - o0)] = acc[o / NC][o % NC];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's partial sums are in LDS
        const int o = o0 + lane;
        float sum = 0.0f;
        if (o < NO) {
#pragma unroll 16
            for (int i = 0; i < 64; ++i) sum += buf[i * LD + lane];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0xc07f);  // every lane has read before the next chunk is written
        const int r = o / NC, c = o % NC;
        if (o < NO && r0 + r < nrows) dst[(int64_t)c * dst_col_stride + r0 + r] = sum;
    }
}

// K-split GEMV (small row counts and long rows): the four waves of a
// workgroup share RPW rows and take a quarter of the K-steps each; their
// partial sums meet in LDS and are added in wave order.
template <int TYPE, int NC, int RPW>
__global__ __launch_bounds__(256) void gemv_ks_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t Kp, float *__restrict__ dst, int64_t dst_col_stride) {
    using F = Fmt<TYPE>;
    __shared__ float part[WAVES_PER_BLOCK][RPW * NC];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = (int64_t)blockIdx.x * RPW;
    const uint8_t *rowp[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rowp[r] = w + (row0 + r < nrows ? row0 + r : nrows - 1) * row_stride;
    float acc[RPW][NC];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    constexpr int STEP = 64 * F::W;
    const int K32 = (int)K;
    const int nsteps = (K32 + STEP - 1) / STEP;
    const int s0 = nsteps * wave / WAVES_PER_BLOCK, s1 = nsteps * (wave + 1) / WAVES_PER_BLOCK;
    for (int st = s0; st < s1; ++st) {
        const int kl = st * STEP + lane * F::W;
        if (kl < K32) {
            Wt<TYPE> wt[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) wt[r].load(rowp[r], kl);
            Act<TYPE> a[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) a[c].load(yqs + c * Kp, yds + c * (Kp / QK8), kl);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    int S[F::NSUB];
                    wt[r].dots(a[c], S, kl);
                    acc[r][c] += wt[r].combine(a[c], S, kl);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float v = wave_sum(acc[r][c]);
            if (lane == 0) part[wave][r * NC + c] = v;
        }
    __syncthreads();
    if (wave == 0 && lane < RPW * NC) {
        float v = part[0][lane];
#pragma unroll
        for (int i = 1; i < WAVES_PER_BLOCK; ++i) v += part[i][lane];
        const int r = lane / NC, c = lane % NC;
        if (row0 + r < nrows) dst[(int64_t)c * dst_col_stride + row0 + r] = v;
    }
}

// One f32 column with the reference's mul_mat_vec fusion epilogue
// (ggml_cuda_mm_fusion_args_device, src/ggml/cuda/common.zig:1448-1459):
//   u[r] = W[r] . x (+ bias[r]);  GATE: g[r] = Wg[r] . x (+ gate_bias[r]),
//   dst[r] = glu(g[r], u[r]);  otherwise dst[r] = u[r].
// The quantize-in-GEMV prologue (the fusion arguments of mmvq.zig:552-622):
// each workgroup issues its activation loads, then its rows' weight loads, and
// quantizes the column to Q8_1 with the standalone quantizer's per-quad code
// (identical bytes) into dynamic LDS of K + K/8 bytes while the weights are in
// flight; one barrier, and the Q8_1 copy never reaches memory.  Each wave owns R
// rows of W (and the same R rows of Wg), one K-step of 64 lanes x W weights
// at a time; the first step's weights are in flight during the prologue.
// The dots and their combination are the two-rows-per-wave kernel's, in the
// same order, so u and g equal that kernel's outputs bit for bit.  Biases are read at the start, from a valid address when absent (the
// value is then unused), so no load sits behind a branch.
//
// KS > 1 (long rows): the workgroup's FW waves are FW / KS row groups times KS
// K shares; share h of a row group contracts K-steps [h n / KS, (h + 1) n / KS)
// of the n steps of the row, so each wave has its first (often only) step in
// flight during the prologue.  Shares 1..KS-1 leave their segment sums in LDS
// behind the Q8_1 copy and share 0 adds them in share order after a second
// barrier (deterministic; one wave per row group runs the epilogue).
//
// IDS (MUL_MAT_ID with few tokens, the reference's MMVQ-with-ids path,
// mmvq.zig:116-125, 531-622): grid y enumerates the (token t, slot s) pairs;
// the pair's expert e = ids[t, s] selects the weights (w + e * expert_stride),
// its column is x row t * ne11 + s % ne11, its result dst row t * n_ids + s.
// An id outside [0, n_as) yields a zero row, as the CPU path's -1 does
// (src/ggml/cpu/mulmat.zig:555-777).  A shared expert (the reference's
// shared_up / shared_gate / shared_dst fusion arguments, mmvq.zig:300-320,
// 574-590) is one more row of workgroups after the pairs: grid y = n_pairs +
// t runs token t's column through the shared weights into shared_dst.
constexpr int FX_MAXK = 32768;

// Byte offset of the K-share partial sums in the fused GEMV's dynamic LDS:
// after the Q8_1 copy (K bytes + K / 32 scale words), 16-aligned.
__host__ __device__ constexpr int fx_part_offset(int K) { return (K + K / 8 + 15) & ~15; }

struct FxIds {
    const int32_t *ids;
    int64_t ids_stride, x_row_stride, expert_stride, dst_row_stride;
    int n_ids, ne11, n_as, n_pairs;
    // shared expert (gated): grid y rows n_pairs .. n_pairs + n_shared - 1
    // are token t = y - n_pairs through shared_up / shared_gate, into
    // shared_dst + t * shared_dst_row_stride
    const uint8_t *shared_up, *shared_gate;
    float *shared_dst;
    int64_t shared_dst_row_stride;
    int n_shared;
    // per-expert biases (ADD_ID): the routed rows of expert e add bias +
    // e * bias_expert_stride (and gate_bias likewise)
    int64_t bias_expert_stride;
};

template <int TYPE, int FW, int R, bool GATE, bool IDS, int SEG, int KS>
__global__ __launch_bounds__(64 * FW) void gemv_fx_kernel(const uint8_t *__restrict__ w,
                                                             const uint8_t *__restrict__ wg, int K32, int64_t nrows,
                                                             int64_t row_stride, const float *x,
                                                             const float *bias, const float *gbias, int glu_op,
                                                             float alpha, float limit, float *__restrict__ dst,
                                                             FxIds fi) {
    using F = Fmt<TYPE>;
    int expert = 0;
    bool shared = false;  // uniform per workgroup
    if constexpr (IDS) {
        const int p = blockIdx.y;
        if (p < fi.n_pairs) {
            const int t = p / fi.n_ids, slot = p - t * fi.n_ids;
            x += (int64_t)(t * fi.ne11 + slot % fi.ne11) * fi.x_row_stride;
            dst += (int64_t)p * fi.dst_row_stride;
            // no ids: every pair runs through the one matrix (the op's columns, qmm_mul_mat_fx_percol)
            expert = fi.ids ? __builtin_amdgcn_readfirstlane(fi.ids[(int64_t)t * fi.ids_stride + slot]) : 0;
        } else {
            const int t = p - fi.n_pairs;
            x += (int64_t)t * fi.ne11 * fi.x_row_stride;
            dst = fi.shared_dst + (int64_t)t * fi.shared_dst_row_stride;
            shared = true;
        }
    }
    constexpr int NM = GATE ? 2 : 1;
    constexpr int NSEG = 64 / SEG;            // weight rows side by side in a wave
    constexpr int CH = 8 * 64 * FW;           // activation values per prologue pass
    constexpr int STEP = SEG * F::W;          // K per step of a segment
    constexpr int FWR = FW / KS;              // row groups per workgroup
    static_assert(FW % KS == 0 && (KS == 1 || SEG == 64), "K shares: whole waves, one row per lane group");
    extern __shared__ __align__(16) uint8_t fx_lds[];
    int8_t *aq = reinterpret_cast<int8_t *>(fx_lds);
    uint32_t *ad = reinterpret_cast<uint32_t *>(fx_lds + K32);  // K32 % 32 == 0
    // First pass of activation loads, then the biases, then the weights:
    // loads complete in issue order, so the quantization waits only for the
    // activations.
    const int kq = 8 * (int)threadIdx.x;
    const int kqc = kq < K32 ? kq : 0;
    const float4 xa = *reinterpret_cast<const float4 *>(x + kqc);
    const float4 xb = *reinterpret_cast<const float4 *>(x + kqc + 4);
    // K shares serve long rows: their second pass goes out ahead of the weights too
    constexpr int PRE = KS > 1 ? 2 : 1;
    float4 xc{}, xd{};
    if constexpr (PRE > 1) {
        const int k2 = kq + CH < K32 ? kq + CH : 0;
        xc = *reinterpret_cast<const float4 *>(x + k2);
        xd = *reinterpret_cast<const float4 *>(x + k2 + 4);
    }
    const int lane = threadIdx.x & 63;
    const int seg = lane / SEG, sl = lane % SEG;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = wave / FWR, wr = wave - kh * FWR;  // K share, row group
    const int64_t row0 = ((int64_t)blockIdx.x * FWR + wr) * (R * NSEG);  // the wave's first row
    // the share's K-steps [s0, s1) (KS = 1: all of them)
    const int nsteps = (K32 + STEP - 1) / STEP;
    const int s0 = kh * nsteps / KS, s1 = (kh + 1) * nsteps / KS;
    // IDS: the routed expert's bias rows (the id clamped to a valid expert
    // for the address; an invalid id's row is zero and the value unused)
    if constexpr (IDS) {
        if (!shared) {
            const int64_t eb = (int64_t)(expert >= 0 && expert < fi.n_as ? expert : 0) * fi.bias_expert_stride;
            if (bias) bias += eb;
            if (gbias) gbias += eb;
        }
    }
    // lane rows: row0 + r * NSEG + seg, clamped for loading
    int64_t rowc[R];
    float bu[R], bg[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = row0 + r * NSEG + seg;
        rowc[r] = row < nrows ? row : nrows - 1;
        bu[r] = *(bias ? bias + rowc[r] : x);
        bg[r] = GATE ? *(gbias ? gbias + rowc[r] : x) : 0.0f;
    }
    asm volatile("" ::: "memory");  // keep them ahead of the weight loads
    if constexpr (IDS) {
        if (shared) {
            w = fi.shared_up;
            if constexpr (GATE) wg = fi.shared_gate;
        } else {
            if (expert < 0 || expert >= fi.n_as) {  // uniform per workgroup, before its barriers
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (kh == 0 && sl == SEG - 1 && row0 + r * NSEG + seg < nrows) dst[row0 + r * NSEG + seg] = 0.0f;
                return;
            }
            w += (int64_t)expert * fi.expert_stride;
            if constexpr (GATE) wg += (int64_t)expert * fi.expert_stride;
        }
    }
    const uint8_t *rows[NM][R];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) rows[m][r] = (m ? wg : w) + rowc[r] * row_stride;
    int kl = s0 * STEP + sl * F::W;
    bool live = s0 < s1 && kl < K32;
    int klc = live ? kl : 0;  // lanes past K load a valid slice and add nothing
    Wt<TYPE> wt[NM][R];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) wt[m][r].load(rows[m][r], klc);
    if (kq < K32) {
        const float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const Q8Quad q = q8_1_quantize_quad(v);
        *reinterpret_cast<uint2 *>(aq + kq) = make_uint2(q.lo, q.hi);
        if ((threadIdx.x & 3) == 0) ad[kq / QK8] = q.ds;
    }
    if (PRE > 1 && kq + CH < K32) {
        const float v[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
        const Q8Quad q = q8_1_quantize_quad(v);
        *reinterpret_cast<uint2 *>(aq + kq + CH) = make_uint2(q.lo, q.hi);
        if ((threadIdx.x & 3) == 0) ad[(kq + CH) / QK8] = q.ds;
    }
    for (int k = kq + PRE * CH; k < K32; k += CH) {  // columns longer than the passes above
        const float4 ya = *reinterpret_cast<const float4 *>(x + k);
        const float4 yb = *reinterpret_cast<const float4 *>(x + k + 4);
        const float v[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
        const Q8Quad q = q8_1_quantize_quad(v);
        *reinterpret_cast<uint2 *>(aq + k) = make_uint2(q.lo, q.hi);
        if ((threadIdx.x & 3) == 0) ad[k / QK8] = q.ds;
    }
    __syncthreads();
    // uniform per wave, after the workgroup's last barrier (K shares meet again
    // at the end: their waves past the rows compute clamped rows and store nothing)
    if (KS == 1 && row0 >= nrows) return;
    float acc[NM][R];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
    auto contract = [&](const Wt<TYPE> (&cur)[NM][R]) {
        Act<TYPE> a;
        a.load(aq, ad, klc);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int S[F::NSUB];
                cur[m][r].dots(a, S, klc);
                const float v = cur[m][r].combine(a, S, klc);
                acc[m][r] += live ? v : 0.0f;
            }
    };
    contract(wt);
    // Rows longer than one step: load, then contract.  No prefetch into a
    // second register set: that would cost the occupancy the single-step
    // case runs on, and with many waves per SIMD the other waves cover the
    // latency.
    for (int k0 = (s0 + 1) * STEP; k0 < s1 * STEP; k0 += STEP) {  // s1 <= nsteps: k0 < K32
        kl = k0 + sl * F::W;
        live = kl < K32;
        klc = live ? kl : 0;
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) wt[m][r].load(rows[m][r], klc);
        contract(wt);
    }
    // Segment sums land in each segment's last lane, which writes its rows.
    float us[R], gs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        us[r] = seg_sum<SEG>(acc[0][r]);
        gs[r] = GATE ? seg_sum<SEG>(acc[NM - 1][r]) : 0.0f;
    }
    if constexpr (KS > 1) {
        // shares 1..KS-1: part[(h - 1) * FWR + group][m * R + r], behind the Q8_1 copy
        float *part = reinterpret_cast<float *>(fx_lds + fx_part_offset(K32));
        if (kh > 0 && sl == SEG - 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                part[((kh - 1) * FWR + wr) * (NM * R) + r] = us[r];
                if constexpr (GATE) part[((kh - 1) * FWR + wr) * (NM * R) + R + r] = gs[r];
            }
        }
        __syncthreads();
        if (kh > 0) return;
        if (sl == SEG - 1) {
#pragma unroll
            for (int h = 1; h < KS; ++h)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    us[r] += part[((h - 1) * FWR + wr) * (NM * R) + r];
                    if constexpr (GATE) gs[r] += part[((h - 1) * FWR + wr) * (NM * R) + R + r];
                }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float u = us[r];
        const float g = gs[r];
        const int64_t row = row0 + r * NSEG + seg;
        if (sl == SEG - 1 && row < nrows) {
            if (bias) u += bu[r];
            if constexpr (GATE) u = glu_apply(glu_op, gbias ? g + bg[r] : g, u, alpha, limit);
            dst[row] = u;
        }
    }
}

// 2-4 f32 columns with the quantization fused in (no gate, bias or ids): the
// one-column kernel's prologue once per column -- all columns' first-pass
// loads first, then the weights -- into NC LDS copies of K + K/8 bytes, then
// each K-step's weights contract against every column in turn.  Column c of
// x starts at x + c * x_col_stride, of dst at dst + c * dst_col_stride; grid
// row y takes columns NC * y .. NC * y + NC - 1.  The
// per-column arithmetic is the one-column kernel's with one K share, so a
// column equals hip_qmm_mul_mat_vec_f32 on it bit for bit wherever that runs
// one share.
template <int TYPE, int FW, int R, int NC>
__global__ __launch_bounds__(64 * FW) void gemv_fxn_kernel(const uint8_t *__restrict__ w, int K32, int64_t nrows,
                                                             int64_t row_stride, const float *x,
                                                             int64_t x_col_stride, float *__restrict__ dst,
                                                             int64_t dst_col_stride) {
    using F = Fmt<TYPE>;
    constexpr int CH = 8 * 64 * FW;
    constexpr int STEP = 64 * F::W;
    extern __shared__ __align__(16) uint8_t fx_lds[];
    const int cb = fx_part_offset(K32);  // bytes per column copy
    x += (int64_t)blockIdx.y * NC * x_col_stride;
    dst += (int64_t)blockIdx.y * NC * dst_col_stride;
    const int kq = 8 * (int)threadIdx.x;
    const int kqc = kq < K32 ? kq : 0;
    float4 xa[NC], xb[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        xa[c] = *reinterpret_cast<const float4 *>(x + c * x_col_stride + kqc);
        xb[c] = *reinterpret_cast<const float4 *>(x + c * x_col_stride + kqc + 4);
    }
    asm volatile("" ::: "memory");  // keep them ahead of the weight loads
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = ((int64_t)blockIdx.x * FW + wave) * R;
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = w + (row0 + r < nrows ? row0 + r : nrows - 1) * row_stride;
    int kl = lane * F::W;
    bool live = kl < K32;
    int klc = live ? kl : 0;
    Wt<TYPE> wt[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wt[r].load(rows[r], klc);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int8_t *aq = reinterpret_cast<int8_t *>(fx_lds + c * cb);
        uint32_t *ad = reinterpret_cast<uint32_t *>(fx_lds + c * cb + K32);
        if (kq < K32) {
            const float v[8] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w, xb[c].x, xb[c].y, xb[c].z, xb[c].w};
            const Q8Quad q = q8_1_quantize_quad(v);
            *reinterpret_cast<uint2 *>(aq + kq) = make_uint2(q.lo, q.hi);
            if ((threadIdx.x & 3) == 0) ad[kq / QK8] = q.ds;
        }
        for (int k = kq + CH; k < K32; k += CH) {
            const float4 ya = *reinterpret_cast<const float4 *>(x + c * x_col_stride + k);
            const float4 yb = *reinterpret_cast<const float4 *>(x + c * x_col_stride + k + 4);
            const float v[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
            const Q8Quad q = q8_1_quantize_quad(v);
            *reinterpret_cast<uint2 *>(aq + k) = make_uint2(q.lo, q.hi);
            if ((threadIdx.x & 3) == 0) ad[k / QK8] = q.ds;
        }
    }
    __syncthreads();
    if (row0 >= nrows) return;  // uniform per wave, after the workgroup's only barrier
    float acc[NC][R];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[c][r] = 0.0f;
    for (int k0 = 0;;) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            Act<TYPE> a;
            a.load(reinterpret_cast<const int8_t *>(fx_lds + c * cb),
                   reinterpret_cast<const uint32_t *>(fx_lds + c * cb + K32), klc);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int S[F::NSUB];
                wt[r].dots(a, S, klc);
                const float v = wt[r].combine(a, S, klc);
                acc[c][r] += live ? v : 0.0f;
            }
        }
        k0 += STEP;
        if (k0 >= K32) break;
        kl = k0 + lane * F::W;
        live = kl < K32;
        klc = live ? kl : 0;
#pragma unroll
        for (int r = 0; r < R; ++r) wt[r].load(rows[r], klc);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float u = seg_sum<64>(acc[c][r]);
            if (lane == 63 && row0 + r < nrows) dst[c * dst_col_stride + row0 + r] = u;
        }
}

template <int TYPE, int NC, int R, int D>
int launch_rows(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                const uint32_t *yds, float *dst, int64_t dst_col_stride, hipStream_t s) {
    const int64_t units = (nrows + R - 1) / R;
    const int64_t nblocks = (units + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_rows_kernel<TYPE, NC, R, D>), dim3((unsigned)nblocks), dim3(64 * WAVES_PER_BLOCK), 0,
                       s, w, K, nrows, row_stride, yqs, yds, pad_k(K), dst, dst_col_stride);
    return (int)hipGetLastError();
}

template <int TYPE, int NC, int RPW>
int launch_ks(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
              const uint32_t *yds, float *dst, int64_t dst_col_stride, hipStream_t s) {
    const int64_t nblocks = (nrows + RPW - 1) / RPW;
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_ks_kernel<TYPE, NC, RPW>), dim3((unsigned)nblocks), dim3(64 * WAVES_PER_BLOCK), 0, s,
                       w, K, nrows, row_stride, yqs, yds, pad_k(K), dst, dst_col_stride);
    return (int)hipGetLastError();
}

template <int TYPE, int NC, int MODE>
int launch_nc(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
              const uint32_t *yds, float *dst, int64_t dst_col_stride, int32_t *dots, hipStream_t s) {
    const int64_t Kp = pad_k(K);
    // rows per wave: 2 measured best for one column (more waves in flight);
    // with more columns the activation registers grow and fewer rows fit
    constexpr int RPW = 2;
    const int64_t rows_per_block = (int64_t)WAVES_PER_BLOCK * RPW;
    const int64_t nblocks = (nrows + rows_per_block - 1) / rows_per_block;
    if (nblocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_kernel<TYPE, NC, RPW, MODE>), dim3((unsigned)nblocks), dim3(64 * WAVES_PER_BLOCK), 0,
                       s, w, K, nrows, row_stride, yqs, yds, Kp, dst, dst_col_stride, dots);
    return (int)hipGetLastError();
}

// Kernel choice for the scaled GEMV (measured on MI355X over the decode and
// cross-quant shapes of bench.py):
//   - Q4_K, K <= 4096, 2..8 columns, >= 4096 rows (>= 8192 at 2 columns):
//     row-streaming, 16 rows per wave from 8192 rows (8 at 2 columns), else 4;
//   - at most 2048 rows, or (K-quants) K >= 8192 with at most 4096 rows: the
//     K-split kernel (1 row per workgroup at <= 2048 rows -- 2 for Q4_K at
//     5-8 columns -- and 4 otherwise);
//   - everything else: the two-rows-per-wave kernel.
enum class GemvKind { pairs, rows16, rows8, rows4, ks1, ks2, ks4 };

GemvKind choose(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (type == TYPE_Q4_K && K <= 4096 && ncols >= 2 && nrows >= (ncols == 2 ? 8192 : 4096))
        return nrows >= 8192 ? (ncols == 2 ? GemvKind::rows8 : GemvKind::rows16) : GemvKind::rows4;
    if (nrows <= 2048) return type == TYPE_Q4_K && ncols >= 5 ? GemvKind::ks2 : GemvKind::ks1;
    if (type != TYPE_Q8_0 && type != TYPE_Q4_0 && K >= 8192 && nrows <= 4096) return GemvKind::ks4;
    return GemvKind::pairs;
}

template <int TYPE, int NC>
int launch_scaled(GemvKind kind, const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                  const uint32_t *yds, float *dst, int64_t dst_col_stride, hipStream_t s) {
    constexpr int D = NC <= 4 ? 4 : 2;  // weight loads in flight (register budget)
    if constexpr (TYPE == TYPE_Q4_K && NC >= 2) {
        switch (kind) {
        case GemvKind::rows16: return launch_rows<TYPE, NC, 16, D>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
        case GemvKind::rows8: return launch_rows<TYPE, NC, 8, 4>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
        case GemvKind::rows4: return launch_rows<TYPE, NC, 4, 4>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
        default: break;
        }
    }
    switch (kind) {
    case GemvKind::ks1: return launch_ks<TYPE, NC, 1>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
    case GemvKind::ks2: return launch_ks<TYPE, NC, 2>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
    case GemvKind::ks4: return launch_ks<TYPE, NC, 4>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
    default: return launch_nc<TYPE, NC, 0>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, nullptr, s);
    }
}

template <int TYPE, int MODE>
int launch_type(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                const uint32_t *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int32_t *dots,
                hipStream_t s) {
    if constexpr (MODE == 0) {
        const GemvKind kind = choose(TYPE, K, nrows, ncols);
        {
            switch (ncols) {
            case 1: return launch_scaled<TYPE, 1>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 2: return launch_scaled<TYPE, 2>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 3: return launch_scaled<TYPE, 3>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 4: return launch_scaled<TYPE, 4>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 5: return launch_scaled<TYPE, 5>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 6: return launch_scaled<TYPE, 6>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 7: return launch_scaled<TYPE, 7>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            case 8: return launch_scaled<TYPE, 8>(kind, w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, s);
            default: return (int)hipErrorInvalidValue;
            }
        }
    }
    switch (ncols) {
    case 1: return launch_nc<TYPE, 1, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 2: return launch_nc<TYPE, 2, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 3: return launch_nc<TYPE, 3, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 4: return launch_nc<TYPE, 4, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 5: return launch_nc<TYPE, 5, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 6: return launch_nc<TYPE, 6, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 7: return launch_nc<TYPE, 7, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    case 8: return launch_nc<TYPE, 8, MODE>(w, K, nrows, row_stride, yqs, yds, dst, dst_col_stride, dots, s);
    default: return (int)hipErrorInvalidValue;
    }
}

int check_shape(int type, int64_t K, int64_t nrows, int64_t row_stride) {
    if (K <= 0 || nrows <= 0) return (int)hipErrorInvalidValue;
    int64_t bs, bb;
    switch (type) {
    case TYPE_Q4_K: bs = QK_K; bb = Q4K_BYTES; break;
    case TYPE_Q5_K: bs = QK_K; bb = Q5K_BYTES; break;
    case TYPE_Q6_K: bs = QK_K; bb = Q6K_BYTES; break;
    case TYPE_Q8_0: bs = QK8; bb = Q80_BYTES; break;
    case TYPE_Q4_0: bs = QK8; bb = Q40_BYTES; break;
    case TYPE_IQ4_XS: bs = QK_K; bb = IQ4XS_BYTES; break;
    default: return (int)hipErrorInvalidValue;
    }
    if (K % bs != 0 || K > (1 << 30) || row_stride < K / bs * bb) return (int)hipErrorInvalidValue;
    // row bases keep the blocks' natural alignment: 16 bytes for Q4_K (144-byte
    // blocks, read as dwordx4), 2 bytes for Q6_K / Q8_0 (read by ld16_u / ld16_a2)
    if (row_stride % block_align(type)) return (int)hipErrorInvalidValue;
    return 0;
}

template <int MODE>
int dispatch(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
             const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int32_t *dots, void *stream) {
    if (int e = check_shape(type, K, nrows, row_stride)) return e;
    if (!w || !yqs || ncols < 1 || ncols > 8) return (int)hipErrorInvalidValue;
    if (MODE == 0 && (!yds || !dst || dst_col_stride < nrows)) return (int)hipErrorInvalidValue;
    if (MODE == 1 && !dots) return (int)hipErrorInvalidValue;
    if ((uintptr_t)w % block_align(type)) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    switch (type) {
    case TYPE_Q4_K: return launch_type<TYPE_Q4_K, MODE>(wb, K, nrows, row_stride, yqs, ds, ncols, dst, dst_col_stride, dots, s);
    case TYPE_Q5_K: return launch_type<TYPE_Q5_K, MODE>(wb, K, nrows, row_stride, yqs, ds, ncols, dst, dst_col_stride, dots, s);
    case TYPE_Q6_K: return launch_type<TYPE_Q6_K, MODE>(wb, K, nrows, row_stride, yqs, ds, ncols, dst, dst_col_stride, dots, s);
    case TYPE_Q4_0: return launch_type<TYPE_Q4_0, MODE>(wb, K, nrows, row_stride, yqs, ds, ncols, dst, dst_col_stride, dots, s);
    case TYPE_IQ4_XS: return launch_type<TYPE_IQ4_XS, MODE>(wb, K, nrows, row_stride, yqs, ds, ncols, dst, dst_col_stride, dots, s);
    default: return launch_type<TYPE_Q8_0, MODE>(wb, K, nrows, row_stride, yqs, ds, ncols, dst, dst_col_stride, dots, s);
    }
}

}  // namespace

extern "C" int hip_qmm_gemv_mfma(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                 const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                                 int64_t dst_col_stride, void *stream);

// The int8-MFMA GEMV takes 8 columns of K-quant weights on large matrices
// that the row-streaming GEMV does not cover (Q6_K, or rows longer than 4096).
static bool use_gemv_mfma(int type, int64_t K, int64_t nrows, int64_t ncols) {
    const bool rows = type == TYPE_Q4_K && K <= 4096 && nrows >= 4096;
    return (type == TYPE_Q4_K || type == TYPE_Q6_K) && !rows && ncols >= 8 && nrows > 2048 && K % QK_K == 0;
}

extern "C" int hip_qmm_mul_mat_vec(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                   const int8_t *y_qs, const void *y_ds, int64_t ncols, float *dst,
                                   int64_t dst_col_stride, void *stream) {
    if (use_gemv_mfma(type, K, nrows, ncols))
        return hip_qmm_gemv_mfma(type, w, K, nrows, row_stride, y_qs, y_ds, ncols, dst, dst_col_stride, stream);
    return dispatch<0>(type, w, K, nrows, row_stride, y_qs, y_ds, ncols, dst, dst_col_stride, nullptr, stream);
}

extern "C" int hip_qmm_block_dots(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                  const int8_t *y_qs, int64_t ncols, int32_t *out, void *stream) {
    // The Q8_1 scales are not read in this mode; pass the qs plane for both.
    return dispatch<1>(type, w, K, nrows, row_stride, y_qs, y_qs, ncols, nullptr, 0, out, stream);
}

// One f32 activation column, quantized to Q8_1 inside the GEMV (no separate
// quantizer launch, no Q8_1 copy in memory): the fused entry point without a
// gate or a bias.  Same result as hip_qmm_quantize_q8_1_planar followed by
// hip_qmm_mul_mat_vec with one column on the two-rows-per-wave kernel.
extern "C" int hip_qmm_mul_mat_vec_f32(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                       const float *x, float *dst, void *stream) {
    return hip_qmm_mul_mat_vec_fused(type, w, nullptr, K, nrows, row_stride, x, nullptr, nullptr, 0, 0.0f, 0.0f, dst,
                                     stream);
}

namespace {

template <int TYPE, int FW, int R, bool GATE, int SEG = 64>
void launch_fx(const uint8_t *w, const uint8_t *wg, int64_t K, int64_t nrows, int64_t row_stride, const float *x,
               const float *bias, const float *gbias, int op, float alpha, float limit, float *dst, const FxIds *fi,
               hipStream_t s) {
    constexpr int64_t ROWS = (int64_t)FW * R * (64 / SEG);  // rows per workgroup
    const int64_t nblocks = (nrows + ROWS - 1) / ROWS;
    const size_t lds = (size_t)K + (size_t)(K / QK8) * 4;
    if (fi)
        hipLaunchKernelGGL((gemv_fx_kernel<TYPE, FW, R, GATE, true, SEG, 1>),
                           dim3((unsigned)nblocks, (unsigned)(fi->n_pairs + fi->n_shared)), dim3(64 * FW), lds, s, w, wg,
                           (int)K, nrows,
                           row_stride, x, bias, gbias, op, alpha, limit, dst, *fi);
    else
        hipLaunchKernelGGL((gemv_fx_kernel<TYPE, FW, R, GATE, false, SEG, 1>), dim3((unsigned)nblocks), dim3(64 * FW),
                           lds, s, w, wg, (int)K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, FxIds{});
}

// The K-share form (no gate): FW / KS row groups of R rows per workgroup.
template <int TYPE, int FW, int R, int KS>
void launch_fx_ks(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x, const float *bias,
                  float *dst, const FxIds *fi, hipStream_t s) {
    constexpr int64_t ROWS = (int64_t)(FW / KS) * R;
    const int64_t nblocks = (nrows + ROWS - 1) / ROWS;
    const size_t lds = (size_t)fx_part_offset((int)K) + (size_t)(KS - 1) * (FW / KS) * R * 4;
    if (fi)
        hipLaunchKernelGGL((gemv_fx_kernel<TYPE, FW, R, false, true, 64, KS>),
                           dim3((unsigned)nblocks, (unsigned)fi->n_pairs), dim3(64 * FW), lds, s, w, nullptr, (int)K,
                           nrows, row_stride, x, bias, nullptr, 0, 0.0f, 0.0f, dst, *fi);
    else
        hipLaunchKernelGGL((gemv_fx_kernel<TYPE, FW, R, false, false, 64, KS>), dim3((unsigned)nblocks),
                           dim3(64 * FW), lds, s, w, nullptr, (int)K, nrows, row_stride, x, bias, nullptr, 0, 0.0f,
                           0.0f, dst, FxIds{});
}

// CUs of the current device (the host's cached attribute; 256 on MI355X).
int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}

// Waves per workgroup for the plain one-launch GEMV on large matrices (2 rows
// per wave): 16 or 14, whichever puts fewer rows on the busiest CU when the
// workgroups are spread over the CUs (ties: 16, fewer column reads).  At
// 14336 rows 16 waves make 448 workgroups, 2 on 192 CUs and 1 on 64 (64 rows
// on the busiest), 14 waves make 512, 2 on every CU (56 rows): 8.15 against
// 8.35 us, the same bits.
int fx_plain_waves(int64_t nrows) {
    const int64_t cus = device_cus();
    auto busiest = [&](int64_t fw) {
        const int64_t wgs = (nrows + 2 * fw - 1) / (2 * fw);
        return (wgs + cus - 1) / cus * 2 * fw;
    };
    return busiest(14) < busiest(16) ? 14 : 16;
}

template <int TYPE>
void launch_fx_type(const uint8_t *w, const uint8_t *wg, int64_t K, int64_t nrows, int64_t row_stride,
                    const float *x, const float *bias, const float *gbias, int op, float alpha, float limit,
                    float *dst, const FxIds *fi, hipStream_t s) {
    // Without a gate: 16 or 14 waves per workgroup on large matrices
    // (fx_plain_waves), 8 otherwise (the plain fused GEMV's measured
    // choice).  Gated, measured on Q4_K
    // (K = 2048..8192): from 8192 rows 8 waves of 2 rows of each matrix
    // (15.4 vs 15.9 us for 16 waves of 1 at 14336x4096), from 2048 rows 8
    // waves of 1, below that 4 waves of 1 (3.1 vs 3.4 us at 768x2048: more
    // workgroups on a small grid).  Q6_K and Q8_0 keep 16 waves of 1 row on
    // large matrices: two rows of each matrix would cost Q6_K 131 VGPRs.
    // Rows of at most 16 (32) lane slices share a wave 4 (2) to a wave, one
    // segment of lanes each, so short rows do not leave most lanes idle.
    const int64_t lanes = (K + Fmt<TYPE>::W - 1) / Fmt<TYPE>::W;
    if (lanes <= 16) {
        if (wg) launch_fx<TYPE, 4, 1, true, 16>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else launch_fx<TYPE, 8, 1, false, 16>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        return;
    }
    if (lanes <= 32) {
        if (wg) launch_fx<TYPE, 4, 1, true, 32>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else launch_fx<TYPE, 8, 1, false, 32>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        return;
    }
    const bool big = nrows >= 8192;
    // Rows of two or more K-steps on fewer than 8192 rows (ffn_down and the
    // like), plain: K shares, sized for about one 16-wave workgroup per CU
    // (rows / 256 rows each), with no more shares than steps.  Measured at
    // K = 14336 (op us, against the one-share kernel): Q4_K 4096 rows 8.99 vs
    // 10.91 (16 rows per workgroup, R = 2), 2048 rows 6.31 vs 8.95 (8 rows,
    // R = 1), 1024 rows 5.00 vs 8.50 (4 rows, 4 shares); Q6_K 4096 rows 14.95
    // vs 18.8 (R = 1: Q6_K and Q5_K take 76-84 registers at R = 2, and came
    // out slower there), 6144 rows 21.3 vs 30.3; Q6_K 1024x8192 4.35 vs 9.1.
    // Not for K <= 4096 above 2048 rows (Q8_0 / Q4_0, two steps of 2048):
    // 4096x4096 took 5.80 / 4.94 us against 5.57 / 4.22 with one share.  The
    // ids form takes the layout of the same rows without ids, so each of its
    // rows equals the one-column op on that expert bit for bit (Mixtral's
    // ffn_down experts, 4096x14336, run here).
    const int64_t nsteps = (K + 64 * Fmt<TYPE>::W - 1) / (64 * Fmt<TYPE>::W);
    if (!wg && !big && nsteps >= 2 && (K > 4096 || nrows <= 2048)) {
        constexpr bool heavy = TYPE == TYPE_Q6_K || TYPE == TYPE_Q5_K;
        if (nrows <= 1024) {
            if (nsteps >= 4) launch_fx_ks<TYPE, 16, 1, 4>(w, K, nrows, row_stride, x, bias, dst, fi, s);
            else launch_fx_ks<TYPE, 8, 1, 2>(w, K, nrows, row_stride, x, bias, dst, fi, s);
        } else if (nrows <= 2048 || heavy) {
            launch_fx_ks<TYPE, 16, 1, 2>(w, K, nrows, row_stride, x, bias, dst, fi, s);
        } else if (nrows <= 4096 || nsteps < 4) {
            launch_fx_ks<TYPE, 16, 2, 2>(w, K, nrows, row_stride, x, bias, dst, fi, s);
        } else {
            launch_fx_ks<TYPE, 16, 2, 4>(w, K, nrows, row_stride, x, bias, dst, fi, s);
        }
        return;
    }
    if (wg) {
        if (big && TYPE == TYPE_Q4_K)
            launch_fx<TYPE, 8, 2, true>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else if (big)
            launch_fx<TYPE, 16, 1, true>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else if (nrows >= 2048)
            launch_fx<TYPE, 8, 1, true>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else launch_fx<TYPE, 4, 1, true>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
    } else {
        if (big && fx_plain_waves(nrows) == 14)
            launch_fx<TYPE, 14, 2, false>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else if (big)
            launch_fx<TYPE, 16, 2, false>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
        else launch_fx<TYPE, 8, 2, false>(w, wg, K, nrows, row_stride, x, bias, gbias, op, alpha, limit, dst, fi, s);
    }
}

template <int TYPE, int FW, int R, int NC>
void launch_fxn(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x, int64_t xs,
                float *dst, int64_t ds, int groups, hipStream_t s) {
    const int64_t nblocks = (nrows + FW * R - 1) / (FW * R);
    const size_t lds = (size_t)NC * fx_part_offset((int)K);
    hipLaunchKernelGGL((gemv_fxn_kernel<TYPE, FW, R, NC>), dim3((unsigned)nblocks, (unsigned)groups), dim3(64 * FW),
                       lds, s, w, (int)K,
                       nrows, row_stride, x, xs, dst, ds);
}

template <int TYPE, int NC>
void launch_fxn_shape(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x, int64_t xs,
                      float *dst, int64_t ds, hipStream_t s, int groups = 1) {
    // the one-column kernel's workgroup shape below 8192 rows (8 waves of 2 rows)
    launch_fxn<TYPE, 8, 2, NC>(w, K, nrows, row_stride, x, xs, dst, ds, groups, s);
}

// Most columns per launch: 2 for the K-quants, 3 for IQ4_XS, 4 for Q8_0 /
// Q4_0 (more spill registers or take over 128 of them).
constexpr int fxn_max_cols(int type) {
    return type == TYPE_Q8_0 || type == TYPE_Q4_0 ? 4 : type == TYPE_IQ4_XS ? 3 : 2;
}

template <int TYPE>
void launch_fxn_type(const uint8_t *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x, int64_t ncols,
                     int64_t xs, float *dst, int64_t ds, hipStream_t s) {
    constexpr int MC = fxn_max_cols(TYPE);
    if (ncols == 2 * MC) return launch_fxn_shape<TYPE, MC>(w, K, nrows, row_stride, x, xs, dst, ds, s, 2);
    if constexpr (fxn_max_cols(TYPE) >= 4)
        if (ncols == 4) return launch_fxn_shape<TYPE, 4>(w, K, nrows, row_stride, x, xs, dst, ds, s);
    if constexpr (fxn_max_cols(TYPE) >= 3)
        if (ncols == 3) return launch_fxn_shape<TYPE, 3>(w, K, nrows, row_stride, x, xs, dst, ds, s);
    launch_fxn_shape<TYPE, 2>(w, K, nrows, row_stride, x, xs, dst, ds, s);
}

}  // namespace

namespace {

// Shared checks and launch of the fusion-epilogue GEMV; fi selects the ids
// mode (one grid row per (token, slot) pair).
int fused_launch(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows, int64_t row_stride,
                 const float *x, const float *bias, const float *gate_bias, int glu_op, float glu_alpha,
                 float glu_limit, float *dst, const FxIds *fi, void *stream) {
    if (int e = check_shape(type, K, nrows, row_stride)) return e;
    if (!w || !x || !dst || K % QK8 != 0 || K > FX_MAXK || (uintptr_t)x % 16) return (int)hipErrorInvalidValue;
    const uintptr_t walign = (uintptr_t)block_align(type);
    if ((uintptr_t)w % walign || (uintptr_t)w_gate % walign) return (int)hipErrorInvalidValue;
    if (!w_gate && gate_bias) return (int)hipErrorInvalidValue;
    if (w_gate && !glu_op_valid(glu_op)) return (int)hipErrorInvalidValue;
    if ((nrows + 7) / 8 > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wb = (const uint8_t *)w, *gb = (const uint8_t *)w_gate;
    switch (type) {
    case TYPE_Q4_K:
        launch_fx_type<TYPE_Q4_K>(wb, gb, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                                  fi, s);
        break;
    case TYPE_Q5_K:
        launch_fx_type<TYPE_Q5_K>(wb, gb, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                                  fi, s);
        break;
    case TYPE_Q6_K:
        launch_fx_type<TYPE_Q6_K>(wb, gb, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                                  fi, s);
        break;
    case TYPE_Q4_0:
        launch_fx_type<TYPE_Q4_0>(wb, gb, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                                  fi, s);
        break;
    case TYPE_IQ4_XS:
        launch_fx_type<TYPE_IQ4_XS>(wb, gb, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit,
                                    dst, fi, s);
        break;
    default:
        launch_fx_type<TYPE_Q8_0>(wb, gb, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                                  fi, s);
        break;
    }
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int hip_qmm_mul_mat_vec_fused(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                         int64_t row_stride, const float *x, const float *bias,
                                         const float *gate_bias, int glu_op, float glu_alpha, float glu_limit,
                                         float *dst, void *stream) {
    return fused_launch(type, w, w_gate, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                        nullptr, stream);
}

namespace {

struct FxShared {
    const void *up, *gate;
    float *dst;
    int64_t dst_row_stride;
};

int id_vec_fused(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows, int64_t row_stride,
                 int64_t expert_stride, int64_t n_as, const float *x, int64_t ne11, int64_t n_tokens,
                 int64_t x_row_stride, const int32_t *ids, int64_t n_ids, int64_t ids_stride, int glu_op,
                 float glu_alpha, float glu_limit, float *dst, int64_t dst_row_stride, const FxShared *sh,
                 const float *bias, const float *gate_bias, int64_t bias_expert_stride, void *stream) {
    if ((bias || gate_bias) && (sh || bias_expert_stride < nrows)) return (int)hipErrorInvalidValue;
    if (!ids || n_as <= 0 || n_as > 0x7FFFFFFF || n_tokens <= 0 || n_ids <= 0 || ids_stride < n_ids ||
        (ne11 != 1 && ne11 != n_ids) || x_row_stride < K || x_row_stride % 4 || dst_row_stride < nrows)
        return (int)hipErrorInvalidValue;
    const int64_t n_shared = sh ? n_tokens : 0;
    if (n_tokens * n_ids + n_shared > 65535 || n_tokens * ne11 > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    const int64_t walign = block_align(type);
    if (expert_stride < nrows * row_stride || expert_stride % walign || expert_stride > ((int64_t)1 << 40))
        return (int)hipErrorInvalidValue;
    if (sh && (!w_gate || !sh->up || !sh->gate || !sh->dst || ne11 != 1 || sh->dst_row_stride < nrows ||
               (uintptr_t)sh->up % (uintptr_t)walign || (uintptr_t)sh->gate % (uintptr_t)walign))
        return (int)hipErrorInvalidValue;
    FxIds fi{ids, ids_stride, x_row_stride, expert_stride, dst_row_stride,
             (int)n_ids, (int)ne11, (int)n_as, (int)(n_tokens * n_ids),
             nullptr, nullptr, nullptr, 0, (int)n_shared, bias_expert_stride};
    if (sh) {
        fi.shared_up = (const uint8_t *)sh->up;
        fi.shared_gate = (const uint8_t *)sh->gate;
        fi.shared_dst = sh->dst;
        fi.shared_dst_row_stride = sh->dst_row_stride;
    }
    return fused_launch(type, w, w_gate, K, nrows, row_stride, x, bias, gate_bias, glu_op, glu_alpha, glu_limit, dst,
                        &fi, stream);
}

}  // namespace

extern "C" int hip_qmm_mul_mat_id_vec_fused(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                            int64_t row_stride, int64_t expert_stride, int64_t n_as, const float *x,
                                            int64_t ne11, int64_t n_tokens, int64_t x_row_stride, const int32_t *ids,
                                            int64_t n_ids, int64_t ids_stride, int glu_op, float glu_alpha,
                                            float glu_limit, float *dst, int64_t dst_row_stride, void *stream) {
    return id_vec_fused(type, w, w_gate, K, nrows, row_stride, expert_stride, n_as, x, ne11, n_tokens, x_row_stride,
                        ids, n_ids, ids_stride, glu_op, glu_alpha, glu_limit, dst, dst_row_stride, nullptr, nullptr,
                        nullptr, 0, stream);
}

extern "C" int hip_qmm_mul_mat_id_vec_fused_bias(int type, const void *w, const void *w_gate, int64_t K,
                                                 int64_t nrows, int64_t row_stride, int64_t expert_stride,
                                                 int64_t n_as, const float *x, int64_t ne11, int64_t n_tokens,
                                                 int64_t x_row_stride, const int32_t *ids, int64_t n_ids,
                                                 int64_t ids_stride, const float *bias, const float *gate_bias,
                                                 int64_t bias_expert_stride, int glu_op, float glu_alpha,
                                                 float glu_limit, float *dst, int64_t dst_row_stride, void *stream) {
    return id_vec_fused(type, w, w_gate, K, nrows, row_stride, expert_stride, n_as, x, ne11, n_tokens, x_row_stride,
                        ids, n_ids, ids_stride, glu_op, glu_alpha, glu_limit, dst, dst_row_stride, nullptr, bias,
                        gate_bias, bias_expert_stride, stream);
}

extern "C" int hip_qmm_mul_mat_id_vec_fused_shared(int type, const void *w, const void *w_gate, int64_t K,
                                                   int64_t nrows, int64_t row_stride, int64_t expert_stride,
                                                   int64_t n_as, const float *x, int64_t n_tokens,
                                                   int64_t x_row_stride, const int32_t *ids, int64_t n_ids,
                                                   int64_t ids_stride, int glu_op, float glu_alpha, float glu_limit,
                                                   float *dst, int64_t dst_row_stride, const void *shared_up,
                                                   const void *shared_gate, float *shared_dst,
                                                   int64_t shared_dst_row_stride, void *stream) {
    const FxShared sh{shared_up, shared_gate, shared_dst, shared_dst_row_stride};
    return id_vec_fused(type, w, w_gate, K, nrows, row_stride, expert_stride, n_as, x, 1, n_tokens, x_row_stride, ids,
                        n_ids, ids_stride, glu_op, glu_alpha, glu_limit, dst, dst_row_stride, &sh, nullptr, nullptr, 0,
                        stream);
}

// 2-8 f32 columns of a small matrix as rows of the one-column kernel's grid
// (the ids form with no ids: grid y is the column, x + c * x_col_stride in,
// dst + c * dst_col_stride out), each quantizing its own column.  On a grid
// that leaves most CUs idle the columns run side by side and read the
// weights from the L2 / MALL after the first, and no quantizer launch comes
// first.  Each column equals hip_qmm_mul_mat_vec_f32 on it bit for bit.
// Returns hipErrorNotSupported outside the shapes where it measured faster
// (fx_percol_wins), so the caller goes on to its other paths.
//
// Measured (op us, graph-timed, the other paths against this): Q4_K 1024x4096
// at 2 / 4 / 8 columns 4.12 / 5.68 / 7.17 against 3.71 / 3.79 / 4.96, 2048x4096
// 4.57 / 8.06 / 11.33 against 4.20 / 5.46 / 7.62, 1024x2048 3.66 / 5.40 / 6.80
// against 3.01 / 3.05 / 3.75; Q6_K 1024x4096 5.08 / 7.46 / 9.83 against 4.68 /
// 4.69 / 6.65, 2048x4096 5.64 / 10.54 / 17.33 against 5.54 / 7.40 / 11.24; Q5_K
// and IQ4_XS alike.  Larger grids lose (Q4_K 4096x4096 at 2 / 8: 4.96 / 9.67
// against 5.84 / 12.98; Q6_K 3072x4096 at 8: 10.79 against 15.37), and so do
// long rows (Q4_K 1024x14336 at 4: 9.70 against 12.42), which keep the other
// paths.  The legacy types win up to 1024 rows at 2-4 columns (Q8_0 1024x4096
// 5.60 / 7.29 against 4.35 / 5.76; Q4_0 4.48 / 6.63 against 3.96 / 5.59) and
// at every column count on rows of K <= 2048 (Q4_0 1024x2048 at 8: 5.49
// against 3.83; Q8_0 4.51 / 5.45 against 3.45 / 4.39 at 4 / 8), but lose at 6-8
// columns of K = 4096 (Q8_0 1024x4096 at 8: 6.85 against 8.93) and on 2048
// rows (Q8_0 2048x4096 at 4: 7.47 against 9.08; Q4_0 7.12 against 8.49).
static bool fx_percol_wins(int type, int64_t K, int64_t nrows, int64_t ncols) {
    if (ncols < 2 || ncols > 8 || K > 4096) return false;
    if (type == TYPE_Q8_0 || type == TYPE_Q4_0) return nrows <= 1024 && (ncols <= 4 || K <= 2048);
    return nrows <= 2048;
}

extern "C" int hip_qmm_mul_mat_per_column(int type, int64_t K, int64_t nrows, int64_t ncols) {
    return nrows > 0 && K > 0 && K % QK8 == 0 && fx_percol_wins(type, K, nrows, ncols) ? 1 : 0;
}

int qmm_mul_mat_fx_percol(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x,
                          int64_t ncols, int64_t x_col_stride, float *dst, int64_t dst_col_stride, void *stream) {
    if (!fx_percol_wins(type, K, nrows, ncols) || K % QK8 != 0 || (uintptr_t)x % 16 || x_col_stride % 4)
        return (int)hipErrorNotSupported;
    if (dst_col_stride < nrows || x_col_stride < K || !dst) return (int)hipErrorInvalidValue;
    const FxIds fi{nullptr, 1, x_col_stride, 0, dst_col_stride, 1, 1, 1, (int)ncols, nullptr, nullptr, nullptr, 0, 0, 0};
    return fused_launch(type, w, nullptr, K, nrows, row_stride, x, nullptr, nullptr, 0, 0.0f, 0.0f, dst, &fi, stream);
}

// 2-4 f32 columns through the quantize-in-GEMV kernel (hip_qmm_mul_mat's
// path for few columns; no workspace).  Returns hipErrorNotSupported when the
// shape is outside what the kernel takes or where quantizer + GEMV measured
// faster, so the caller quantizes first.  Measured (op us, quantizer + GEMV
// against this): 4096x4096 Q4_K 2 columns 6.90 vs 5.09, Q8_0 4 columns 10.40
// vs 8.24, IQ4_XS 3 columns 7.48 vs 6.42, 1024x4096 Q4_K 2 columns 5.47 vs
// 4.42; slower from 8192 rows (14336x4096 Q4_K 2 columns 11.19 vs 12.08,
// IQ4_XS 12.44 vs 14.10: the doubled registers halve the workgroups per CU)
// but for Q8_0 at 3-4 columns (14336x4096, 4 columns: 24.56 vs 20.77) and
// Q4_K / Q4_0 rows of K <= 2048 (8192x2048 Q4_K 2 columns 7.71 vs 5.86; the
// other types were not measured there and keep quantizer + GEMV); slower on rows
// of K > 4096 (4096x14336 Q4_K 13.08 vs 14.63: no K shares here).  Twice the
// kernel's columns (4 for the K-quants, 6 for IQ4_XS, 8 for Q8_0) run as two
// rows of its grid up to 4096 rows: Q4_K 4096x4096 at 4 columns 7.82 vs 7.08,
// 3072x4096 8.32 vs 6.82, 4096x2048 7.28 vs 5.58; Q5_K 4096x4096 8.93 vs 8.42;
// Q6_K 4096x2048 8.52 vs 7.48 (4096x4096 9.56 vs 9.40); IQ4_XS 4096x4096 at 6
// 9.71 vs 9.19; Q8_0 4096x4096 at 8 11.63 vs 10.53.  Three groups lost (Q5_K
// 4096x4096 at 6: 10.37 vs 11.28), and so did two from 8192 rows (Q5_K
// 8192x4096 at 4: 12.32 vs 14.96); Q4_0 was not measured there.
int qmm_mul_mat_fx_cols(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const float *x,
                        int64_t ncols, int64_t x_col_stride, float *dst, int64_t dst_col_stride, void *stream) {
    const bool big_wins = (K <= 2048 && (type == TYPE_Q4_K || type == TYPE_Q4_0)) || (type == TYPE_Q8_0 && ncols >= 3);
    const bool two_groups = ncols == 2 * fxn_max_cols(type) && nrows <= 4096 && type != TYPE_Q4_0;
    if (ncols < 2 || (ncols > fxn_max_cols(type) && !two_groups) || K % QK8 != 0 || K > 4096 ||
        (nrows >= 8192 && !big_wins) ||
        (uintptr_t)x % 16 || x_col_stride % 4)
        return (int)hipErrorNotSupported;
    if (dst_col_stride < nrows || x_col_stride < K) return (int)hipErrorInvalidValue;
    if (int e = check_shape(type, K, nrows, row_stride)) return e;
    if ((uintptr_t)w % (uintptr_t)block_align(type) || !dst || nrows <= 0) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wb = (const uint8_t *)w;
    switch (type) {
    case TYPE_Q4_K: launch_fxn_type<TYPE_Q4_K>(wb, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, s); break;
    case TYPE_Q5_K: launch_fxn_type<TYPE_Q5_K>(wb, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, s); break;
    case TYPE_Q6_K: launch_fxn_type<TYPE_Q6_K>(wb, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, s); break;
    case TYPE_Q4_0: launch_fxn_type<TYPE_Q4_0>(wb, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, s); break;
    case TYPE_IQ4_XS: launch_fxn_type<TYPE_IQ4_XS>(wb, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, s); break;
    default: launch_fxn_type<TYPE_Q8_0>(wb, K, nrows, row_stride, x, ncols, x_col_stride, dst, dst_col_stride, s); break;
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------- the reference's MMVQ launch
//
// hip_qmm_mul_mat_vec_q: one launch over the channels and samples (or the
// MUL_MAT_ID slots and tokens) of a batched GEMV, on AoS block_q8_1
// activations as hip_qmm_quantize_q8_1 writes them, with the launch arguments
// of the reference's mul_mat_vec_q (the Common struct, src/ggml/cuda/mmvq.zig
// :260-280, filled at :349-420 from mulMatVecQ's strides, :531-696).  The
// arithmetic is the two-rows-per-wave kernel's (Act::load_aos reads the same
// slices from the AoS blocks).  Grid: x = row pairs of 4-wave workgroups,
// y = destination channel (the slot with ids), z = sample (the token column
// with ids).

namespace {

struct VecQArgs {
    const uint8_t *vx, *vy;
    const int32_t *ids;
    float *dst;
    int64_t ncols_x, nrows_x;
    int64_t row_x;                           // bytes between weight rows
    int64_t col_y, col_dst;                  // bytes of Q8_1 / floats between columns
    int64_t nchannels_x, nchannels_y;
    int64_t channel_x, channel_y, channel_dst;  // bytes, bytes, floats
    int64_t channel_ratio, sample_ratio;
    int64_t sample_x, sample_y, sample_dst;     // bytes, bytes, floats
    int64_t ids_stride;
};

template <int TYPE, int NC, bool IDS>
__global__ __launch_bounds__(64 * WAVES_PER_BLOCK) void gemv_vecq_kernel(const VecQArgs a) {
    using F = Fmt<TYPE>;
    constexpr int RPW = 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = ((int64_t)blockIdx.x * WAVES_PER_BLOCK + wave) * RPW;
    if (row0 >= a.nrows_x) return;
    const int64_t ch = blockIdx.y, z = blockIdx.z;
    const uint8_t *x, *y;
    float *d;
    if constexpr (IDS) {
        // one token column per grid z; its slot's expert from ids
        const int64_t e = a.ids[z * a.ids_stride + ch];
        d = a.dst + z * a.col_dst + ch * a.channel_dst;
        if (e < 0 || e >= a.nchannels_x) {  // a dropped slot: a zero row
            if (lane < RPW && row0 + lane < a.nrows_x) d[row0 + lane] = 0.0f;
            return;
        }
        x = a.vx + e * a.channel_x;
        y = a.vy + z * a.col_y + (ch % a.nchannels_y) * a.channel_y;
    } else {
        x = a.vx + (ch / a.channel_ratio) * a.channel_x + (z / a.sample_ratio) * a.sample_x;
        y = a.vy + ch * a.channel_y + z * a.sample_y;
        d = a.dst + ch * a.channel_dst + z * a.sample_dst;
    }
    const uint8_t *rowp[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rowp[r] = x + (row0 + r < a.nrows_x ? row0 + r : a.nrows_x - 1) * a.row_x;
    float acc[RPW][NC];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    constexpr int STEP = 64 * F::W;
    const int K32 = (int)a.ncols_x;
    for (int k0 = 0; k0 < K32; k0 += STEP) {
        const int kl = k0 + lane * F::W;
        if (kl < K32) {
            Wt<TYPE> wt[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) wt[r].load(rowp[r], kl);
            Act<TYPE> av[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) av[c].load_aos(y + c * a.col_y, kl);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    int S[F::NSUB];
                    wt[r].dots(av[c], S, kl);
                    acc[r][c] += wt[r].combine(av[c], S, kl);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float v = wave_sum(acc[r][c]);
            if (lane == r * NC + c && row0 + r < a.nrows_x) d[c * a.col_dst + row0 + r] = v;
        }
}

template <int TYPE, bool IDS>
int launch_vecq(const VecQArgs &a, int64_t ncols, dim3 grid, hipStream_t s) {
    const dim3 block(64 * WAVES_PER_BLOCK);
    if constexpr (IDS) {
        hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 1, true>), grid, block, 0, s, a);
    } else {
        switch (ncols) {
        case 1: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 1, false>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 2, false>), grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 3, false>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 4, false>), grid, block, 0, s, a); break;
        case 5: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 5, false>), grid, block, 0, s, a); break;
        case 6: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 6, false>), grid, block, 0, s, a); break;
        case 7: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 7, false>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((gemv_vecq_kernel<TYPE, 8, false>), grid, block, 0, s, a); break;
        }
    }
    return (int)hipGetLastError();
}

template <bool IDS>
int launch_vecq_type(int type, const VecQArgs &a, int64_t ncols, dim3 grid, hipStream_t s) {
    switch (type) {
    case TYPE_Q4_K: return launch_vecq<TYPE_Q4_K, IDS>(a, ncols, grid, s);
    case TYPE_Q5_K: return launch_vecq<TYPE_Q5_K, IDS>(a, ncols, grid, s);
    case TYPE_Q6_K: return launch_vecq<TYPE_Q6_K, IDS>(a, ncols, grid, s);
    case TYPE_Q4_0: return launch_vecq<TYPE_Q4_0, IDS>(a, ncols, grid, s);
    case TYPE_IQ4_XS: return launch_vecq<TYPE_IQ4_XS, IDS>(a, ncols, grid, s);
    default: return launch_vecq<TYPE_Q8_0, IDS>(a, ncols, grid, s);
    }
}

int64_t block_bytes(int type) {
    switch (type) {
    case TYPE_Q4_K: return Q4K_BYTES;
    case TYPE_Q5_K: return Q5K_BYTES;
    case TYPE_Q6_K: return Q6K_BYTES;
    case TYPE_Q4_0: return Q40_BYTES;
    case TYPE_IQ4_XS: return IQ4XS_BYTES;
    case TYPE_Q8_0: return Q80_BYTES;
    default: return 0;
    }
}

}  // namespace

extern "C" int hip_qmm_mul_mat_vec_q(int type, const void *vx, const void *vy, const int32_t *ids, float *dst,
                                     int64_t ncols_x, int64_t nrows_x, int64_t ncols_dst, int64_t stride_row_x,
                                     int64_t stride_col_y, int64_t stride_col_dst, int64_t nchannels_x,
                                     int64_t nchannels_y, int64_t nchannels_dst, int64_t stride_channel_x,
                                     int64_t stride_channel_y, int64_t stride_channel_dst, int64_t nsamples_x,
                                     int64_t nsamples_dst, int64_t stride_sample_x, int64_t stride_sample_y,
                                     int64_t stride_sample_dst, int64_t ids_stride, void *stream) {
    const int64_t bb = block_bytes(type);
    if (!bb || !vx || !vy || !dst || ncols_dst < 1 || ncols_dst > 8) return (int)hipErrorInvalidValue;
    if (nchannels_x < 1 || nchannels_y < 1 || nchannels_dst < 1 || nsamples_x < 1 || nsamples_dst < 1)
        return (int)hipErrorInvalidValue;
    if (int e = check_shape(type, ncols_x, nrows_x, stride_row_x * bb)) return e;
    const int64_t walign = block_align(type);
    if ((uintptr_t)vx % walign || (stride_channel_x * bb) % walign || (stride_sample_x * bb) % walign ||
        (uintptr_t)vy % 4 || stride_channel_x < 0 || stride_sample_x < 0)
        return (int)hipErrorInvalidValue;
    // each activation column holds the row's Q8_1 blocks
    if (stride_col_y < ncols_x / QK8 || stride_channel_y < 0 || stride_sample_y < 0 || stride_col_dst < 0 ||
        stride_channel_dst < 0 || stride_sample_dst < 0)
        return (int)hipErrorInvalidValue;
    const bool has_ids = ids != nullptr;
    if (has_ids && (nsamples_x != 1 || nsamples_dst != 1 || ids_stride < nchannels_dst)) return (int)hipErrorInvalidValue;
    if (!has_ids && (nchannels_dst % nchannels_x || nsamples_dst % nsamples_x || nchannels_y != nchannels_dst))
        return (int)hipErrorInvalidValue;
    if (!has_ids && ncols_dst > 1 && stride_col_dst < nrows_x) return (int)hipErrorInvalidValue;
    const int64_t gz = has_ids ? ncols_dst : nsamples_dst;
    const int64_t gx = (nrows_x + 2 * WAVES_PER_BLOCK - 1) / (2 * WAVES_PER_BLOCK);
    if (gx > 0x7FFFFFFF || nchannels_dst > 65535 || gz > 65535) return (int)hipErrorInvalidValue;
    VecQArgs a{};
    a.vx = (const uint8_t *)vx;
    a.vy = (const uint8_t *)vy;
    a.ids = ids;
    a.dst = dst;
    a.ncols_x = ncols_x;
    a.nrows_x = nrows_x;
    a.row_x = stride_row_x * bb;
    a.col_y = stride_col_y * Q81_BYTES;
    a.col_dst = stride_col_dst;
    a.nchannels_x = nchannels_x;
    a.nchannels_y = nchannels_y;
    a.channel_x = stride_channel_x * bb;
    a.channel_y = stride_channel_y * Q81_BYTES;
    a.channel_dst = stride_channel_dst;
    a.channel_ratio = has_ids ? 1 : nchannels_dst / nchannels_x;
    a.sample_ratio = nsamples_dst / nsamples_x;
    a.sample_x = stride_sample_x * bb;
    a.sample_y = stride_sample_y * Q81_BYTES;
    a.sample_dst = stride_sample_dst;
    a.ids_stride = ids_stride;
    const dim3 grid((unsigned)gx, (unsigned)nchannels_dst, (unsigned)gz);
    hipStream_t s = (hipStream_t)stream;
    return has_ids ? launch_vecq_type<true>(type, a, ncols_dst, grid, s)
                   : launch_vecq_type<false>(type, a, ncols_dst, grid, s);
}
