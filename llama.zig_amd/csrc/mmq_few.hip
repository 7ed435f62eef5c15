// mmq_few.hip -- Q4_K / Q5_K / Q6_K / Q8_0 / Q4_0 / IQ4_XS GEMM for few
// activation columns (up to 32), on 16x16 int8 MFMA.
//
// The reference sends 2-24 src1 columns to a separate "few-row" MMQ kernel
// (src/ggml/cuda/mmq_few.zig:1-20, mulMatQFew :204-255, shouldUseMmqFew
// :270-281): at that width the weights are streamed once and the 128 x 32
// MMQ tile is mostly empty.  This is the CDNA4 kernel for that regime.
//
// Arithmetic (as mmq.hip / mmq_q4k_dma.hip, on the 16x16 MFMA shapes):
//   out = sum_b d_b * sum_j (sc_bj*d8_j) * S_bj - dmin_b * sum_j m_bj*s8_j
// S_bj, the exact integer dot of sub-block j against the Q8_1 block, comes
// from v_mfma_i32_16x16x32_i8; the scale sc_bj*d8_j is an exact f16 outer
// product from v_mfma_f32_16x16x16_f16 with one live K slot; one convert + FMA
// per output and sub-block; d, dmin and the min term (a K=8 f16 MFMA of
// m_j x s8_j) once per super-block.
//
// Mapping: a workgroup of 4 waves owns 64 rows (16 per wave, one MFMA tile
// high) and all <= 32 columns (one or two 16-column tiles), over its share of
// the K-steps (split K over grid z when the row tiles alone do not fill the
// chip).  Each K-step (one Q4_K super-block) moves from global memory straight
// into LDS with global_load_lds_dwordx4, in 1 KiB transfers (14 per step with
// one column tile, 18 with two):
//   - A: the 64 rows' 144-byte blocks as stored (contiguous 144-byte runs);
//   - B: the columns' 256 Q8_1 codes, 16-byte chunk c of column n at position
//     c ^ n, so the operand reads of 16 columns spread over the banks;
//   - D: the columns' (d8 | s8 << 16) headers.
// Three LDS stages form a ring: while step k is contracted, steps k+1 and k+2
// are in flight, and a wave waits only for its own transfers of step k
// (vmcnt = its transfer count of one step) before the step's barrier.  The
// weight decode (nibbles, scales) is shared by the column tiles.
//
// Q5_K (176-byte blocks, 16-byte aligned like Q4_K) takes the Q4_K path with
// the fifth bit of each element merged from qh (bit g of qh[l] for element l
// of sub-block g).
//
// The 2-byte-aligned types (the reference routes them here too,
// mmq_few.zig:246-266): a K-step is still 256 weights of a row.
//   - Q4_0: 8 blocks of 18 bytes, 144 bytes, 16-byte aligned when the rows
//     are; the Q8_0 path with the lane's 8 nibbles taken as q - 8 (bytewise).
//   - IQ4_XS: one 136-byte block at 8-byte alignment; the step moves the 144
//     aligned bytes around it (from (136 * k) & ~15, the block 0 or 8 bytes
//     in), which stay inside the row when K % 512 == 0.
//   - Q8_0: 8 blocks of 34 bytes, 272 bytes, 16-byte aligned when the rows
//     are; per block S_b from one int8 MFMA and the scale d_w * d8 from the
//     f16 scale MFMA; no super-block terms.
//   - Q6_K: one 210-byte block, which sits at 2-byte alignment.  The step
//     moves the 224 aligned bytes around it (14 x 16, from (210 * k) & ~15:
//     the block starts (2 * k) % 16 bytes in), which stay inside the row when
//     its block count is a multiple of 8 (K % 2048 == 0).  Each 32 weights hold
//     two 16-weight sub-blocks with their own int8 scale: two int8 MFMAs, each
//     with the other sub-block's lanes zeroed, against the same Q8_1 block;
//     the weights go in as q - 32 (bytewise, no carries); d once per step.
// Operand reads at 2-byte alignment in LDS take two byte funnel shifts of
// three aligned dwords.
//
// 16x16 MFMA operand convention: lane l supplies row (l % 16) of A and column
// (l % 16) of B over the K-slice [(l / 16) * K/4, +K/4); the result value i of
// lane l is row 4*(l/16) + i, column l % 16.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

constexpr int FBN = 32;  // most columns (two 16-column MFMA tiles)

// Bytes of one row's K-step as moved to LDS, and where step k starts in the row.
template <int TYPE>
struct FewFmt;
template <>
struct FewFmt<TYPE_Q4_K> {
    static constexpr int WROW = Q4K_BYTES;
    __device__ static int64_t aoff(int kb) { return (int64_t)kb * Q4K_BYTES; }
};
template <>
struct FewFmt<TYPE_Q5_K> {
    static constexpr int WROW = Q5K_BYTES;  // 176, 16-byte aligned
    __device__ static int64_t aoff(int kb) { return (int64_t)kb * Q5K_BYTES; }
};
template <>
struct FewFmt<TYPE_Q4_0> {
    static constexpr int WROW = 8 * Q40_BYTES;  // 144
    __device__ static int64_t aoff(int kb) { return (int64_t)kb * (8 * Q40_BYTES); }
};
template <>
struct FewFmt<TYPE_IQ4_XS> {
    static constexpr int WROW = 144;  // the aligned window around one 136-byte block
    __device__ static int64_t aoff(int kb) { return ((int64_t)kb * IQ4XS_BYTES) & ~(int64_t)15; }
};
template <>
struct FewFmt<TYPE_Q8_0> {
    static constexpr int WROW = 8 * Q80_BYTES;  // 272
    __device__ static int64_t aoff(int kb) { return (int64_t)kb * (8 * Q80_BYTES); }
};
template <>
struct FewFmt<TYPE_Q6_K> {
    static constexpr int WROW = 224;  // the aligned window around one 210-byte block
    __device__ static int64_t aoff(int kb) { return ((int64_t)kb * Q6K_BYTES) & ~(int64_t)15; }
};

// Workgroup geometry for NW waves of 16 rows each and NCT tiles of 16
// columns: the step's LDS stage and its 1 KiB transfers (transfer q goes to
// wave q % NW).
template <int TYPE, int NW, int NCT>
struct FewGeo {
    static constexpr int WROW = FewFmt<TYPE>::WROW;
    static constexpr int BM = 16 * NW;                 // rows per workgroup
    static constexpr int NT = 64 * NW;                 // threads
    static constexpr int A = BM * WROW;                // weights per step
    static_assert(A % 1024 == 0, "whole weight transfers");
    static constexpr int B = 16 * NCT * QK_K;          // codes per step
    static constexpr int D = 16 * NCT * 8 * 4;         // headers per step
    static constexpr int NQ = (A + B + D + 1023) / 1024;
    static constexpr int STAGE = NQ * 1024;
    static constexpr int PER = (NQ + NW - 1) / NW;     // most transfers of one wave
    static constexpr int transfers_of(int w) { return NQ / NW + (w < NQ % NW ? 1 : 0); }
};

__device__ __forceinline__ uint32_t f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// f16 bits of byte b of v (an integer 0..255, exact in f16), zero-extended
__device__ __forceinline__ uint32_t byte_f16(uint32_t v, int b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(uint16_t)((v >> (8 * b)) & 0xFFu));
}

__device__ __forceinline__ long as_long(uint2 v) { return (long)(((uint64_t)v.y << 32) | v.x); }

// 8 bytes at a 2-byte-aligned LDS address: three aligned dwords, funnel-shifted
// (may read up to 4 bytes past p + 8, inside the stage).
__device__ __forceinline__ uint2 lds8_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 2u);
    const uint32_t *b = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t a0 = b[0], a1 = b[1], a2 = b[2];
    return make_uint2(__builtin_amdgcn_alignbyte(a1, a0, sh), __builtin_amdgcn_alignbyte(a2, a1, sh));
}

// Q6_K weights q (0..63 per byte) to q - 32 as signed bytes: q + 96 stays
// below 256 (no carry between bytes), and flipping its bit 7 gives q + 224,
// which is q - 32 mod 256.
__device__ __forceinline__ uint32_t q6_signed(uint32_t q) { return (q + 0x60606060u) ^ 0x80808080u; }

// Q4_0 nibbles q (0..15 per byte) to q - 8 as signed bytes: q ^ 8 is
// (q - 8) mod 16; its bit 3 copied into bits 4-7 sign-extends it.
__device__ __forceinline__ uint32_t q4_0_signed(uint32_t q) {
    const uint32_t x = q ^ 0x08080808u, t = x & 0x08080808u;
    return x | (t << 1) | (t << 2) | (t << 3) | (t << 4);
}

// 16 bytes per lane from global memory to LDS at base + 16 * lane (base is
// wave-uniform).  Issued as inline assembly on purpose: the compiler does not
// track it, so it inserts no vmcnt(0) of its own before the LDS reads of the
// other stages (it cannot tell the stages apart), and the waits of the ring
// (wait_step) are the only ones.  The "memory" clobber keeps LDS reads and
// writes in program order around it.  M0, bound by the "{m0}" operand so
// the compiler sets it, holds the LDS base; the s_nop separates that write
// from the transfer.
__device__ __forceinline__ void dma16(const void *g, void *lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr)lds_base;
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
}

// Wait until at most n of this wave's memory operations are outstanding
// (vmcnt(n); expcnt and lgkmcnt not waited).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));  // vmcnt bits 3:0 and 15:14
}

// Workgroup barrier that orders LDS only.  __syncthreads() also orders
// global memory, so the compiler puts vmcnt(0) before it, which would wait
// for the transfers of the steps still in flight.  Here: this wave's LDS
// reads of the previous step are done (its stage may be refilled after the
// barrier), the acquire fence keeps the next stage's reads below the
// barrier, and wait_step has already waited for this wave's transfers.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// This wave's transfers of step k are complete while those of the `ahead`
// steps issued after it (0 <= ahead <= A) may still be in flight; `big`:
// this wave issues NBIG transfers per step, else NSMALL.  Both are uniform
// over the wave.
template <int A, int NBIG, int NSMALL>
__device__ __forceinline__ void wait_step(bool big, int ahead) {
    if constexpr (A > 0) {
        if (ahead == A) {
            if (big) wait_vm<A * NBIG>();
            else wait_vm<A * NSMALL>();
            return;
        }
        wait_step<A - 1, NBIG, NSMALL>(big, ahead);
    } else {
        wait_vm<0>();
    }
}

// workgroups per CU that the LDS (160 KiB) holds with KH NST-stage rings
template <int TYPE, int NW, int NCT>
constexpr int few_occupancy(int nst, int kh = 1) { return 163840 / (kh * nst * FewGeo<TYPE, NW, NCT>::STAGE); }

// KH K halves: the workgroup's waves are KH groups of NW, each with its own
// ring over an equal share of the workgroup's K-steps (the launcher makes the
// step count a multiple of KH), so two waves with independent work share a
// SIMD; the groups meet at every ring barrier (equal step counts) and add
// their sums through LDS at the end, group 0 first (deterministic).
template <int TYPE, int NST, int NW, int NCT, bool PACK, int KH>
__global__ __launch_bounds__((KH * FewGeo<TYPE, NW, NCT>::NT), (few_occupancy<TYPE, NW, NCT>(NST, KH))) void mmq_few_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int ncols, float *__restrict__ dst, int64_t dst_col_stride,
    float *__restrict__ partial) {
    static_assert(!PACK || (NCT == 1 && (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K || TYPE == TYPE_Q6_K)),
                  "packed: one tile, K-quants");
    using G = FewGeo<TYPE, NW, NCT>;
    using FF = FewFmt<TYPE>;
    constexpr int FA = G::A, FB = G::B, FD = G::D, FNQ = G::NQ, PER = G::PER, WROW = G::WROW;
    constexpr int NQA = FA / 1024;  // transfers 0 .. NQA-1 move weights
    static_assert(NST >= 2 && few_occupancy<TYPE, NW, NCT>(NST, KH) >= 1, "ring depth");
    static_assert((NST - 2) * G::transfers_of(0) <= 63, "vmcnt field");
    static_assert(KH == 1 || NCT * NW * 1024 <= G::STAGE, "K-half sums fit one stage");
    __shared__ alignas(16) uint8_t rings[KH][NST][G::STAGE];
    __shared__ alignas(16) uint4 zero16;  // the packed path's B operand for the lanes of the other sub-block
    if (PACK && threadIdx.x == 0) zero16 = make_uint4(0u, 0u, 0u, 0u);  // published by the ring's first barrier

    const int64_t Kp = pad_k(K);
    const int lane = threadIdx.x & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = wave_all / NW, wave = wave_all - kh * NW;  // K half, wave within it
    uint8_t(*st)[G::STAGE] = rings[kh];
    const int li = lane & 15, kq = lane >> 4;
    const int64_t row0 = (int64_t)blockIdx.x * G::BM;
    const int nkb = (int)(K / QK_K);
    const int gz = (int)gridDim.z, z = (int)blockIdx.z;
    const int kz0 = (int)((int64_t)nkb * z / gz), kz1 = (int)((int64_t)nkb * (z + 1) / gz);
    const int nkh = (kz1 - kz0) / KH;  // steps per K half (the launcher makes them equal)
    const int kb0 = kz0 + kh * nkh, kb1 = kb0 + nkh;

    // Per-lane sources of this wave's transfers (q = wave + NW*i), as a base
    // at K-step 0 and the bytes one K-step adds.
    const uint8_t *src[PER];
    int kstep[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int q = wave + NW * i;
        const int pos = (q < FNQ ? q : 0) * 1024 + lane * 16;
        if (pos < FA) {
            const int r = pos / WROW, off = pos - r * WROW;
            const int64_t grow = row0 + r < nrows ? row0 + r : nrows - 1;  // rows past the end: duplicates
            src[i] = w + grow * row_stride + off;
            kstep[i] = 0;  // the weights' step offset is FF::aoff
        } else if (pos < FA + FB) {
            const int p = pos - FA, n = p >> 8, c = ((p >> 4) & 15) ^ (n & 15);
            const int col = n < ncols ? n : ncols - 1;  // columns past the end: duplicates
            src[i] = reinterpret_cast<const uint8_t *>(yqs + (int64_t)col * Kp) + 16 * c;
            kstep[i] = QK_K;
        } else {
            // headers; the rest of the last transfer re-reads the first column's
            const int p = pos - FA - FB;
            const int n = p < FD ? p >> 5 : 0, h = (p >> 4) & 1;
            const int col = n < ncols ? n : ncols - 1;
            src[i] = reinterpret_cast<const uint8_t *>(yds + (int64_t)col * (Kp / QK8)) + 16 * h;
            kstep[i] = 8 * 4;
        }
    }
    auto dma = [&](int kb, uint8_t *st) {
        const int64_t ao = FF::aoff(kb);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int q = wave + NW * i;  // uniform
            if (q < FNQ) dma16(src[i] + (q < NQA ? ao : (int64_t)kb * kstep[i]), st + q * 1024);
        }
    };

    v4f acc[NCT];
#pragma unroll
    for (int j = 0; j < NCT; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // K-slot carriers: slot 0 and 2 of the scale MFMA live in lanes 0-15,
    // slots 0-7 of the min MFMA in lanes 0-31; the other lanes' A values are
    // zero, so their (finite) B values add nothing.
    const uint32_t m_sc = kq == 0 ? 0xFFFFFFFFu : 0u;
    const uint32_t m_mn = kq < 2 ? 0xFFFFFFFFu : 0u;

    // per column tile j: the lane's column 16j + li, its codes and its
    // (d8 | s8 << 16) headers of the step's 8 blocks
    auto col_headers = [&](const uint8_t *st, int j, const uint8_t *&bcol, uint4 &dh0, uint4 &dh1) {
        bcol = st + FA + (16 * j + li) * QK_K;
        const uint32_t *dcol = reinterpret_cast<const uint32_t *>(st + FA + FB) + (16 * j + li) * 8;
        dh0 = *reinterpret_cast<const uint4 *>(dcol);
        dh1 = *reinterpret_cast<const uint4 *>(dcol + 4);
    };
    // the scale MFMA's B operand for block g: the headers of blocks 2h, 2h+1
    // (h = g/2) as stored, d8 of block g in K slot 0 (g even) or 2 (g odd)
    auto scale_b = [&](int g, const uint4 &dh0, const uint4 &dh1) {
        const uint4 &dh = g < 4 ? dh0 : dh1;
        return __builtin_bit_cast(v4h, (g & 2) ? make_uint2(dh.z, dh.w) : make_uint2(dh.x, dh.y));
    };
    // ... and its A operand: the row's f16 scale bits in the slot of block g
    auto scale_a = [&](int g, uint32_t f16bits) {
        return __builtin_bit_cast(v4h, (g & 1) ? make_uint2(0u, f16bits) : make_uint2(f16bits, 0u));
    };

    auto compute_q8_0 = [&](const uint8_t *st) {
        const uint8_t *arow = st + (wave * 16 + li) * WROW;
        const uint8_t *bcol[NCT];
        uint4 dh0[NCT], dh1[NCT];
#pragma unroll
        for (int j = 0; j < NCT; ++j) col_headers(st, j, bcol[j], dh0[j], dh1[j]);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            // Q8_0: the lane's 8 codes of block g; Q4_0: byte j of the 16 holds
            // element j (low nibble) and j + 16 (high), taken as q - 8
            const uint8_t *blk = arow + g * (TYPE == TYPE_Q4_0 ? Q40_BYTES : Q80_BYTES);
            uint2 a;
            if constexpr (TYPE == TYPE_Q4_0) {
                const uint2 q = lds8_a2(blk + 2 + 8 * (kq & 1));
                const int sh = 4 * (kq >> 1);
                a = make_uint2(q4_0_signed((q.x >> sh) & 0x0F0F0F0Fu), q4_0_signed((q.y >> sh) & 0x0F0F0F0Fu));
            } else {
                a = lds8_a2(blk + 2 + 8 * kq);
            }
            const uint32_t dw = (uint32_t)*reinterpret_cast<const uint16_t *>(blk) & m_sc;
            const v4h sa = scale_a(g, dw);
            const int c = 2 * g + (kq >> 1);
#pragma unroll
            for (int j = 0; j < NCT; ++j) {
                const uint2 b = *reinterpret_cast<const uint2 *>(bcol[j] + 16 * (c ^ li) + 8 * (kq & 1));
                const v4i zi = {0, 0, 0, 0};
                const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a), as_long(b), zi, 0, 0, 0);
                const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
                const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, scale_b(g, dh0[j], dh1[j]), zf, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[j][v] = fmaf((float)S[v], SC[v], acc[j][v]);
            }
        }
    };

    auto compute_q6_k = [&](const uint8_t *st, int kb) {
        const int delta = (int)(((int64_t)kb * Q6K_BYTES) & 15);  // the block's start in the window
        const uint8_t *blk = st + (wave * 16 + li) * WROW + delta;
        const uint8_t *bcol[NCT];
        uint4 dh0[NCT], dh1[NCT];
#pragma unroll
        for (int j = 0; j < NCT; ++j) col_headers(st, j, bcol[j], dh0[j], dh1[j]);
        v4f accb[NCT];
#pragma unroll
        for (int j = 0; j < NCT; ++j) accb[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        // two 32-weight chunks per pass keep the registers below the spill line
#pragma unroll 2
        for (int g = 0; g < 8; ++g) {
            const int n = g >> 2, m = g & 3;
            const uint2 ql = lds8_a2(blk + 64 * n + 32 * (m & 1) + 8 * kq);
            const uint2 qh = lds8_a2(blk + 128 + 32 * n + 8 * kq);
            const int sl = 4 * (m >> 1), shh = 2 * m;
            const uint32_t v0 = q6_signed(((ql.x >> sl) & 0x0F0F0F0Fu) | (((qh.x >> shh) & 0x03030303u) << 4));
            const uint32_t v1 = q6_signed(((ql.y >> sl) & 0x0F0F0F0Fu) | (((qh.y >> shh) & 0x03030303u) << 4));
            // sub-block 2g is the lanes' K-slices 0, 1 (kq < 2), sub-block 2g+1 slices 2, 3
            const uint2 a_lo = kq < 2 ? make_uint2(v0, v1) : make_uint2(0u, 0u);
            const uint2 a_hi = kq < 2 ? make_uint2(0u, 0u) : make_uint2(v0, v1);
            // the row's int8 scales of sub-blocks 2g and 2g+1
            const uint32_t w2 = *reinterpret_cast<const uint16_t *>(blk + 192 + 2 * g);
            const uint32_t sc0 = f16_bits((float)(int8_t)w2) & m_sc;
            const uint32_t sc1 = f16_bits((float)(int8_t)(w2 >> 8)) & m_sc;
            const v4h sa0 = scale_a(g, sc0), sa1 = scale_a(g, sc1);
            const int c = 2 * g + (kq >> 1);
#pragma unroll
            for (int j = 0; j < NCT; ++j) {
                const uint2 b = *reinterpret_cast<const uint2 *>(bcol[j] + 16 * (c ^ li) + 8 * (kq & 1));
                const v4i zi = {0, 0, 0, 0};
                const v4i S0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a_lo), as_long(b), zi, 0, 0, 0);
                const v4i S1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a_hi), as_long(b), zi, 0, 0, 0);
                const v4h sb = scale_b(g, dh0[j], dh1[j]);
                const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
                const v4f SC0 = __builtin_amdgcn_mfma_f32_16x16x16f16(sa0, sb, zf, 0, 0, 0);
                const v4f SC1 = __builtin_amdgcn_mfma_f32_16x16x16f16(sa1, sb, zf, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) accb[j][v] = fmaf((float)S1[v], SC1[v], fmaf((float)S0[v], SC0[v], accb[j][v]));
            }
        }
        // d of the output rows (4*kq + v of this wave's 16)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint8_t *ob = st + (wave * 16 + 4 * kq + v) * WROW + delta;
            const float d = h2f((uint32_t)*reinterpret_cast<const uint16_t *>(ob + 208));
#pragma unroll
            for (int j = 0; j < NCT; ++j) acc[j][v] = fmaf(d, accb[j][v], acc[j][v]);
        }
    };

    // Q4_K, and Q5_K (block {d, dmin, scales[12], qh[32], qs[128]}: the same
    // header, the fifth bit of element l of sub-block g is bit g of qh[l])
    // IQ4_XS (block {d, scales_h, scales_l[4], qs[128]}, 136 bytes): byte j of
    // sub-block g's 16 holds elements j (low nibble) and j + 16 (high), which
    // index the 16 int8 levels; sub-block g's scale is scales_l nibble g |
    // scales_h bits 2g..2g+1 << 4, minus 32 (exact in f16, the scale MFMA's
    // A); d once per step.  The window is 8-byte aligned around the block.
    auto compute_iq4_xs = [&](const uint8_t *st, int kb) {
        const int delta = (int)(((int64_t)kb * IQ4XS_BYTES) & 15);  // 0 or 8
        const uint8_t *blk = st + (wave * 16 + li) * WROW + delta;
        const uint2 hdr = *reinterpret_cast<const uint2 *>(blk);  // d | scales_h << 16, scales_l[4]
        const uint8_t *bcol[NCT];
        uint4 dh0[NCT], dh1[NCT];
#pragma unroll
        for (int j = 0; j < NCT; ++j) col_headers(st, j, bcol[j], dh0[j], dh1[j]);
        v4f accb[NCT];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint2 q = *reinterpret_cast<const uint2 *>(blk + 8 + 16 * g + 8 * (kq & 1));
            const int sh = 4 * (kq >> 1);
            const uint2 a = make_uint2(iq4nl_levels((q.x >> sh) & 0x0F0F0F0Fu), iq4nl_levels((q.y >> sh) & 0x0F0F0F0Fu));
            const int ls = (int)(((hdr.y >> (4 * g)) & 0xFu) | (((hdr.x >> (16 + 2 * g)) & 3u) << 4)) - 32;
            const v4h sa = scale_a(g, f16_bits((float)ls) & m_sc);
            const int c = 2 * g + (kq >> 1);
#pragma unroll
            for (int j = 0; j < NCT; ++j) {
                const uint2 b = *reinterpret_cast<const uint2 *>(bcol[j] + 16 * (c ^ li) + 8 * (kq & 1));
                const v4i zi = {0, 0, 0, 0};
                const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a), as_long(b), zi, 0, 0, 0);
                const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
                const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, scale_b(g, dh0[j], dh1[j]), zf, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    accb[j][v] = g == 0 ? (float)S[v] * SC[v] : fmaf((float)S[v], SC[v], accb[j][v]);
            }
        }
        // d of the output rows (4*kq + v of this wave's 16)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint8_t *ob = st + (wave * 16 + 4 * kq + v) * WROW + delta;
            const float d = h2f((uint32_t)*reinterpret_cast<const uint16_t *>(ob));
#pragma unroll
            for (int j = 0; j < NCT; ++j) acc[j][v] = fmaf(d, accb[j][v], acc[j][v]);
        }
    };

    auto compute = [&](const uint8_t *st) {
        constexpr bool Q5 = TYPE == TYPE_Q5_K;
        constexpr int QS = Q5 ? 48 : 16;  // the nibbles' offset in the block
        const uint8_t *arow = st + (wave * 16 + li) * WROW;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(arow);
        uint2 qh = make_uint2(0u, 0u);  // fifth bits of the lane's 8 elements of every sub-block
        if constexpr (Q5) qh = *reinterpret_cast<const uint2 *>(arow + 16 + 8 * kq);
        // getScaleMinK4 for all 8 sub-blocks, four per dword (bytes)
        const uint32_t sc_lo = hdr.y & 0x3F3F3F3Fu & m_sc;
        const uint32_t sc_hi = ((hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u)) & m_sc;
        const uint32_t mn_lo = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mn_hi = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        // per column tile j: the lane's column 16j + li, its codes and its
        // (d8 | s8 << 16) of the step's 8 blocks (and of blocks 4*(kq&1) .. +3
        // for the min MFMA)
        const uint8_t *bcol[NCT];
        uint4 dh0[NCT], dh1[NCT], dm[NCT];
#pragma unroll
        for (int j = 0; j < NCT; ++j) {
            bcol[j] = st + FA + (16 * j + li) * QK_K;
            const uint32_t *dcol = reinterpret_cast<const uint32_t *>(st + FA + FB) + (16 * j + li) * 8;
            dh0[j] = *reinterpret_cast<const uint4 *>(dcol);
            dh1[j] = *reinterpret_cast<const uint4 *>(dcol + 4);
            dm[j] = *reinterpret_cast<const uint4 *>(dcol + 4 * (kq & 1));
        }
        v4f accb[NCT];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint2 q = *reinterpret_cast<const uint2 *>(arow + QS + 32 * (g >> 1) + 8 * kq);
            const int sh = 4 * (g & 1);
            uint2 a = make_uint2((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
            if constexpr (Q5) {
                a.x |= ((qh.x >> g) & 0x01010101u) << 4;
                a.y |= ((qh.y >> g) & 0x01010101u) << 4;
            }
            // d8 of block g sits in K slot 0 (g even) or 2 (g odd) of the
            // headers of blocks 2h, 2h+1 (h = g/2) as stored; A puts sc there
            const uint32_t scf = byte_f16(g < 4 ? sc_lo : sc_hi, g & 3);
            const v4h sa = __builtin_bit_cast(v4h, (g & 1) ? make_uint2(0u, scf) : make_uint2(scf, 0u));
            const int c = 2 * g + (kq >> 1);
#pragma unroll
            for (int j = 0; j < NCT; ++j) {
                const uint2 b = *reinterpret_cast<const uint2 *>(bcol[j] + 16 * (c ^ li) + 8 * (kq & 1));
                const v4i zi = {0, 0, 0, 0};
                const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a), as_long(b), zi, 0, 0, 0);
                const uint4 &dh = g < 4 ? dh0[j] : dh1[j];
                const v4h sb = __builtin_bit_cast(v4h, (g & 2) ? make_uint2(dh.z, dh.w) : make_uint2(dh.x, dh.y));
                const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
                const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, sb, zf, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    accb[j][v] = g == 0 ? (float)S[v] * SC[v] : fmaf((float)S[v], SC[v], accb[j][v]);
            }
        }
        // min term: K slot 4*kq + t holds sub-block 4*kq + t for kq < 2
        const uint32_t mb = ((kq & 1) ? mn_hi : mn_lo) & m_mn;
        const v4h am = __builtin_bit_cast(
            v4h, make_uint2(byte_f16(mb, 0) | (byte_f16(mb, 1) << 16), byte_f16(mb, 2) | (byte_f16(mb, 3) << 16)));
        float dr[4], dn[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t dd = *reinterpret_cast<const uint32_t *>(st + (wave * 16 + 4 * kq + v) * WROW);
            dr[v] = h2f(dd);
            dn[v] = -h2f(dd >> 16);
        }
#pragma unroll
        for (int j = 0; j < NCT; ++j) {
            const v4h bm = __builtin_bit_cast(v4h, make_uint2(__builtin_amdgcn_perm(dm[j].y, dm[j].x, 0x07060302u),
                                                              __builtin_amdgcn_perm(dm[j].w, dm[j].z, 0x07060302u)));
            const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f P = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[j][v] = fmaf(dr[v], accb[j][v], fmaf(dn[v], P[v], acc[j][v]));
        }
    };

    // Up to 8 columns (PACK): one v_mfma_i32_16x16x64_i8 takes sub-blocks 2c
    // and 2c + 1 of the step.  Lane group kq >> 1 supplies the sub-block (low
    // nibbles of the 32 bytes qs[32c..], then high), kq & 1 its elements
    // 16 (kq & 1) .. +16.  Output column li holds activation column li & 7
    // against sub-block 2c + (li >> 3): B is that column's Q8_1 codes in the
    // lane groups of its sub-block and zero in the other two, so every output
    // is a live (column, sub-block) dot, and the scale MFMA puts sc_{2c} * d8
    // in K slot 0 for columns 0-7 and sc_{2c+1} * d8 in slot 1 for columns
    // 8-15.  The min term goes to columns 0-7 only, and the two halves of an
    // output column are added at the end.  Against one 16x16x32 MFMA per
    // sub-block with columns 8-15 idle, it halves the MFMAs and the
    // per-output convert + FMA of a step.
    const int phi = li >> 3, pj = li & 7;  // output column half, activation column
    const bool plive = (kq >> 1) == phi;   // this lane group's codes belong to its column's sub-block
    auto compute_pack = [&](const uint8_t *st) {
        constexpr bool Q5 = TYPE == TYPE_Q5_K;
        constexpr int QS = Q5 ? 48 : 16;  // the nibbles' offset in the block
        const uint8_t *arow = st + (wave * 16 + li) * WROW;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(arow);
        uint4 qh5 = make_uint4(0u, 0u, 0u, 0u);  // fifth bits of the lane's 16 elements of every sub-block
        if constexpr (Q5) qh5 = *reinterpret_cast<const uint4 *>(arow + 16 + 16 * (kq & 1));
        // getScaleMinK4 for all 8 sub-blocks, four per dword (bytes)
        const uint32_t sc_lo = hdr.y & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        const uint32_t mn_lo = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mn_hi = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        const uint8_t *bcol = st + FA + pj * QK_K;
        const uint32_t *dcol = reinterpret_cast<const uint32_t *>(st + FA + FB) + pj * 8;
        const uint4 dh0 = *reinterpret_cast<const uint4 *>(dcol), dh1 = *reinterpret_cast<const uint4 *>(dcol + 4);
        const uint4 dm = *reinterpret_cast<const uint4 *>(dcol + 4 * (kq & 1));
        v4f accb;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 q = *reinterpret_cast<const uint4 *>(arow + QS + 32 * c + 16 * (kq & 1));
            const int sh = 4 * (kq >> 1);
            const uint32_t m4 = 0x0F0F0F0Fu;
            uint4 a4 = make_uint4((q.x >> sh) & m4, (q.y >> sh) & m4, (q.z >> sh) & m4, (q.w >> sh) & m4);
            if constexpr (Q5) {
                const int bit = 2 * c + (kq >> 1);
                a4.x |= ((qh5.x >> bit) & 0x01010101u) << 4;
                a4.y |= ((qh5.y >> bit) & 0x01010101u) << 4;
                a4.z |= ((qh5.z >> bit) & 0x01010101u) << 4;
                a4.w |= ((qh5.w >> bit) & 0x01010101u) << 4;
            }
            const v4i a = __builtin_bit_cast(v4i, a4);
            // column pj's codes of block 2c + phi, elements 16 (kq & 1) .. +16: chunk 4c + 2 phi + (kq & 1)
            const uint4 *bp = plive ? reinterpret_cast<const uint4 *>(bcol + 16 * ((4 * c + 2 * phi + (kq & 1)) ^ pj))
                                    : &zero16;
            const v4i b = __builtin_bit_cast(v4i, *bp);
            const v4i zi = {0, 0, 0, 0};
            const v4i S = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, zi, 0, 0, 0);
            // A: (sc_{2c}, sc_{2c+1}) in K slots 0, 1 of lane group 0; B: d8 of block 2c + phi in slot phi
            const uint32_t scb = c < 2 ? sc_lo : sc_hi;
            const int sb = 16 * (c & 1);
            const uint32_t sa2 = (byte_f16(scb >> sb, 0) | (byte_f16(scb >> sb, 1) << 16)) & m_sc;
            const uint4 &dh = c < 2 ? dh0 : dh1;
            const uint32_t d8 = ((c & 1) ? (phi ? dh.w : dh.z) : (phi ? dh.y : dh.x)) & 0xFFFFu;
            const v4h sa = __builtin_bit_cast(v4h, make_uint2(sa2, 0u));
            const v4h sbv = __builtin_bit_cast(v4h, make_uint2(d8 << (16 * phi), 0u));
            const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, sbv, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) accb[v] = c == 0 ? (float)S[v] * SC[v] : fmaf((float)S[v], SC[v], accb[v]);
        }
        // min term, columns 0-7 only: K slot 4*kq + t holds sub-block 4*kq + t for kq < 2
        const uint32_t mb = ((kq & 1) ? mn_hi : mn_lo) & m_mn;
        const v4h am = __builtin_bit_cast(
            v4h, make_uint2(byte_f16(mb, 0) | (byte_f16(mb, 1) << 16), byte_f16(mb, 2) | (byte_f16(mb, 3) << 16)));
        const uint32_t m_lo = phi ? 0u : 0xFFFFFFFFu;
        const v4h bm = __builtin_bit_cast(v4h, make_uint2(__builtin_amdgcn_perm(dm.y, dm.x, 0x07060302u) & m_lo,
                                                          __builtin_amdgcn_perm(dm.w, dm.z, 0x07060302u) & m_lo));
        const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
        const v4f P = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, zf, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t dd = *reinterpret_cast<const uint32_t *>(st + (wave * 16 + 4 * kq + v) * WROW);
            acc[0][v] = fmaf(h2f(dd), accb[v], fmaf(-h2f(dd >> 16), P[v], acc[0][v]));
        }
    };

    // Q6_K up to 8 columns (PACK): one v_mfma_i32_16x16x32_i8 per 32-weight
    // window g takes both of its 16-weight sub-blocks.  Lane groups kq < 2 hold
    // sub-block 2g and kq >= 2 sub-block 2g + 1 (as in compute_q6_k); output
    // column li holds activation column li & 7 against sub-block 2g + (li >> 3):
    // B is that column's codes in the lane groups of its sub-block and zero in
    // the other two.  The scale MFMA puts sc_{2g} * d8 in K slot 0 for columns
    // 0-7 and sc_{2g+1} * d8 in slot 1 for columns 8-15; d once per step; the
    // two halves of an output column are added at the end.  Against two masked
    // MFMAs per window it halves the MFMAs and the per-output convert + FMA.
    auto compute_q6_k_pack = [&](const uint8_t *st, int kb) {
        const int delta = (int)(((int64_t)kb * Q6K_BYTES) & 15);  // the block's start in the window
        const uint8_t *blk = st + (wave * 16 + li) * WROW + delta;
        const uint8_t *bcol = st + FA + pj * QK_K;
        const uint32_t *dcol = reinterpret_cast<const uint32_t *>(st + FA + FB) + pj * 8;
        const uint4 dh0 = *reinterpret_cast<const uint4 *>(dcol), dh1 = *reinterpret_cast<const uint4 *>(dcol + 4);
        v4f accb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int n = g >> 2, m = g & 3;
            const uint2 ql = lds8_a2(blk + 64 * n + 32 * (m & 1) + 8 * kq);
            const uint2 qh = lds8_a2(blk + 128 + 32 * n + 8 * kq);
            const int sl = 4 * (m >> 1), shh = 2 * m;
            const uint2 a = make_uint2(q6_signed(((ql.x >> sl) & 0x0F0F0F0Fu) | (((qh.x >> shh) & 0x03030303u) << 4)),
                                       q6_signed(((ql.y >> sl) & 0x0F0F0F0Fu) | (((qh.y >> shh) & 0x03030303u) << 4)));
            // column pj's codes of sub-block 2g + phi, elements 8 (kq & 1) .. +8: chunk 2g + phi
            const uint2 *bp = plive ? reinterpret_cast<const uint2 *>(bcol + 16 * ((2 * g + phi) ^ pj) + 8 * (kq & 1))
                                    : reinterpret_cast<const uint2 *>(&zero16);
            const uint2 b = *bp;
            const v4i zi = {0, 0, 0, 0};
            const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a), as_long(b), zi, 0, 0, 0);
            // A: the row's int8 scales of sub-blocks 2g, 2g+1 in K slots 0, 1 of
            // lane group 0; B: d8 of block g of column pj in slot phi
            const uint32_t w2 = *reinterpret_cast<const uint16_t *>(blk + 192 + 2 * g);
            const uint32_t sa2 = (f16_bits((float)(int8_t)w2) | (f16_bits((float)(int8_t)(w2 >> 8)) << 16)) & m_sc;
            const uint4 &dh = g < 4 ? dh0 : dh1;
            const uint32_t hw = (g & 2) ? ((g & 1) ? dh.w : dh.z) : ((g & 1) ? dh.y : dh.x);
            const v4h sa = __builtin_bit_cast(v4h, make_uint2(sa2, 0u));
            const v4h sbv = __builtin_bit_cast(v4h, make_uint2((hw & 0xFFFFu) << (16 * phi), 0u));
            const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, sbv, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) accb[v] = fmaf((float)S[v], SC[v], accb[v]);
        }
        // d of the output rows (4*kq + v of this wave's 16)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint8_t *ob = st + (wave * 16 + 4 * kq + v) * WROW + delta;
            const float d = h2f((uint32_t)*reinterpret_cast<const uint16_t *>(ob + 208));
            acc[0][v] = fmaf(d, accb[v], acc[0][v]);
        }
    };

    // NST-stage ring: step kb0 + i lives in stage i % NST; while a step is
    // contracted, the next NST - 2 are in flight and one more is issued
    const bool big = wave < FNQ % NW || FNQ % NW == 0;
#pragma unroll
    for (int i = 0; i < NST - 1; ++i)
        if (kb0 + i < kb1) dma(kb0 + i, st[i]);
    for (int kb = kb0; kb < kb1;) {
#pragma unroll
        for (int i = 0; i < NST; ++i) {
            const int left = kb1 - 1 - kb;  // steps after kb already issued: min(left, NST - 2)
            wait_step<NST - 2, G::transfers_of(0), G::transfers_of(NW - 1)>(big, left < NST - 2 ? left : NST - 2);
            lds_barrier();
            if (kb + NST - 1 < kb1) dma(kb + NST - 1, st[(i + NST - 1) % NST]);
            if constexpr (PACK && TYPE == TYPE_Q6_K) compute_q6_k_pack(st[i], kb);
            else if constexpr (PACK) compute_pack(st[i]);
            else if constexpr (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) compute(st[i]);
            else if constexpr (TYPE == TYPE_Q8_0 || TYPE == TYPE_Q4_0) compute_q8_0(st[i]);
            else if constexpr (TYPE == TYPE_IQ4_XS) compute_iq4_xs(st[i], kb);
            else compute_q6_k(st[i], kb);
            if (++kb >= kb1) break;
        }
    }
    if constexpr (KH > 1) {
        // every wave's ring reads (and transfers: the last wait was vmcnt(0))
        // are done; K half 1 hands its sums to half 0 through the first stage
        lds_barrier();
        v4f *part = reinterpret_cast<v4f *>(&rings[0][0][0]);
        if (kh == 1) {
#pragma unroll
            for (int j = 0; j < NCT; ++j) part[(j * NW + wave) * 64 + lane] = acc[j];
        }
        lds_barrier();
        if (kh == 1) return;
#pragma unroll
        for (int j = 0; j < NCT; ++j) acc[j] += part[(j * NW + wave) * 64 + lane];
    }

    if constexpr (PACK) {
        // the odd sub-blocks' half of each output column (lanes li + 8) onto the even half
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[0][v] += __shfl_xor(acc[0][v], 8, 64);
        if (li >= 8 || li >= ncols) return;
        float *o = partial ? partial + ((int64_t)z * ncols + li) * nrows : dst + (int64_t)li * dst_col_stride;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t r = row0 + wave * 16 + 4 * kq + v;
            if (r < nrows) o[r] = acc[0][v];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < NCT; ++j) {
        const int c = 16 * j + li;
        if (c >= ncols) continue;
        float *o = partial ? partial + ((int64_t)z * ncols + c) * nrows : dst + (int64_t)c * dst_col_stride;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t r = row0 + wave * 16 + 4 * kq + v;
            if (r < nrows) o[r] = acc[j][v];
        }
    }
}

}  // namespace

// Shape of the few-column kernel: 3 ring stages, 4 waves per workgroup.  A
// sweep of 2-6 stages, 4 or 8 waves and 256-2560 workgroups (Q4_K, 16
// columns, 1024-14336 rows, K 4096 / 14336) found this best or within noise
// everywhere: pure transfer streaming of the same pattern takes ~8 us for
// 33 MB, and the rest is contraction that a deeper ring or more workgroups
// per CU did not hide.
constexpr int FEW_NST = 3, FEW_NW = 4;
constexpr int FEW_PACK_COLS = 8;  // most columns of the packed (two sub-blocks per MFMA) path

// K-split for the few-column kernel.  From 192 row tiles (3/4 of the CUs)
// the kernel runs unsplit: the partials' reduction is a second launch of
// ~3-4 us, more than a fuller grid saves (14336 rows at 16 columns: 14.7 us
// unsplit, 13.3 + 4.0 us in 2 shares).  Below that, about two workgroups per
// CU (4096 rows: 8 shares), at least 2 K-steps per share, equal shares.
int mmq_few_split_k(int64_t K, int64_t nrows) {
    const int64_t bm = 16 * FEW_NW;
    const int64_t wgs = (nrows + bm - 1) / bm;
    const int64_t nkb = K / QK_K;
    if (wgs >= 192) return 1;
    int64_t split = (512 + wgs - 1) / wgs;
    const int64_t cap = nkb / 2 < 16 ? nkb / 2 : 16;
    if (split > cap) split = cap;
    if (split < 1) split = 1;
    while (nkb % split) --split;
    return (int)split;
}

// Whether a workgroup runs two K halves of its K part (KH = 2): K parts of
// an even step count, at least 4, on grids of at most 256 workgroups (two
// rings take twice the LDS, so a workgroup fills a CU's LDS by itself: a
// larger grid would run a second round).  Against one ring of 4 waves (graph-timed,
// same box): Q4_K 14336x4096 at 8 columns 13.4-13.5 -> 11.9-12.0 us, at 16
// 13.9-14.1 -> 13.0-13.1, at 32 18.9-19.0 -> 18.3; Q5_K at 8 15.6-15.8 ->
// 13.7, Q4_0 18.0-18.1 -> 14.5, IQ4_XS 18.7-18.9 -> 15.5-15.6, Q8_0
// 17.2 -> 16.7.  Two waves with independent work share each SIMD, where one
// wave alone stalled on its own LDS and MFMA latencies.  Halving the K
// shares of the split grids (4096 rows) in exchange for K halves measured
// level (and slower on 1024 rows), so those keep one ring.  Split grids of
// more than 256 workgroups with K halves ran a second round: 6144x4096 /
// 8192x4096 / 10240x4096 / 8192x8192 / 2048x14336 at 8 columns 12.9 / 13.5 /
// 17.4 / 17.6 / 14.4 us against 10.3 / 10.7 / 12.4 / 14.0 / 11.7 with one ring.
bool few_k_halves(int64_t K, int64_t gx, int split) {
    const int64_t per = K / QK_K / split;
    return per % 2 == 0 && per >= 4 && gx * split <= 256;
}

// Whether the few-column kernel takes this weight layout: Q4_K and Q5_K;
// Q8_0, Q4_0, Q6_K and IQ4_XS with 16-byte-aligned rows (and, Q6_K,
// K % 2048 == 0, IQ4_XS K % 512 == 0, so that their aligned windows stay
// inside the row).
bool mmq_few_takes(int type, int64_t K, const void *w, int64_t row_stride) {
    if (type == TYPE_Q4_K || type == TYPE_Q5_K) return true;
    if (type != TYPE_Q8_0 && type != TYPE_Q4_0 && type != TYPE_Q6_K && type != TYPE_IQ4_XS) return false;
    if ((uintptr_t)w % 16 || row_stride % 16 || K % QK_K) return false;
    if (type == TYPE_IQ4_XS) return K % 512 == 0;
    return type != TYPE_Q6_K || K % 2048 == 0;
}

// Launch for mmq.hip's dispatch: the rows as mmq_few_takes says, the
// activation planes 16-byte aligned, 1 <= ncols <= 32 (Q6_K: 16), K % 256 ==
// 0, which the caller checks.  `partial` (split * nrows * ncols floats) takes the
// split-K partials when split > 1.
int mmq_few_launch(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                   const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int split, float *partial,
                   hipStream_t s) {
    const int64_t gx = (nrows + 16 * FEW_NW - 1) / (16 * FEW_NW);
    if (ncols < 1 || ncols > FBN || gx > 0x7FFFFFFF || split < 1 || split > 16 || K / QK_K > 0x7FFFFFFF ||
        !mmq_few_takes(type, K, w, row_stride))
        return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)gx, 1, (unsigned)split);
    // two K halves per workgroup where the K parts split evenly
    const bool khalves = few_k_halves(K, gx, split);
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    float *pp = split > 1 ? partial : nullptr;
#define FEW_LAUNCH_P(TYPE, NCT, PK)                                                                                    \
    if (khalves)                                                                                                       \
        hipLaunchKernelGGL((mmq_few_kernel<TYPE, FEW_NST, FEW_NW, NCT, PK, 2>), grid, dim3(128 * FEW_NW), 0, s, wb, K, \
                           nrows, row_stride, yqs, ds, (int)ncols, dst, dst_col_stride, pp);                           \
    else                                                                                                               \
        hipLaunchKernelGGL((mmq_few_kernel<TYPE, FEW_NST, FEW_NW, NCT, PK, 1>), grid, dim3(64 * FEW_NW), 0, s, wb, K,  \
                           nrows, row_stride, yqs, ds, (int)ncols, dst, dst_col_stride, pp)
#define FEW_LAUNCH(TYPE, NCT) FEW_LAUNCH_P(TYPE, NCT, false)
    // up to 8 columns of the K-quant nibble types: two sub-blocks per MFMA
    const bool pack = ncols <= FEW_PACK_COLS;
    switch (type) {
    case TYPE_Q8_0:
        if (ncols > 16) FEW_LAUNCH(TYPE_Q8_0, 2);
        else FEW_LAUNCH(TYPE_Q8_0, 1);
        break;
    case TYPE_Q6_K:  // one column tile: two measured slower than the 128-row MMQ tile
        if (ncols > 16) return (int)hipErrorInvalidValue;
        if (pack) FEW_LAUNCH_P(TYPE_Q6_K, 1, true);
        else FEW_LAUNCH(TYPE_Q6_K, 1);
        break;
    case TYPE_Q5_K:
        if (ncols > 16) FEW_LAUNCH(TYPE_Q5_K, 2);
        else if (pack) FEW_LAUNCH_P(TYPE_Q5_K, 1, true);
        else FEW_LAUNCH(TYPE_Q5_K, 1);
        break;
    case TYPE_Q4_0:
        if (ncols > 16) FEW_LAUNCH(TYPE_Q4_0, 2);
        else FEW_LAUNCH(TYPE_Q4_0, 1);
        break;
    case TYPE_IQ4_XS:
        if (ncols > 16) FEW_LAUNCH(TYPE_IQ4_XS, 2);
        else FEW_LAUNCH(TYPE_IQ4_XS, 1);
        break;
    default:
        if (ncols > 16) FEW_LAUNCH(TYPE_Q4_K, 2);
        else if (pack) FEW_LAUNCH_P(TYPE_Q4_K, 1, true);
        else FEW_LAUNCH(TYPE_Q4_K, 1);
        break;
    }
#undef FEW_LAUNCH
#undef FEW_LAUNCH_P
    return (int)hipGetLastError();
}
