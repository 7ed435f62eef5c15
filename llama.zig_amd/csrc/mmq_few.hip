// mmq_few.hip -- Q4_K GEMM for few activation columns (up to 32), on 16x16 int8 MFMA.
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

// Workgroup geometry for NW waves of 16 rows each and NCT tiles of 16
// columns: the step's LDS stage and its 1 KiB transfers (transfer q goes to
// wave q % NW).
template <int NW, int NCT>
struct FewGeo {
    static constexpr int BM = 16 * NW;                 // rows per workgroup
    static constexpr int NT = 64 * NW;                 // threads
    static constexpr int A = BM * Q4K_BYTES;           // weights per step
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

// workgroups per CU that the LDS (160 KiB) holds with an NST-stage ring
template <int NW, int NCT>
constexpr int few_occupancy(int nst) { return 163840 / (nst * FewGeo<NW, NCT>::STAGE); }

template <int NST, int NW, int NCT>
__global__ __launch_bounds__((FewGeo<NW, NCT>::NT), (few_occupancy<NW, NCT>(NST))) void mmq_few_q4k_kernel(const uint8_t *__restrict__ w, int64_t K, int64_t nrows,
                                                            int64_t row_stride, const int8_t *__restrict__ yqs,
                                                            const uint32_t *__restrict__ yds, int ncols,
                                                            float *__restrict__ dst, int64_t dst_col_stride,
                                                            float *__restrict__ partial) {
    using G = FewGeo<NW, NCT>;
    constexpr int FA = G::A, FB = G::B, FD = G::D, FNQ = G::NQ, PER = G::PER;
    static_assert(NST >= 2 && few_occupancy<NW, NCT>(NST) >= 1, "ring depth");
    static_assert((NST - 2) * G::transfers_of(0) <= 63, "vmcnt field");
    __shared__ alignas(16) uint8_t st[NST][G::STAGE];

    const int64_t Kp = pad_k(K);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, kq = lane >> 4;
    const int64_t row0 = (int64_t)blockIdx.x * G::BM;
    const int nkb = (int)(K / QK_K);
    const int gz = (int)gridDim.z, z = (int)blockIdx.z;
    const int kb0 = (int)((int64_t)nkb * z / gz), kb1 = (int)((int64_t)nkb * (z + 1) / gz);

    // Per-lane sources of this wave's transfers (q = wave + NW*i), as a base
    // at K-step 0 and the bytes one K-step adds.
    const uint8_t *src[PER];
    int kstep[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int q = wave + NW * i;
        const int pos = (q < FNQ ? q : 0) * 1024 + lane * 16;
        if (pos < FA) {
            const int r = pos / Q4K_BYTES, off = pos - r * Q4K_BYTES;
            const int64_t grow = row0 + r < nrows ? row0 + r : nrows - 1;  // rows past the end: duplicates
            src[i] = w + grow * row_stride + off;
            kstep[i] = Q4K_BYTES;
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
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (wave + NW * i < FNQ) dma16(src[i] + (int64_t)kb * kstep[i], st + (wave + NW * i) * 1024);
    };

    v4f acc[NCT];
#pragma unroll
    for (int j = 0; j < NCT; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // K-slot carriers: slot 0 and 2 of the scale MFMA live in lanes 0-15,
    // slots 0-7 of the min MFMA in lanes 0-31; the other lanes' A values are
    // zero, so their (finite) B values add nothing.
    const uint32_t m_sc = kq == 0 ? 0xFFFFFFFFu : 0u;
    const uint32_t m_mn = kq < 2 ? 0xFFFFFFFFu : 0u;

    auto compute = [&](const uint8_t *st) {
        const uint8_t *arow = st + (wave * 16 + li) * Q4K_BYTES;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(arow);
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
            const uint2 q = *reinterpret_cast<const uint2 *>(arow + 16 + 32 * (g >> 1) + 8 * kq);
            const int sh = 4 * (g & 1);
            const uint2 a = make_uint2((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
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
            const uint32_t dd = *reinterpret_cast<const uint32_t *>(st + (wave * 16 + 4 * kq + v) * Q4K_BYTES);
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
            compute(st[i]);
            if (++kb >= kb1) break;
        }
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

// Launch for mmq.hip's dispatch: Q4_K rows 16-byte aligned (row_stride % 16 ==
// 0), the activation planes 16-byte aligned, 1 <= ncols <= 32, K % 256 == 0,
// which the caller checks.  `partial` (split * nrows * ncols floats) takes the
// split-K partials when split > 1.
int mmq_few_q4k_launch(const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                       const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int split, float *partial,
                       hipStream_t s) {
    const int64_t gx = (nrows + 16 * FEW_NW - 1) / (16 * FEW_NW);
    if (ncols < 1 || ncols > FBN || gx > 0x7FFFFFFF || split < 1 || split > 16 || K / QK_K > 0x7FFFFFFF)
        return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)gx, 1, (unsigned)split);
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    float *pp = split > 1 ? partial : nullptr;
#define FEW_LAUNCH(NST, NW, NCT)                                                                                       \
    hipLaunchKernelGGL((mmq_few_q4k_kernel<NST, NW, NCT>), grid, dim3(64 * NW), 0, s, wb, K, nrows, row_stride, yqs,   \
                       ds, (int)ncols, dst, dst_col_stride, pp)
    if (ncols > 16) FEW_LAUNCH(FEW_NST, FEW_NW, 2);
    else FEW_LAUNCH(FEW_NST, FEW_NW, 1);
#undef FEW_LAUNCH
    return (int)hipGetLastError();
}
