// mmq_few.hip -- Q4_K GEMM for few activation columns (9-16), on 16x16 int8 MFMA.
//
// The reference sends 2-24 src1 columns to a separate "few-row" MMQ kernel
// (src/ggml/cuda/mmq_few.zig:1-20, mulMatQFew :204-255, shouldUseMmqFew
// :847-860): at that width the weights are streamed once and the 128 x 32
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
// Mapping: a workgroup of 4 waves owns 64 rows (16 per wave, one MFMA tile)
// and all <= 16 columns, over its share of the K-steps (split K over grid z
// when the row tiles alone do not fill the chip).  Each K-step (one Q4_K
// super-block) moves from global memory straight into LDS with
// global_load_lds_dwordx4, 14 transfers of 1 KiB per step:
//   - A: the 64 rows' 144-byte blocks as stored (contiguous 144-byte runs);
//   - B: the columns' 256 Q8_1 codes, 16-byte chunk c of column n at position
//     c ^ n, so the operand reads of 16 columns spread over the banks;
//   - D: the columns' (d8 | s8 << 16) headers.
// Three LDS stages form a ring: while step k is contracted, steps k+1 and k+2
// are in flight, and a wave waits only for its own transfers of step k
// (vmcnt = its transfer count of one step) before the step's barrier.
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

constexpr int FBM = 64;                    // rows per workgroup
constexpr int FBN = 16;                    // columns
constexpr int FNT = 256;                   // threads per workgroup
constexpr int FA = FBM * Q4K_BYTES;        // 9216 B of weights per step
constexpr int FB = FBN * QK_K;             // 4096 B of codes per step
constexpr int FD = FBN * 8 * 4;            // 512 B of headers per step
constexpr int FNQ = (FA + FB + FD + 1023) / 1024;  // 14 transfers per step
constexpr int FSTAGE = FNQ * 1024;

// transfers per step issued by wave w (transfer q goes to wave q % 4)
__host__ __device__ constexpr int transfers_of(int w) { return FNQ / 4 + (w < FNQ % 4 ? 1 : 0); }
static_assert(transfers_of(0) <= 15 && transfers_of(3) >= 1, "vmcnt immediates below assume 1..15");

__device__ __forceinline__ uint32_t f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
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
    static_assert(N >= 0 && N <= 15, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
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

// this wave's step k is complete; `ahead`: step k+1 was issued after it
__device__ __forceinline__ void wait_step(int wave, bool ahead) {
    if (!ahead) {
        wait_vm<0>();
    } else if (wave < FNQ % 4) {
        wait_vm<transfers_of(0)>();
    } else {
        wait_vm<transfers_of(3)>();
    }
}

__global__ __launch_bounds__(FNT, 3) void mmq_few_q4k_kernel(const uint8_t *__restrict__ w, int64_t K, int64_t nrows,
                                                            int64_t row_stride, const int8_t *__restrict__ yqs,
                                                            const uint32_t *__restrict__ yds, int ncols,
                                                            float *__restrict__ dst, int64_t dst_col_stride,
                                                            float *__restrict__ partial) {
    __shared__ alignas(16) uint8_t st0[FSTAGE], st1[FSTAGE], st2[FSTAGE];

    const int64_t Kp = pad_k(K);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, kq = lane >> 4;
    const int64_t row0 = (int64_t)blockIdx.x * FBM;
    const int nkb = (int)(K / QK_K);
    const int gz = (int)gridDim.z, z = (int)blockIdx.z;
    const int kb0 = (int)((int64_t)nkb * z / gz), kb1 = (int)((int64_t)nkb * (z + 1) / gz);

    // Per-lane sources of this wave's transfers (q = wave + 4i), as a base at
    // K-step 0 and the bytes one K-step adds.
    const uint8_t *src[4];
    int kstep[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = wave + 4 * i;
        const int pos = (q < FNQ ? q : 0) * 1024 + lane * 16;
        if (pos < FA) {
            const int r = pos / Q4K_BYTES, off = pos - r * Q4K_BYTES;
            const int64_t grow = row0 + r < nrows ? row0 + r : nrows - 1;  // rows past the end: duplicates
            src[i] = w + grow * row_stride + off;
            kstep[i] = Q4K_BYTES;
        } else if (pos < FA + FB) {
            const int p = pos - FA, n = p >> 8, c = ((p >> 4) & 15) ^ n;
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
        for (int i = 0; i < 4; ++i)
            if (wave + 4 * i < FNQ) dma16(src[i] + (int64_t)kb * kstep[i], st + (wave + 4 * i) * 1024);
    };

    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // K-slot carriers: slot 0 and 2 of the scale MFMA live in lanes 0-15,
    // slots 0-7 of the min MFMA in lanes 0-31; the other lanes' A values are
    // zero, so their (finite) B values add nothing.
    const uint32_t m_sc = kq == 0 ? 0xFFFFFFFFu : 0u;
    const uint32_t m_mn = kq < 2 ? 0xFFFFFFFFu : 0u;

    auto compute = [&](const uint8_t *st) {
        const uint8_t *arow = st + (wave * 16 + li) * Q4K_BYTES;
        const uint8_t *bcol = st + FA + li * QK_K;
        const uint32_t *dcol = reinterpret_cast<const uint32_t *>(st + FA + FB) + li * 8;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(arow);
        // getScaleMinK4 for all 8 sub-blocks, four per dword (bytes)
        const uint32_t sc_lo = hdr.y & 0x3F3F3F3Fu & m_sc;
        const uint32_t sc_hi = ((hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u)) & m_sc;
        const uint32_t mn_lo = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mn_hi = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        // the columns' (d8 | s8 << 16) of the step's 8 blocks, and of blocks
        // 4*(kq&1) .. +3 for the min MFMA
        const uint4 dh0 = *reinterpret_cast<const uint4 *>(dcol);
        const uint4 dh1 = *reinterpret_cast<const uint4 *>(dcol + 4);
        const uint4 dm = *reinterpret_cast<const uint4 *>(dcol + 4 * (kq & 1));
        v4f accb;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint2 q = *reinterpret_cast<const uint2 *>(arow + 16 + 32 * (g >> 1) + 8 * kq);
            const int sh = 4 * (g & 1);
            const uint2 a = make_uint2((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
            const int c = 2 * g + (kq >> 1);
            const uint2 b = *reinterpret_cast<const uint2 *>(bcol + 16 * (c ^ li) + 8 * (kq & 1));
            const v4i zi = {0, 0, 0, 0};
            const v4i S = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a), as_long(b), zi, 0, 0, 0);
            // B = the headers of blocks 2h, 2h+1 (h = g/2) as stored: d8 of
            // block g sits in K slot 0 (g even) or 2 (g odd), where A puts sc
            const uint32_t scf = f16_bits((float)(((g < 4 ? sc_lo : sc_hi) >> (8 * (g & 3))) & 0xFFu));
            const uint4 &dh = g < 4 ? dh0 : dh1;
            const uint2 hb = (g & 2) ? make_uint2(dh.z, dh.w) : make_uint2(dh.x, dh.y);
            const v4h sa = __builtin_bit_cast(v4h, (g & 1) ? make_uint2(0u, scf) : make_uint2(scf, 0u));
            const v4h sb = __builtin_bit_cast(v4h, hb);
            const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f SC = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, sb, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) accb[v] = g == 0 ? (float)S[v] * SC[v] : fmaf((float)S[v], SC[v], accb[v]);
        }
        // min term: K slot 4*kq + t holds sub-block 4*kq + t for kq < 2
        const uint32_t mb = ((kq & 1) ? mn_hi : mn_lo) & m_mn;
        const v4h am = __builtin_bit_cast(
            v4h, make_uint2(f16_bits((float)(mb & 0xFFu)) | (f16_bits((float)((mb >> 8) & 0xFFu)) << 16),
                            f16_bits((float)((mb >> 16) & 0xFFu)) | (f16_bits((float)(mb >> 24)) << 16)));
        const v4h bm = __builtin_bit_cast(v4h, make_uint2(__builtin_amdgcn_perm(dm.y, dm.x, 0x07060302u),
                                                          __builtin_amdgcn_perm(dm.w, dm.z, 0x07060302u)));
        const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
        const v4f P = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, zf, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t dd = *reinterpret_cast<const uint32_t *>(st + (wave * 16 + 4 * kq + v) * Q4K_BYTES);
            acc[v] = fmaf(h2f(dd), accb[v], fmaf(-h2f(dd >> 16), P[v], acc[v]));
        }
    };

    // three-stage ring: step kb + s lives in stage s % 3
    if (kb0 < kb1) dma(kb0, st0);
    if (kb0 + 1 < kb1) dma(kb0 + 1, st1);
    for (int kb = kb0; kb < kb1;) {
        wait_step(wave, kb + 1 < kb1);
        lds_barrier();
        if (kb + 2 < kb1) dma(kb + 2, st2);
        compute(st0);
        if (++kb >= kb1) break;
        wait_step(wave, kb + 1 < kb1);
        lds_barrier();
        if (kb + 2 < kb1) dma(kb + 2, st0);
        compute(st1);
        if (++kb >= kb1) break;
        wait_step(wave, kb + 1 < kb1);
        lds_barrier();
        if (kb + 2 < kb1) dma(kb + 2, st1);
        compute(st2);
        ++kb;
    }

    if (li < ncols) {
        float *o = partial ? partial + ((int64_t)z * ncols + li) * nrows : dst + (int64_t)li * dst_col_stride;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t r = row0 + wave * 16 + 4 * kq + v;
            if (r < nrows) o[r] = acc[v];
        }
    }
}

}  // namespace

// K-split for the few-column kernel: about three workgroups per CU (the LDS
// ring holds three per CU), at least 2 K-steps per share, equal shares.
int mmq_few_split_k(int64_t K, int64_t nrows) {
    const int64_t wgs = (nrows + FBM - 1) / FBM;
    const int64_t nkb = K / QK_K;
    int64_t split = (768 + wgs - 1) / wgs;
    const int64_t cap = nkb / 2 < 16 ? nkb / 2 : 16;
    if (split > cap) split = cap;
    if (split < 1) split = 1;
    while (nkb % split) --split;
    return (int)split;
}

// Launch for mmq.hip's dispatch: Q4_K rows 16-byte aligned (row_stride % 16 ==
// 0), the activation planes 16-byte aligned, 1 <= ncols <= 16, K % 256 == 0,
// which the caller checks.  `partial` (split * nrows * ncols floats) takes the
// split-K partials when split > 1.
int mmq_few_q4k_launch(const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                       const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, int split, float *partial,
                       hipStream_t s) {
    const int64_t gx = (nrows + FBM - 1) / FBM;
    if (ncols < 1 || ncols > FBN || gx > 0x7FFFFFFF || split < 1 || split > 16 || K / QK_K > 0x7FFFFFFF)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(mmq_few_q4k_kernel, dim3((unsigned)gx, 1, (unsigned)split), dim3(FNT), 0, s,
                       (const uint8_t *)w, K, nrows, row_stride, yqs, (const uint32_t *)yds, (int)ncols, dst,
                       dst_col_stride, split > 1 ? partial : nullptr);
    return (int)hipGetLastError();
}
