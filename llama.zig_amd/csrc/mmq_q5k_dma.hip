// mmq_q5k_dma.hip -- the dense Q5_K MMQ with direct global->LDS loads.
//
// Arithmetic as in mmq.hip's Q5_K path (the Q4_K arithmetic on 5-bit
// values): the 32-deep sub-block dot of the values 0..31 on
// v_mfma_i32_32x32x32_i8 (exact), the per-(row, column, sub-block) scale
// sc_j * d8_j as an exact f16 outer product (v_mfma_f32_32x32x8_f16, one live
// K slot), one convert + FMA per output and sub-block, and per super-block
//   out += d * accb - dmin * sum_j m_j * s8_j
// with the min term on one more f16 MFMA (K = 8: the eight sub-blocks).
//
// Data path.  block_q5_K {d, dmin, scales[12], qh[32], qs[128]} is 176 bytes,
// a multiple of 16, so every super-block of a 16-byte aligned row goes from
// global memory straight into LDS with global_load_lds_dwordx4, rows back to
// back.  Lane half h of a wave takes elements 16h..16h+15 of each sub-block:
// sub-block j's nibbles from qs[32 (j / 2) + 16 h ..] (low for even j, high
// for odd), its fifth bits as bit j of qh[16 h ..], and decodes the scales and
// mins of sub-blocks 4h..4h+3 only.  The columns' Q8_1 codes (256 per column)
// and their eight block headers come the same way; chunk c of column n sits
// at slot c ^ (n & 15).  Two buffers: the next super-block's transfers run
// while the current one is contracted, one barrier per step.  d and dmin of
// the output rows are read from the block headers in LDS, so the kernel needs
// no table beside the two buffers (80 KB at 64 columns: two workgroups per CU).
#include "../../include/ggml_hip_qmm.h"
#include "mmq_dma.h"
#include "qmm_device.h"

using namespace qmm;
using namespace qmm_dma;

namespace {

constexpr int ABYTES = BM * Q5K_BYTES;  // 22528: 22 transfers of 1 KiB
constexpr int NA = ABYTES / 1024;

template <int BN, bool GROUPED>
__global__ __launch_bounds__(NTHREADS, 2) void mmq_q5k_dma_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t ncols, float *__restrict__ dst, int64_t dst_col_stride,
    float *__restrict__ partial, int gx, int gy, int gz, MmqGroups grp, MmqGlu glu) {
    constexpr int TJ = BN / 32;
    constexpr int NQB = BN / 4;   // 1 KiB transfers of the B codes per step (4 columns each)
    constexpr int NQD = BN / 32;  // 1 KiB transfers of the B headers per step (32 columns each)
    __shared__ alignas(16) uint8_t sA0[ABYTES], sA1[ABYTES];
    __shared__ alignas(16) uint8_t sB0[BN * 256], sB1[BN * 256];
    __shared__ alignas(16) uint32_t sD0[BN * 8], sD1[BN * 8];

    const int64_t Kp = pad_k(K);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int wr = wave * 32;

    int bx = (int)blockIdx.x, by = (int)blockIdx.y;
    int64_t col0, col_end = ncols;
    // gate/up/GLU fusion (glu.gate != nullptr): 64 output rows per tile, tile
    // row t from the gate (t % 4 < 2) or up weights of output row
    // mmq_glu_tile_row(t); no K split
    const bool fused = glu.gate != nullptr;  // uniform
    const uint8_t *wexp = w, *wgexp = glu.gate;
    if constexpr (GROUPED) {
        if ((int)blockIdx.y >= *grp.n_tiles) return;  // uniform per workgroup
        const int4 t = *reinterpret_cast<const int4 *>(grp.tiles + 4 * blockIdx.y);
        wexp = w + (int64_t)t.x * grp.expert_stride;
        if (fused) wgexp = glu.gate + (int64_t)t.x * grp.expert_stride;
        col0 = t.y;
        col_end = t.z;
    } else {
        if (gz == 1) mmq_tile_order(bx + gx * by, gx, gy, bx, by);
        col0 = (int64_t)by * BN;
    }
    // activation row of tile column c (clamped into the tile)
    auto src_col = [&](int64_t c) -> int64_t {
        const int64_t cc = c < col_end ? c : col0;
        return GROUPED ? (int64_t)grp.col_src[cc] : cc;
    };
    const int64_t row0 = (int64_t)bx * (fused ? BM / 2 : BM);  // first output row
    const int nkb = (int)(K / QK_K);
    const int kb0 = nkb * (int)blockIdx.z / gz, kb1 = nkb * ((int)blockIdx.z + 1) / gz;

    // per-lane transfer sources (fixed over the K loop)
    const uint8_t *a_src[(NA + 3) / 4];
#pragma unroll
    for (int i = 0; i < (NA + 3) / 4; ++i) {
        const int t = wave + 4 * i < NA ? wave + 4 * i : 0;
        const int pos = t * 1024 + lane * 16, r = pos / Q5K_BYTES;
        const int64_t orow = row0 + (fused ? mmq_glu_tile_row(r) : r);
        const int64_t rr = orow < nrows ? orow : nrows - 1;
        a_src[i] = (fused && (r & 2) == 0 ? wgexp : wexp) + rr * row_stride + (pos - r * Q5K_BYTES);
    }
    const int8_t *b_src[(NQB + 3) / 4];
#pragma unroll
    for (int i = 0; i < (NQB + 3) / 4; ++i) {
        const int t = wave + 4 * i < NQB ? wave + 4 * i : 0;
        const int n = 4 * t + (lane >> 4);
        b_src[i] = yqs + src_col(col0 + n) * Kp + 16 * ((lane & 15) ^ (n & 15));
    }
    // column headers (waves 2 .. 1 + NQD, which take 5 of the 22 A transfers
    // to waves 0-1's 6):
    // transfer t, lane l -> column 32 t + l / 2, blocks 4 (l & 1) .. +3
    const uint32_t *d_src;
    {
        const int n = 32 * (wave >= 2 && wave - 2 < NQD ? wave - 2 : 0) + (lane >> 1);
        d_src = yds + src_col(col0 + n) * (Kp / QK8) + 4 * (lane & 1);
    }

    auto dma = [&](int kb, uint8_t *sA, uint8_t *sB, uint32_t *sD) {
        const int64_t woff = (int64_t)kb * Q5K_BYTES;
#pragma unroll
        for (int i = 0; i < (NA + 3) / 4; ++i)
            if (wave + 4 * i < NA) dma16(a_src[i] + woff, sA + (wave + 4 * i) * 1024);
#pragma unroll
        for (int i = 0; i < (NQB + 3) / 4; ++i)
            if (wave + 4 * i < NQB) dma16(b_src[i] + (int64_t)kb * QK_K, sB + (wave + 4 * i) * 1024);
        if (wave >= 2 && wave - 2 < NQD) dma16(d_src + 8 * kb, reinterpret_cast<uint8_t *>(sD) + (wave - 2) * 1024);
    };

    v16f acc[TJ], accb[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;

    // Scale outer product per sub-block g on the f16 MFMA with one live K
    // slot.  A lane of half h decodes only the scales and mins of sub-blocks
    // 4h..4h+3; its A operand for sub-block g is sc of sub-block 4h + g % 4,
    // live when h == g / 4 and zero in the other half.  The A operand sits in
    // slot 0 (g even) or slot 2 (g odd); the B operand is the raw pair of
    // (d8 | s8 << 16) headers of groups 2(g/2), 2(g/2)+1, unmasked (a zero
    // block after each header table, as the Q4_K kernel reads for the dead
    // half, would take this kernel's LDS past 80 KiB and one workgroup per CU).
    const uint32_t live_lo = lh ? 0u : 0xFFFFFFFFu;  // groups 0-3 are live in lane half 0
    const uint32_t sel_s8 = 0x07060302u;  // s8 halves of two headers -> one dword

    auto compute = [&](const uint8_t *sA, const uint8_t *sB, const uint32_t *sD) {
        const uint8_t *arow = sA + (wr + li) * Q5K_BYTES;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(arow);
        // getScaleMinK4 for sub-blocks 4 lh .. 4 lh + 3, four at a time (bytes)
        const uint32_t hsel = 0u - (uint32_t)lh;  // all ones in lane half 1
        const uint32_t scb = (hsel & ((hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u))) |
                             (~hsel & hdr.y & 0x3F3F3F3Fu);
        const uint32_t mnb = (hsel & (((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u))) |
                             (~hsel & hdr.z & 0x3F3F3F3Fu);
        uint32_t sa[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) sa[t] = f16_bits((float)((scb >> (8 * t)) & 0xFFu));
        // the mins as packed f16 pairs: 0x64nn is 1024 + nn in f16 (nn < 64),
        // so a byte permute against 0x64 bytes and one packed subtract of 1024
        // give the exact values
        const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const uint32_t mh01 = __builtin_bit_cast(
            uint32_t, __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, mnb, 0x07010700u)) - k1024);
        const uint32_t mh23 = __builtin_bit_cast(
            uint32_t, __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, mnb, 0x07030702u)) - k1024);
        // fifth bits of elements 16 lh .. 16 lh + 15 (bit j: sub-block j)
        const uint4 qh = *reinterpret_cast<const uint4 *>(arow + 16 + 16 * lh);
        uint4 hd[TJ][2];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            hd[j][0] = *reinterpret_cast<const uint4 *>(sD + (32 * j + li) * 8);
            hd[j][1] = *reinterpret_cast<const uint4 *>(sD + (32 * j + li) * 8 + 4);
        }
        auto hpair = [&](int j, int g) -> uint2 {
            const uint4 &v = hd[j][g >> 2];
            return (g & 2) ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y);
        };
        struct BOps {
            v4i b;
            v4h sb;
        };
        v4i aop[2];
        // sub-block g's 16 values of this lane half: nibble g % 2 of
        // qs[32 (g / 2) + 16 lh ..] with bit g of qh[16 lh ..] above it
        auto load_a = [&](int g) {
            const uint4 q = *reinterpret_cast<const uint4 *>(arow + 48 + 32 * (g >> 1) + 16 * lh);
            const int sh = 4 * (g & 1);
            const uint32_t m = 0x0F0F0F0Fu, one = 0x01010101u;
            aop[g & 1] = v4i{(int)(((q.x >> sh) & m) | (((qh.x >> g) & one) << 4)),
                             (int)(((q.y >> sh) & m) | (((qh.y >> g) & one) << 4)),
                             (int)(((q.z >> sh) & m) | (((qh.z >> g) & one) << 4)),
                             (int)(((q.w >> sh) & m) | (((qh.w >> g) & one) << 4))};
        };
        auto load_b = [&](int p, BOps &o) {
            const int g = p / TJ, j = p % TJ;
            const int n = 32 * j + li;
            o.b = *reinterpret_cast<const v4i *>(sB + n * 256 + 16 * ((2 * g + lh) ^ (n & 15)));
            o.sb = __builtin_bit_cast(v4h, hpair(j, g));
        };
        auto issue = [&](int p, const BOps &o, v16i &S, v16f &SC) {
            const int g = p / TJ;
            const v16i z = {0};
            const v16f zf = {0};
            S = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[g & 1], o.b, z, 0, 0, 0);
            const uint32_t a = sa[g & 3] & (g < 4 ? live_lo : ~live_lo);
            const uint2 as = (g & 1) ? make_uint2(0u, a) : make_uint2(a, 0u);
            SC = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, as), o.sb, zf, 0, 0, 0);
        };
        auto consume = [&](int p, const v16i &S, const v16f &SC) {
            const int g = p / TJ, j = p % TJ;
            if (g == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) accb[j][v] = (float)S[v] * SC[v];
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v) accb[j][v] = fmaf((float)S[v], SC[v], accb[j][v]);
            }
            // keep the FMAs here: sunk to the super-block's end they would
            // hold every pair's MFMA results live at once
            asm volatile("" : "+v"(accb[j]));
        };
        // pair p = (sub-block p / TJ, column tile p % TJ); pair p+1's MFMAs
        // and pair p+2's LDS reads go out before pair p's epilogue
        constexpr int NP = 8 * TJ;
        BOps ops[2];
        v16i Sb[2];
        v16f SCb[2];
        load_a(0);
        load_b(0, ops[0]);
        if (1 / TJ != 0) load_a(1);
        load_b(1, ops[1]);
        issue(0, ops[0], Sb[0], SCb[0]);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            __builtin_amdgcn_sched_barrier(0);
            if (p + 1 < NP) issue(p + 1, ops[(p + 1) & 1], Sb[(p + 1) & 1], SCb[(p + 1) & 1]);
            if (p + 2 < NP) {
                if ((p + 2) % TJ == 0) load_a((p + 2) / TJ);
                load_b(p + 2, ops[p & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
            consume(p, Sb[p & 1], SCb[p & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        // acc += d[r] * accb - dmin[r] * sum_j m_j[r] * s8_j[c] for the lane's
        // rows 8 q + 4 lh + i, their d | dmin read from the block headers; lane
        // half h supplies K slots 4h..4h+3 of the K=8 MFMA: sub-blocks 4h..4h+3
        float dr[16], dm[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t dd = *reinterpret_cast<const uint32_t *>(
                sA + (wr + 8 * (v >> 2) + 4 * lh + (v & 3)) * Q5K_BYTES);
            dr[v] = h2f(dd);
            dm[v] = h2f(dd >> 16);
        }
        const v4h am = __builtin_bit_cast(v4h, make_uint2(mh01, mh23));
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const uint4 s = *reinterpret_cast<const uint4 *>(sD + (32 * j + li) * 8 + 4 * lh);
            const v4h bm = __builtin_bit_cast(
                v4h, make_uint2(__builtin_amdgcn_perm(s.y, s.x, sel_s8), __builtin_amdgcn_perm(s.w, s.z, sel_s8)));
            const v16f zf = {0};
            const v16f P = __builtin_amdgcn_mfma_f32_32x32x8f16(am, bm, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[j][v] = fmaf(dr[v], accb[j][v], fmaf(-dm[v], P[v], acc[j][v]));
        }
    };

    dma(kb0, sA0, sB0, sD0);
    wait_vmem();
    __syncthreads();
    for (int kb = kb0; kb < kb1; kb += 2) {
        if (kb + 1 < kb1) dma(kb + 1, sA1, sB1, sD1);
        compute(sA0, sB0, sD0);
        wait_vmem();
        __syncthreads();
        if (kb + 1 < kb1) {
            if (kb + 2 < kb1) dma(kb + 2, sA0, sB0, sD0);
            compute(sA1, sB1, sD1);
            wait_vmem();
            __syncthreads();
        }
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int64_t c = col0 + 32 * j + li;
        if (c >= col_end) continue;
        float *o = GROUPED   ? dst + (int64_t)grp.col_dst[c] * dst_col_stride
                   : partial ? partial + ((int64_t)blockIdx.z * ncols + c) * nrows
                             : dst + c * dst_col_stride;
        if (fused) store_glu_column(o, row0 + wr / 2 + 2 * lh, nrows, acc[j], glu);
        else store_tile_column(o, row0 + wr + 4 * lh, nrows, acc[j]);
    }
}

}  // namespace

// Launch for mmq.hip's dispatch: Q5_K on 16-byte aligned rows, row strides
// and activation planes (the caller checks).  `grid` is (row tiles, column
// tiles, K parts); with `grp`, (row tiles, the tile table's bound, 1).
int mmq_q5k_dma_launch(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                       const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, dim3 grid, float *partial,
                       const MmqGroups *grp, const MmqGlu &glu, hipStream_t s) {
    if (K % QK_K || (int64_t)grid.x * grid.y * grid.z > 0x7FFFFFFF || nrows > 0x7FFFFFFF || ncols > 0x7FFFFFFF ||
        ((grp || glu.gate) && (grid.z != 1 || partial)))
        return (int)hipErrorInvalidValue;
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    const MmqGroups g = grp ? *grp : MmqGroups{};
#define Q5K_LAUNCH(BNV, GR)                                                                                            \
    hipLaunchKernelGGL((mmq_q5k_dma_kernel<BNV, GR>), grid, dim3(NTHREADS), 0, s, wb, K, nrows, row_stride, yqs, ds,  \
                       ncols, dst, dst_col_stride, partial, (int)grid.x, (int)grid.y, (int)grid.z, g, glu)
    if (grp) {
        if (bn == 32) Q5K_LAUNCH(32, true);
        else Q5K_LAUNCH(64, true);
    } else {
        if (bn == 32) Q5K_LAUNCH(32, false);
        else Q5K_LAUNCH(64, false);
    }
#undef Q5K_LAUNCH
    return (int)hipGetLastError();
}
