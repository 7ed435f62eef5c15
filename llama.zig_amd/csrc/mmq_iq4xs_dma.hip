// mmq_iq4xs_dma.hip -- the IQ4_XS MMQ with direct global->LDS loads.
//
// Arithmetic as in mmq.hip's IQ4_XS path: the 32-deep sub-block dot of the
// int8 levels (kvalues_iq4nl[index]) on v_mfma_i32_32x32x32_i8 (exact), the
// per-(row, column, sub-block) scale (ls_j - 32) * d8_j as an exact f16 outer
// product (v_mfma_f32_32x32x8_f16, one live K slot), one convert + FMA per
// output and sub-block, and d once per super-block:
//   out = sum_b d_b * sum_j ((ls_bj - 32) * d8_j) * dot_bj(levels, q8)
//
// Data path.  block_iq4_xs {d, scales_h, scales_l[4], qs[128]} is 136 bytes,
// 8-byte aligned.  IQ4_XS rows of K % 512 == 0 are a multiple of 272 bytes,
// so super-block s starts at 136 s, 16-byte aligned for even s and 8 bytes
// past a boundary for odd s; the 144-byte aligned window around it (never
// past the row: the last super-block is odd and its window ends at the row's
// end) goes straight from global memory into LDS with
// global_load_lds_dwordx4, rows back to back.  The levels are looked up when
// the operands are read (three byte permutes per four indices), by the wave
// that owns the row, as the staged kernel does when it unpacks into LDS.
// The columns' Q8_1 codes (256 per column) and their eight block headers come
// the same way; chunk c of column n sits at slot c ^ (n & 15).  Two buffers:
// the next super-block's transfers run while the current one is contracted,
// one barrier per step.
#include "../../include/ggml_hip_qmm.h"
#include "mmq_dma.h"
#include "qmm_device.h"

using namespace qmm;
using namespace qmm_dma;

namespace {

constexpr int WIN = 144;          // bytes of a row's window in LDS
constexpr int ABYTES = BM * WIN;  // 18432: 18 transfers of 1 KiB

template <int BN, bool GROUPED>
__global__ __launch_bounds__(NTHREADS, 2) void mmq_iq4xs_dma_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t ncols, float *__restrict__ dst, int64_t dst_col_stride,
    float *__restrict__ partial, int gx, int gy, int gz, MmqGroups grp, MmqGlu glu) {
    constexpr int TJ = BN / 32;
    constexpr int NQB = BN / 4;   // 1 KiB transfers of the B codes per step (4 columns each)
    constexpr int NQD = BN / 32;  // 1 KiB transfers of the B headers per step (32 columns each)
    __shared__ alignas(16) uint8_t sA0[ABYTES], sA1[ABYTES];
    __shared__ alignas(16) uint8_t sB0[BN * 256], sB1[BN * 256];
    // each stage's header table and, after it, a zero block of 4 words that
    // the transfers never write (read by the scale MFMA's dead lane half)
    __shared__ alignas(16) uint32_t sD0[BN * 8 + 4], sD1[BN * 8 + 4];
    __shared__ alignas(16) float rowd[4][32];

    const int64_t Kp = pad_k(K);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int wr = wave * 32;
    // the zero blocks (published by the first barrier, before any contraction)
    if (threadIdx.x < 8) (threadIdx.x < 4 ? sD0 : sD1)[BN * 8 + (threadIdx.x & 3)] = 0u;

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
    const int nkb = (int)(K / QK_K);  // even
    const int kb0 = nkb * (int)blockIdx.z / gz, kb1 = nkb * ((int)blockIdx.z + 1) / gz;

    // per-lane transfer sources (fixed over the K loop)
    const uint8_t *a_src[(18 + 3) / 4];
#pragma unroll
    for (int i = 0; i < (18 + 3) / 4; ++i) {
        const int t = wave + 4 * i < 18 ? wave + 4 * i : 0;
        const int pos = t * 1024 + lane * 16, r = pos / WIN;
        const int64_t orow = row0 + (fused ? mmq_glu_tile_row(r) : r);
        const int64_t rr = orow < nrows ? orow : nrows - 1;
        a_src[i] = (fused && (r & 2) == 0 ? wgexp : wexp) + rr * row_stride + (pos - r * WIN);
    }
    const int8_t *b_src[(NQB + 3) / 4];
#pragma unroll
    for (int i = 0; i < (NQB + 3) / 4; ++i) {
        const int t = wave + 4 * i < NQB ? wave + 4 * i : 0;
        const int n = 4 * t + (lane >> 4);
        b_src[i] = yqs + src_col(col0 + n) * Kp + 16 * ((lane & 15) ^ (n & 15));
    }
    // column headers (waves 2 .. 1 + NQD, which take one A transfer fewer):
    // transfer t, lane l -> column 32 t + l / 2, blocks 4 (l & 1) .. +3
    const uint32_t *d_src;
    {
        const int n = 32 * (wave >= 2 && wave - 2 < NQD ? wave - 2 : 0) + (lane >> 1);
        d_src = yds + src_col(col0 + n) * (Kp / QK8) + 4 * (lane & 1);
    }

    auto dma = [&](int kb, uint8_t *sA, uint8_t *sB, uint32_t *sD) {
        const int64_t woff = ((int64_t)kb * IQ4XS_BYTES) & ~(int64_t)15;
#pragma unroll
        for (int i = 0; i < (18 + 3) / 4; ++i)
            if (wave + 4 * i < 18) dma16(a_src[i] + woff, sA + (wave + 4 * i) * 1024);
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
    // slot.  A lane of half h decodes only the scales of sub-blocks 4h..4h+3;
    // its A operand for sub-block g is (ls - 32) of sub-block 4h + g % 4, live
    // when h == g / 4 (the other half reads zero headers below).
    // The A operand sits in slot 0 (g even) or slot 2 (g odd); the B operand is
    // the raw pair of (d8 | s8 << 16) headers of groups 2(g/2), 2(g/2)+1.  A
    // lane reads its own half's four headers and, for the other half's
    // groups, the zero block after the stage's header table.
    int hoff[TJ][2];  // word offsets of the lane's header reads from the stage's table
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        hoff[j][0] = lh ? BN * 8 : (32 * j + li) * 8;
        hoff[j][1] = lh ? (32 * j + li) * 8 + 4 : BN * 8;
    }

    auto compute = [&](int kb, const uint8_t *sA, const uint8_t *sB, const uint32_t *sD) {
        const int shift = (kb * IQ4XS_BYTES) & 15;  // 0 or 8, uniform
        const uint8_t *arow = sA + (wr + li) * WIN + shift;
        const uint2 hdr = *reinterpret_cast<const uint2 *>(arow);  // d | scales_h << 16, scales_l
        uint32_t sa[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int j = 4 * lh + t;
            const uint32_t ls = ((hdr.y >> (4 * j)) & 0xFu) | (((hdr.x >> (16 + 2 * j)) & 3u) << 4);
            sa[t] = f16_bits((float)((int)ls - 32));
        }
        rowd[wave][li] = h2f(hdr.x);  // the two lanes of a row store the same value
        uint4 hd[TJ][2];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            hd[j][0] = *reinterpret_cast<const uint4 *>(sD + hoff[j][0]);
            hd[j][1] = *reinterpret_cast<const uint4 *>(sD + hoff[j][1]);
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
        // sub-block g's 16 levels of this lane half: the low (h = 0) or high
        // (h = 1) nibbles of qs[16g .. 16g+15] as indices
        auto load_a = [&](int g) {
            const uint4 q = *reinterpret_cast<const uint4 *>(arow + 8 + 16 * g);  // 8-byte aligned
            const int sh = 4 * lh;
            const uint32_t m = 0x0F0F0F0Fu;
            aop[g & 1] = v4i{(int)iq4nl_levels((q.x >> sh) & m), (int)iq4nl_levels((q.y >> sh) & m),
                             (int)iq4nl_levels((q.z >> sh) & m), (int)iq4nl_levels((q.w >> sh) & m)};
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
            const uint2 as = (g & 1) ? make_uint2(0u, sa[g & 3]) : make_uint2(sa[g & 3], 0u);
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
        // acc += d[r] * accb (rows 8q + 4h + i of the lane)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
            const float4 t = *reinterpret_cast<const float4 *>(&rowd[wave][8 * v4 + 4 * lh]);
            const float dr[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][4 * v4 + i] = fmaf(dr[i], accb[j][4 * v4 + i], acc[j][4 * v4 + i]);
        }
    };

    dma(kb0, sA0, sB0, sD0);
    wait_vmem();
    __syncthreads();
    for (int kb = kb0; kb < kb1; kb += 2) {
        dma(kb + 1, sA1, sB1, sD1);  // the part holds an even number of super-blocks
        compute(kb, sA0, sB0, sD0);
        wait_vmem();
        __syncthreads();
        if (kb + 2 < kb1) dma(kb + 2, sA0, sB0, sD0);
        compute(kb + 1, sA1, sB1, sD1);
        wait_vmem();
        __syncthreads();
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

// Launch for mmq.hip's dispatch: IQ4_XS on rows of K % 512 == 0 at 16-byte
// aligned addresses and strides, 16-byte aligned activation planes, K parts
// of an even number of super-blocks (the caller checks).  `grid` is (row
// tiles, column tiles, K parts); with `grp`, (row tiles, the tile table's
// bound, 1).
int mmq_iq4xs_dma_launch(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *yqs,
                         const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride, dim3 grid, float *partial,
                         const MmqGroups *grp, const MmqGlu &glu, hipStream_t s) {
    if (K % 512 || (K / QK_K) % (2 * (int64_t)grid.z) || (int64_t)grid.x * grid.y * grid.z > 0x7FFFFFFF ||
        nrows > 0x7FFFFFFF || ncols > 0x7FFFFFFF || ((grp || glu.gate) && (grid.z != 1 || partial)))
        return (int)hipErrorInvalidValue;
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    const MmqGroups g = grp ? *grp : MmqGroups{};
#define IQ4XS_LAUNCH(BNV, GR)                                                                                          \
    hipLaunchKernelGGL((mmq_iq4xs_dma_kernel<BNV, GR>), grid, dim3(NTHREADS), 0, s, wb, K, nrows, row_stride, yqs, ds,\
                       ncols, dst, dst_col_stride, partial, (int)grid.x, (int)grid.y, (int)grid.z, g, glu)
    if (grp) {
        if (bn == 32) IQ4XS_LAUNCH(32, true);
        else IQ4XS_LAUNCH(64, true);
    } else {
        if (bn == 32) IQ4XS_LAUNCH(32, false);
        else IQ4XS_LAUNCH(64, false);
    }
#undef IQ4XS_LAUNCH
    return (int)hipGetLastError();
}
