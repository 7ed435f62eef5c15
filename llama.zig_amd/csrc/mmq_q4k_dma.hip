// mmq_q4k_dma.hip -- the Q4_K MMQ with direct global->LDS loads.
//
// Same arithmetic as mmq.hip's kernel: exact int8 block dots on
// v_mfma_i32_32x32x32_i8, the per-(row, column, block) scale sc_j * d8_j as an
// exact f16 outer product (v_mfma_f32_32x32x8_f16, one live K slot), one
// convert + FMA per output and block, d and the min term (K=8 f16 MFMA of
// m_j x s8_j) once per super-block:
//   out = sum_b d_b * sum_j (sc_bj*d8_j) * S_bj - dmin_b * sum_j m_bj*s8_j
//
// What differs is the data path.  The staged kernel loads each K-step into
// registers, unpacks it and writes it to LDS between two barriers, so every
// wave stalls on that phase.  Here the step's raw bytes go straight from
// global memory into LDS with global_load_lds_dwordx4 (no registers, no
// VALU), into a second LDS buffer while the current one is contracted:
//   - A: the 128 rows' Q4_K blocks of the step, 144 B per row, as stored;
//     nibbles are unpacked when the MFMA operands are read (each 16-byte read
//     serves sub-blocks 2c and 2c+1);
//   - B: the BN columns' Q8_1 int8 values, 256 B per column, with the 16-byte
//     chunk c of column n stored at chunk position c ^ (n % 16) so that the
//     operand reads of 32 columns spread over all banks;
//   - the columns' raw (d8 | s8 << 16) headers.
// One barrier per K-step.  A wave waits only for its own transfers
// (vmcnt(0)) before that barrier; the barrier publishes every wave's.
// Rows past nrows and columns past the tile load duplicates of a valid row /
// column, whose results are never stored.
#include "../../include/ggml_hip_qmm.h"
#include "mmq_dma.h"
#include "qmm_device.h"

using namespace qmm;
using namespace qmm_dma;

namespace {

constexpr int ABYTES = BM * Q4K_BYTES;  // 18432: 18 transfers of 1 KiB

template <int BN, bool GROUPED>
__global__ __launch_bounds__(NTHREADS, 2) void mmq_q4k_dma_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride,
    const int8_t *__restrict__ yqs, const uint32_t *__restrict__ yds, int64_t ncols, float *__restrict__ dst,
    int64_t dst_col_stride, const int32_t *__restrict__ tiles, const int32_t *__restrict__ n_tiles,
    const int32_t *__restrict__ col_src, const int32_t *__restrict__ col_dst, float *__restrict__ partial, int gx,
    int gy, int gz, MmqGlu glu) {
    constexpr int TJ = BN / 32;
    constexpr int NQB = BN / 4;    // 1 KiB transfers of B int8 per step
    constexpr int NQD = BN / 32;   // 1 KiB transfers of B headers per step
    __shared__ alignas(16) uint8_t sA0[ABYTES], sA1[ABYTES];
    __shared__ alignas(16) uint8_t sB0[BN * 256], sB1[BN * 256];
    // each stage's header table and, after it, a zero block of 4 words that
    // the transfers never write (read by the scale MFMA's dead lane half)
    __shared__ alignas(16) uint32_t sD0[BN * 8 + 4], sD1[BN * 8 + 4];
    __shared__ alignas(16) float rowd[4][2][32];

    const int64_t Kp = pad_k(K);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int wr = wave * 32;
    // the zero blocks (published by the first barrier, before any contraction)
    if (threadIdx.x < 8) (threadIdx.x < 4 ? sD0 : sD1)[BN * 8 + (threadIdx.x & 3)] = 0u;

    // Work items (row tile, column tile, K part), row tiles fastest; the
    // workgroups take items blockIdx.x, +gridDim.x, ...  Grouped mode has
    // *n_tiles live column tiles.
    const int gy_live = GROUPED ? (*n_tiles < gy ? *n_tiles : gy) : gy;  // uniform
    const int nitems = gx * gy_live * gz;  // < 2^31, checked by the host
    const int nkb_all = (int)(K / QK_K);
    // one item's tile, as 32-bit values (the host bounds rows, columns and
    // K-steps below 2^31); wexp is the expert's weights in grouped mode (wgexp
    // its gate weights when fused).  row0 is the tile's first output row: a
    // fused tile has 64 of them.
    const bool fused = glu.gate != nullptr;  // uniform
    const int tile_rows = fused ? BM / 2 : BM;
    struct Item {
        int row0, col0, col_end, kb0, kb1, z;
        const uint8_t *wexp, *wgexp;
    };
    auto item_xyz = [&](int bx, int by, int bz) {
        Item I;
        I.row0 = bx * tile_rows;
        I.z = bz;
        I.kb0 = nkb_all * bz / gz;
        I.kb1 = nkb_all * (bz + 1) / gz;
        I.col0 = by * BN;
        I.col_end = (int)ncols;
        I.wexp = w;
        I.wgexp = glu.gate;
        if constexpr (GROUPED) {
            const int4 t = *reinterpret_cast<const int4 *>(tiles + 4 * by);  // {expert, col_low, col_high, -}
            I.wexp = w + (int64_t)t.x * expert_stride;
            I.wgexp = fused ? glu.gate + (int64_t)t.x * expert_stride : nullptr;
            I.col0 = t.y;
            I.col_end = t.z;
        }
        return I;
    };

    // per-lane sources of this wave's transfers for one item (fixed over its K-steps)
    const uint8_t *a_src[(18 + 3) / 4];
    const int8_t *b_src[(NQB + 3) / 4];
    const uint32_t *d_src = yds;
    // tile column whose activations lane `lane` moves in B transfer i, and in
    // the header transfer (waves < NQD)
    auto b_col = [&](int i) {
        const int q = wave + 4 * i;
        return ((q < NQB ? q : 0) * 1024 + lane * 16) >> 8;
    };
    const int d_col = (wave * 1024 + lane * 16) >> 5;
    auto set_a = [&](const Item &I) {
#pragma unroll
        for (int i = 0; i < (18 + 3) / 4; ++i) {
            const int q = wave + 4 * i;
            const int pos = (q < 18 ? q : 0) * 1024 + lane * 16;
            const int r = pos / Q4K_BYTES, ch = (pos - r * Q4K_BYTES) / 16;
            const int64_t orow = (int64_t)I.row0 + (fused ? mmq_glu_tile_row(r) : r);
            const int64_t grow = orow < nrows ? orow : nrows - 1;
            a_src[i] = (fused && (r & 2) == 0 ? I.wgexp : I.wexp) + grow * row_stride + ch * 16;
        }
    };
    // activation rows (planar Q8_1 columns) of the lane's B and header transfers
    struct Rows {
        int b[(NQB + 3) / 4];
        int d;
    };
    auto set_b = [&](const Rows &R) {
#pragma unroll
        for (int i = 0; i < (NQB + 3) / 4; ++i) {
            const int q = wave + 4 * i;
            const int pos = (q < NQB ? q : 0) * 1024 + lane * 16;
            const int n = pos >> 8, p = (pos >> 4) & 15;
            b_src[i] = yqs + (int64_t)R.b[i] * Kp + 16 * (p ^ (n & 15));
        }
        if (wave < NQD) d_src = yds + (int64_t)R.d * (Kp / QK8) + 4 * ((wave * 1024 + lane * 16) >> 4 & 1);
    };
    // the rows of an item's columns; past col_end a tile column repeats its
    // first column (loaded, never stored)
    auto rows_of = [&](int col0, int col_end) {
        auto src = [&](int n) -> int {
            const int cc = col0 + n < col_end ? col0 + n : col0;
            return GROUPED ? col_src[cc] : cc;
        };
        Rows R;
#pragma unroll
        for (int i = 0; i < (NQB + 3) / 4; ++i) R.b[i] = src(b_col(i));
        R.d = wave < NQD ? src(d_col) : 0;
        return R;
    };
    auto set_sources = [&](const Item &I) {
        set_a(I);
        set_b(rows_of(I.col0, I.col_end));
    };

    auto dma = [&](int64_t kb, uint8_t *sA, uint8_t *sB, uint32_t *sD) {
#pragma unroll
        for (int i = 0; i < (18 + 3) / 4; ++i)
            if (wave + 4 * i < 18) dma16(a_src[i] + kb * Q4K_BYTES, sA + (wave + 4 * i) * 1024);
#pragma unroll
        for (int i = 0; i < (NQB + 3) / 4; ++i)
            if (wave + 4 * i < NQB) dma16(b_src[i] + kb * 256, sB + (wave + 4 * i) * 1024);
        if (wave < NQD) dma16(d_src + kb * 8, reinterpret_cast<uint8_t *>(sD) + wave * 1024);
    };

    v16f acc[TJ], accb[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;

    // Scale outer product per group g on the f16 MFMA with one live K slot.
    // A lane of half h decodes only sub-blocks 4h..4h+3 (their scales and
    // mins); its A operand for group g is sc_{4h + g%4} in slot 0 (g even)
    // or slot 2 (g odd), zero elsewhere.  Its B operand is the raw pair of
    // (d8 | s8 << 16) headers of groups 2(g/2), 2(g/2)+1, so slot 0 / 2 hold
    // d8 of the even / odd group.  A lane reads its own half's headers (groups
    // 4h..4h+3) and, for the other half's groups, the zero block that follows
    // each stage's header table: a group is live in one lane half only.
    const uint32_t sel_s8 = 0x07060302u;  // s8 halves of two headers -> one dword
    int hoff[TJ][2];  // word offsets of the lane's header reads from the stage's table
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        hoff[j][0] = lh ? BN * 8 : (32 * j + li) * 8;
        hoff[j][1] = lh ? (32 * j + li) * 8 + 4 : BN * 8;
    }

    auto compute = [&](const uint8_t *sA, const uint8_t *sB, const uint32_t *sD) {
        const uint8_t *arow = sA + (wr + li) * Q4K_BYTES;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(arow);
        // getScaleMinK4 for sub-blocks 4*lh .. 4*lh+3, four at a time (bytes)
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
        // row d / dmin into this wave's table (the two lanes of a row store the same values)
        rowd[wave][0][li] = h2f(hdr.x);
        rowd[wave][1][li] = h2f(hdr.x >> 16);
        // the tile columns' (d8 | s8 << 16) headers of the step
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
        uint4 qa, qc;  // weight bytes as read (two pairs ahead) and in use
        auto load_ops = [&](int p, BOps &o) {
            const int g = p / TJ, j = p % TJ;
            // the weight bytes are only read here; unpacking them at issue time
            // keeps the LDS latency off the critical path
            if (j == 0 && (g & 1) == 0) qa = *reinterpret_cast<const uint4 *>(arow + 16 + 32 * (g >> 1) + 16 * lh);
            const int n = 32 * j + li;
            o.b = *reinterpret_cast<const v4i *>(sB + n * 256 + 16 * ((2 * g + lh) ^ (n & 15)));
            o.sb = __builtin_bit_cast(v4h, hpair(j, g));
        };
        auto issue = [&](int p, const BOps &o, v16i &S, v16f &SC) {
            const int g = p / TJ, j = p % TJ;
            if (j == 0) {
                if ((g & 1) == 0) qc = qa;
                const uint32_t m4 = 0x0F0F0F0Fu;
                const int sh = 4 * (g & 1);
                aop[g & 1] = v4i{(int)((qc.x >> sh) & m4), (int)((qc.y >> sh) & m4), (int)((qc.z >> sh) & m4),
                                 (int)((qc.w >> sh) & m4)};
            }
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
        };
        // pair p+1's MFMAs and pair p+2's LDS reads are issued before pair p's
        // epilogue; the fences keep the scheduler from collapsing that
        constexpr int NP = 8 * TJ;
        BOps ops[2];
        v16i Sb[2];
        v16f SCb[2];
        load_ops(0, ops[0]);
        load_ops(1, ops[1]);
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

        // acc += d[r] * accb - dmin[r] * sum_j m_j[r] * s8_j[c]; lane half h
        // supplies K slots 4h..4h+3 of the K=8 MFMA: sub-blocks 4h..4h+3
        float dr[16], dm[16];
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
            const float4 t = *reinterpret_cast<const float4 *>(&rowd[wave][0][8 * v4 + 4 * lh]);
            const float4 u = *reinterpret_cast<const float4 *>(&rowd[wave][1][8 * v4 + 4 * lh]);
            dr[4 * v4 + 0] = t.x; dr[4 * v4 + 1] = t.y; dr[4 * v4 + 2] = t.z; dr[4 * v4 + 3] = t.w;
            dm[4 * v4 + 0] = u.x; dm[4 * v4 + 1] = u.y; dm[4 * v4 + 2] = u.z; dm[4 * v4 + 3] = u.w;
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

    // Grouped 32-column tiles (the MoE case: a few K-steps per tile) are
    // walked by persistent workgroups; everything else takes one tile per
    // workgroup (the persistent loop's extra state spills at 64 columns).
    constexpr bool PERSIST = GROUPED && BN == 32;
    if constexpr (!PERSIST) {
        // one tile per workgroup: grid (row tiles, column tiles, K parts)
        if ((int)blockIdx.y >= gy_live) return;  // grouped: past the live tiles (uniform)
        int bx = (int)blockIdx.x, by = (int)blockIdx.y;
        if (!GROUPED && gz == 1) mmq_tile_order(bx + gx * by, gx, gy, bx, by);
        const Item C = item_xyz(bx, by, (int)blockIdx.z);
        set_sources(C);
        dma(C.kb0, sA0, sB0, sD0);
        wait_vmem();
        __syncthreads();
        for (int kb = C.kb0; kb < C.kb1; kb += 2) {
            if (kb + 1 < C.kb1) dma(kb + 1, sA1, sB1, sD1);
            compute(sA0, sB0, sD0);
            wait_vmem();
            __syncthreads();
            if (kb + 1 < C.kb1) {
                if (kb + 2 < C.kb1) dma(kb + 2, sA0, sB0, sD0);
                compute(sA1, sB1, sD1);
                wait_vmem();
                __syncthreads();
            }
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int64_t c = (int64_t)C.col0 + 32 * j + li;
            if (c >= C.col_end) continue;
            float *o;
            if constexpr (GROUPED) o = dst + (int64_t)col_dst[c] * dst_col_stride;
            else o = partial ? partial + ((int64_t)C.z * ncols + c) * nrows : dst + c * dst_col_stride;
            if (fused) store_glu_column(o, (int64_t)C.row0 + wr / 2 + 2 * lh, nrows, acc[j], glu);
            else store_tile_column(o, (int64_t)C.row0 + wr + 4 * lh, nrows, acc[j]);
        }
    } else {
        // Persistent workgroups walk items blockIdx.x, +G, +2G, ... (G =
        // gridDim.x; one K part).  The transfer cursor (item it_n, step kb_n)
        // runs one step ahead of the contraction (item it_c, step kb_c) and
        // crosses into the next item while the current one finishes, so a
        // tile's first transfer is not exposed.  The tables an item needs
        // are fetched ahead, so no item boundary waits on a dependent load:
        // the tile entries of the items two ahead of the transfer cursor and
        // one ahead of the contraction, the gather rows (col_src) of the item
        // one ahead of the transfer cursor, and the scatter rows (col_dst) of
        // the contraction's item as it starts.
        const int G = (int)gridDim.x;
        int it_c = (int)blockIdx.x;
        if (it_c >= nitems) return;  // uniform per workgroup
        auto tile_of = [&](int it) { return *reinterpret_cast<const int4 *>(tiles + 4 * ((it / gx) % gy_live)); };
        auto item_of = [&](int it, const int4 &t) {
            Item I;
            I.row0 = (it % gx) * tile_rows;
            I.z = 0;
            I.kb0 = 0;
            I.kb1 = nkb_all;
            I.wexp = w + (int64_t)t.x * expert_stride;
            I.wgexp = fused ? glu.gate + (int64_t)t.x * expert_stride : nullptr;
            I.col0 = t.y;
            I.col_end = t.z;
            return I;
        };
        int drow[TJ];  // scatter rows of the contraction item's lane columns
        auto load_drows = [&](const Item &I) {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int c = I.col0 + 32 * j + li;
                drow[j] = col_dst[c < I.col_end ? c : I.col0];
            }
        };
        const int4 t0 = tile_of(it_c);
        Item C = item_of(it_c, t0);
        load_drows(C);
        set_a(C);
        set_b(rows_of(t0.y, t0.z));
        int4 tc1 = it_c + G < nitems ? tile_of(it_c + G) : t0;  // contraction: next item's tile
        int4 tn1 = tc1, tn2 = t0;                                 // transfer: tiles one and two ahead
        Rows rn1 = {};                                            // transfer: rows one ahead
        if (it_c + G < nitems) rn1 = rows_of(tn1.y, tn1.z);
        if (it_c + 2 * G < nitems) tn2 = tile_of(it_c + 2 * G);
        int it_n = it_c;
        int kb_n = 0, kb_c = 0;
        bool dma_live = true;
        auto advance = [&]() {
            if (++kb_n < nkb_all) return;
            it_n += G;
            if (it_n < nitems) {
                kb_n = 0;
                set_a(item_of(it_n, tn1));
                set_b(rn1);
                tn1 = tn2;
                if (it_n + G < nitems) rn1 = rows_of(tn1.y, tn1.z);
                if (it_n + 2 * G < nitems) tn2 = tile_of(it_n + 2 * G);
            } else {
                dma_live = false;
            }
        };
        auto store = [&]() {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int64_t c = (int64_t)C.col0 + 32 * j + li;
                if (c >= C.col_end) continue;
                float *o = dst + (int64_t)drow[j] * dst_col_stride;
                if (fused) store_glu_column(o, (int64_t)C.row0 + wr / 2 + 2 * lh, nrows, acc[j], glu);
                else store_tile_column(o, (int64_t)C.row0 + wr + 4 * lh, nrows, acc[j]);
            }
        };
        // after a step's contraction: at an item's last step store it and move on
        auto finish_step = [&]() -> bool {
            if (++kb_c < nkb_all) return true;
            store();
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
            it_c += G;
            if (it_c >= nitems) return false;
            C = item_of(it_c, tc1);
            kb_c = 0;
            load_drows(C);
            if (it_c + G < nitems) tc1 = tile_of(it_c + G);
            return true;
        };

        dma(kb_n, sA0, sB0, sD0);
        advance();
        wait_vmem();
        __syncthreads();
        for (;;) {
            if (dma_live) {
                dma(kb_n, sA1, sB1, sD1);
                advance();
            }
            compute(sA0, sB0, sD0);
            wait_vmem();
            __syncthreads();
            if (!finish_step()) break;
            if (dma_live) {
                dma(kb_n, sA0, sB0, sD0);
                advance();
            }
            compute(sA1, sB1, sD1);
            wait_vmem();
            __syncthreads();
            if (!finish_step()) break;
        }
    }
}

}  // namespace

// Launch for mmq.hip's dispatch (same arguments as its kernel; Q4_K rows and
// the activation planes 16-byte aligned, which the caller checks).  `grid` is
// the tile grid (row tiles, column tiles, K parts).  Grouped 32-column tiles
// are walked by at most two workgroups per CU (the kernel's register and LDS
// budget); otherwise each workgroup takes one tile.
int mmq_q4k_dma_launch(int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride, int64_t expert_stride,
                       const int8_t *yqs, const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride,
                       dim3 grid, const int32_t *tiles, const int32_t *n_tiles, const int32_t *col_src,
                       const int32_t *col_dst, float *partial, const MmqGlu &glu, hipStream_t s) {
    // workgroups resident at once: 2 per CU of the current device (queried per
    // call: a process may drive GPUs of different sizes; the query is a host
    // attribute read)
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    const int resident = 2 * cus;
    const int64_t items = (int64_t)grid.x * grid.y * grid.z;
    if (items > 0x7FFFFFFF || K / QK_K > 0x7FFFFFFF || nrows > 0x7FFFFFFF || ncols > 0x7FFFFFFF)
        return (int)hipErrorInvalidValue;
    // grouped mode walks its tiles with the resident workgroups; a dense
    // launch takes one tile per workgroup
    const dim3 pgrid((unsigned)(items < resident ? items : resident));
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    const int gx = (int)grid.x, gy = (int)grid.y, gz = (int)grid.z;
#define MMQ_DMA_LAUNCH(BNV, GR)                                                                                        \
    hipLaunchKernelGGL((mmq_q4k_dma_kernel<BNV, GR>), GR && BNV == 32 ? pgrid : grid, dim3(NTHREADS), 0, s, wb, K,   \
                       nrows,                                                                                          \
                       row_stride,                                                                                     \
                       expert_stride, yqs, ds, ncols, dst, dst_col_stride, tiles, n_tiles, col_src, col_dst,         \
                       partial, gx, gy, gz, glu)
    if (tiles) {
        if (bn == 32) MMQ_DMA_LAUNCH(32, true);
        else MMQ_DMA_LAUNCH(64, true);
    } else {
        if (bn == 32) MMQ_DMA_LAUNCH(32, false);
        else MMQ_DMA_LAUNCH(64, false);
    }
#undef MMQ_DMA_LAUNCH
    return (int)hipGetLastError();
}
