// mmq_legacy_dma.hip -- the Q8_0 and Q4_0 MMQ with direct global->LDS loads.
//
// Arithmetic as in mmq.hip: the 32-deep block dot on v_mfma_i32_32x32x32_i8
// (exact), the per-(row, column, block) scale d_b * d8_b as an exact f16 outer
// product (v_mfma_f32_32x32x8_f16, one live K slot), one convert + FMA per
// output and block:
//   out = sum_b (d_b * d8_b) * dot_b(q, q8)
// with q the Q8_0 codes or the Q4_0 nibbles minus 8.  These "legacy" types
// (ggml's name) have no super-block, so there is no per-super-block term.
//
// Data path.  Rows of K % 256 == 0 at 16-byte aligned addresses and strides:
//   - Q8_0: a K-step is 128 values, four 34-byte blocks, 136 bytes of a row.
//     A Q8_0 row is a multiple of 272 bytes, so step s starts at 136 s,
//     16-byte aligned for even s and 8 bytes past a boundary for odd s; the
//     144-byte aligned window around it (never past the row: the last step
//     is odd and its window ends at the row's end) is moved.
//   - Q4_0: a K-step is 256 values, eight 18-byte blocks, 144 bytes of a row,
//     always 16-byte aligned; the step's bytes are moved as they are.
// Either way 144 bytes per row go straight from global memory into LDS with
// global_load_lds_dwordx4, rows back to back.  A block's codes start 2 bytes
// in, so a lane reads the aligned 16-byte chunks around its 16 code bytes and
// funnel-shifts them (v_alignbyte_b32) into place.  Q4_0's lane half h
// takes the low (h = 0) or high (h = 1) nibbles of the block's 16 bytes and
// subtracts 8 bytewise ((n + 0x78) ^ 0x80, no carries between bytes).  The
// columns' Q8_1 bytes (one step's worth per column) and their block headers
// come the same way; 16 consecutive columns' reads of one 16-byte chunk cover
// all banks.  Two buffers: the next step's transfers run while the current
// step is contracted, one barrier per step.
#include "../../include/ggml_hip_qmm.h"
#include "mmq_dma.h"
#include "qmm_device.h"

#include <type_traits>

using namespace qmm;
using namespace qmm_dma;

namespace {

constexpr int WIN = 144;          // bytes of a row's step in LDS
constexpr int ABYTES = BM * WIN;  // 18432: 18 transfers of 1 KiB

template <int TYPE>
struct Legacy;
template <>
struct Legacy<TYPE_Q8_0> {
    static constexpr int KSTEP = 128;                // values per step
    static constexpr int NB = 4;                     // blocks per step
    static constexpr int BBYTES = Q80_BYTES;         // 34
    static constexpr int STEP_BYTES = NB * BBYTES;   // 136: the window is the aligned 144 around it
};
template <>
struct Legacy<TYPE_Q4_0> {
    static constexpr int KSTEP = 256;
    static constexpr int NB = 8;
    static constexpr int BBYTES = Q40_BYTES;         // 18
    static constexpr int STEP_BYTES = NB * BBYTES;   // 144: always aligned
};

// A block's codes start 2 bytes past its header, so they are rarely 16-byte
// aligned in the window.  The rows sit 144 bytes (36 dwords) apart, so 4-byte
// reads of one offset by the 32 rows of a wave hit each bank 4 times; 16-byte
// reads (8 lanes per LDS cycle) cover the banks once.  The window is
// therefore read as the aligned 16-byte chunks around the 16 bytes and
// funnel-shifted in registers.
//
// A block's 16 bytes at byte offset R (even, compile-time) of the chunk pair
// [c, c + 1] of a 16-byte aligned row (chunk c + 1 only when R != 0), and the
// f16 two bytes before them (the block's d) when they lie in the pair.
template <int R>
struct Win16 {
    uint32_t w[8];
    __device__ __forceinline__ void load(const uint8_t *row, int c) {
        const uint4 a = *reinterpret_cast<const uint4 *>(row + 16 * c);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        if constexpr (R != 0) {
            const uint4 b = *reinterpret_cast<const uint4 *>(row + 16 * c + 16);
            w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
        }
    }
    __device__ __forceinline__ v4i codes() const {
        constexpr int D = R >> 2, B = R & 3;
        v4i q;
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = B ? (int)__builtin_amdgcn_alignbyte(w[D + k + 1], w[D + k], B) : (int)w[D + k];
        return q;
    }
    // the f16 bits before the codes (R >= 2)
    __device__ __forceinline__ uint32_t before() const {
        static_assert(R >= 2, "the two bytes before the codes are in the previous chunk");
        return (w[(R - 2) >> 2] >> (8 * ((R - 2) & 3))) & 0xFFFFu;
    }
};

// Block I's A operand and scale slot for a step whose window starts SH bytes
// into its 16-byte aligned row (SH = 0, or 8 for odd Q8_0 steps): Q8_0 lane
// half h reads the block's codes 16h .. 16h + 15; Q4_0 lanes read all 16
// bytes and keep the low (h = 0) or high (h = 1) nibbles, minus 8 bytewise
// ((n + 0x78) ^ 0x80, no carries between bytes).  The block's d goes to lanes
// of half 0 only (keep), in K slot 0 (I even) or 2 (I odd).
template <int TYPE, int SH, int I>
__device__ __forceinline__ void legacy_a(const uint8_t *row, int lh, uint32_t keep, v4i &aop, v4h &asc) {
    constexpr int BB = Legacy<TYPE>::BBYTES;
    constexpr int O = SH + BB * I + 2, R = O & 15;
    Win16<R> win;
    win.load(row, (O >> 4) + (TYPE == TYPE_Q8_0 ? lh : 0));
    v4i q = win.codes();
    if constexpr (TYPE == TYPE_Q4_0) {
        const int sh = 4 * lh;
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = (int)((((uint32_t)q[e] >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ (int)0x80808080u;
    }
    aop = q;
    uint32_t d;
    if constexpr (R >= 2) {
        d = win.before();
    } else {
        const uint32_t dw = *reinterpret_cast<const uint32_t *>(row + ((O - 2) & ~3));
        d = ((O - 2) & 3) ? dw >> 16 : dw;
    }
    asc = __builtin_bit_cast(v4h, (I & 1) ? make_uint2(0u, d & keep) : make_uint2(d & keep, 0u));
}

template <int TYPE, int BN, bool GROUPED>
__global__ __launch_bounds__(NTHREADS, 2) void mmq_legacy_dma_kernel(
    const uint8_t *__restrict__ w, int64_t K, int64_t nrows, int64_t row_stride, const int8_t *__restrict__ yqs,
    const uint32_t *__restrict__ yds, int64_t ncols, float *__restrict__ dst, int64_t dst_col_stride,
    float *__restrict__ partial, int gx, int gy, int gz, MmqGroups grp, MmqGlu glu) {
    using L = Legacy<TYPE>;
    constexpr int KSTEP = L::KSTEP, NB = L::NB, STEP_BYTES = L::STEP_BYTES;
    constexpr int TJ = BN / 32;
    constexpr int NCH = KSTEP / 16;                 // 16-byte chunks of a column's step codes
    constexpr int NQB = BN * KSTEP / 1024;          // 1 KiB transfers of the B codes per step
    constexpr int NQD = (BN * NB * 4 + 1023) / 1024;  // 1 KiB transfers of the headers per step
    static_assert(NQB % 4 == 0 && NQD <= 2, "code transfers over 4 waves, headers on waves 2-3");
    // slot of a column's 16-byte chunk c: c ^ bswz(n), so 16 consecutive
    // columns' reads of one chunk spread over all banks (a column's step is
    // 128 bytes for Q8_0, 256 for Q4_0)
    auto bswz = [](int n) { return NCH == 16 ? (n & 15) : ((n >> 1) & 7); };
    __shared__ alignas(16) uint8_t sA0[ABYTES], sA1[ABYTES];
    __shared__ alignas(16) uint8_t sB0[BN * KSTEP], sB1[BN * KSTEP];
    __shared__ alignas(16) uint32_t sD0[NQD * 256], sD1[NQD * 256];  // the columns' block headers

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
    // a K part takes whole 256-value super-steps (SPS steps each), as the
    // split factor counts them; for Q8_0 (SPS = 2) every part starts on an
    // even step
    constexpr int SPS = 256 / KSTEP;
    const int nss = (int)(K / 256);
    const int s_begin = SPS * (nss * (int)blockIdx.z / gz), s_end = SPS * (nss * ((int)blockIdx.z + 1) / gz);

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
        // transfer t covers 1024 / (16 NCH) columns; lane -> (column, slot)
        const int n = t * (64 / NCH) + lane / NCH, slot = lane % NCH;
        b_src[i] = yqs + src_col(col0 + n) * Kp + 16 * (slot ^ bswz(n));
    }
    // column headers (waves 2 .. 1 + NQD): 16-byte runs of NB headers per
    // column; transfer t, lane l -> column (64 t + l) / (NB / 4), part
    const uint32_t *d_src;
    {
        const int per = NB / 4;  // 16-byte runs per column
        const int q = (wave >= 2 && wave - 2 < NQD ? wave - 2 : 0) * 64 + lane;
        const int n0 = q / per, part = q % per;
        const int n = n0 < BN ? n0 : 0;
        d_src = yds + src_col(col0 + n) * (Kp / QK8) + 4 * part;
    }

    auto dma = [&](int s, uint8_t *sA, uint8_t *sB, uint32_t *sD) {
        const int64_t woff = ((int64_t)s * STEP_BYTES) & ~(int64_t)15;
#pragma unroll
        for (int i = 0; i < (18 + 3) / 4; ++i)
            if (wave + 4 * i < 18) dma16(a_src[i] + woff, sA + (wave + 4 * i) * 1024);
#pragma unroll
        for (int i = 0; i < (NQB + 3) / 4; ++i)
            if (wave + 4 * i < NQB) dma16(b_src[i] + (int64_t)s * KSTEP, sB + (wave + 4 * i) * 1024);
        if (wave >= 2 && wave - 2 < NQD)
            dma16(d_src + NB * s, reinterpret_cast<uint8_t *>(sD) + (wave - 2) * 1024);
    };

    v16f acc[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;

    // Scale outer product on the f16 MFMA with one live K slot (slot 0 or 2
    // of lane half 0 for even or odd blocks b): lanes of half 0 hand d_b of
    // their row, lanes of half 1 zeros; the B operand is the column's raw
    // (d8 | s8 << 16) headers of blocks b & ~1 and b | 1 as read.
    const uint32_t keep = lh ? 0u : 0xFFFFu;

    // the step's window starts SH bytes into its row: 0, or 8 for odd Q8_0
    // steps (a part starts at an even step)
    auto compute = [&](auto shc, const uint8_t *sA, const uint8_t *sB, const uint32_t *sD) __attribute__((always_inline)) {
        constexpr int SH = decltype(shc)::value;
        const uint8_t *arow = sA + (wr + li) * WIN;
        struct Ops {
            v4i b;
            v4h sb;
        };
        v4i aop[2];
        v4h asc[2];
        auto load_a = [&](int i, int slot) __attribute__((always_inline)) {
            switch (i) {
#define LEGACY_A_CASE(I)                                                                   \
    case I:                                                                                \
        if constexpr (I < NB) legacy_a<TYPE, SH, I>(arow, lh, keep, aop[slot], asc[slot]); \
        break;
                LEGACY_A_CASE(0) LEGACY_A_CASE(1) LEGACY_A_CASE(2) LEGACY_A_CASE(3)
                LEGACY_A_CASE(4) LEGACY_A_CASE(5) LEGACY_A_CASE(6) LEGACY_A_CASE(7)
#undef LEGACY_A_CASE
            }
        };
        auto load_b = [&](int p, Ops &o) {
            const int i = p / TJ, j = p % TJ;
            const int n = 32 * j + li;
            o.b = *reinterpret_cast<const v4i *>(sB + n * KSTEP + 16 * ((2 * i + lh) ^ bswz(n)));
            o.sb = __builtin_bit_cast(v4h, *reinterpret_cast<const uint2 *>(sD + NB * n + (i & ~1)));
        };
        auto issue = [&](int p, const Ops &o, v16i &S, v16f &SC) {
            const int i = p / TJ;
            const v16i z = {0};
            const v16f zf = {0};
            S = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[i & 1], o.b, z, 0, 0, 0);
            SC = __builtin_amdgcn_mfma_f32_32x32x8f16(asc[i & 1], o.sb, zf, 0, 0, 0);
        };
        auto consume = [&](int p, const v16i &S, const v16f &SC) {
            const int j = p % TJ;
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[j][v] = fmaf((float)S[v], SC[v], acc[j][v]);
            // keep the FMAs at their pair: nothing reads acc before the
            // stores, and sinking them there would hold every S and SC
            asm volatile("" : "+v"(acc[j]));
        };
        // pair p = (block p / TJ, column tile p % TJ); pair p+1's MFMAs and
        // pair p+2's LDS reads go out before pair p's epilogue
        constexpr int NP = NB * TJ;
        Ops ops[2];
        v16i Sb[2];
        v16f SCb[2];
        load_a(0, 0);
        load_b(0, ops[0]);
        if (1 / TJ != 0) load_a(1, 1);
        load_b(1, ops[1]);
        issue(0, ops[0], Sb[0], SCb[0]);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            __builtin_amdgcn_sched_barrier(0);
            if (p + 1 < NP) issue(p + 1, ops[(p + 1) & 1], Sb[(p + 1) & 1], SCb[(p + 1) & 1]);
            if (p + 2 < NP) {
                if ((p + 2) % TJ == 0) load_a((p + 2) / TJ, ((p + 2) / TJ) & 1);
                load_b(p + 2, ops[p & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
            consume(p, Sb[p & 1], SCb[p & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    dma(s_begin, sA0, sB0, sD0);
    wait_vmem();
    __syncthreads();
    // steps in pairs from an even s_begin (Q8_0: window shift 0, then 8);
    // a Q4_0 part may end on an odd step
    for (int s = s_begin; s < s_end; s += 2) {
        if (s + 1 < s_end) dma(s + 1, sA1, sB1, sD1);
        compute(std::integral_constant<int, 0>{}, sA0, sB0, sD0);
        wait_vmem();
        __syncthreads();
        if (s + 1 < s_end) {
            if (s + 2 < s_end) dma(s + 2, sA0, sB0, sD0);
            compute(std::integral_constant<int, STEP_BYTES & 15>{}, sA1, sB1, sD1);
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

// Launch for mmq.hip's dispatch: Q8_0 or Q4_0, rows of K % 256 == 0 at
// 16-byte aligned addresses and strides, 16-byte aligned activation planes
// (the caller checks).  `grid` is (row tiles, column tiles, K parts), with
// `grp` (row tiles, the tile table's bound, 1).
int mmq_legacy_dma_launch(int type, int bn, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                          const int8_t *yqs, const void *yds, int64_t ncols, float *dst, int64_t dst_col_stride,
                          dim3 grid, float *partial, const MmqGroups *grp, const MmqGlu &glu, hipStream_t s) {
    if (K % 256 || (int64_t)grid.x * grid.y * grid.z > 0x7FFFFFFF || nrows > 0x7FFFFFFF || ncols > 0x7FFFFFFF ||
        ((grp || glu.gate) && (grid.z != 1 || partial)))
        return (int)hipErrorInvalidValue;
    const uint8_t *wb = (const uint8_t *)w;
    const uint32_t *ds = (const uint32_t *)yds;
    const MmqGroups g = grp ? *grp : MmqGroups{};
#define LEGACY_LAUNCH(T, BNV, GR)                                                                                      \
    hipLaunchKernelGGL((mmq_legacy_dma_kernel<T, BNV, GR>), grid, dim3(NTHREADS), 0, s, wb, K, nrows, row_stride, yqs, \
                       ds, ncols, dst, dst_col_stride, partial, (int)grid.x, (int)grid.y, (int)grid.z, g, glu)
#define LEGACY_TYPE(T)                                                                                                 \
    if (grp) {                                                                                                         \
        if (bn == 32) LEGACY_LAUNCH(T, 32, true);                                                                      \
        else LEGACY_LAUNCH(T, 64, true);                                                                               \
    } else {                                                                                                           \
        if (bn == 32) LEGACY_LAUNCH(T, 32, false);                                                                     \
        else LEGACY_LAUNCH(T, 64, false);                                                                              \
    }
    if (type == TYPE_Q8_0) {
        LEGACY_TYPE(TYPE_Q8_0)
    } else if (type == TYPE_Q4_0) {
        LEGACY_TYPE(TYPE_Q4_0)
    } else {
        return (int)hipErrorInvalidValue;
    }
#undef LEGACY_TYPE
#undef LEGACY_LAUNCH
    return (int)hipGetLastError();
}
