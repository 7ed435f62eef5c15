// qmm_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Block layouts follow the reference's ggml-common.h restatement
// (src/ggml/quants/blocks.zig:67-222): block_q4_K {d, dmin, scales[12],
// qs[128]} 144 B; block_q6_K {ql[128], qh[64], scales[16], d} 210 B;
// block_q8_0 {d, qs[32]} 34 B.  Q6_K and Q8_0 blocks sit at 2-byte alignment
// inside a row.  Two ways read 16 of their bytes: dword-aligned loads plus a
// byte funnel shift (v_alignbyte_b32, ld16_a2), or one unaligned vector load
// (ld16_u).  Each kernel uses the one that measured faster for it: ld16_u for
// the MMQ staging loads and the Q6_K GEMV, ld16_a2 for the Q8_0 and Q4_0
// GEMVs.  Neither reads outside the block.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm {

constexpr int QK_K = 256;
constexpr int QK8 = 32;
constexpr int Q4K_BYTES = 144;
constexpr int Q5K_BYTES = 176;
constexpr int Q6K_BYTES = 210;
constexpr int Q80_BYTES = 34;
constexpr int Q81_BYTES = 36;  // block_q8_1: d, s (f16), qs[32]
constexpr int Q40_BYTES = 18;
constexpr int IQ4XS_BYTES = 136;
constexpr int64_t ROW_PAD = 512;  // activation row padding (MATRIX_ROW_PADDING)

constexpr int TYPE_Q4_0 = 2;
constexpr int TYPE_Q8_0 = 8;
constexpr int TYPE_Q4_K = 12;
constexpr int TYPE_Q5_K = 13;
constexpr int TYPE_Q6_K = 14;
constexpr int TYPE_IQ4_XS = 23;

__host__ __device__ constexpr int64_t pad_k(int64_t k) { return (k + ROW_PAD - 1) / ROW_PAD * ROW_PAD; }

// Alignment of a weight type's blocks inside its rows, which the kernels read
// at: 16 bytes for the 144- and 176-byte K-quant blocks (dwordx4 loads), 8 for
// IQ4_XS's 136, 2 for Q6_K's 210, Q8_0's 34 and Q4_0's 18.
__host__ __device__ constexpr int64_t block_align(int type) {
    return type == TYPE_Q4_K || type == TYPE_Q5_K ? 16 : type == TYPE_IQ4_XS ? 8 : 2;
}

// IQ4_XS / IQ4_NL level lookup: four 4-bit indices (one per byte, 0..15) to
// their int8 levels {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38,
// 53, 69, 89, 113} (kvalues_iq4nl, the format's table, reached by the
// reference through @cImport, src/ggml/quants/iq4.zig:12-14).  Two byte
// permutes look the index up in levels 0-7 and 8-15, a third picks per byte
// by the index's bit 3.
__device__ __forceinline__ uint32_t iq4nl_levels(uint32_t idx) {
    constexpr uint32_t T0 = 0xBFAD9881u, T1 = 0xF6EADDCFu, T2 = 0x26190D01u, T3 = 0x71594535u;
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(T3, T2, sel);
    const uint32_t pick = ((idx >> 1) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(hi, lo, pick);
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xFFFFu)));
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }
__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }


// 16 bytes at a 2-byte-aligned address, read without touching any byte
// outside [p, p+16): four dwords from the dword below p, plus a 16-bit load
// of the last two bytes (redundant when p is 4-aligned), then funnel-shifted.
__device__ __forceinline__ uint4 ld16_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 2u);
    const uint8_t *base = p - sh;
    const uint32_t a0 = ld_u32(base + 0), a1 = ld_u32(base + 4), a2 = ld_u32(base + 8), a3 = ld_u32(base + 12);
    const uint32_t t = ld_u16(p + 14);
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(a1, a0, sh);
    r.y = __builtin_amdgcn_alignbyte(a2, a1, sh);
    r.z = __builtin_amdgcn_alignbyte(a3, a2, sh);
    r.w = __builtin_amdgcn_alignbyte(t, a3, sh);
    return r;
}

// The same 16 bytes with one instruction: a memcpy from a pointer known to be
// 2-byte aligned compiles to a single global_load_dwordx4 (global memory
// accepts unaligned vector loads on gfx950).  It reads exactly [p, p+16).
// Measured faster for the MMQ's Q6_K staging loads and the Q6_K GEMV (its
// op at 4096x14336: 13.0 against 15.1 us), slower for the Q8_0 and Q4_0
// GEMVs (13.7 against 15.9 us at 4096x14336 Q8_0), where the aligned dwords
// above stay.
__device__ __forceinline__ uint4 ld16_u(const uint8_t *p) {
    uint4 r;
    __builtin_memcpy(&r, __builtin_assume_aligned(p, 2), 16);
    return r;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t byte_of(uint4 v, int i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// Sub-block j's 6-bit scale and min from block_q4_K.scales (getScaleMinK4,
// src/ggml/quants/helpers.zig:621-629).  `s` holds the 12 scale bytes in
// its low three words (.x = bytes 0..3).
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc,
                                              uint32_t &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int jj = j - 4;
        const uint32_t b8 = (s2 >> (8 * jj)) & 0xFFu;     // scales[j + 4]
        const uint32_t blo = (s0 >> (8 * jj)) & 0xFFu;    // scales[j - 4]
        const uint32_t bhi = (s1 >> (8 * jj)) & 0xFFu;    // scales[j]
        sc = (b8 & 0xFu) | ((blo >> 6) << 4);
        m = (b8 >> 4) | ((bhi >> 6) << 4);
    }
}

// Q8_1 code of one value (quantize_row_q8_1_ref, src/ggml/quants/legacy.zig:
// 451-484): roundf (half away from zero) of x * id, narrowed with the
// reference's clamping C cast (src/ggml/impl.zig:744-752).
// Branch-free.  roundf(v) is computed as trunc(v + copysign(h, v)) with h the
// float just below 0.5: the two agree for every float (checked for all
// non-negative floats below 2^24, the formula is odd in v, and above 2^24
// every float is an integer that v + h rounds back to).  The clamp is one
// v_med3_f32, NaN maps to 0 by a select, and the clamped value is integral,
// so the convert is exact.
__device__ __forceinline__ int8_t q8_1_code(float x, float id) {
    // The product is pinned in a register so that it is rounded to f32 on its
    // own, as the reference's x * id is: HIP's default contraction otherwise
    // fuses it with the add below into one FMA (one rounding of the sum),
    // which moves ties such as x * id = 63.5 - 5e-7 from 64 to 63.
    float v = x * id;
    asm volatile("" : "+v"(v));
    const float r = __builtin_truncf(v + __builtin_copysignf(0.49999997f, v));
    const float c = __builtin_amdgcn_fmed3f(r, -128.0f, 127.0f);
    return (int8_t)(int)(r == r ? c : 0.0f);
}

// Q8_1 block header: f16 d in the low half, f16 s = fp16(f32(sum * d)) in the
// high half.  The f32 product is pinned in a register before its f16
// conversion: the AMDGPU backend otherwise folds multiply + convert into
// v_fma_mixlo_f16 (one rounding, where the reference rounds to f32 first and
// then to f16), which changes `s` whenever the f32 product is an exact f16
// tie.  `#pragma clang fp contract(off)` does not stop that fold.
__device__ __forceinline__ uint32_t q8_1_pack_ds(float d, int sum) {
    float sd = (float)sum * d;
    asm volatile("" : "+v"(sd));
    const uint32_t hd = __half_as_ushort(__float2half_rn(d));
    const uint32_t hs = __half_as_ushort(__float2half_rn(sd));
    return hd | (hs << 16);
}

// Lane values of the quad partner (lane ^ 1, lane ^ 2): DPP quad_perm
// [1,0,3,2] and [2,3,0,1].
__device__ __forceinline__ float quad_x1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_x2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ int quad_x1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int quad_x2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }

// One Q8_1 block held by the 4 lanes of a quad, 8 consecutive values per lane
// (quantize_row_q8_1_ref, src/ggml/quants/legacy.zig:451-484): amax and the
// code sum take two DPP exchanges each; the max and the integer sum do not
// depend on the order, so the bytes equal a one-value-per-lane quantizer's.
// lo / hi pack this lane's 8 codes; ds is the block header (every lane).  All
// 4 lanes of the quad must be active.
struct Q8Quad {
    uint32_t lo, hi, ds;
};
__device__ __forceinline__ Q8Quad q8_1_quantize_quad(const float v[8]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, quad_x1(amax));
    amax = fmaxf(amax, quad_x2(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    Q8Quad r;
    r.lo = 0;
    r.hi = 0;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int8_t q = q8_1_code(v[i], id);
        sum += q;
        if (i < 4) r.lo |= (uint32_t)(uint8_t)q << (8 * i);
        else r.hi |= (uint32_t)(uint8_t)q << (8 * (i - 4));
    }
    sum += quad_x1(sum);
    sum += quad_x2(sum);
    r.ds = q8_1_pack_ds(d, sum);
    return r;
}

// Sum over the 64 lanes of a wavefront with DPP: an inclusive prefix sum
// inside each row of 16 lanes (row_shr 1, 2, 4, 8), then row_bcast:15 and
// row_bcast:31 carry the row totals forward, leaving the total in lane 63,
// which is broadcast.  Every lane of the wave must be active.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_or_zero(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf,
                                                                 false));
}

__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_or_zero<0x111, 0xf>(x);  // row_shr:1
    x += dpp_or_zero<0x112, 0xf>(x);  // row_shr:2
    x += dpp_or_zero<0x114, 0xf>(x);  // row_shr:4
    x += dpp_or_zero<0x118, 0xf>(x);  // row_shr:8
    x += dpp_or_zero<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    x += dpp_or_zero<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// Sums over segments of SEG consecutive lanes (16, 32 or 64) with wave_sum's
// first steps: the total of segment q lands in its last lane, (q+1)*SEG - 1,
// with the same additions in the same order as wave_sum for those lanes (at
// SEG = 64, lane 63 holds exactly wave_sum's result).
template <int SEG>
__device__ __forceinline__ float seg_sum(float x) {
    static_assert(SEG == 16 || SEG == 32 || SEG == 64, "segments of 16, 32 or 64 lanes");
    x += dpp_or_zero<0x111, 0xf>(x);  // row_shr:1
    x += dpp_or_zero<0x112, 0xf>(x);  // row_shr:2
    x += dpp_or_zero<0x114, 0xf>(x);  // row_shr:4
    x += dpp_or_zero<0x118, 0xf>(x);  // row_shr:8
    if constexpr (SEG >= 32) x += dpp_or_zero<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    if constexpr (SEG == 64) x += dpp_or_zero<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}

// ggml_glu_op values: positions in GGML_GLU_OP_NAME (src/ggml/types.zig:103-106).
enum : int {
    GLU_REGLU = 0,
    GLU_GEGLU = 1,
    GLU_SWIGLU = 2,
    GLU_SWIGLU_OAI = 3,
    GLU_SWIGLU_CLAMP = 6,
};

__host__ __device__ constexpr bool glu_op_valid(int op) {
    return op == GLU_REGLU || op == GLU_GEGLU || op == GLU_SWIGLU || op == GLU_SWIGLU_OAI || op == GLU_SWIGLU_CLAMP;
}

// out = glu(gate g, value u) for one element, as the CPU ops define it:
//   REGLU         g > 0 ? g*u : 0                      (vecinline.zig:507-511)
//   GEGLU         gelu from the f16 table: g rounded to f16, gelu of that,
//                 rounded to f16, times u; 0 at g <= -10, g*u at g >= 10
//                 (vecinline.zig:522-536; table entries convert.zig:224-260,
//                 gelu = 0.5x(1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2))) with
//                 the inner 1 + a*x*x as one fused multiply-add)
//   SWIGLU        g / (1 + exp(-g)) * u                (vec.zig:658-668)
//   SWIGLU_OAI    x = min(g, limit), y = clamp(u, -limit, limit),
//                 x / (1 + exp(alpha * -x)) * (y + 1)  (activation.zig:475-503)
//   SWIGLU_CLAMP  x = min(g, limit), y = clamp(u, -limit, limit),
//                 x / (1 + exp(-x)) * y                (activation.zig:523-548)
// min and clamp keep the C++ library's NaN behaviour (a NaN g or u passes
// through).  The host validates op.
__device__ __forceinline__ float glu_apply(int op, float g, float u, float alpha, float limit) {
    if (op == GLU_REGLU) return g > 0.0f ? g * u : 0.0f;
    if (op == GLU_GEGLU) {
        if (g <= -10.0f) return 0.0f;
        if (g >= 10.0f) return g * u;
        const float t = (float)(_Float16)g;
        const float inner = 0.79788456080286535587989211986876f * t * __builtin_fmaf(0.044715f * t, t, 1.0f);
        const float gl = 0.5f * t * (1.0f + tanhf(inner));
        return (float)(_Float16)gl * u;
    }
    if (op == GLU_SWIGLU) return g / (1.0f + expf(-g)) * u;
    const float x = limit < g ? limit : g;
    const float y = u < -limit ? -limit : (limit < u ? limit : u);
    if (op == GLU_SWIGLU_OAI) return x / (1.0f + expf(alpha * (-x))) * (y + 1.0f);
    return x / (1.0f + expf(-x)) * y;  // GLU_SWIGLU_CLAMP
}

// Tile order of a dense MMQ grid (gx row tiles x gy column tiles, one K part),
// from the workgroup's linear id L = blockIdx.x + gx * blockIdx.y.  The
// dispatcher deals consecutive workgroups to the 8 XCDs in turn, and each XCD
// has its own L2, so the workgroups of one XCD (ids L = xcd mod 8) get one
// contiguous run v of the tile sequence.  The sequence walks bands of
// MMQ_BAND row tiles: within a band every column tile in turn, and for each
// the band's row tiles, so the tiles an XCD holds at once share a few weight
// row tiles and a few activation column tiles in its L2.  A bijection of
// [0, gx*gy).
constexpr int MMQ_BAND = 8;
__device__ __forceinline__ void mmq_tile_order(int L, int gx, int gy, int &bx, int &by) {
    const int n = gx * gy, q = n >> 3, r = n & 7, xcd = L & 7, slot = L >> 3;
    const int v = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
    const int band = v / (MMQ_BAND * gy), idx = v - band * (MMQ_BAND * gy);
    const int rows = gx - band * MMQ_BAND < MMQ_BAND ? gx - band * MMQ_BAND : MMQ_BAND;
    bx = band * MMQ_BAND + idx % rows;
    by = idx / rows;
}

// Gate/up/GLU fusion of the MMQ kernels (the reference's mul_mat_q with a
// gate, src/ggml/cuda/mmq.zig:568-640).  With gate != nullptr a 128-row tile
// holds 64 output rows: tile row t reads output row 2 * (t / 4) + t % 2 of the
// tile from the gate weights (t % 4 < 2) or the up weights (t % 4 >= 2).  A
// 32x32 MFMA result gives lane half h rows 8q + 4h + i (i = 0..3), so each
// lane holds gate (i = 0, 1) and up (i = 2, 3) of the same two output rows,
// and the epilogue writes glu(gate, up) without any exchange.
struct MmqGlu {
    const uint8_t *gate;
    int op;
    float alpha, limit;
};

__device__ __forceinline__ int mmq_glu_tile_row(int t) { return 2 * (t >> 2) + (t & 1); }

// One lane's 8 fused outputs of a 32x32 tile column: rows r0 + 4q + {0, 1}
// (q = 0..3) of the column at o, from accumulators a[4q + i].
template <typename V>
__device__ __forceinline__ void store_glu_column(float *o, int64_t r0, int64_t nrows, const V &a, const MmqGlu &g) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float v0 = glu_apply(g.op, a[4 * q], a[4 * q + 2], g.alpha, g.limit);
        const float v1 = glu_apply(g.op, a[4 * q + 1], a[4 * q + 3], g.alpha, g.limit);
        const int64_t r = r0 + 4 * q;
        if (((uintptr_t)(o + r) & 7) == 0 && r + 1 < nrows) {
            *reinterpret_cast<float2 *>(o + r) = make_float2(v0, v1);
        } else {
            if (r < nrows) o[r] = v0;
            if (r + 1 < nrows) o[r + 1] = v1;
        }
    }
}

}  // namespace qmm
