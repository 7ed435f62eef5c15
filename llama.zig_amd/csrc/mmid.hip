// mmid.hip -- MUL_MAT_ID (mixture-of-experts) on the GPU without a host
// round trip: a grouping kernel builds, on the device, the per-expert lists
// of routed (token, slot) pairs and the table of column tiles, and the
// expert-grouped MMQ consumes them.
//
// Semantics follow ggml_compute_forward_mul_mat_id
// (src/ggml/cpu/mulmat.zig:555-777): dst row (t, s) = W[ids[t][s]] x
// x[t][s % ne11]; an id of -1 leaves a zero row (mulmat.zig:670-676).  The
// reference's CUDA path builds the same grouping with mm_ids_helper
// (src/ggml/cuda/mmid.zig:32-90) and, for larger batches, falls back to a
// host-synchronising sort (cuda/mulmat.zig:728-800); this path never syncs.
// Ids outside [-1, n_as) are treated as -1 (zero row) rather than read out
// of bounds.
#include "../../include/ggml_hip_qmm.h"
#include "qmm_device.h"

using namespace qmm;

extern "C" int hip_qmm_mmq_grouped(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                   int64_t expert_stride, const int8_t *y_qs, const void *y_ds, float *dst,
                                   int64_t dst_row_stride, int bn, int64_t max_tiles, const int32_t *tiles,
                                   const int32_t *n_tiles, const int32_t *col_src, const int32_t *col_dst,
                                   void *stream);

namespace {

constexpr int MAX_EXPERTS = 1024;
constexpr int PREP_THREADS = 256;
constexpr int IDS_PER_THREAD = 16;                          // consecutive pairs per thread and chunk
constexpr int CHUNK = PREP_THREADS * IDS_PER_THREAD;        // pairs per chunk
constexpr int QUANT_VALS = PREP_THREADS * 8;                // K values one quantizing workgroup covers

// Exclusive prefix sum of one value per thread over the workgroup, with the
// total.  `buf` is PREP_THREADS / 64 ints of LDS; ends with a barrier.
__device__ __forceinline__ int block_excl_scan(int a, int &total, int *buf) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int ia = a;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(ia, off);
        if (lane >= off) ia += u;
    }
    if (lane == 63) buf[wave] = ia;
    __syncthreads();
    int pre = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < PREP_THREADS / 64; ++w) {
        const int v = buf[w];
        if (w < wave) pre += v;
        total += v;
    }
    __syncthreads();  // buf may be reused by the caller's next scan
    return pre + ia - a;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP (row_shr 1, 2, 4, 8
// inside rows of 16, then row_bcast:15 and row_bcast:31 carry the row totals
// forward).  Every lane of the wave must be active.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
    return x;
}

// Exclusive prefix sum of one value per thread over the workgroup, with the
// total, on DPP wave scans and one barrier.  `buf` is PREP_THREADS / 64 ints of
// LDS that no other thread reads or writes until the caller's next barrier
// (consecutive calls alternate two buffers).
__device__ __forceinline__ int block_excl_scan_dpp(int a, int &total, int *buf) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int incl = wave_incl_scan(a);
    if (lane == 63) buf[wave] = incl;
    __syncthreads();
    int pre = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < PREP_THREADS / 64; ++w) {
        const int v = buf[w];
        if (w < wave) pre += v;
        total += v;
    }
    return pre + incl - a;
}

// Most chunks of CHUNK pairs the register path of the grouping keeps.
constexpr int FAST_CHUNKS = 4;

// One launch that prepares a MUL_MAT_ID: workgroups [0, n_group) build the
// expert grouping, the rest quantize the activation rows to planar Q8_1 (the
// 8-values-per-lane form of quantize_q8_1.hip); the two parts are independent.
//
// Grouping, in the shape of the reference's mm_ids_helper (one block per
// expert, src/ggml/cuda/mmid.zig:30-70): every grouping workgroup counts the
// pairs of all experts (the ids are a few KB, read from L2 by all of them),
// scans the counts into column and tile offsets, and then writes, for its own
// experts e = g, g + n_group, ..., the pairs routed to e in pair order
// (col_src: activation row, col_dst: output row) and e's column tiles
// {expert, col_low, col_high, 0}.  Workgroup 0 also writes the tile count.
// Pairs whose id is -1 or out of
// [0, n_as) get a zero output row (mulmat.zig:670-676), written by one thread
// of the grouping workgroups.  The result does not depend on scheduling:
// every position is a function of the ids alone.
__global__ __launch_bounds__(PREP_THREADS) void mmid_prepare(
    const int32_t *__restrict__ ids, int64_t ids_stride, int64_t n_tokens, int64_t n_ids, int n_as, int64_t ne11,
    int bn, int n_group, int32_t *__restrict__ col_src, int32_t *__restrict__ col_dst,
    int32_t *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    float *__restrict__ dst, int64_t dst_row_stride, int64_t nrows, const float *__restrict__ x, int64_t K,
    int64_t x_row_stride, int64_t Kp, int nq_per_row, int rows_per_wg, int64_t nrows_x, int8_t *__restrict__ qs,
    uint32_t *__restrict__ ds) {
    const int tid = threadIdx.x;
    if ((int)blockIdx.x >= n_group) {
        // quantize: workgroup (row, K slice of QUANT_VALS values), or for rows
        // shorter than QUANT_VALS, rows_per_wg whole rows; Kp is a multiple of
        // 512, so a quad (one 32-block) is wholly inside one row and inside or
        // past Kp
        const int b = (int)blockIdx.x - n_group;
        int64_t c, k;
        if (rows_per_wg > 1) {
            c = (int64_t)b * rows_per_wg + (tid * 8) / Kp;
            k = (tid * 8) % Kp;
            if (c >= nrows_x || (tid * 8) / Kp >= rows_per_wg) return;
        } else {
            c = b / nq_per_row;
            k = (int64_t)(b - c * nq_per_row) * QUANT_VALS + tid * 8;
            if (k >= Kp) return;
        }
        float v[8];
        if (k < K) {  // K % 32 == 0
            const float4 a0 = *reinterpret_cast<const float4 *>(x + c * x_row_stride + k);
            const float4 a1 = *reinterpret_cast<const float4 *>(x + c * x_row_stride + k + 4);
            v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
            v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        const Q8Quad r = q8_1_quantize_quad(v);
        *reinterpret_cast<uint2 *>(qs + c * Kp + k) = make_uint2(r.lo, r.hi);
        if ((tid & 3) == 0) ds[c * (Kp / QK8) + k / QK8] = r.ds;
        return;
    }

    __shared__ int count[MAX_EXPERTS];
    __shared__ int coff[MAX_EXPERTS], toff[MAX_EXPERTS];
    __shared__ int sbuf[2][PREP_THREADS / 64];
    const int g = (int)blockIdx.x;
    // pair indices fit in 32 bits (checked by the host): 32-bit division
    const uint32_t npairs = (uint32_t)(n_tokens * n_ids), nid = (uint32_t)n_ids;
    const bool dense_ids = ids_stride == n_ids;  // uniform; the usual layout, no division per id
    auto id_of = [&](uint32_t p) -> int {
        int e;
        if (dense_ids) {
            e = ids[p];
        } else {
            const uint32_t t = p / nid;
            e = ids[(int64_t)t * ids_stride + (p - t * nid)];
        }
        return e >= 0 && e < n_as ? e : -1;
    };

    // Register path (up to FAST_CHUNKS chunks of pairs, at most PREP_THREADS
    // experts; uniform): the ids are read once, IDS_PER_THREAD consecutive pairs
    // per thread and chunk, and counting, placement and the zero rows all work
    // from registers; the column and tile offsets come from one scan of both
    // counts packed in 16-bit fields (both totals stay below 2^16 here).  Same
    // results as the general path below: positions depend on the ids alone.
    if (npairs <= (uint32_t)(FAST_CHUNKS * CHUNK) && n_as <= PREP_THREADS) {
        const int nch = (int)((npairs + CHUNK - 1) / CHUNK);
        int ev[FAST_CHUNKS][IDS_PER_THREAD];
#pragma unroll
        for (int c = 0; c < FAST_CHUNKS; ++c) {
            const uint32_t p0 = (uint32_t)c * CHUNK + (uint32_t)tid * IDS_PER_THREAD;
            if (c < nch) {
                if (dense_ids && p0 + IDS_PER_THREAD <= npairs && ((uintptr_t)(ids + p0) & 15) == 0) {
#pragma unroll
                    for (int q = 0; q < IDS_PER_THREAD / 4; ++q) {
                        const int4 v = *reinterpret_cast<const int4 *>(ids + p0 + 4 * q);
                        ev[c][4 * q] = v.x; ev[c][4 * q + 1] = v.y; ev[c][4 * q + 2] = v.z; ev[c][4 * q + 3] = v.w;
                    }
#pragma unroll
                    for (int k = 0; k < IDS_PER_THREAD; ++k) ev[c][k] = ev[c][k] >= 0 && ev[c][k] < n_as ? ev[c][k] : -1;
                } else {
#pragma unroll
                    for (int k = 0; k < IDS_PER_THREAD; ++k) {
                        const uint32_t p = p0 + (uint32_t)k;
                        ev[c][k] = p < npairs ? id_of(p) : -2;  // -2: past the end
                    }
                }
            }
        }
        if (tid < n_as) count[tid] = 0;
        __syncthreads();
#pragma unroll
        for (int c = 0; c < FAST_CHUNKS; ++c)
            if (c < nch)
#pragma unroll
                for (int k = 0; k < IDS_PER_THREAD; ++k)
                    if (ev[c][k] >= 0) atomicAdd(&count[ev[c][k]], 1);
        __syncthreads();
        const int ce_t = tid < n_as ? count[tid] : 0;
        const int packed = ce_t | (((ce_t + bn - 1) / bn) << 16);
        int tot;
        const int pre = block_excl_scan_dpp(packed, tot, sbuf[0]);
        if (tid < n_as) {
            coff[tid] = pre & 0xFFFF;
            toff[tid] = pre >> 16;
        }
        __syncthreads();
        if (g == 0 && tid == 0) *n_tiles = tot >> 16;
        for (int e = g; e < n_as; e += n_group) {
            const int ce = count[e], c0 = coff[e], t0 = toff[e];
            for (int i = tid; i * bn < ce; i += PREP_THREADS) {
                const int lo = c0 + i * bn, hi = lo + bn < c0 + ce ? lo + bn : c0 + ce;
                *reinterpret_cast<int4 *>(tiles + 4 * (t0 + i)) = make_int4(e, lo, hi, 0);
            }
            int pos = c0;
#pragma unroll
            for (int c = 0; c < FAST_CHUNKS; ++c) {
                if (c >= nch) break;  // uniform
                uint32_t mask = 0;
#pragma unroll
                for (int k = 0; k < IDS_PER_THREAD; ++k) mask |= (ev[c][k] == e ? 1u : 0u) << k;
                int ctot;
                int at = pos + block_excl_scan_dpp(__builtin_popcount(mask), ctot, sbuf[(c + 1) & 1]);
                const uint32_t p0 = (uint32_t)c * CHUNK + (uint32_t)tid * IDS_PER_THREAD, n11 = (uint32_t)ne11;
                while (mask) {
                    const int k = __builtin_ctz(mask);
                    mask &= mask - 1;
                    const uint32_t p = p0 + k, t = p / nid, sl = p - t * nid;
                    col_src[at] = (int32_t)(t * n11 + (n11 == 1 ? 0u : sl));
                    col_dst[at] = (int32_t)p;
                    ++at;
                }
                pos += ctot;
            }
        }
        // zero rows for invalid ids: thread slot (c, tid) belongs to grouping
        // workgroup (c * PREP_THREADS + tid) % n_group
#pragma unroll
        for (int c = 0; c < FAST_CHUNKS; ++c) {
            if (c >= nch || (c * PREP_THREADS + tid) % n_group != g) continue;
#pragma unroll
            for (int k = 0; k < IDS_PER_THREAD; ++k) {
                if (ev[c][k] != -1) continue;
                float *row = dst + (int64_t)((uint32_t)c * CHUNK + (uint32_t)tid * IDS_PER_THREAD + k) * dst_row_stride;
                for (int64_t r = 0; r < nrows; ++r) row[r] = 0.0f;
            }
        }
        return;
    }
    for (int e = tid; e < n_as; e += PREP_THREADS) count[e] = 0;
    __syncthreads();
    // ids of pair p, or -1 past the end; the loads are unconditional (index
    // clamped) so that a thread's loads are all in flight before the first use
    auto id_or_none = [&](uint32_t p) -> int {
        const int e = id_of(p < npairs ? p : npairs - 1);
        return p < npairs ? e : -1;
    };
    for (uint32_t base = 0; base < npairs; base += CHUNK) {
        int ev[IDS_PER_THREAD];
#pragma unroll
        for (int k = 0; k < IDS_PER_THREAD; ++k) ev[k] = id_or_none(base + (uint32_t)k * PREP_THREADS + tid);
#pragma unroll
        for (int k = 0; k < IDS_PER_THREAD; ++k)
            if (ev[k] >= 0) atomicAdd(&count[ev[k]], 1);
    }
    __syncthreads();
    // column and tile offsets of every expert: each thread scans a run of
    // consecutive experts, then the runs are scanned across the workgroup
    constexpr int EPT = MAX_EXPERTS / PREP_THREADS;
    int c_run = 0, t_run = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid * EPT + i;
        if (e < n_as) {
            c_run += count[e];
            t_run += (count[e] + bn - 1) / bn;
        }
    }
    int c_tot, t_tot;
    int c_pre = block_excl_scan(c_run, c_tot, sbuf[0]);
    int t_pre = block_excl_scan(t_run, t_tot, sbuf[0]);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid * EPT + i;
        if (e < n_as) {
            coff[e] = c_pre;
            toff[e] = t_pre;
            c_pre += count[e];
            t_pre += (count[e] + bn - 1) / bn;
        }
    }
    __syncthreads();
    if (g == 0 && tid == 0) *n_tiles = t_tot;
    for (int e = g; e < n_as; e += n_group) {
        const int ce = count[e], c0 = coff[e], t0 = toff[e];
        for (int i = tid; i * bn < ce; i += PREP_THREADS) {
            const int lo = c0 + i * bn, hi = lo + bn < c0 + ce ? lo + bn : c0 + ce;
            *reinterpret_cast<int4 *>(tiles + 4 * (t0 + i)) = make_int4(e, lo, hi, 0);
        }
        // e's pairs in pair order: thread tid takes IDS_PER_THREAD consecutive
        // pairs of each chunk, counts its matches and scans for its position
        int pos = c0;
        for (uint32_t base = 0; base < npairs; base += CHUNK) {
            const uint32_t p0 = base + (uint32_t)tid * IDS_PER_THREAD;
            int ev[IDS_PER_THREAD];
#pragma unroll
            for (int k = 0; k < IDS_PER_THREAD; ++k) ev[k] = id_or_none(p0 + k);
            uint32_t mask = 0;
#pragma unroll
            for (int k = 0; k < IDS_PER_THREAD; ++k) mask |= (ev[k] == e ? 1u : 0u) << k;
            int tot;
            int at = pos + block_excl_scan(__builtin_popcount(mask), tot, sbuf[0]);
            const uint32_t n11 = (uint32_t)ne11;  // 1 or n_ids
            while (mask) {
                const int k = __builtin_ctz(mask);
                mask &= mask - 1;
                const uint32_t p = p0 + k, t = p / nid, sl = p - t * nid;
                col_src[at] = (int32_t)(t * n11 + (n11 == 1 ? 0u : sl));
                col_dst[at] = (int32_t)p;
                ++at;
            }
            pos += tot;
        }
    }
    // zero rows for invalid ids: one pair per thread, the pairs spread over
    // the grouping workgroups (independent loads, no chain of round trips)
    for (uint32_t p = (uint32_t)g * PREP_THREADS + tid; p < npairs; p += (uint32_t)n_group * PREP_THREADS) {
        if (id_of(p) >= 0) continue;
        float *row = dst + (int64_t)p * dst_row_stride;
        for (int64_t r = 0; r < nrows; ++r) row[r] = 0.0f;
    }
}

struct MmidLayout {
    int64_t Kp, nrows_x, npairs, max_tiles;
    size_t off_qs, off_ds, off_src, off_dst, off_tiles, off_ntiles, total;
};

MmidLayout layout(int64_t K, int64_t n_as, int64_t ne11, int64_t n_tokens, int64_t n_ids, int bn) {
    MmidLayout L;
    L.Kp = pad_k(K);
    L.nrows_x = ne11 * n_tokens;
    L.npairs = n_tokens * n_ids;
    L.max_tiles = (L.npairs + bn - 1) / bn + n_as;
    auto a256 = [](size_t v) { return (v + 255) / 256 * 256; };
    size_t o = 0;
    L.off_qs = o;     o = a256(o + (size_t)(L.nrows_x * L.Kp));
    L.off_ds = o;     o = a256(o + (size_t)(L.nrows_x * (L.Kp / QK8)) * 4);
    L.off_src = o;    o = a256(o + (size_t)L.npairs * 4);
    L.off_dst = o;    o = a256(o + (size_t)L.npairs * 4);
    L.off_tiles = o;  o = a256(o + (size_t)L.max_tiles * 16);
    L.off_ntiles = o; o = a256(o + 4);
    L.total = o;
    return L;
}

// Column-tile width for the grouped GEMM: the mean number of columns per
// expert picks the narrowest tile that is not mostly empty.
int grouped_bn(int64_t npairs, int64_t n_as) {
    const int64_t mean = (npairs + n_as - 1) / n_as;
    return mean <= 32 ? 32 : 64;
}

}  // namespace

extern "C" size_t hip_qmm_mul_mat_id_workspace_size(int type, int64_t K, int64_t n_as, int64_t ne11,
                                                    int64_t n_tokens, int64_t n_ids) {
    (void)type;
    if (K <= 0 || n_as <= 0 || ne11 <= 0 || n_tokens <= 0 || n_ids <= 0) return 0;
    return layout(K, n_as, ne11, n_tokens, n_ids, grouped_bn(n_tokens * n_ids, n_as)).total;
}

namespace {

// MUL_MAT_ID, and with w_gate its gate/up/GLU fusion (glu_op etc. unused
// without it).
int mul_mat_id(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows, int64_t row_stride,
               int64_t expert_stride, int64_t n_as, const float *x, int64_t ne11, int64_t n_tokens,
               int64_t x_row_stride, const int32_t *ids, int64_t n_ids, int64_t ids_stride, int glu_op,
               float glu_alpha, float glu_limit, float *dst, int64_t dst_row_stride, void *workspace,
               size_t workspace_size, void *stream) {
    if (!w || !x || !ids || !dst || !workspace || K <= 0 || nrows <= 0 || n_as <= 0 || n_as > MAX_EXPERTS ||
        ne11 <= 0 || n_tokens <= 0 || n_ids <= 0 || ids_stride < n_ids || dst_row_stride < nrows ||
        x_row_stride < K || expert_stride < nrows * row_stride)
        return (int)hipErrorInvalidValue;
    if (ne11 != 1 && ne11 != n_ids) return (int)hipErrorInvalidValue;  // ggml_mul_mat_id's b.ne1 rule
    if (n_tokens * n_ids > 0x7FFFFFFF || n_tokens * ne11 > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    // Up to 8 tokens (the reference's MMVQ-with-ids limit on AMD,
    // mmvq.zig:116-125): one GEMV launch over the (token, slot) pairs, each
    // quantizing its own column in LDS; no grouping, no workspace used.
    const int64_t walign = block_align(type);
    if (n_tokens <= 8 && n_tokens * n_ids <= 65535 && K % 32 == 0 && K <= 32768 && (uintptr_t)x % 16 == 0 &&
        x_row_stride % 4 == 0 && expert_stride % walign == 0)
        return hip_qmm_mul_mat_id_vec_fused(type, w, w_gate, K, nrows, row_stride, expert_stride, n_as, x, ne11,
                                            n_tokens, x_row_stride, ids, n_ids, ids_stride, glu_op, glu_alpha,
                                            glu_limit, dst, dst_row_stride, stream);
    const int bn = grouped_bn(n_tokens * n_ids, n_as);
    const MmidLayout L = layout(K, n_as, ne11, n_tokens, n_ids, bn);
    if (workspace_size < L.total || (uintptr_t)workspace % 256) return (int)hipErrorInvalidValue;
    if (L.max_tiles > 65535) return (int)hipErrorInvalidValue;
    uint8_t *ws = (uint8_t *)workspace;
    int8_t *qs = (int8_t *)(ws + L.off_qs);
    void *ds = ws + L.off_ds;
    int32_t *col_src = (int32_t *)(ws + L.off_src), *col_dst = (int32_t *)(ws + L.off_dst);
    int32_t *tiles = (int32_t *)(ws + L.off_tiles);
    int32_t *ntiles = (int32_t *)(ws + L.off_ntiles);
    hipStream_t s = (hipStream_t)stream;

    const int n_group = n_as < 256 ? (int)n_as : 256;
    if ((uintptr_t)x % 16 == 0 && x_row_stride % 4 == 0 && K % QK8 == 0) {
        // one launch: grouping and quantization
        const int nq_per_row = (int)((L.Kp + QUANT_VALS - 1) / QUANT_VALS);
        // short rows (Kp < QUANT_VALS): whole rows per workgroup
        const int rows_per_wg = L.Kp < QUANT_VALS ? (int)(QUANT_VALS / L.Kp) : 1;
        const int64_t nq = rows_per_wg > 1 ? (L.nrows_x + rows_per_wg - 1) / rows_per_wg : L.nrows_x * nq_per_row;
        const int64_t nwg = n_group + nq;
        if (nwg > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
        hipLaunchKernelGGL(mmid_prepare, dim3((unsigned)nwg), dim3(PREP_THREADS), 0, s, ids, ids_stride, n_tokens,
                           n_ids, (int)n_as, ne11, bn, n_group, col_src, col_dst, tiles, ntiles, dst,
                           dst_row_stride, nrows, x, K, x_row_stride, L.Kp, nq_per_row, rows_per_wg, L.nrows_x, qs,
                           (uint32_t *)ds);
    } else {
        if (int e = hip_qmm_quantize_q8_1_planar(x, K, L.nrows_x, x_row_stride, qs, ds, stream)) return e;
        hipLaunchKernelGGL(mmid_prepare, dim3((unsigned)n_group), dim3(PREP_THREADS), 0, s, ids, ids_stride, n_tokens,
                           n_ids, (int)n_as, ne11, bn, n_group, col_src, col_dst, tiles, ntiles, dst,
                           dst_row_stride, nrows, x, K, x_row_stride, L.Kp, 1, 1, L.nrows_x, qs, (uint32_t *)ds);
    }
    if (int e = (int)hipGetLastError()) return e;
    if (w_gate)
        return hip_qmm_mmq_grouped_glu(type, w, w_gate, K, nrows, row_stride, expert_stride, qs, ds, dst,
                                       dst_row_stride, bn, L.max_tiles, tiles, ntiles, col_src, col_dst, glu_op,
                                       glu_alpha, glu_limit, stream);
    return hip_qmm_mmq_grouped(type, w, K, nrows, row_stride, expert_stride, qs, ds, dst, dst_row_stride, bn,
                               L.max_tiles, tiles, ntiles, col_src, col_dst, stream);
}

}  // namespace

extern "C" int hip_qmm_mul_mat_id(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                  int64_t expert_stride, int64_t n_as, const float *x, int64_t ne11,
                                  int64_t n_tokens, int64_t x_row_stride, const int32_t *ids, int64_t n_ids,
                                  int64_t ids_stride, float *dst, int64_t dst_row_stride, void *workspace,
                                  size_t workspace_size, void *stream) {
    return mul_mat_id(type, w, nullptr, K, nrows, row_stride, expert_stride, n_as, x, ne11, n_tokens, x_row_stride,
                      ids, n_ids, ids_stride, 0, 0.0f, 0.0f, dst, dst_row_stride, workspace, workspace_size, stream);
}

// Gate/up/GLU over the routed pairs (the reference's MUL_MAT_ID fusion,
// src/ggml/cuda/fusion.zig:1153-1306 into mmvq or mmq with ids): the same
// grouping and one Q8_1 copy feed both weights; dst row (t, s) =
// glu(Wg_e . x, W_e . x), a zero row for an id outside [0, n_as).
extern "C" int hip_qmm_mul_mat_id_glu(int type, const void *w, const void *w_gate, int64_t K, int64_t nrows,
                                      int64_t row_stride, int64_t expert_stride, int64_t n_as, const float *x,
                                      int64_t ne11, int64_t n_tokens, int64_t x_row_stride, const int32_t *ids,
                                      int64_t n_ids, int64_t ids_stride, int glu_op, float glu_alpha,
                                      float glu_limit, float *dst, int64_t dst_row_stride, void *workspace,
                                      size_t workspace_size, void *stream) {
    if (!w_gate || !glu_op_valid(glu_op)) return (int)hipErrorInvalidValue;
    return mul_mat_id(type, w, w_gate, K, nrows, row_stride, expert_stride, n_as, x, ne11, n_tokens, x_row_stride,
                      ids, n_ids, ids_stride, glu_op, glu_alpha, glu_limit, dst, dst_row_stride, workspace,
                      workspace_size, stream);
}
