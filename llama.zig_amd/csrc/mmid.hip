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
                                   const int32_t *n_tiles, const int32_t *expert_off, const int32_t *col_src,
                                   const int32_t *col_dst, void *stream);

namespace {

constexpr int GROUP_THREADS = 1024;
constexpr int MAX_EXPERTS = 1024;

constexpr int IDS_PER_THREAD = 16;  // ids held in registers between the passes

// Exclusive prefix sums of two per-thread values over the workgroup (thread i
// holds the values of expert i), with the totals.
__device__ __forceinline__ void block_excl_scan2(int &a, int &b, int &tot_a, int &tot_b) {
    __shared__ int wa[GROUP_THREADS / 64], wb[GROUP_THREADS / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int ia = a, ib = b;  // inclusive scans inside the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int ua = __shfl_up(ia, off), ub = __shfl_up(ib, off);
        if (lane >= off) {
            ia += ua;
            ib += ub;
        }
    }
    if (lane == 63) {
        wa[wave] = ia;
        wb[wave] = ib;
    }
    __syncthreads();
    int pa = 0, pb = 0;
    tot_a = 0;
    tot_b = 0;
    for (int w = 0; w < GROUP_THREADS / 64; ++w) {
        if (w < wave) {
            pa += wa[w];
            pb += wb[w];
        }
        tot_a += wa[w];
        tot_b += wb[w];
    }
    a = pa + ia - a;
    b = pb + ib - b;
}

// One workgroup.  Every thread first loads its ids into registers (all loads
// in flight at once); pass 1 counts the pairs routed to each expert (LDS
// atomics); parallel exclusive scans give each expert its column range and
// its tile range, and thread e writes expert e's tiles; pass 2 places every
// pair at its expert's cursor.  The order of pairs inside an expert's range is
// whatever the atomics give: each pair writes its own output row, so the
// order does not change any result.
__global__ __launch_bounds__(GROUP_THREADS) void mmid_group(
    const int32_t *__restrict__ ids, int64_t ids_stride, int64_t n_tokens, int64_t n_ids, int n_as, int64_t ne11,
    int bn, int32_t *__restrict__ col_src, int32_t *__restrict__ col_dst, int32_t *__restrict__ expert_off,
    int32_t *__restrict__ tiles, int32_t *__restrict__ n_tiles, float *__restrict__ dst, int64_t dst_row_stride,
    int64_t nrows) {
    __shared__ int count[MAX_EXPERTS];
    __shared__ int cursor[MAX_EXPERTS];
    // pair indices fit in 32 bits (checked by the host): 32-bit division
    // instead of the much longer 64-bit sequence
    const uint32_t npairs = (uint32_t)(n_tokens * n_ids), nid = (uint32_t)n_ids;
    const int tid = threadIdx.x;
    auto id_of = [&](uint32_t p) -> int {
        const uint32_t t = p / nid;
        const int e = ids[(int64_t)t * ids_stride + (p - t * nid)];
        return e >= 0 && e < n_as ? e : -1;
    };
    int eid[IDS_PER_THREAD];
#pragma unroll
    for (int k = 0; k < IDS_PER_THREAD; ++k) {
        const uint32_t p = tid + (uint32_t)k * GROUP_THREADS;
        eid[k] = p < npairs ? id_of(p) : -1;
    }
    for (int e = tid; e < n_as; e += GROUP_THREADS) count[e] = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < IDS_PER_THREAD; ++k)
        if (eid[k] >= 0) atomicAdd(&count[eid[k]], 1);
    for (uint32_t p = tid + (uint32_t)IDS_PER_THREAD * GROUP_THREADS; p < npairs; p += GROUP_THREADS) {
        const int e = id_of(p);
        if (e >= 0) atomicAdd(&count[e], 1);
    }
    __syncthreads();
    {
        int c = tid < n_as ? count[tid] : 0;
        int nt = (c + bn - 1) / bn;
        const int nt_own = nt;
        int total_c, total_t;
        block_excl_scan2(c, nt, total_c, total_t);
        if (tid < n_as) {
            cursor[tid] = c;
            expert_off[tid] = c;
            for (int i = 0; i < nt_own; ++i) {
                tiles[2 * (nt + i)] = tid;
                tiles[2 * (nt + i) + 1] = c + i * bn;
            }
        }
        if (tid == 0) {
            expert_off[n_as] = total_c;
            *n_tiles = total_t;
        }
    }
    __syncthreads();
    const uint32_t n11 = (uint32_t)ne11;  // 1 or n_ids
    auto place = [&](uint32_t p, int e) {
        if (e >= 0) {
            const int pos = atomicAdd(&cursor[e], 1);
            const uint32_t t = p / nid, sl = p - t * nid;
            col_src[pos] = (int32_t)(t * n11 + (n11 == 1 ? 0u : sl));
            col_dst[pos] = (int32_t)p;
        } else {
            float *row = dst + (int64_t)p * dst_row_stride;
            for (int64_t r = 0; r < nrows; ++r) row[r] = 0.0f;
        }
    };
#pragma unroll
    for (int k = 0; k < IDS_PER_THREAD; ++k) {
        const uint32_t p = tid + (uint32_t)k * GROUP_THREADS;
        if (p < npairs) place(p, eid[k]);
    }
    for (uint32_t p = tid + (uint32_t)IDS_PER_THREAD * GROUP_THREADS; p < npairs; p += GROUP_THREADS) place(p, id_of(p));
}

struct MmidLayout {
    int64_t Kp, nrows_x, npairs, max_tiles;
    size_t off_qs, off_ds, off_src, off_dst, off_eoff, off_tiles, off_ntiles, total;
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
    L.off_eoff = o;   o = a256(o + (size_t)(n_as + 1) * 4);
    L.off_tiles = o;  o = a256(o + (size_t)L.max_tiles * 8);
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

extern "C" int hip_qmm_mul_mat_id(int type, const void *w, int64_t K, int64_t nrows, int64_t row_stride,
                                  int64_t expert_stride, int64_t n_as, const float *x, int64_t ne11,
                                  int64_t n_tokens, int64_t x_row_stride, const int32_t *ids, int64_t n_ids,
                                  int64_t ids_stride, float *dst, int64_t dst_row_stride, void *workspace,
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
        return hip_qmm_mul_mat_id_vec_fused(type, w, nullptr, K, nrows, row_stride, expert_stride, n_as, x, ne11,
                                            n_tokens, x_row_stride, ids, n_ids, ids_stride, 0, 0.0f, 0.0f, dst,
                                            dst_row_stride, stream);
    const int bn = grouped_bn(n_tokens * n_ids, n_as);
    const MmidLayout L = layout(K, n_as, ne11, n_tokens, n_ids, bn);
    if (workspace_size < L.total || (uintptr_t)workspace % 256) return (int)hipErrorInvalidValue;
    if (L.max_tiles > 65535) return (int)hipErrorInvalidValue;
    uint8_t *ws = (uint8_t *)workspace;
    int8_t *qs = (int8_t *)(ws + L.off_qs);
    void *ds = ws + L.off_ds;
    int32_t *col_src = (int32_t *)(ws + L.off_src), *col_dst = (int32_t *)(ws + L.off_dst);
    int32_t *eoff = (int32_t *)(ws + L.off_eoff), *tiles = (int32_t *)(ws + L.off_tiles);
    int32_t *ntiles = (int32_t *)(ws + L.off_ntiles);
    hipStream_t s = (hipStream_t)stream;

    if (int e = hip_qmm_quantize_q8_1_planar(x, K, L.nrows_x, x_row_stride, qs, ds, stream)) return e;
    hipLaunchKernelGGL(mmid_group, dim3(1), dim3(GROUP_THREADS), 0, s, ids, ids_stride, n_tokens, n_ids, (int)n_as,
                       ne11, bn, col_src, col_dst, eoff, tiles, ntiles, dst, dst_row_stride, nrows);
    if (int e = (int)hipGetLastError()) return e;
    return hip_qmm_mmq_grouped(type, w, K, nrows, row_stride, expert_stride, qs, ds, dst, dst_row_stride, bn,
                               L.max_tiles, tiles, ntiles, eoff, col_src, col_dst, stream);
}
