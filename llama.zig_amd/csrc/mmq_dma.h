// mmq_dma.h -- pieces shared by the MMQ kernels fed by direct global->LDS
// loads (mmq_q4k_dma.hip, mmq_q5k_dma.hip, mmq_legacy_dma.hip,
// mmq_iq4xs_dma.hip): the workgroup shape, the MFMA operand types, the
// 16-byte transfer, its wait, and the tile-column store.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm_dma {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void *lds_ptr;

constexpr int BM = 128;        // weight rows per workgroup tile: four waves of 32
constexpr int NTHREADS = 256;

__device__ __forceinline__ uint32_t f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// 16 bytes per lane from global memory to LDS at base + 16 * lane (base is
// wave-uniform).
__device__ __forceinline__ void dma16(const void *g, void *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds_base, 16, 0, 0);
}

__device__ __forceinline__ void wait_vmem() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt / lgkmcnt not waited
}

// Expert-grouped (MUL_MAT_ID) mode of the dense direct-transfer kernels:
// workgroup (x, y) takes row tile x of column tile y of the device tile table
// {expert, col_low, col_high, -} (mmid.hip's grouping; workgroups past
// *n_tiles exit at once).  Its activation columns are gathered through
// col_src and its output columns scattered through col_dst (dst's column
// stride is then the output row stride).  No K split.
struct MmqGroups {
    const int32_t *tiles, *n_tiles, *col_src, *col_dst;
    int64_t expert_stride;
};

// One lane's 16 outputs of a 32x32 MFMA tile (column fixed, rows r0 + 8q +
// 0..3 for q = 0..3, r0 a multiple of 4) into the column at o: four 16-byte
// stores when the column is 16-byte aligned and all rows are below nrows,
// else one store per row below nrows.
__device__ __forceinline__ void store_tile_column(float *o, int64_t r0, int64_t nrows, const v16f &a) {
    if (((uintptr_t)(o + r0) & 15) == 0 && r0 + 27 < nrows) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<float4 *>(o + r0 + 8 * q) = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
    } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
            if (r < nrows) o[r] = a[v];
        }
    }
}

}  // namespace qmm_dma
