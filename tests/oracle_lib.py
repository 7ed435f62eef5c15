"""ctypes wrapper around oracle/liborc_qmm.so -- the CPU checker.

Test infrastructure: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg only.
"""
import ctypes
import os
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = ROOT / "oracle" / "liborc_qmm.so"

TYPE_F32, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q8_1, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_K = 0, 2, 8, 9, 12, 13, 14, 15
TYPE_IQ4_XS = 23
TYPE_IDS = {"Q4_0": TYPE_Q4_0, "Q8_0": TYPE_Q8_0, "Q8_1": TYPE_Q8_1, "Q4_K": TYPE_Q4_K, "Q5_K": TYPE_Q5_K, "Q6_K": TYPE_Q6_K,
            "Q8_K": TYPE_Q8_K, "IQ4_XS": TYPE_IQ4_XS}
BLOCK = {TYPE_Q4_0: (32, 18), TYPE_Q8_0: (32, 34), TYPE_Q8_1: (32, 36), TYPE_Q4_K: (256, 144), TYPE_Q5_K: (256, 176), TYPE_Q6_K: (256, 210),
         TYPE_Q8_K: (256, 292), TYPE_IQ4_XS: (256, 136)}
_NAMES = {TYPE_Q4_0: "q4_0", TYPE_Q4_K: "q4_K", TYPE_Q5_K: "q5_K", TYPE_Q6_K: "q6_K", TYPE_Q8_0: "q8_0", TYPE_Q8_1: "q8_1",
          TYPE_Q8_K: "q8_K", TYPE_IQ4_XS: "iq4_xs"}
IMPL_GENERIC, IMPL_AVX2 = 0, 1

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, f32p = ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p
        L.orc_fp32_to_fp16.restype = ctypes.c_uint16
        L.orc_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.orc_fp16_to_fp32.restype = ctypes.c_float
        L.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.orc_nearest_int.restype = ctypes.c_int
        L.orc_nearest_int.argtypes = [ctypes.c_float]
        for n in ("q4_0", "q4_K", "q5_K", "q6_K", "q8_0", "q8_1", "q8_K", "iq4_xs"):
            f = getattr(L, f"orc_quantize_row_{n}_ref")
            f.restype = None
            f.argtypes = [vp, vp, i64]
        for n in ("q4_0", "q4_K", "q5_K", "q6_K", "q8_0", "q8_K", "iq4_xs"):
            f = getattr(L, f"orc_dequantize_row_{n}")
            f.restype = None
            f.argtypes = [vp, vp, i64]
        L.orc_quantize_row_q8_0_avx2.restype = None
        L.orc_quantize_row_q8_0_avx2.argtypes = [vp, vp, i64]
        L.orc_quantize_chunk.restype = ctypes.c_size_t
        L.orc_quantize_chunk.argtypes = [ctypes.c_int, vp, vp, i64, i64, i64, vp]
        L.orc_vec_dot.restype = ctypes.c_float
        L.orc_vec_dot.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        L.orc_block_dots_q8_1.restype = None
        L.orc_block_dots_q8_1.argtypes = [ctypes.c_int, vp, i64, i64, vp, vp]
        L.orc_mul_mat_q8_1_f64.restype = None
        L.orc_mul_mat_q8_1_f64.argtypes = [ctypes.c_int, vp, i64, i64, vp, i64, vp]
        L.orc_mul_mat.restype = None
        L.orc_mul_mat.argtypes = [ctypes.c_int, ctypes.c_int, vp, i64, i64, f32p, i64, f32p, ctypes.c_int]
        L.orc_mul_mat_tiled.restype = ctypes.c_int
        L.orc_mul_mat_tiled.argtypes = [ctypes.c_int, vp, i64, i64, f32p, i64, f32p, ctypes.c_int]
        L.orc_tinyblas_q0.restype = ctypes.c_int
        L.orc_tinyblas_q0.argtypes = [ctypes.c_int, vp, i64, i64, vp, i64, f32p, ctypes.c_int]
        L.orc_tinyblas_q0_per_output.restype = ctypes.c_int
        L.orc_tinyblas_q0_per_output.argtypes = [ctypes.c_int, vp, i64, i64, vp, i64, f32p, ctypes.c_int]
        L.orc_mul_mat_tinyblas.restype = ctypes.c_int
        L.orc_mul_mat_tinyblas.argtypes = [ctypes.c_int, vp, i64, i64, f32p, i64, f32p, ctypes.c_int]
        L.orc_mul_mat_id.restype = None
        L.orc_mul_mat_id.argtypes = [ctypes.c_int, ctypes.c_int, vp, i64, i64, i64, f32p, i64, i64, vp, i64,
                                     f32p, ctypes.c_int]
        L.orc_fill_normal.restype = None
        L.orc_fill_normal.argtypes = [ctypes.c_uint64, i64, ctypes.c_float, ctypes.c_float, f32p]
        L.orc_fill_normal_mt.restype = None
        L.orc_fill_normal_mt.argtypes = [ctypes.c_uint64, i64, ctypes.c_float, ctypes.c_float, f32p, ctypes.c_int]
        L.orc_quantize_rows_mt.restype = None
        L.orc_quantize_rows_mt.argtypes = [ctypes.c_int, vp, vp, i64, i64, ctypes.c_int]
        L.orc_fnv1a.restype = ctypes.c_uint64
        L.orc_fnv1a.argtypes = [vp, ctypes.c_size_t]
        L.orc_has_avx2.restype = ctypes.c_int
        L.orc_gelu_f32.restype = ctypes.c_float
        L.orc_gelu_f32.argtypes = [ctypes.c_float]
        L.orc_glu_f32.restype = None
        L.orc_glu_f32.argtypes = [ctypes.c_int, i64, f32p, f32p, ctypes.c_float, ctypes.c_float, f32p]
        L.orc_glu_f32_rows.restype = None
        L.orc_glu_f32_rows.argtypes = [ctypes.c_int, i64, i64, f32p, f32p, ctypes.c_float, ctypes.c_float, f32p]
        L.orc_v_expf.restype = ctypes.c_float
        L.orc_v_expf.argtypes = [ctypes.c_float]
        L.orc_v_silu.restype = ctypes.c_float
        L.orc_v_silu.argtypes = [ctypes.c_float]
        L.orc_v_expf_n.restype = None
        L.orc_v_expf_n.argtypes = [i64, f32p, f32p]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def fnv1a(buf):
    b = np.ascontiguousarray(buf).view(np.uint8)
    return int(lib().orc_fnv1a(_p(b), b.nbytes))


def row_bytes(t, k):
    bs, ts = BLOCK[t]
    assert k % bs == 0
    return (k // bs) * ts


def quantize_ref(t, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(row_bytes(t, x.size), dtype=np.uint8)
    getattr(lib(), f"orc_quantize_row_{_NAMES[t]}_ref")(_p(x), _p(out), x.size)
    return out


def gen_threads():
    """Threads for the input generators: the CPUs this process may use, at
    most 16 (a GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def quantize_rows(t, w, nth=None):
    """Quantize a [nrows, K] f32 matrix row by row (quantize_row_*_ref); rows
    are independent, so threads split them (same bytes as one thread)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    nrows, k = w.shape
    if t in (TYPE_Q8_1, TYPE_Q8_K):
        return quantize_ref(t, w.reshape(-1)).reshape(nrows, -1)
    out = np.zeros((nrows, row_bytes(t, k)), dtype=np.uint8)
    lib().orc_quantize_rows_mt(t, _p(w), _p(out), nrows, k, gen_threads() if nth is None else nth)
    return out


def dequantize(t, q, k):
    out = np.zeros(k, dtype=np.float32)
    q = np.ascontiguousarray(q)
    getattr(lib(), f"orc_dequantize_row_{_NAMES[t]}")(_p(q), _p(out), k)
    return out


def quantize_chunk(t, src, nrows, n_per_row, imatrix=None):
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.zeros(nrows * row_bytes(t, n_per_row), dtype=np.uint8)
    im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
    n = lib().orc_quantize_chunk(t, _p(src), _p(out), 0, nrows, n_per_row, None if im is None else _p(im))
    return out[:n]


def vec_dot(t, impl, n, xq, yq):
    return float(lib().orc_vec_dot(t, impl, n, _p(np.ascontiguousarray(xq)), _p(np.ascontiguousarray(yq))))


def block_dots_q8_1(t, wq, nrows, K, yq8_1):
    nsub = K // 16 if t == TYPE_Q6_K else K // 32
    out = np.zeros(nrows * nsub, dtype=np.int32)
    lib().orc_block_dots_q8_1(t, _p(np.ascontiguousarray(wq)), nrows, K, _p(np.ascontiguousarray(yq8_1)), _p(out))
    return out.reshape(nrows, nsub)


def mul_mat_q8_1_f64(t, wq, nrows, K, yq8_1, ncols):
    out = np.zeros(ncols * nrows, dtype=np.float64)
    lib().orc_mul_mat_q8_1_f64(t, _p(np.ascontiguousarray(wq)), nrows, K, _p(np.ascontiguousarray(yq8_1)), ncols,
                               _p(out))
    return out.reshape(ncols, nrows)


def mul_mat(t, wq, nrows, K, x, nth=4, impl=IMPL_GENERIC):
    """x: [ncols, K] f32 -> [ncols, nrows] f32 (ggml's dst with ne0 = nrows)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ncols = x.shape[0]
    out = np.zeros((ncols, nrows), dtype=np.float32)
    lib().orc_mul_mat(t, impl, _p(np.ascontiguousarray(wq)), nrows, K, _p(x), ncols, _p(out), nth)
    return out


def mul_mat_tiled(t, wq, nrows, K, x, nth=4):
    """The reference's x86 tiled GEMM (AVX2 arm) for Q4_K / Q5_K / Q6_K /
    IQ4_XS: x [ncols, K] f32 -> [ncols, nrows] f32, or None where the host
    lacks AVX2 or the type is not tiled."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ncols = x.shape[0]
    out = np.full((ncols, nrows), np.nan, dtype=np.float32)
    ok = lib().orc_mul_mat_tiled(t, _p(np.ascontiguousarray(wq)), nrows, K, _p(x), ncols, _p(out), nth)
    return out if ok else None


def tinyblas_q0(t, wq, nrows, K, y_q8_0, ncols, nth=4):
    """tinyBLAS_Q0_AVX's outputs for Q8_0 / Q4_0 weights against columns
    already quantized to Q8_0 (ncols x K/32 blocks) -> [ncols, nrows], or None
    for other types."""
    out = np.full((ncols, nrows), np.nan, dtype=np.float32)
    ok = lib().orc_tinyblas_q0(t, _p(np.ascontiguousarray(wq)), nrows, K, _p(np.ascontiguousarray(y_q8_0)), ncols,
                               _p(out), nth)
    return out if ok else None


def tinyblas_q0_per_output(t, wq, nrows, K, y_q8_0, ncols, nth=4):
    """The same outputs one at a time (the per-output restatement the tile
    loops are checked against)."""
    out = np.full((ncols, nrows), np.nan, dtype=np.float32)
    ok = lib().orc_tinyblas_q0_per_output(t, _p(np.ascontiguousarray(wq)), nrows, K,
                                          _p(np.ascontiguousarray(y_q8_0)), ncols, _p(out), nth)
    return out if ok else None


def mul_mat_tinyblas(t, wq, nrows, K, x, nth=4):
    """The reference's x86 Q8_0 / Q4_0 mul_mat for 2+ columns (x86
    quantize_row_q8_0, then tinyBLAS_Q0_AVX): x [ncols, K] -> [ncols, nrows],
    or None where it does not apply."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ncols = x.shape[0]
    out = np.full((ncols, nrows), np.nan, dtype=np.float32)
    ok = lib().orc_mul_mat_tinyblas(t, _p(np.ascontiguousarray(wq)), nrows, K, _p(x), ncols, _p(out), nth)
    return out if ok else None


def mul_mat_x86(t, wq, nrows, K, x, nth=4):
    """ggml_compute_forward_mul_mat as an x86 AVX2 host runs it
    (src/ggml/cpu/mulmat.zig:218-220, 336-367): the tiled GEMM for the tiled
    K-quants from 8 columns, tinyBLAS for Q8_0 / Q4_0 from 2 columns, else
    the AVX2 vec_dot route."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    if x.shape[0] >= 8:
        out = mul_mat_tiled(t, wq, nrows, K, x, nth=nth)
        if out is not None:
            return out
    out = mul_mat_tinyblas(t, wq, nrows, K, x, nth=nth)
    if out is not None:
        return out
    return mul_mat(t, wq, nrows, K, x, nth=nth, impl=IMPL_AVX2)


def mul_mat_id(t, wq, n_as, nrows, K, x, ids, nth=4, impl=IMPL_GENERIC):
    """x: [n_tokens, ne11, K]; ids: [n_tokens, n_ids] int32 -> [n_tokens, n_ids, nrows]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n_tokens, ne11, _ = x.shape
    n_ids = ids.shape[1]
    out = np.full((n_tokens, n_ids, nrows), np.nan, dtype=np.float32)
    lib().orc_mul_mat_id(t, impl, _p(np.ascontiguousarray(wq)), n_as, nrows, K, _p(x), ne11, n_tokens, _p(ids),
                         n_ids, _p(out), nth)
    return out


GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI, GLU_SWIGLU_CLAMP = 0, 1, 2, 3, 6


def gelu_f32(x):
    return float(lib().orc_gelu_f32(x))


def glu(op, gate, up, alpha=0.0, limit=0.0):
    """The CPU GLU op, split form: out = glu(gate, up) over rows of the last
    dimension, as an AVX2 host runs it (SWIGLU's 8-lane vector arm and
    scalar tail per row)."""
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    assert gate.shape == up.shape
    out = np.empty_like(gate)
    nc = gate.shape[-1] if gate.ndim else 1
    lib().orc_glu_f32_rows(op, gate.size // max(nc, 1), nc, _p(gate), _p(up), alpha, limit, _p(out))
    return out


def glu_elementwise(op, gate, up, alpha=0.0, limit=0.0):
    """Every element by the scalar formula (the row tail's)."""
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(gate)
    lib().orc_glu_f32(op, gate.size, _p(gate), _p(up), alpha, limit, _p(out))
    return out


def v_expf(x):
    """ggml_v_expf (the vector arm's exp) elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_v_expf_n(x.size, _p(x), _p(out))
    return out


def fill_normal(seed, n, mean=0.0, std=1.0, nth=None):
    """SplitMix64 -> Box-Muller normals; threads split the array at even
    indices (same values as one thread)."""
    out = np.zeros(n, dtype=np.float32)
    nth = (gen_threads() if n >= (1 << 20) else 1) if nth is None else nth
    if nth == 1:
        lib().orc_fill_normal(seed, n, mean, std, _p(out))
    else:
        lib().orc_fill_normal_mt(seed, n, mean, std, _p(out), nth)
    return out


def has_avx2():
    return bool(lib().orc_has_avx2())
