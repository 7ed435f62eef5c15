"""Host-side mirror of the ggml quantized-matmul path, over libggml_hip_qmm.so.

The functions mirror the reference's operator interface for this path:
``mul_mat(w, x)`` is ``ggml_mul_mat(a, b)`` (src/ggml/ops.zig:1072-1083: a is
the [K, M] quantized weight, b the [K, N] f32 activation, result [M, N] f32)
and ``mul_mat_id(as_, x, ids)`` is ``ggml_mul_mat_id`` (ops.zig:1104-1125).
Compute runs only in the HIP library; there is no CPU fallback.  If the
library is missing or no GPU is present the calls raise.

Tensors are torch tensors on the GPU (torch provides device memory and
streams); weights are uint8 tensors holding ggml blocks row by row.
"""
from __future__ import annotations

import ctypes
import pathlib

import torch

from .qtypes import BLOCK, TYPE_IDS, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, row_size  # noqa: F401

PKG_DIR = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = PKG_DIR / "libggml_hip_qmm.so"

_lib = None


class HipQmmError(RuntimeError):
    pass


def lib():
    """Load the HIP library; raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipQmmError(f"{LIB_PATH} not built: run `make -C {PKG_DIR}` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.hip_qmm_version.restype = i32
        L.hip_qmm_row_padding.restype = i64
        L.hip_qmm_quantize_q8_1.restype = i32
        L.hip_qmm_quantize_q8_1.argtypes = [vp, vp, i64, i64, i64, i64, i64, i64, i64, i64, vp]
        L.hip_qmm_quantize_q8_1_planar.restype = i32
        L.hip_qmm_quantize_q8_1_planar.argtypes = [vp, i64, i64, i64, vp, vp, vp]
        L.hip_qmm_mul_mat_workspace_size.restype = ctypes.c_size_t
        L.hip_qmm_mul_mat_workspace_size.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mul_mat_uses_mmq.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mul_mat_per_column.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mul_mat_vec.restype = i32
        L.hip_qmm_mul_mat_vec.argtypes = [i32, vp, i64, i64, i64, vp, vp, i64, vp, i64, vp]
        L.hip_qmm_gemv_mfma.restype = i32
        L.hip_qmm_gemv_mfma.argtypes = [i32, vp, i64, i64, i64, vp, vp, i64, vp, i64, vp]
        L.hip_qmm_mul_mat_vec_f32.restype = i32
        L.hip_qmm_mul_mat_vec_f32.argtypes = [i32, vp, i64, i64, i64, vp, vp, vp]
        L.hip_qmm_mul_mat_vec_fused.restype = i32
        L.hip_qmm_mul_mat_vec_fused.argtypes = [i32, vp, vp, i64, i64, i64, vp, vp, vp, i32, ctypes.c_float,
                                                ctypes.c_float, vp, vp]
        L.hip_qmm_mul_mat_id_vec_fused.restype = i32
        L.hip_qmm_mul_mat_id_vec_fused.argtypes = [i32, vp, vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64,
                                                   i64, i32, ctypes.c_float, ctypes.c_float, vp, i64, vp]
        L.hip_qmm_mul_mat_id_vec_fused_shared.restype = i32
        L.hip_qmm_mul_mat_id_vec_fused_shared.argtypes = [i32, vp, vp, i64, i64, i64, i64, i64, vp, i64, i64, vp,
                                                          i64, i64, i32, ctypes.c_float, ctypes.c_float, vp, i64, vp,
                                                          vp, vp, i64, vp]
        L.hip_qmm_mul_mat_id_vec_fused_bias.restype = i32
        L.hip_qmm_mul_mat_id_vec_fused_bias.argtypes = [i32, vp, vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp,
                                                        i64, i64, vp, vp, i64, i32, ctypes.c_float, ctypes.c_float, vp,
                                                        i64, vp]
        L.hip_qmm_add_id_f32.restype = i32
        L.hip_qmm_add_id_f32.argtypes = [i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, vp, i64, i64, vp]
        L.hip_qmm_glu_f32.restype = i32
        L.hip_qmm_glu_f32.argtypes = [i32, ctypes.c_float, ctypes.c_float, i64, i64, vp, i64, vp, i64, vp, i64, vp]
        L.hip_qmm_add_f32.restype = i32
        L.hip_qmm_add_f32.argtypes = [i64, i64, vp, i64, vp, i64, vp, i64, vp]
        L.hip_qmm_mmq.restype = i32
        L.hip_qmm_mmq.argtypes = [i32, vp, i64, i64, i64, vp, vp, i64, vp, i64, vp, ctypes.c_size_t, vp]
        L.hip_qmm_mmq_workspace_size.restype = ctypes.c_size_t
        L.hip_qmm_mmq_workspace_size.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mmq_split_k.restype = i32
        L.hip_qmm_mmq_split_k.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mul_mat.restype = i32
        L.hip_qmm_mul_mat.argtypes = [i32, vp, i64, i64, i64, vp, i64, i64, vp, i64, vp, ctypes.c_size_t, vp]
        L.hip_qmm_mmq_tile_n.restype = i32
        L.hip_qmm_mmq_tile_n.argtypes = [i64]
        L.hip_qmm_mul_mat_id_workspace_size.restype = ctypes.c_size_t
        L.hip_qmm_mul_mat_id_workspace_size.argtypes = [i32, i64, i64, i64, i64, i64]
        L.hip_qmm_mul_mat_id.restype = i32
        L.hip_qmm_mul_mat_id.argtypes = [i32, vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64, vp, i64,
                                         vp, ctypes.c_size_t, vp]
        L.hip_qmm_mmq_glu.restype = i32
        L.hip_qmm_mmq_glu.argtypes = [i32, vp, vp, i64, i64, i64, vp, vp, i64, i32, ctypes.c_float, ctypes.c_float,
                                      vp, i64, vp]
        L.hip_qmm_mmq_grouped_glu.restype = i32
        L.hip_qmm_mmq_grouped_glu.argtypes = [i32, vp, vp, i64, i64, i64, i64, vp, vp, vp, i64, i32, i64, vp, vp,
                                              vp, vp, i32, ctypes.c_float, ctypes.c_float, vp]
        L.hip_qmm_mul_mat_glu_workspace_size.restype = ctypes.c_size_t
        L.hip_qmm_mul_mat_glu_workspace_size.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mul_mat_glu_fused.restype = i32
        L.hip_qmm_mul_mat_glu_fused.argtypes = [i32, i64, i64, i64]
        L.hip_qmm_mul_mat_glu.restype = i32
        L.hip_qmm_mul_mat_glu.argtypes = [i32, vp, vp, i64, i64, i64, vp, i64, i64, i32, ctypes.c_float,
                                          ctypes.c_float, vp, i64, vp, ctypes.c_size_t, vp]
        L.hip_qmm_mul_mat_id_glu.restype = i32
        L.hip_qmm_mul_mat_id_glu.argtypes = [i32, vp, vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64,
                                             i32, ctypes.c_float, ctypes.c_float, vp, i64, vp, ctypes.c_size_t, vp]
        L.hip_qmm_mul_mat_vec_q.restype = i32
        L.hip_qmm_mul_mat_vec_q.argtypes = [i32, vp, vp, vp, vp] + [i64] * 18 + [vp]
        L.hip_qmm_block_dots.restype = i32
        L.hip_qmm_block_dots.argtypes = [i32, vp, i64, i64, i64, vp, i64, vp, vp]
        _lib = L
    return _lib


def _check(err, what):
    if err != 0:
        raise HipQmmError(f"{what} failed with hipError {err}")


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _require_cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise HipQmmError("tensors must live on the GPU")
        if not t.is_contiguous():
            raise HipQmmError("tensors must be contiguous")


def padded_k(K: int) -> int:
    pad = int(lib().hip_qmm_row_padding())
    return (K + pad - 1) // pad * pad


def quantize_q8_1(x: torch.Tensor, ne0_padded: int | None = None) -> torch.Tensor:
    """f32 [N, K] -> uint8 [N, ne0_padded/32*36] in block_q8_1 layout, bit-exact
    with quantize_row_q8_1_ref (src/ggml/quants/legacy.zig:451-484)."""
    _require_cuda(x)
    if x.dtype != torch.float32 or x.dim() != 2:
        raise HipQmmError("x must be a 2-D float32 tensor [ncols, K]")
    n, K = x.shape
    ne0_padded = padded_k(K) if ne0_padded is None else ne0_padded
    y = torch.empty((n, ne0_padded // 32 * 36), dtype=torch.uint8, device=x.device)
    _check(lib().hip_qmm_quantize_q8_1(_ptr(x), _ptr(y), K, K, K * n, K * n, ne0_padded, n, 1, 1, _stream()),
           "hip_qmm_quantize_q8_1")
    return y


def quantize_q8_1_planar(x: torch.Tensor):
    """f32 [N, K] -> (qs int8 [N, Kp], ds int32 [N, Kp/32]) in the library's planar layout."""
    _require_cuda(x)
    n, K = x.shape
    Kp = padded_k(K)
    qs = torch.empty((n, Kp), dtype=torch.int8, device=x.device)
    ds = torch.empty((n, Kp // 32), dtype=torch.int32, device=x.device)
    _check(lib().hip_qmm_quantize_q8_1_planar(_ptr(x), K, n, K, _ptr(qs), _ptr(ds), _stream()),
           "hip_qmm_quantize_q8_1_planar")
    return qs, ds


def _weight_args(qtype, w, K):
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    _require_cuda(w)
    if w.dtype != torch.uint8 or w.dim() != 2:
        raise HipQmmError("weights must be a 2-D uint8 tensor [nrows, row_bytes]")
    if w.shape[1] < row_size(t, K):
        raise HipQmmError("weight rows are shorter than K elements of this type")
    return t, w.shape[0], w.stride(0)


def mul_mat_vec(qtype, w: torch.Tensor, K: int, qs: torch.Tensor, ds: torch.Tensor, out=None):
    """GEMV against planar Q8_1 activations (1..8 columns)."""
    t, nrows, rs = _weight_args(qtype, w, K)
    n = qs.shape[0]
    out = torch.empty((n, nrows), dtype=torch.float32, device=w.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_vec(t, _ptr(w), K, nrows, rs, _ptr(qs), _ptr(ds), n, _ptr(out), out.stride(0),
                                     _stream()), "hip_qmm_mul_mat_vec")
    return out


def mul_mat_vec_f32(qtype, w: torch.Tensor, K: int, x: torch.Tensor, out=None):
    """GEMV of one f32 column [1, K] with the Q8_1 quantization fused into the kernel."""
    _require_cuda(x)
    t, nrows, rs = _weight_args(qtype, w, K)
    x = x.reshape(-1)
    if x.numel() != K or not x.is_contiguous():
        raise ValueError("x must be one contiguous column of K values")
    out = torch.empty((1, nrows), dtype=torch.float32, device=w.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_vec_f32(t, _ptr(w), K, nrows, rs, _ptr(x), _ptr(out), _stream()),
           "hip_qmm_mul_mat_vec_f32")
    return out


GLU_OPS = {"REGLU": 0, "GEGLU": 1, "SWIGLU": 2, "SWIGLU_OAI": 3, "SWIGLU_CLAMP": 6}


def _vec(t, n, name):
    if t is None:
        return None
    _require_cuda(t)
    if t.dtype != torch.float32 or t.numel() != n or not t.is_contiguous():
        raise ValueError(f"{name} must be {n} contiguous float32 values")
    return t


def mul_mat_vec_fused(qtype, w: torch.Tensor, K: int, x: torch.Tensor, w_gate=None, bias=None, gate_bias=None,
                      glu="SWIGLU", alpha=1.702, limit=7.0, out=None):
    """One f32 column through the quantizing GEMV with the fusion epilogue:
    u = W x (+ bias); with w_gate, out = glu(Wg x (+ gate_bias), u), else u."""
    _require_cuda(x)
    t, nrows, rs = _weight_args(qtype, w, K)
    if w_gate is not None:
        tg, ng, rg = _weight_args(qtype, w_gate, K)
        if (ng, rg) != (nrows, rs):
            raise ValueError("w_gate must match w")
    x = x.reshape(-1)
    if x.numel() != K or not x.is_contiguous():
        raise ValueError("x must be one contiguous column of K values")
    _vec(bias, nrows, "bias")
    _vec(gate_bias, nrows, "gate_bias")
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    out = torch.empty((1, nrows), dtype=torch.float32, device=w.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_vec_fused(t, _ptr(w), _ptr(w_gate) if w_gate is not None else None, K, nrows, rs,
                                           _ptr(x), _ptr(bias) if bias is not None else None,
                                           _ptr(gate_bias) if gate_bias is not None else None, op, alpha, limit,
                                           _ptr(out), _stream()), "hip_qmm_mul_mat_vec_fused")
    return out


def mul_mat_id_vec_fused(qtype, w: torch.Tensor, x: torch.Tensor, ids: torch.Tensor, w_gate=None, glu="SWIGLU",
                         alpha=1.702, limit=7.0, out=None):
    """MUL_MAT_ID over few tokens in one launch: row (t, s) = W_e x[t, s % ne11]
    with e = ids[t, s], or glu(Wg_e x, W_e x) with w_gate; zero rows for ids
    outside [0, n_as).  w / w_gate: uint8 [n_as, nrows, row_bytes]; x: f32
    [n_tokens, ne11, K]; ids: int32 [n_tokens, n_ids]."""
    _require_cuda(w, x, ids)
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    n_as, nrows, rb = w.shape
    n_tokens, ne11, K = x.shape
    n_ids = ids.shape[1]
    if rb < row_size(t, K) or ids.shape[0] != n_tokens or ids.dtype != torch.int32:
        raise HipQmmError("bad mul_mat_id shapes")
    if w_gate is not None:
        _require_cuda(w_gate)
        if w_gate.shape != w.shape:
            raise HipQmmError("w_gate must match w")
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    out = torch.empty((n_tokens, n_ids, nrows), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_id_vec_fused(t, _ptr(w), _ptr(w_gate) if w_gate is not None else None, K, nrows,
                                              w.stride(1), w.stride(0), n_as, _ptr(x), ne11, n_tokens, K, _ptr(ids),
                                              n_ids, n_ids, op, alpha, limit, _ptr(out), nrows, _stream()),
           "hip_qmm_mul_mat_id_vec_fused")
    return out


def mul_mat_id_vec_fused_bias(qtype, w: torch.Tensor, x: torch.Tensor, ids: torch.Tensor, bias: torch.Tensor,
                              w_gate=None, gate_bias=None, glu="SWIGLU", alpha=1.702, limit=7.0, out=None):
    """mul_mat_id_vec_fused with per-expert biases: bias / gate_bias f32
    [n_as, nrows] (row e for expert e), added to u / g before the GLU."""
    _require_cuda(w, x, ids, bias)
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    n_as, nrows, rb = w.shape
    n_tokens, ne11, K = x.shape
    n_ids = ids.shape[1]
    if (rb < row_size(t, K) or ids.shape[0] != n_tokens or tuple(bias.shape) != (n_as, nrows) or
            (gate_bias is not None and (w_gate is None or gate_bias.shape != bias.shape))):
        raise HipQmmError("bad mul_mat_id bias shapes")
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    out = torch.empty((n_tokens, n_ids, nrows), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_id_vec_fused_bias(
        t, _ptr(w), _ptr(w_gate) if w_gate is not None else None, K, nrows, w.stride(1), w.stride(0), n_as, _ptr(x),
        ne11, n_tokens, K, _ptr(ids), n_ids, n_ids, _ptr(bias), _ptr(gate_bias) if gate_bias is not None else None,
        bias.stride(0), op, alpha, limit, _ptr(out), nrows, _stream()), "hip_qmm_mul_mat_id_vec_fused_bias")
    return out


def add_id_f32(a: torch.Tensor, b: torch.Tensor, ids: torch.Tensor, out=None):
    """ggml_add_id: a [n_tokens, n_slots, nc] + b[ids[t, s]] (b [n_b, nc]); -1 ids copy a."""
    _require_cuda(a, b, ids)
    n_tokens, n_slots, nc = a.shape
    out = torch.empty_like(a) if out is None else out
    _check(lib().hip_qmm_add_id_f32(nc, n_slots, n_tokens, _ptr(a), a.stride(1), a.stride(0), _ptr(b), b.stride(0),
                                    b.shape[0], _ptr(ids), ids.stride(0), _ptr(out), out.stride(1), out.stride(0),
                                    _stream()), "hip_qmm_add_id_f32")
    return out


def mul_mat_id_vec_fused_shared(qtype, w: torch.Tensor, w_gate: torch.Tensor, x: torch.Tensor, ids: torch.Tensor,
                                shared_up: torch.Tensor, shared_gate: torch.Tensor, glu="SWIGLU", alpha=1.702,
                                limit=7.0, out=None, shared_out=None):
    """The routed experts' gate / up / GLU over the (token, slot) pairs and a
    shared expert's gate / up / GLU on every token, one launch.  w / w_gate:
    uint8 [n_as, nrows, row_bytes]; shared_up / shared_gate: uint8 [nrows,
    row_bytes]; x: f32 [n_tokens, 1, K]; ids: int32 [n_tokens, n_ids].
    Returns (routed [n_tokens, n_ids, nrows], shared [n_tokens, nrows])."""
    _require_cuda(w, w_gate, x, ids, shared_up, shared_gate)
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    n_as, nrows, rb = w.shape
    n_tokens, ne11, K = x.shape
    n_ids = ids.shape[1]
    if (rb < row_size(t, K) or ne11 != 1 or ids.shape[0] != n_tokens or ids.dtype != torch.int32 or
            w_gate.shape != w.shape or tuple(shared_up.shape) != (nrows, rb) or shared_gate.shape != shared_up.shape):
        raise HipQmmError("bad shared-expert shapes")
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    out = torch.empty((n_tokens, n_ids, nrows), dtype=torch.float32, device=x.device) if out is None else out
    shared_out = (torch.empty((n_tokens, nrows), dtype=torch.float32, device=x.device) if shared_out is None
                  else shared_out)
    _check(lib().hip_qmm_mul_mat_id_vec_fused_shared(t, _ptr(w), _ptr(w_gate), K, nrows, w.stride(1), w.stride(0),
                                                     n_as, _ptr(x), n_tokens, K, _ptr(ids), n_ids, n_ids, op, alpha,
                                                     limit, _ptr(out), nrows, _ptr(shared_up), _ptr(shared_gate),
                                                     _ptr(shared_out), nrows, _stream()),
           "hip_qmm_mul_mat_id_vec_fused_shared")
    return out, shared_out


def glu_f32(gate: torch.Tensor, up: torch.Tensor, glu="SWIGLU", alpha=1.702, limit=7.0, out=None):
    """Standalone GLU over [rows, n] f32 tensors (rows may be strided)."""
    if not (gate.is_cuda and up.is_cuda):
        raise HipQmmError("tensors must live on the GPU")
    if gate.shape != up.shape or gate.dim() != 2 or gate.stride(1) != 1 or up.stride(1) != 1:
        raise ValueError("gate and up must be [rows, n] with contiguous rows")
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    out = torch.empty(gate.shape, dtype=torch.float32, device=gate.device) if out is None else out
    _check(lib().hip_qmm_glu_f32(op, alpha, limit, gate.shape[1], gate.shape[0], _ptr(gate), gate.stride(0),
                                 _ptr(up), up.stride(0), _ptr(out), out.stride(0), _stream()), "hip_qmm_glu_f32")
    return out


def add_f32(a: torch.Tensor, b: torch.Tensor, out=None):
    """Same-shape f32 add over [rows, n] tensors (rows may be strided)."""
    if not (a.is_cuda and b.is_cuda):
        raise HipQmmError("tensors must live on the GPU")
    if a.shape != b.shape or a.dim() != 2 or a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("a and b must be [rows, n] with contiguous rows")
    out = torch.empty(a.shape, dtype=torch.float32, device=a.device) if out is None else out
    _check(lib().hip_qmm_add_f32(a.shape[1], a.shape[0], _ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(out),
                                 out.stride(0), _stream()), "hip_qmm_add_f32")
    return out


def gemv_mfma(qtype, w: torch.Tensor, K: int, qs: torch.Tensor, ds: torch.Tensor, out=None):
    """Small-batch GEMV on int8 MFMA against planar Q8_1 activations (1..16 columns)."""
    t, nrows, rs = _weight_args(qtype, w, K)
    n = qs.shape[0]
    out = torch.empty((n, nrows), dtype=torch.float32, device=w.device) if out is None else out
    _check(lib().hip_qmm_gemv_mfma(t, _ptr(w), K, nrows, rs, _ptr(qs), _ptr(ds), n, _ptr(out), out.stride(0),
                                   _stream()), "hip_qmm_gemv_mfma")
    return out


def mmq(qtype, w: torch.Tensor, K: int, qs: torch.Tensor, ds: torch.Tensor, out=None, workspace=None):
    """int8-MFMA GEMM against planar Q8_1 activations (any column count).
    `workspace` (uint8, >= mmq_workspace_size) enables the K split."""
    t, nrows, rs = _weight_args(qtype, w, K)
    n = qs.shape[0]
    out = torch.empty((n, nrows), dtype=torch.float32, device=w.device) if out is None else out
    need = int(lib().hip_qmm_mmq_workspace_size(t, K, nrows, n))
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=w.device)
    wp, wn = (_ptr(workspace), workspace.numel()) if workspace is not None else (None, 0)
    _check(lib().hip_qmm_mmq(t, _ptr(w), K, nrows, rs, _ptr(qs), _ptr(ds), n, _ptr(out), out.stride(0), wp, wn,
                             _stream()), "hip_qmm_mmq")
    return out


def _glu_weights(qtype, w, w_gate, K):
    t, nrows, rs = _weight_args(qtype, w, K)
    tg, ng, rg = _weight_args(qtype, w_gate, K)
    if (ng, rg) != (nrows, rs):
        raise HipQmmError("w_gate must match w")
    return t, nrows, rs


def mmq_glu(qtype, w: torch.Tensor, w_gate: torch.Tensor, K: int, qs: torch.Tensor, ds: torch.Tensor,
            glu="SWIGLU", alpha=1.702, limit=7.0, out=None):
    """Gate/up/GLU fused MMQ: out[c] = glu(Wg y_c, W y_c) over planar Q8_1 columns."""
    t, nrows, rs = _glu_weights(qtype, w, w_gate, K)
    n = qs.shape[0]
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    out = torch.empty((n, nrows), dtype=torch.float32, device=w.device) if out is None else out
    _check(lib().hip_qmm_mmq_glu(t, _ptr(w), _ptr(w_gate), K, nrows, rs, _ptr(qs), _ptr(ds), n, op, alpha, limit,
                                 _ptr(out), out.stride(0), _stream()), "hip_qmm_mmq_glu")
    return out


def mul_mat_glu(qtype, w: torch.Tensor, w_gate: torch.Tensor, x: torch.Tensor, glu="SWIGLU", alpha=1.702,
                limit=7.0, out=None, workspace=None):
    """{MUL_MAT gate, MUL_MAT up, GLU}: x f32 [N, K] -> glu(Wg x, W x) f32 [N, nrows]."""
    _require_cuda(x)
    if x.dtype != torch.float32 or x.dim() != 2:
        raise HipQmmError("x must be a 2-D float32 tensor [ncols, K]")
    n, K = x.shape
    t, nrows, rs = _glu_weights(qtype, w, w_gate, K)
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    need = int(lib().hip_qmm_mul_mat_glu_workspace_size(t, K, nrows, n))
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    elif workspace.numel() < need:
        raise HipQmmError(f"workspace too small: {workspace.numel()} < {need}")
    out = torch.empty((n, nrows), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_glu(t, _ptr(w), _ptr(w_gate), K, nrows, rs, _ptr(x), n, x.stride(0), op, alpha,
                                     limit, _ptr(out), out.stride(0), _ptr(workspace), workspace.numel(), _stream()),
           "hip_qmm_mul_mat_glu")
    return out


def mul_mat_vec_q(qtype, w: torch.Tensor, y_q8_1: torch.Tensor, K: int, ncols_dst: int, dst: torch.Tensor, *,
                  nchannels_x=1, nchannels_y=1, nchannels_dst=1, nsamples_x=1, nsamples_dst=1,
                  stride_col_y, stride_col_dst, stride_channel_x=0, stride_channel_y=0, stride_channel_dst=0,
                  stride_sample_x=0, stride_sample_y=0, stride_sample_dst=0, ids=None, ids_stride=0, nrows=None):
    """hip_qmm_mul_mat_vec_q: the reference's mul_mat_vec_q launch on AoS
    block_q8_1 activations (strides of x in weight blocks, of y in Q8_1
    blocks, of dst in floats; w's first matrix gives the row stride)."""
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    _require_cuda(w, y_q8_1, dst)
    bs, bb = BLOCK[t]
    nrows = w.shape[-2] if nrows is None else nrows
    row_stride = w.stride(-2)
    if row_stride % bb:
        raise HipQmmError("weight rows must be whole blocks apart")
    _check(lib().hip_qmm_mul_mat_vec_q(t, _ptr(w), _ptr(y_q8_1), _ptr(ids) if ids is not None else None, _ptr(dst),
                                       K, nrows, ncols_dst, row_stride // bb, stride_col_y, stride_col_dst,
                                       nchannels_x, nchannels_y, nchannels_dst, stride_channel_x, stride_channel_y,
                                       stride_channel_dst, nsamples_x, nsamples_dst, stride_sample_x,
                                       stride_sample_y, stride_sample_dst, ids_stride, _stream()),
           "hip_qmm_mul_mat_vec_q")
    return dst


def block_dots(qtype, w: torch.Tensor, K: int, qs: torch.Tensor):
    """The GEMV's integer block dot products: int32 [N, nrows, K/32 or K/16]."""
    t, nrows, rs = _weight_args(qtype, w, K)
    n = qs.shape[0]
    nsub = K // 16 if t == TYPE_Q6_K else K // 32
    out = torch.empty((n, nrows, nsub), dtype=torch.int32, device=w.device)
    _check(lib().hip_qmm_block_dots(t, _ptr(w), K, nrows, rs, _ptr(qs), n, _ptr(out), _stream()),
           "hip_qmm_block_dots")
    return out


def workspace_size(qtype, K: int, ncols: int, nrows: int = 0) -> int:
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    return int(lib().hip_qmm_mul_mat_workspace_size(t, K, nrows, ncols))


def mul_mat(qtype, w: torch.Tensor, x: torch.Tensor, out=None, workspace=None):
    """ggml_mul_mat(w, x): w quantized [nrows, row_bytes], x f32 [N, K] -> f32 [N, nrows]."""
    _require_cuda(x)
    if x.dtype != torch.float32 or x.dim() != 2:
        raise HipQmmError("x must be a 2-D float32 tensor [ncols, K]")
    n, K = x.shape
    t, nrows, rs = _weight_args(qtype, w, K)
    need = workspace_size(t, K, n, nrows)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    elif workspace.numel() < need:
        raise HipQmmError(f"workspace too small: {workspace.numel()} < {need}")
    out = torch.empty((n, nrows), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().hip_qmm_mul_mat(t, _ptr(w), K, nrows, rs, _ptr(x), n, x.stride(0), _ptr(out), out.stride(0),
                                 _ptr(workspace), workspace.numel(), _stream()), "hip_qmm_mul_mat")
    return out


def mul_mat_id(qtype, w: torch.Tensor, x: torch.Tensor, ids: torch.Tensor, out=None, workspace=None):
    """ggml_mul_mat_id(as, b, ids) (src/ggml/ops.zig:1104-1125).

    w: uint8 [n_as, nrows, row_bytes] stacked expert weights; x: f32
    [n_tokens, ne11, K] with ne11 = 1 (one row per token) or n_ids (one per
    slot); ids: int32 [n_tokens, n_ids] expert per slot (-1: zero row).
    Returns f32 [n_tokens, n_ids, nrows].
    """
    _require_cuda(w, x, ids)
    if w.dtype != torch.uint8 or w.dim() != 3:
        raise HipQmmError("w must be a 3-D uint8 tensor [n_as, nrows, row_bytes]")
    if x.dtype != torch.float32 or x.dim() != 3:
        raise HipQmmError("x must be a 3-D float32 tensor [n_tokens, ne11, K]")
    if ids.dtype != torch.int32 or ids.dim() != 2:
        raise HipQmmError("ids must be a 2-D int32 tensor [n_tokens, n_ids]")
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    n_as, nrows, rb = w.shape
    n_tokens, ne11, K = x.shape
    n_ids = ids.shape[1]
    if ids.shape[0] != n_tokens:
        raise HipQmmError("ids and x disagree on the token count")
    if rb < row_size(t, K):
        raise HipQmmError("weight rows are shorter than K elements of this type")
    need = int(lib().hip_qmm_mul_mat_id_workspace_size(t, K, n_as, ne11, n_tokens, n_ids))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    elif workspace.numel() < need:
        raise HipQmmError(f"workspace too small: {workspace.numel()} < {need}")
    out = torch.empty((n_tokens, n_ids, nrows), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_id(t, _ptr(w), K, nrows, w.stride(1), w.stride(0), n_as, _ptr(x), ne11, n_tokens,
                                    K, _ptr(ids), n_ids, n_ids, _ptr(out), nrows, _ptr(workspace),
                                    workspace.numel(), _stream()), "hip_qmm_mul_mat_id")
    return out


def mul_mat_id_glu(qtype, w: torch.Tensor, w_gate: torch.Tensor, x: torch.Tensor, ids: torch.Tensor, glu="SWIGLU",
                   alpha=1.702, limit=7.0, out=None, workspace=None):
    """Gate/up/GLU over ggml_mul_mat_id's routed pairs: f32 [n_tokens, n_ids, nrows] =
    glu(Wg_e x, W_e x) with e = ids[t, s] (zero rows for ids outside [0, n_as))."""
    _require_cuda(w, w_gate, x, ids)
    if w.shape != w_gate.shape or w.stride() != w_gate.stride() or w.dtype != torch.uint8 or w.dim() != 3:
        raise HipQmmError("w and w_gate must be matching 3-D uint8 tensors [n_as, nrows, row_bytes]")
    if x.dtype != torch.float32 or x.dim() != 3 or ids.dtype != torch.int32 or ids.dim() != 2:
        raise HipQmmError("x must be f32 [n_tokens, ne11, K] and ids int32 [n_tokens, n_ids]")
    t = TYPE_IDS[qtype] if isinstance(qtype, str) else int(qtype)
    n_as, nrows, rb = w.shape
    n_tokens, ne11, K = x.shape
    n_ids = ids.shape[1]
    if ids.shape[0] != n_tokens or rb < row_size(t, K):
        raise HipQmmError("ids, x and w disagree on the shape")
    op = GLU_OPS[glu] if isinstance(glu, str) else int(glu)
    need = int(lib().hip_qmm_mul_mat_id_workspace_size(t, K, n_as, ne11, n_tokens, n_ids))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    elif workspace.numel() < need:
        raise HipQmmError(f"workspace too small: {workspace.numel()} < {need}")
    out = torch.empty((n_tokens, n_ids, nrows), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().hip_qmm_mul_mat_id_glu(t, _ptr(w), _ptr(w_gate), K, nrows, w.stride(1), w.stride(0), n_as, _ptr(x),
                                        ne11, n_tokens, K, _ptr(ids), n_ids, n_ids, op, alpha, limit, _ptr(out), nrows,
                                        _ptr(workspace), workspace.numel(), _stream()), "hip_qmm_mul_mat_id_glu")
    return out
