"""Decode GEMV (1..8 columns) parity: integer block dots exact, fp32 outputs
within NMSE < 5e-4 of the CPU ggml path (and within 1e-5 relative of the
f64 evaluation of the same Q8_1 formula)."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, max_rel, nmse, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4  # test-backend-ops' gate for mul_mat
F64_TOL = 2e-6    # fp32 epilogue vs exact f64 of the same Q8_1 formula, / max|out|

TYPES = {"Q4_K": O.TYPE_Q4_K, "Q5_K": O.TYPE_Q5_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0,
         "Q4_0": O.TYPE_Q4_0, "IQ4_XS": O.TYPE_IQ4_XS}


def _run(tname, nrows, K, ncols):
    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    got = G.mul_mat_vec(tname, w_d, K, qs, ds).cpu().numpy()
    return t, wq, x, w_d, x_d, qs, got


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("ncols", [1, 2, 3, 8])
def test_block_dots_exact(tname, ncols):
    import ggml_hip as G
    nrows, K = 64, 2048
    t, wq, x, w_d, x_d, qs, _ = _run(tname, nrows, K, ncols)
    got = G.block_dots(tname, w_d, K, qs).cpu().numpy()
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    for c in range(ncols):
        want = O.block_dots_q8_1(t, wq, nrows, K, y[c])
        np.testing.assert_array_equal(got[c], want)


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("nrows,K,ncols", [(4096, 4096, 1), (1024, 4096, 2), (1024, 4096, 4), (1000, 4096, 8),
                                           (333, 14336, 3), (96, 768, 5)])
def test_gemv_parity(tname, nrows, K, ncols):
    import ggml_hip as G
    t, wq, x, w_d, x_d, qs, got = _run(tname, nrows, K, ncols)
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    assert nmse(got, ideal) < 1e-11
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    e = nmse(got, cpu)
    assert e < NMSE_GATE, f"NMSE {e:.3g}, max rel {max_rel(got, cpu):.3g}"


# Shapes that reach each GEMV kernel of hip_qmm_mul_mat_vec's shape-based
# choice: Q4_K row-streaming with 4 / 8 / 16 rows per wave (ragged row counts,
# 7 columns = more outputs per wave than lanes), the K-split kernel with 4
# rows per workgroup (long rows, at most 4096 rows), and the int8-MFMA GEMV
# beside them.
@pytest.mark.parametrize("tname,nrows,K,ncols", [
    ("Q4_K", 4100, 4096, 3), ("Q4_K", 4096, 2048, 8), ("Q4_K", 8195, 1024, 2), ("Q4_K", 8195, 1024, 7),
    ("Q4_K", 2500, 8192, 2), ("Q6_K", 2500, 8192, 4), ("Q6_K", 3000, 8192, 8), ("Q8_0", 2500, 8192, 3),
    ("Q5_K", 4100, 4096, 3), ("Q5_K", 2500, 8192, 8), ("Q5_K", 8195, 1024, 2), ("Q4_0", 2500, 8192, 3),
    ("Q4_0", 4100, 4096, 8), ("Q4_0", 8195, 1056, 2), ("IQ4_XS", 4100, 4096, 3), ("IQ4_XS", 2500, 8192, 8),
    ("IQ4_XS", 8195, 1024, 2)])
def test_gemv_kernel_paths(tname, nrows, K, ncols):
    import ggml_hip as G
    t, wq, x, w_d, x_d, qs, got = _run(tname, nrows, K, ncols)
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    e = nmse(got, cpu)
    assert e < NMSE_GATE, f"NMSE {e:.3g}, max rel {max_rel(got, cpu):.3g}"


@pytest.mark.parametrize("tname,nrows,K", [("Q4_K", 4096, 4096), ("Q4_K", 5000, 1024), ("Q6_K", 4100, 4096),
                                           ("Q8_0", 4096, 2048), ("Q8_0", 333, 96), ("Q4_K", 4096, 768),
                                           ("Q6_K", 4100, 1536), ("Q8_0", 4097, 1024), ("Q5_K", 4096, 4096),
                                           ("Q5_K", 4100, 768), ("Q4_0", 4096, 4096), ("Q4_0", 4096, 2048),
                                           ("Q4_0", 333, 96), ("Q4_0", 4097, 1024), ("IQ4_XS", 4096, 4096),
                                           ("IQ4_XS", 4100, 768), ("Q4_K", 14336, 4096), ("Q6_K", 11008, 4096),
                                           ("IQ4_XS", 16390, 2048), ("Q8_0", 8192, 2048)])
def test_gemv_fused_quantize(tname, nrows, K):
    """Quantize-in-GEMV for one column: bit-identical to the separate Q8_1
    quantizer followed by the two-rows-per-wave GEMV (which the unfused path
    takes for one column on >= 4096 rows) when a row is one K-step of 64 lane
    slices, and within the gates of the CPU path always.  Over several steps
    the two kernels accumulate a lane's steps with different roundings (one
    contracts the add into an fma), so only the tolerances apply there.  Short
    rows (at most 16 or 32 lane slices) run several rows per wave in lane
    segments; their sums must still match bit for bit."""
    import ggml_hip as G
    t, wq, x, w_d, x_d, qs, got = _run(tname, nrows, K, 1)
    fused = G.mul_mat_vec_f32(tname, w_d, K, x_d[0]).cpu().numpy()
    one_step = K <= 64 * (32 if tname in ("Q8_0", "Q4_0") else 64)
    if nrows >= 4096 and one_step:
        np.testing.assert_array_equal(fused, got)
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, 1)
    assert max_err_scaled(fused, ideal) < F64_TOL, max_err_scaled(fused, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    assert nmse(fused, cpu) < NMSE_GATE
    # the op-level entry point takes the fused kernel for this shape
    op = G.mul_mat(tname, w_d, x_d).cpu().numpy()
    np.testing.assert_array_equal(op.reshape(fused.shape), fused)


# One column on long rows (two or more K-steps of 64 lane slices) below 8192
# rows: K shares of one workgroup, one case per share layout of the fused
# GEMV's choice (4 shares of 1 row at <= 1024 rows, 2 shares of 1 row for 2-3
# steps there, 2 of 1 row up to 2048 rows and for Q6_K / Q5_K, 2 of 2 rows up
# to 4096 rows or under 4 steps, else 4 of 2 rows), with ragged row counts
# (row groups past the end), part-filled last steps and a bias.
@pytest.mark.parametrize("tname,nrows,K", [("Q4_K", 1001, 14336), ("Q8_0", 777, 8192), ("Q6_K", 1023, 8192),
                                           ("Q4_0", 500, 4096), ("Q4_K", 2047, 11008), ("Q6_K", 4100, 14336),
                                           ("Q5_K", 3001, 9216), ("IQ4_XS", 4095, 14336), ("Q4_K", 7000, 8192),
                                           ("Q4_0", 6001, 14336), ("Q4_K", 5000, 16384), ("IQ4_XS", 257, 12288)])
def test_gemv_fused_k_shares(tname, nrows, K):
    import ggml_hip as G
    t, wq, x, w_d, x_d, qs, got = _run(tname, nrows, K, 1)
    fused = G.mul_mat_vec_f32(tname, w_d, K, x_d[0]).cpu().numpy()
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, 1)
    assert max_err_scaled(fused, ideal) < F64_TOL, max_err_scaled(fused, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    assert nmse(fused, cpu) < NMSE_GATE
    op = G.mul_mat(tname, w_d, x_d).cpu().numpy()
    np.testing.assert_array_equal(op.reshape(fused.shape), fused)
    # the bias is one fp32 add after the share sums
    b = np.random.default_rng(nrows).standard_normal(nrows).astype(np.float32)
    with_b = G.mul_mat_vec_fused(tname, w_d, K, x_d[0], bias=torch.from_numpy(b).cuda()).cpu().numpy()
    np.testing.assert_array_equal(with_b.reshape(-1), fused.reshape(-1) + b)


def _one_column_op_splits_k(tname, nrows, K):
    """Whether the one-column op splits this row into K shares: rows of two or
    more 64-lane steps (2048 elements for Q8_0 / Q4_0, 4096 for the others)
    below 8192 rows, when K > 4096 or there are at most 2048 rows."""
    step = 64 * (32 if tname in ("Q8_0", "Q4_0") else 64)
    return nrows < 8192 and K > step and (K > 4096 or nrows <= 2048)


# 2-4 f32 columns on at most 4096-long rows below 8192 rows (and above, for
# Q8_0 at 3-4 columns and rows of K <= 2048): the op runs the
# quantize-in-GEMV kernel over all columns in one launch (2 columns for the
# K-quants, 3 for IQ4_XS, 4 for Q8_0 / Q4_0).  Where the one-column op runs
# one K share, each column equals it bit for bit; where the one-column op
# splits the row into K shares (Q8_0 / Q4_0 rows of two 2048-steps on at most
# 2048 rows: attn_k / attn_v shapes) the one-launch kernel adds both steps in
# each lane before the wave sum, another rounding order, so only the f64 and
# CPU gates apply.
@pytest.mark.parametrize("tname,nrows,K,ncols", [("Q4_K", 4096, 4096, 2), ("Q5_K", 1000, 4096, 2),
                                                 ("Q6_K", 1024, 4096, 2), ("IQ4_XS", 777, 2048, 3),
                                                 ("Q8_0", 4100, 4096, 4), ("Q4_0", 333, 96, 3),
                                                 ("Q8_0", 5000, 1024, 3), ("Q4_0", 4097, 4096, 2),
                                                 ("IQ4_XS", 6000, 4096, 2), ("Q8_0", 9000, 4096, 4),
                                                 ("Q4_K", 8200, 2048, 2), ("Q4_0", 8195, 1024, 4),
                                                 ("Q8_0", 1024, 4096, 2), ("Q4_0", 500, 4096, 3),
                                                 ("Q8_0", 2048, 4096, 4)])
def test_op_few_columns_one_launch(tname, nrows, K, ncols):
    import ggml_hip as G
    t, wq, x, w_d, x_d, qs, _ = _run(tname, nrows, K, ncols)
    got = G.mul_mat(tname, w_d, x_d).cpu().numpy()
    for c in range(ncols):
        one = G.mul_mat_vec_f32(tname, w_d, K, x_d[c]).cpu().numpy().reshape(-1)
        if _one_column_op_splits_k(tname, nrows, K):
            assert max_err_scaled(got[c], one) < 1e-6
        else:
            np.testing.assert_array_equal(got[c], one)
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE


def test_gemv_config0_op_level():
    """Config 0: 4096x4096 Q4_K (seed 42) times a 4096x1 activation through the
    op-level entry point, against the CPU ggml path."""
    import ggml_hip as G
    K = nrows = 4096
    wq = weights_q(O.TYPE_Q4_K, nrows, K)
    x = acts(1, K)
    got = G.mul_mat("Q4_K", torch.from_numpy(np.array(wq)).cuda(),
                    torch.from_numpy(np.array(x)).cuda()).cpu().numpy()
    cpu = O.mul_mat(O.TYPE_Q4_K, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    assert np.all(np.isfinite(got))


def test_op_rejects_overlapping_columns():
    """hip_qmm_mul_mat refuses column strides below the column length (outputs
    or inputs that would overlap) for every column count, with
    hipErrorInvalidValue, before any launch."""
    import ctypes
    import ggml_hip as G
    nrows, K = 1024, 4096
    wq = weights_q(O.TYPE_Q4_K, nrows, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    for ncols in (2, 4, 8, 16):
        x_d = torch.from_numpy(np.array(acts(ncols, K))).cuda()
        out = torch.zeros((ncols, nrows), device="cuda")
        ws = torch.empty(G.workspace_size("Q4_K", K, ncols, nrows), dtype=torch.uint8, device="cuda")
        for xs, ds in ((K, nrows - 1), (K - 32, nrows)):
            e = G.lib().hip_qmm_mul_mat(O.TYPE_Q4_K, G._ptr(w_d), K, nrows, w_d.stride(0), G._ptr(x_d), ncols, xs,
                                        G._ptr(out), ds, G._ptr(ws), ctypes.c_size_t(ws.numel()), G._stream())
            assert e == 1, (ncols, xs, ds, e)
    torch.cuda.synchronize()
    assert float(out.abs().sum()) == 0.0
