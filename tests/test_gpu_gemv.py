"""Decode GEMV (1..8 columns) parity: integer block dots exact, fp32 outputs
within NMSE < 5e-4 of the CPU ggml path (and within 1e-5 relative of the
f64 evaluation of the same Q8_1 formula)."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, max_rel, nmse, weights_f32, weights_q

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
# Q8_0 at 3-4 columns and rows of K <= 2048), where the per-column grid below
# does not take them: the op runs the
# quantize-in-GEMV kernel over all columns in one launch (2 columns for the
# K-quants, 3 for IQ4_XS, 4 for Q8_0 / Q4_0; twice that on at most 4096 rows
# as two rows of its grid, except Q4_0).  Where the one-column op runs
# one K share, each column equals it bit for bit; where the one-column op
# splits the row into K shares (Q8_0 / Q4_0 rows of two 2048-steps on at most
# 2048 rows: attn_k / attn_v shapes) the one-launch kernel adds both steps in
# each lane before the wave sum, another rounding order, so only the f64 and
# CPU gates apply.
@pytest.mark.parametrize("tname,nrows,K,ncols", [("Q4_K", 4096, 4096, 2), ("Q5_K", 1000, 4096, 2),
                                                 ("Q6_K", 1024, 4096, 2), ("IQ4_XS", 777, 2048, 3),
                                                 ("Q8_0", 4100, 4096, 4), ("Q4_0", 333, 96, 3),
                                                 ("Q8_0", 5000, 1024, 3), ("Q4_0", 4097, 4096, 2),
                                                 ("IQ4_XS", 6000, 4096, 2), ("Q8_0", 9000, 4096, 3),
                                                 ("Q4_K", 8200, 2048, 2), ("Q4_0", 8195, 1024, 4),
                                                 ("Q8_0", 1024, 4096, 2), ("Q4_0", 500, 4096, 3),
                                                 ("Q8_0", 2048, 4096, 4), ("Q4_K", 4096, 4096, 4),
                                                 ("Q6_K", 3000, 4096, 4), ("Q5_K", 2500, 3072, 4),
                                                 ("IQ4_XS", 4096, 2048, 6), ("Q8_0", 4096, 4096, 8),
                                                 ("Q8_0", 4000, 1024, 8)])
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


# 2-8 f32 columns of matrices of at most 2048 rows of at most 4096 elements
# (Q8_0 / Q4_0: 1024 rows, up to 4 columns unless K <= 2048): the op runs every column
# through the one-column kernel as one row of its grid
# (qmm_mul_mat_fx_percol, gemv.hip), so each column equals the one-column op
# on it bit for bit, K shares included.  Columns strided in and out; nothing
# is written past a column's rows.
@pytest.mark.parametrize("tname,nrows,K,ncols", [("Q4_K", 1024, 4096, 8), ("Q4_K", 2048, 4096, 3),
                                                 ("Q5_K", 1000, 2048, 5), ("Q6_K", 1024, 4096, 4),
                                                 ("Q6_K", 777, 4096, 8), ("IQ4_XS", 2048, 4096, 6),
                                                 ("Q8_0", 1024, 4096, 4), ("Q8_0", 520, 1024, 2),
                                                 ("Q4_K", 300, 256, 7), ("Q6_K", 64, 2048, 2),
                                                 ("Q4_0", 1024, 4096, 3), ("Q4_0", 1000, 2048, 8),
                                                 ("Q8_0", 700, 2048, 6)])
def test_op_few_columns_per_column_grid(tname, nrows, K, ncols):
    import ctypes

    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    xb = torch.zeros((ncols, K + 64), dtype=torch.float32, device="cuda")
    xb[:, :K] = torch.from_numpy(np.array(x)).cuda()
    x_d = xb[:, :K]
    ob = torch.full((ncols, nrows + 40), 7.0, dtype=torch.float32, device="cuda")
    ws = torch.empty(max(16, G.workspace_size(tname, K, ncols, nrows)), dtype=torch.uint8, device="cuda")
    e = G.lib().hip_qmm_mul_mat(t, G._ptr(w_d), K, nrows, w_d.stride(0), G._ptr(x_d), ncols, K + 64, G._ptr(ob),
                                nrows + 40, G._ptr(ws), ctypes.c_size_t(ws.numel()), G._stream())
    assert e == 0, e
    got = ob.cpu().numpy()
    assert np.all(got[:, nrows:] == 7.0)
    got = got[:, :nrows]
    for c in range(ncols):
        one = G.mul_mat_vec_f32(tname, w_d, K, x_d[c]).cpu().numpy().reshape(-1)
        np.testing.assert_array_equal(got[c], one)
    y = G.quantize_q8_1(x_d.contiguous(), K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)


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


# ---------------------------------------------------------------- the reference's MMVQ launch

def _aos(G, x2d, K, padded=True):
    xd = torch.from_numpy(np.ascontiguousarray(x2d, dtype=np.float32)).cuda()
    return G.quantize_q8_1(xd) if padded else G.quantize_q8_1(xd, K)


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
def test_mul_mat_vec_q_broadcast_channels_and_samples(tname):
    """hip_qmm_mul_mat_vec_q without ids: 3 columns x 4 destination channels x
    2 samples in one launch, weights broadcast over channels (ratio 2) and
    samples (ratio 2), AoS Q8_1 activations padded to 512 as the reference's
    quantizer leaves them; every (channel, sample) slice against the f64
    formula and the CPU path on its own weight matrix."""
    import ggml_hip as G
    t = TYPES[tname]
    K, M, N = 2048, 300, 3
    ncx, nsx, ncd, nsd = 2, 1, 4, 2
    bs, bb = O.BLOCK[t]
    wq = np.stack([np.array(weights_q(t, M, K, idx)) for idx in range(ncx * nsx)])
    rb_blocks = wq.shape[2] // bb
    x = np.array(acts(nsd * ncd * N, K)).reshape(nsd, ncd, N, K)
    y = _aos(G, x.reshape(-1, K), K)
    cb = G.padded_k(K) // 32
    dst = torch.full((nsd, ncd, N, M), float("nan"), device="cuda")
    G.mul_mat_vec_q(tname, torch.from_numpy(wq).cuda(), y, K, N, dst, nchannels_x=ncx, nchannels_y=ncd,
                    nchannels_dst=ncd, nsamples_x=nsx, nsamples_dst=nsd, stride_col_y=cb, stride_col_dst=M,
                    stride_channel_x=M * rb_blocks, stride_channel_y=N * cb, stride_channel_dst=N * M,
                    stride_sample_x=ncx * M * rb_blocks, stride_sample_y=ncd * N * cb, stride_sample_dst=ncd * N * M)
    got = dst.cpu().numpy()
    yk = _aos(G, x.reshape(-1, K), K, padded=False).cpu().numpy().reshape(nsd, ncd, N, -1)
    for s in range(nsd):
        for ch in range(ncd):
            wsl = wq[(s // (nsd // nsx)) * ncx + ch // (ncd // ncx)]
            ideal = O.mul_mat_q8_1_f64(t, wsl, M, K, yk[s, ch], N)
            assert max_err_scaled(got[s, ch], ideal) < F64_TOL, (s, ch, max_err_scaled(got[s, ch], ideal))
            assert nmse(got[s, ch], O.mul_mat(t, wsl, M, K, x[s, ch], nth=8)) < NMSE_GATE


@pytest.mark.parametrize("tname", ["Q4_K", "Q6_K", "Q8_0", "IQ4_XS"])
@pytest.mark.parametrize("ne11", [1, 4])
def test_mul_mat_vec_q_ids(tname, ne11):
    """hip_qmm_mul_mat_vec_q with ids (MUL_MAT_ID): 3 tokens x 4 slots, one
    activation row per token (ne11 = 1) or per slot, ids of -1 and past the
    expert count writing zero rows; against mul_mat_id on the CPU and the f64
    formula per expert."""
    import ggml_hip as G
    t = TYPES[tname]
    n_as, M, K, n_tokens, n_ids = 5, 200, 1024, 3, 4
    bs, bb = O.BLOCK[t]
    wq = O.quantize_rows(t, np.array(weights_f32(n_as * M, K, 3))).reshape(n_as, M, -1)
    rb_blocks = wq.shape[2] // bb
    ids = np.random.default_rng(ne11).integers(0, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    ids[0, 1] = -1
    ids[2, 3] = n_as + 2
    x = np.array(acts(n_tokens * ne11, K, 2)).reshape(n_tokens, ne11, K)
    y = _aos(G, x.reshape(-1, K), K)
    cb = G.padded_k(K) // 32
    dst = torch.full((n_tokens, n_ids, M), float("nan"), device="cuda")
    G.mul_mat_vec_q(tname, torch.from_numpy(wq).cuda(), y, K, n_tokens, dst, nchannels_x=n_as, nchannels_y=ne11,
                    nchannels_dst=n_ids, stride_col_y=ne11 * cb, stride_col_dst=n_ids * M,
                    stride_channel_x=M * rb_blocks, stride_channel_y=cb, stride_channel_dst=M,
                    ids=torch.from_numpy(ids).cuda(), ids_stride=n_ids)
    got = dst.cpu().numpy()
    bad = (ids < 0) | (ids >= n_as)
    assert np.all(got[bad] == 0.0)
    ok_ids = np.where(bad, -1, ids).astype(np.int32)
    assert nmse(got, O.mul_mat_id(t, wq, n_as, M, K, x, ok_ids, nth=8)) < NMSE_GATE
    yk = _aos(G, x.reshape(-1, K), K, padded=False).cpu().numpy()
    from cases import mul_mat_id_f64
    ideal = mul_mat_id_f64(t, wq, M, K, yk, ne11, ok_ids)
    assert max_err_scaled(got, ideal) < F64_TOL


@pytest.mark.parametrize("tname,nrows,K,ncols", [("Q8_0", 4100, 2048, 1), ("Q4_0", 4100, 2048, 2),
                                                 ("Q6_K", 4100, 4096, 3), ("Q4_K", 4100, 4096, 1),
                                                 ("IQ4_XS", 4100, 4096, 1), ("Q5_K", 4100, 4096, 1)])
def test_mul_mat_vec_q_equals_the_planar_gemv(tname, nrows, K, ncols):
    """On shapes where hip_qmm_mul_mat_vec runs the two-rows-per-wave kernel,
    the AoS launch gives the same bits: the same slices, dots and order."""
    import ggml_hip as G
    t, wq, x, w_d, x_d, qs, planar = _run(tname, nrows, K, ncols)
    y = G.quantize_q8_1(x_d)
    cb = G.padded_k(K) // 32
    dst = torch.full((ncols, nrows), float("nan"), device="cuda")
    G.mul_mat_vec_q(tname, w_d, y, K, ncols, dst, stride_col_y=cb, stride_col_dst=nrows)
    np.testing.assert_array_equal(dst.cpu().numpy(), planar)


def test_mul_mat_vec_q_rejects_bad_launches():
    import ggml_hip as G
    t = O.TYPE_Q4_K
    K, M = 1024, 64
    w_d = torch.from_numpy(np.array(weights_q(t, M, K))).cuda()
    y = G.quantize_q8_1(torch.zeros((2, K), device="cuda"))
    dst = torch.zeros((2, M), device="cuda")
    cb = G.padded_k(K) // 32
    ok = dict(stride_col_y=cb, stride_col_dst=M)
    with pytest.raises(G.HipQmmError):  # channel ratio not whole
        G.mul_mat_vec_q("Q4_K", w_d, y, K, 1, dst, nchannels_x=2, nchannels_y=3, nchannels_dst=3, **ok)
    with pytest.raises(G.HipQmmError):  # columns shorter than the row
        G.mul_mat_vec_q("Q4_K", w_d, y, K, 2, dst, stride_col_y=K // 32 - 1, stride_col_dst=M)
    with pytest.raises(G.HipQmmError):  # more than 8 columns
        G.mul_mat_vec_q("Q4_K", w_d, y, K, 9, dst, **ok)
    with pytest.raises(G.HipQmmError):  # overlapping output columns
        G.mul_mat_vec_q("Q4_K", w_d, y, K, 2, dst, stride_col_y=cb, stride_col_dst=M - 1)
    torch.cuda.synchronize()
    assert float(dst.abs().sum()) == 0.0
