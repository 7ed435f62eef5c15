"""MMQ (int8 MFMA) parity: fp32 outputs within NMSE < 5e-4 of the CPU ggml
path and within 1e-5 relative of the f64 evaluation of the Q8_1 formula."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, max_rel, nmse, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
F64_TOL = 2e-6  # vs the f64 Q8_1 formula, error / max|out|
TYPES = {"Q4_K": O.TYPE_Q4_K, "Q5_K": O.TYPE_Q5_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0,
         "Q4_0": O.TYPE_Q4_0, "IQ4_XS": O.TYPE_IQ4_XS}


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("nrows,K,ncols", [(256, 4096, 128), (200, 2048, 77), (128, 14336, 9), (384, 768, 300),
                                           (1000, 4096, 17), (200, 2048, 24), (64, 512, 32), (70, 1024, 3)])
def test_mmq_parity(tname, nrows, K, ncols):
    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    got = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE


def test_mmq_config2_rows_subset():
    """Config 2 shape (Q4_K 14336x4096, T=512) at full size on the GPU, checked
    on a row subset against the oracle, plus the op-level entry point."""
    import ggml_hip as G
    nrows, K, T = 14336, 4096, 512
    wq = weights_q(O.TYPE_Q4_K, nrows, K)
    x = acts(T, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    got = G.mul_mat("Q4_K", w_d, x_d).cpu().numpy()
    rows = np.r_[0:64, 7000:7064, nrows - 64:nrows]
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(O.TYPE_Q4_K, wq[rows], len(rows), K, y, T)
    assert max_err_scaled(got[:, rows], ideal) < F64_TOL
    cpu = O.mul_mat(O.TYPE_Q4_K, wq[rows], len(rows), K, x, nth=8)
    assert nmse(got[:, rows], cpu) < NMSE_GATE


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("nrows,K,ncols", [(128, 14336, 9), (256, 4096, 40), (2048, 14336, 32)])
def test_mmq_split_k(tname, nrows, K, ncols):
    """Under-filled grids split K over workgroups; the partials are summed in a
    fixed order, so two runs agree bit for bit, and split and unsplit results
    both match the f64 formula."""
    import ggml_hip as G
    t = TYPES[tname]
    split = G.lib().hip_qmm_mmq_split_k(t, K, nrows, ncols)
    assert split > 1 and (K // 256) % split == 0
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    a = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    b = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    assert np.array_equal(a, b)
    # a workspace too small for the partials runs the GEMM unsplit
    tiny = torch.empty(16, dtype=torch.uint8, device="cuda")
    u = G.mmq(tname, w_d, K, qs, ds, workspace=tiny).cpu().numpy()
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(a, ideal) < F64_TOL, max_err_scaled(a, ideal)
    assert max_err_scaled(u, ideal) < F64_TOL, max_err_scaled(u, ideal)


@pytest.mark.parametrize("tname,nrows,K,ncols", [("Q4_K", 4096, 8192, 5), ("Q4_K", 2048, 8192, 6),
                                                 ("Q4_K", 6144, 4096, 8), ("Q4_K", 6150, 4096, 7),
                                                 ("Q5_K", 2048, 14336, 4), ("Q5_K", 4096, 4096, 8),
                                                 ("Q8_0", 4096, 8192, 4), ("Q8_0", 1024, 14336, 8),
                                                 ("Q4_0", 2048, 14336, 5), ("Q4_0", 12300, 2048, 5),
                                                 ("IQ4_XS", 2048, 14336, 5), ("IQ4_XS", 1024, 14336, 8),
                                                 ("Q6_K", 1024, 14336, 7), ("Q6_K", 2048, 14336, 8),
                                                 ("Q6_K", 2048, 14336, 6), ("Q6_K", 4096, 14336, 4)])
def test_op_few_columns(tname, nrows, K, ncols):
    """The op sends 4-8 columns of large matrices to the few-column GEMM
    instead of the GEMV (per type, where it measured faster): same bits as
    the kernel-level MMQ on the quantized columns, within the f64 and CPU
    gates, and within rounding of the GEMV."""
    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    got = G.mul_mat(tname, w_d, x_d).cpu().numpy()
    qs, ds = G.quantize_q8_1_planar(x_d)
    np.testing.assert_array_equal(got, G.mmq(tname, w_d, K, qs, ds).cpu().numpy())
    gemv = G.mul_mat_vec(tname, w_d, K, qs, ds).cpu().numpy()
    assert max_err_scaled(got, gemv) < 1e-6
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE


def test_op_few_columns_unaligned_rows_keep_the_gemv():
    """Rows the few-column kernel does not take (2-byte-aligned Q8_0 rows)
    keep the GEMV at 4-8 columns, where the 128-row tile would be slower:
    the op equals hip_qmm_mul_mat_vec on the same columns bit for bit."""
    import ggml_hip as G
    nrows, K, ncols = 4096, 8192, 6
    wq = weights_q(O.TYPE_Q8_0, nrows, K)
    w_d = _offset_copy(torch.from_numpy(np.array(wq)).cuda())
    x_d = torch.from_numpy(np.array(acts(ncols, K))).cuda()
    got = G.mul_mat("Q8_0", w_d, x_d).cpu().numpy()
    qs, ds = G.quantize_q8_1_planar(x_d)
    np.testing.assert_array_equal(got, G.mul_mat_vec("Q8_0", w_d, K, qs, ds).cpu().numpy())


def _offset_copy(w_d, off=2):
    """The same weight rows at a base `off` bytes past 16-byte alignment (a
    contiguous view into a larger buffer)."""
    buf = torch.zeros(w_d.numel() + 16, dtype=torch.uint8, device="cuda")
    v = buf[off:off + w_d.numel()].view(w_d.shape)
    v.copy_(w_d)
    return v


@pytest.mark.parametrize("tname", ["Q6_K", "Q8_0", "Q4_0"])
@pytest.mark.parametrize("nrows,K,ncols", [(1000, 4096, 3), (4096, 2048, 9), (700, 14336, 17), (4100, 4096, 32),
                                           (64, 2048, 16), (12300, 2048, 12)])
def test_few_columns_q6_k_q8_0(tname, nrows, K, ncols):
    """Q8_0 and Q4_0 with at most 32 columns and Q6_K with at most 16 take the
    few-column kernel on 16-byte-aligned rows (Q6_K from K % 2048 == 0; Q8_0
    and Q4_0 at 17-32 columns only below 8 MiB of weights, else their
    direct-transfer tile): within the f64 and CPU gates, and within rounding
    of the staged 128-row tile that the same rows take at a 2-byte-aligned
    base."""
    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    got = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    tile = G.mmq(tname, _offset_copy(w_d), K, qs, ds).cpu().numpy()
    assert max_err_scaled(got, tile) < 1e-6
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat_x86(t, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    # the op at > 8 columns goes through the same dispatch
    if ncols > 8:
        np.testing.assert_array_equal(G.mul_mat(tname, w_d, x_d).cpu().numpy(), got)


@pytest.mark.parametrize("nrows,K,ncols", [(1000, 4096, 3), (4096, 2048, 9), (700, 14336, 17), (4100, 4096, 32),
                                           (64, 2048, 16), (256, 512, 24)])
@pytest.mark.parametrize("tname", ["Q5_K", "IQ4_XS"])
def test_few_columns_q5_k_iq4_xs(tname, nrows, K, ncols):
    """Q5_K and IQ4_XS (K % 512 == 0) up to 32 columns take the few-column
    kernel (Q5_K: the Q4_K data path with the fifth bits merged from qh;
    IQ4_XS: an 8-byte-aligned window around each block, levels looked up by
    byte permutes): within the f64 and CPU gates; the op above 8 columns runs
    the same kernel."""
    import ggml_hip as G
    t = TYPES[tname]
    assert G.lib().hip_qmm_mmq_split_k(t, K, nrows, ncols) >= 1
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    got = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat_x86(t, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    if ncols > 8:
        np.testing.assert_array_equal(G.mul_mat(tname, w_d, x_d).cpu().numpy(), got)


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q8_0", "Q4_0", "IQ4_XS", "Q6_K"])
@pytest.mark.parametrize("ncols", [9, 16, 24])
def test_few_columns_large_weights(tname, ncols):
    """9-24 columns of a large weight (config 3's 4096x14336): the few-column
    kernel for every type up to 16 columns and for the K-quants and IQ4_XS at
    24, the direct-transfer tile for Q8_0 and Q4_0 at 24 (Q6_K's tile from 17
    columns): checked on a row subset against the f64 formula and the CPU
    path, and equal to the op."""
    import ggml_hip as G
    t = TYPES[tname]
    nrows, K = 4096, 14336
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    got = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    rows = np.r_[0:64, 2000:2064, nrows - 64:nrows]
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq[rows], len(rows), K, y, ncols)
    assert max_err_scaled(got[:, rows], ideal) < F64_TOL, max_err_scaled(got[:, rows], ideal)
    cpu = O.mul_mat_x86(t, wq[rows], len(rows), K, x, nth=8)
    assert nmse(got[:, rows], cpu) < NMSE_GATE
    np.testing.assert_array_equal(G.mul_mat(tname, w_d, x_d).cpu().numpy(), got)


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K"])
@pytest.mark.parametrize("nrows,K,ncols", [(1000, 4096, 1), (1000, 4096, 2), (4100, 4096, 3), (6144, 2048, 5),
                                           (300, 14336, 8), (64, 512, 7), (14336, 4096, 8), (4096, 14336, 6),
                                           (12300, 2048, 8), (12300, 1280, 4)])
def test_few_columns_packed(tname, nrows, K, ncols):
    """Up to 8 columns the few-column kernel packs two sub-blocks into each
    MFMA (Q4_K / Q5_K: two 32-deep sub-blocks per 16x16x64, Q6_K: two 16-deep
    sub-blocks per 16x16x32; output columns 0-7 against the even sub-block,
    8-15 the odd one, halves added at the end): within the f64 and CPU gates,
    split and unsplit (small row counts split K; 14336 rows run two K halves
    per workgroup), and within rounding of the GEMV on the same quantized
    columns.  Q6_K at K = 512 is not the few-column kernel's (its aligned
    windows need K % 2048 == 0) and runs the tile."""
    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = acts(ncols, K)
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(np.array(x)).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    got = G.mmq(tname, w_d, K, qs, ds).cpu().numpy()
    tiny = torch.empty(16, dtype=torch.uint8, device="cuda")
    unsplit = G.mmq(tname, w_d, K, qs, ds, workspace=tiny).cpu().numpy()
    gemv = G.mul_mat_vec(tname, w_d, K, qs, ds).cpu().numpy()
    assert max_err_scaled(got, gemv) < 1e-6, max_err_scaled(got, gemv)
    assert max_err_scaled(unsplit, gemv) < 1e-6, max_err_scaled(unsplit, gemv)
    rows = np.arange(nrows) if nrows <= 1024 else np.r_[0:96, nrows // 2:nrows // 2 + 96, nrows - 96:nrows]
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq[rows], len(rows), K, y, ncols)
    assert max_err_scaled(got[:, rows], ideal) < F64_TOL, max_err_scaled(got[:, rows], ideal)
    cpu = O.mul_mat(t, wq[rows], len(rows), K, x, nth=8)
    assert nmse(got[:, rows], cpu) < NMSE_GATE
