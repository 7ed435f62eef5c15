"""The reference's own boundary cases for this path, from its CUDA op diff
(harness/cuda_ops_diff.c:505-541, 713-726), run on the HIP kernels:

- MUL_MAT of a 64-row weight against one f32 column at the K where the
  upstream MMVQ's per-lane depth decides how the K sum is split: Q8_0 at
  K = 1056, Q4_K / Q5_K / Q6_K at K = 2304, Q4_0 at K = 2080 (the harness's
  Q4_1 / Q5_0 / Q5_1 / IQ4_NL cases are types this backend does not take).
  1056 is 33 blocks of 32 and 2304 is 36 slices of 64 weights: one past the
  32-slice lane segments of this repository's one-column GEMVs, so a lane
  segment runs short.  Every one-column entry point is checked: the op
  (quantization fused into the GEMV), the GEMV on planar Q8_1, the
  reference-shaped hip_qmm_mul_mat_vec_q on AoS block_q8_1, and, for Q4_K
  and Q6_K, the MFMA GEMV;
- MUL_MAT_ID with 8 experts of 64 x 256, 2 used per token, one activation
  row per slot, at 8 and 9 tokens (the GEMV / grouped-MMQ boundary), Q4_0
  and Q4_K.

Gates (as the configuration cells): within 2e-6 (error / max |out|) of the
f64 evaluation of the Q8_1 formula, and NMSE < 5e-4 against the CPU path an
x86 AVX2 host takes."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, nmse, route_top_k, weights_f32, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
F64_TOL = 2e-6
MMVQ_CASES = [("Q8_0", 1056), ("Q4_K", 2304), ("Q5_K", 2304), ("Q6_K", 2304), ("Q4_0", 2080)]


def _gates(got, t, wq, nrows, K, x):
    got = np.asarray(got, dtype=np.float64).reshape(1, nrows)
    assert np.all(np.isfinite(got))
    yq = O.quantize_rows(O.TYPE_Q8_1, np.ascontiguousarray(x, dtype=np.float32).reshape(1, K))
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, yq, 1)
    cpu = O.mul_mat_x86(t, wq, nrows, K, x.reshape(1, K), nth=2)
    assert max_err_scaled(got, ideal) < F64_TOL
    assert nmse(got, cpu) < NMSE_GATE


@pytest.mark.parametrize("tname,K", MMVQ_CASES, ids=[f"{t}-k{K}" for t, K in MMVQ_CASES])
def test_one_column_at_the_reference_mmvq_boundary_k(tname, K):
    import ggml_hip as G
    t = O.TYPE_IDS[tname]
    nrows = 64
    wq = weights_q(t, nrows, K, 3)
    x = np.array(acts(1, K, 3))
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(x).cuda()
    outs = {"op": G.mul_mat(tname, w_d, x_d).cpu().numpy()}
    qs, ds = G.quantize_q8_1_planar(x_d)
    outs["gemv planar"] = G.mul_mat_vec(tname, w_d, K, qs, ds).cpu().numpy()
    y = G.quantize_q8_1(x_d)
    dst = torch.full((1, nrows), float("nan"), device="cuda")
    outs["mul_mat_vec_q"] = G.mul_mat_vec_q(tname, w_d, y, K, 1, dst, stride_col_y=y.shape[1] // 36,
                                            stride_col_dst=nrows).cpu().numpy()
    if K % 256 == 0 and tname in ("Q4_K", "Q6_K"):
        outs["gemv mfma"] = G.gemv_mfma(tname, w_d, K, qs, ds).cpu().numpy()
    for name, got in outs.items():
        try:
            _gates(got, t, wq, nrows, K, x)
        except AssertionError as e:
            raise AssertionError(f"{name}: {e}") from None
    # the AoS entry point reads the same bytes as the planar GEMV (bit for bit
    # where both run the two-rows-per-wave kernel; the Q4_0 planar GEMV streams
    # rows and sums in another order)
    assert max_err_scaled(outs["mul_mat_vec_q"], outs["gemv planar"]) < 1e-6


@pytest.mark.parametrize("tname", ["Q4_0", "Q4_K"])
@pytest.mark.parametrize("n_tokens", [8, 9])
def test_mul_mat_id_at_the_reference_gemv_mmq_boundary(tname, n_tokens):
    import ggml_hip as G
    t = O.TYPE_IDS[tname]
    n_as, n_used, M, K = 8, 2, 64, 256
    wq = O.quantize_rows(t, weights_f32(n_as * M, K, 4)).reshape(n_as, M, -1)
    x = np.array(acts(n_tokens * n_used, K, 4)).reshape(n_tokens, n_used, K)
    ids, _ = route_top_k(n_tokens, n_as, n_used, seed=45)
    out = torch.full((n_tokens, n_used, M), float("nan"), device="cuda")
    got = G.mul_mat_id(tname, torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(),
                       out=out).cpu().numpy()
    assert np.all(np.isfinite(got))
    cpu = O.mul_mat_id(t, wq, n_as, M, K, x, ids, nth=2)
    ys = O.quantize_rows(O.TYPE_Q8_1, x.reshape(-1, K))
    ideal = np.zeros((n_tokens, n_used, M))
    for e in np.unique(ids):
        ts, ss = np.nonzero(ids == e)
        ideal[ts, ss] = O.mul_mat_q8_1_f64(t, wq[e], M, K, ys[ts * n_used + ss], len(ts))
    assert max_err_scaled(got, ideal) < F64_TOL
    assert nmse(got, cpu) < NMSE_GATE
