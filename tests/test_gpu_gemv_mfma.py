"""Small-batch GEMV on int8 MFMA: parity with the CPU ggml path (NMSE gate)
and with the f64 evaluation of the Q8_1 formula, for 1..16 columns, row
counts that are not multiples of the 16-row tile, and K split unevenly over
the workgroup's 4 waves."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, nmse, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
F64_TOL = 2e-6
TYPES = {"Q4_K": O.TYPE_Q4_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0}


@pytest.mark.parametrize("tname", ["Q4_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("nrows,K,ncols", [(256, 4096, 1), (200, 4096, 2), (96, 768, 5), (1024, 4096, 8),
                                           (77, 1536, 16), (64, 14336, 4)])
def test_gemv_mfma_parity(tname, nrows, K, ncols):
    import ggml_hip as G
    t = TYPES[tname]
    wq = weights_q(t, nrows, K)
    x = np.array(acts(ncols, K))
    w_d = torch.from_numpy(np.array(wq)).cuda()
    x_d = torch.from_numpy(x).cuda()
    qs, ds = G.quantize_q8_1_planar(x_d)
    out = torch.full((ncols, nrows), float("nan"), dtype=torch.float32, device="cuda")
    got = G.gemv_mfma(tname, w_d, K, qs, ds, out=out).cpu().numpy()
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, ncols)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    if ncols <= 8:  # same integer dots as the v_dot4 GEMV; fp32 sums in another order
        dot4 = G.mul_mat_vec(tname, w_d, K, qs, ds).cpu().numpy()
        assert max_err_scaled(got, dot4) < F64_TOL
