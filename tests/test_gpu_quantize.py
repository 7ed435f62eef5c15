"""Q8_1 activation quantizer on the GPU: bytes equal quantize_row_q8_1_ref."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts
from golden_patterns import QUANT_PATTERNS, VECDOT_PATTERNS, quant_src, vecdot_fill

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _gpu_q8_1(x_np, ne0_padded=None):
    import ggml_hip as G
    x = torch.from_numpy(np.ascontiguousarray(x_np, dtype=np.float32)).cuda()
    if x.dim() == 1:
        x = x[None, :]
    return G.quantize_q8_1(x, ne0_padded).cpu().numpy()


def _ref_q8_1(x_np, ne0_padded):
    x_np = np.atleast_2d(np.asarray(x_np, dtype=np.float32))
    out = []
    for row in x_np:
        padded = np.zeros(ne0_padded, dtype=np.float32)
        padded[: row.size] = row
        out.append(O.quantize_ref(O.TYPE_Q8_1, padded))
    return np.stack(out)


@pytest.mark.parametrize("pattern", VECDOT_PATTERNS)
def test_q8_1_vecdot_patterns_bit_exact(pattern):
    x, y = vecdot_fill(pattern)
    for v in (x, y):
        np.testing.assert_array_equal(_gpu_q8_1(v, 512), _ref_q8_1(v, 512))


@pytest.mark.parametrize("pattern", QUANT_PATTERNS)
def test_q8_1_quant_patterns_bit_exact(pattern):
    x = quant_src(pattern).reshape(4, 256)
    np.testing.assert_array_equal(_gpu_q8_1(x, 256), _ref_q8_1(x, 256))


@pytest.mark.parametrize("K,ncols", [(4096, 8), (14336, 2), (2048, 512), (768, 5)])
def test_q8_1_config_shapes_bit_exact(K, ncols):
    x = acts(ncols, K)
    Kp = (K + 511) // 512 * 512
    np.testing.assert_array_equal(_gpu_q8_1(x, Kp), _ref_q8_1(x, Kp))


def test_q8_1_ties_and_extremes():
    """Exact halves at the step (round half away from zero), tiny/huge scales,
    and a block holding +-amax only."""
    rows = []
    t = np.zeros(256, dtype=np.float32)
    t[0::32] = 127.0
    for i in range(256):
        if i % 32:
            t[i] = (i % 9 - 4) + 0.5
    rows.append(t)
    rows.append(np.full(256, 1e-30, dtype=np.float32))
    rows.append(np.linspace(-3e4, 3e4, 256, dtype=np.float32))
    rows.append(np.where(np.arange(256) % 2, 1.0, -1.0).astype(np.float32))
    x = np.stack(rows)
    np.testing.assert_array_equal(_gpu_q8_1(x, 512), _ref_q8_1(x, 512))


def test_planar_layout_holds_the_same_bytes():
    import ggml_hip as G
    K, n = 4096, 3
    x = torch.from_numpy(np.array(acts(n, K))).cuda()
    aos = G.quantize_q8_1(x).cpu().numpy().reshape(n, K // 32, 36)
    qs, ds = G.quantize_q8_1_planar(x)
    qs, ds = qs.cpu().numpy(), ds.cpu().numpy()
    np.testing.assert_array_equal(aos[:, :, 4:].reshape(n, K).view(np.int8), qs[:, :K])
    np.testing.assert_array_equal(aos[:, :, :4].copy().view(np.int32).reshape(n, K // 32), ds)
