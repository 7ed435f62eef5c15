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


@pytest.mark.parametrize("K,pad", [(768, 0), (4096, 4), (1024, 1)])
def test_planar_matches_reference_on_ties_and_strides(K, pad):
    """The planar quantizer (8 values per lane with quad reductions for
    16-byte-aligned x, one value per lane otherwise) against
    quantize_row_q8_1_ref, on tie-heavy and extreme rows, with and without
    the 512-padding and with row strides that do and do not allow 16-byte
    loads.  Padding blocks must come out as zero blocks."""
    import ggml_hip as G
    rng = np.random.default_rng(9)
    n = 6
    rows = [np.array(acts(1, K))[0],
            (rng.integers(-254, 255, size=K) * np.float32(0.5)).astype(np.float32),  # x.5 ties after scaling
            np.full(K, 3.0, dtype=np.float32),
            np.where(np.arange(K) % 3 == 0, 1e-30, -7.5).astype(np.float32),
            (rng.standard_normal(K) * 1e4).astype(np.float32),
            np.zeros(K, dtype=np.float32)]
    x = np.zeros((n, K + pad), dtype=np.float32)
    x[:, :K] = np.stack(rows)
    xd = torch.from_numpy(x).cuda()[:, :K]
    Kp = G.padded_k(K)
    qs = torch.empty((n, Kp), dtype=torch.int8, device="cuda")
    ds = torch.empty((n, Kp // 32), dtype=torch.int32, device="cuda")
    L = G.lib()
    assert L.hip_qmm_quantize_q8_1_planar(G._ptr(xd), K, n, K + pad, G._ptr(qs), G._ptr(ds), G._stream()) == 0
    qs, ds = qs.cpu().numpy(), ds.cpu().numpy()
    for r in range(n):
        ref = O.quantize_ref(O.TYPE_Q8_1, x[r, :K]).reshape(-1, 36)
        np.testing.assert_array_equal(qs[r, :K], ref[:, 4:].reshape(-1).view(np.int8))
        np.testing.assert_array_equal(ds[r, :K // 32], ref[:, :4].copy().view(np.int32).reshape(-1))
        assert not qs[r, K:].any() and not ds[r, K // 32:].any()
