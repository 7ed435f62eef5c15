"""hip_qmm_mul_mat_noalloc through the C ABI: the same results as
hip_qmm_mul_mat with a caller-owned workspace, bit for bit, on successive
calls that share the device's scratch array (the later ones with smaller
inputs, so stale scratch from a larger call is present), and shapes whose
workspace exceeds the array rejected before any launch."""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from cases import acts, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # HIP_QMM_NOALLOC_SCRATCH_BYTES


def _lib():
    import ggml_hip as G
    L = G.lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.hip_qmm_mul_mat_noalloc.restype = ctypes.c_int
    L.hip_qmm_mul_mat_noalloc.argtypes = [ctypes.c_int, vp, i64, i64, i64, vp, i64, i64, vp, i64, vp]
    return G, L


# one case per dispatch path, in decreasing workspace: MMQ with split-K
# partials (18.8 MB), the few-column GEMM with split-K (3.3 MB), the MMQ
# (2.4 MB), quantizer + GEMV, the one-launch 2-4 column GEMV (no scratch),
# the one-column fused GEMV (no scratch)
CASES = [("Q4_K", 4096, 14336, 128), ("Q4_K", 4096, 4096, 24), ("Q4_K", 4096, 4096, 512), ("Q6_K", 1024, 4096, 7),
         ("Q8_0", 1024, 4096, 3), ("Q4_K", 4096, 4096, 1)]


def test_noalloc_matches_mul_mat_on_successive_calls():
    G, L = _lib()
    prev = None
    for tname, nrows, K, T in CASES:
        t = O.TYPE_IDS[tname]
        need = G.workspace_size(tname, K, T, nrows)
        assert need <= SCRATCH_BYTES
        if prev is not None:
            assert need <= prev  # each call smaller than the one before
        prev = need
        w_d = torch.from_numpy(np.array(weights_q(t, nrows, K))).cuda()
        x_d = torch.from_numpy(np.array(acts(T, K))).cuda()
        want = G.mul_mat(tname, w_d, x_d).cpu().numpy()
        out = torch.full((T, nrows), float("nan"), device="cuda")
        e = L.hip_qmm_mul_mat_noalloc(t, G._ptr(w_d), K, nrows, w_d.stride(0), G._ptr(x_d), T, K, G._ptr(out),
                                      nrows, G._stream())
        assert e == 0, (tname, nrows, K, T, e)
        np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_noalloc_rejects_a_workspace_beyond_the_array():
    G, L = _lib()
    K, nrows, T = 4096, 256, 8192  # 8192 columns of Q8_1: 37.7 MB > 32 MiB
    assert G.workspace_size("Q4_K", K, T, nrows) > SCRATCH_BYTES
    w_d = torch.from_numpy(np.array(weights_q(O.TYPE_Q4_K, nrows, K))).cuda()
    x_d = torch.zeros((T, K), device="cuda")
    out = torch.zeros((T, nrows), device="cuda")
    e = L.hip_qmm_mul_mat_noalloc(O.TYPE_Q4_K, G._ptr(w_d), K, nrows, w_d.stride(0), G._ptr(x_d), T, K, G._ptr(out),
                                  nrows, G._stream())
    assert e == 1
    torch.cuda.synchronize()
    assert float(out.abs().sum()) == 0.0


def test_noalloc_under_graph_capture():
    """The callers the entry point is for capture it: after one eager call
    (which looks up the scratch array's address), two calls of different
    shapes (the few-column GEMM with split-K partials in the scratch, then
    the quantizer + GEMV) are captured into one HIP graph.  Every replay,
    with eager work and synchronizations between replays, equals
    hip_qmm_mul_mat bit for bit."""
    G, L = _lib()
    cases = [("Q4_K", 4096, 4096, 24), ("Q8_0", 1024, 4096, 3)]
    ins, wants, outs = [], [], []
    for tname, nrows, K, T in cases:
        t = O.TYPE_IDS[tname]
        w_d = torch.from_numpy(np.array(weights_q(t, nrows, K))).cuda()
        x_d = torch.from_numpy(np.array(acts(T, K))).cuda()
        ins.append((t, w_d, x_d, nrows, K, T))
        wants.append(G.mul_mat(tname, w_d, x_d).cpu().numpy())
        outs.append(torch.full((T, nrows), float("nan"), device="cuda"))

    def call(i):
        t, w_d, x_d, nrows, K, T = ins[i]
        return L.hip_qmm_mul_mat_noalloc(t, G._ptr(w_d), K, nrows, w_d.stride(0), G._ptr(x_d), T, K,
                                         G._ptr(outs[i]), nrows, G._stream())

    assert call(0) == 0  # eager first call on the device
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        with torch.cuda.graph(g, stream=cs):
            assert call(0) == 0 and call(1) == 0
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        G.mul_mat("Q4_K", ins[0][1], ins[0][2])  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, want in zip(outs, wants):
            np.testing.assert_array_equal(o.cpu().numpy(), want, err_msg=f"replay {rep}")
