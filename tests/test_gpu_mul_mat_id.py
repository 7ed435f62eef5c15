"""MUL_MAT_ID (expert-grouped MMQ) parity against the CPU ggml path
(ggml_compute_forward_mul_mat_id restated) and the f64 Q8_1 formula."""
import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, mul_mat_id_f64, nmse, route_top_k, weights_f32

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
F64_TOL = 2e-6
TYPES = {"Q4_K": O.TYPE_Q4_K, "Q5_K": O.TYPE_Q5_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0,
         "Q4_0": O.TYPE_Q4_0, "IQ4_XS": O.TYPE_IQ4_XS}


def _experts(t, n_as, nrows, K):
    w = weights_f32(n_as * nrows, K)
    return O.quantize_rows(t, w).reshape(n_as, nrows, -1)


def _run(tname, n_as, nrows, K, x, ids):
    import ggml_hip as G
    t = TYPES[tname]
    wq = _experts(t, n_as, nrows, K)
    got = G.mul_mat_id(tname, torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(),
                       torch.from_numpy(ids).cuda()).cpu().numpy()
    return t, wq, got


def _check(tname, n_as, nrows, K, x, ids):
    import ggml_hip as G
    t, wq, got = _run(tname, n_as, nrows, K, x, ids)
    n_tokens, ne11, _ = x.shape
    cpu = O.mul_mat_id(t, wq, n_as, nrows, K, x, ids, nth=8)
    assert np.all(got[ids < 0] == 0.0)
    assert nmse(got, cpu) < NMSE_GATE, nmse(got, cpu)
    y = G.quantize_q8_1(torch.from_numpy(x.reshape(-1, K)).cuda(), K).cpu().numpy()
    ideal = mul_mat_id_f64(t, wq, nrows, K, y, ne11, ids)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
    return got


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("ne11", [1, 3])
def test_mul_mat_id_random_ids(tname, ne11):
    n_as, nrows, K, n_tokens, n_ids = 8, 160, 512, 37, 3
    rng = np.random.default_rng(5)
    ids = rng.integers(-1, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    x = np.array(acts(n_tokens * ne11, K)).reshape(n_tokens, ne11, K)
    _check(tname, n_as, nrows, K, x, ids)


def test_mul_mat_id_uneven_and_single_expert():
    """Every slot routed to one expert (one long column list, many tiles)."""
    n_as, nrows, K, n_tokens, n_ids = 16, 128, 256, 150, 2
    ids = np.full((n_tokens, n_ids), 11, dtype=np.int32)
    ids[::7, 1] = -1
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    _check("Q4_K", n_as, nrows, K, x, ids)


def test_mul_mat_id_decode_one_token():
    n_as, nrows, K = 32, 256, 1024
    ids = np.array([[3, 17, 31, 0, 9, 22, 5, 30]], dtype=np.int32)
    x = np.array(acts(1, K)).reshape(1, 1, K)
    _check("Q4_K", n_as, nrows, K, x, ids)


def test_mul_mat_id_all_ids_negative():
    import ggml_hip as G
    n_as, nrows, K, n_tokens, n_ids = 4, 64, 256, 5, 2
    ids = np.full((n_tokens, n_ids), -1, dtype=np.int32)
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    wq = _experts(O.TYPE_Q4_K, n_as, nrows, K)
    out = torch.full((n_tokens, n_ids, nrows), float("nan"), device="cuda")
    got = G.mul_mat_id("Q4_K", torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(),
                       torch.from_numpy(ids).cuda(), out=out).cpu().numpy()
    assert np.all(got == 0.0)


def test_mul_mat_id_config4_qwen3_moe_gate():
    """Config 4 (Qwen3-30B-A3B shape): 128 experts of Q4_K 768x2048, 512 tokens
    routed top-8 by softmax over seeded N(0,1) logits; broadcast activations
    (gate/up projection).  Full size on the GPU, oracle on a token subset."""
    import ggml_hip as G
    n_as, nrows, K, n_tokens, k = 128, 768, 2048, 512, 8
    ids, _ = route_top_k(n_tokens, n_as, k)
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    t = O.TYPE_Q4_K
    wq = _experts(t, n_as, nrows, K)
    got = G.mul_mat_id("Q4_K", torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(),
                       torch.from_numpy(ids).cuda()).cpu().numpy()
    sub = np.arange(0, n_tokens, 16)
    cpu = O.mul_mat_id(t, wq, n_as, nrows, K, x[sub], ids[sub], nth=8)
    assert nmse(got[sub], cpu) < NMSE_GATE
    y = G.quantize_q8_1(torch.from_numpy(x[sub].reshape(-1, K)).cuda(), K).cpu().numpy()
    ideal = mul_mat_id_f64(t, wq, nrows, K, y, 1, ids[sub])
    assert max_err_scaled(got[sub], ideal) < F64_TOL


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("n_tokens,ne11", [(1, 1), (3, 1), (8, 1), (2, 4)])
def test_mul_mat_id_few_tokens(tname, n_tokens, ne11):
    """Up to 8 tokens run the one-launch GEMV over (token, slot) pairs: each
    row equals the one-column fused GEMV of its expert bit for bit, ids of -1
    or past n_as give zero rows, and the result passes the CPU gates."""
    import ggml_hip as G
    n_as, nrows, K, n_ids = 12, 320, 1024, 4
    rng = np.random.default_rng(n_tokens * 10 + ne11)
    ids = rng.integers(0, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    ids[0, 1] = -1
    if n_tokens > 1:
        ids[1, 2] = n_as + 3  # out of range: a zero row, like -1
    x = np.array(acts(n_tokens * ne11, K)).reshape(n_tokens, ne11, K)
    t = TYPES[tname]
    wq = _experts(t, n_as, nrows, K)
    w_d, x_d = torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda()
    out = torch.full((n_tokens, n_ids, nrows), float("nan"), device="cuda")
    got = G.mul_mat_id(tname, w_d, x_d, torch.from_numpy(ids).cuda(), out=out).cpu().numpy()
    bad = (ids < 0) | (ids >= n_as)
    assert np.all(got[bad] == 0.0)
    for tt in range(n_tokens):
        for s in range(n_ids):
            if bad[tt, s]:
                continue
            one = G.mul_mat_vec_f32(tname, w_d[ids[tt, s]], K, x_d[tt, s % ne11]).cpu().numpy().reshape(-1)
            np.testing.assert_array_equal(got[tt, s], one)
    ok_ids = np.where(bad, -1, ids).astype(np.int32)
    cpu = O.mul_mat_id(t, wq, n_as, nrows, K, x, ok_ids, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    y = G.quantize_q8_1(x_d.reshape(-1, K), K).cpu().numpy()
    ideal = mul_mat_id_f64(t, wq, nrows, K, y, ne11, ok_ids)
    assert max_err_scaled(got, ideal) < F64_TOL


# Long expert rows (Mixtral's ffn_down is 4096x14336 per expert): the ids form
# splits K into shares with the one-column op's layout for the same rows, one
# case per layout, with a dropped slot (-1) in every case.
@pytest.mark.parametrize("tname,n_as,nrows,K,n_tokens", [("Q4_K", 3, 1000, 14336, 2), ("Q6_K", 3, 2100, 8192, 1),
                                                         ("Q8_0", 3, 3000, 8192, 2), ("IQ4_XS", 2, 4100, 14336, 1),
                                                         ("Q4_0", 3, 700, 4096, 2)])
def test_mul_mat_id_few_tokens_long_rows(tname, n_as, nrows, K, n_tokens):
    import ggml_hip as G
    n_ids = 2
    rng = np.random.default_rng(nrows + K)
    ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    ids[0, 1] = -1
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    got = _check(tname, n_as, nrows, K, x, ids)
    wq = _experts(TYPES[tname], n_as, nrows, K)
    w_d, x_d = torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda()
    for tt in range(n_tokens):
        for s in range(n_ids):
            if ids[tt, s] < 0:
                continue
            one = G.mul_mat_vec_f32(tname, w_d[ids[tt, s]], K, x_d[tt, 0]).cpu().numpy().reshape(-1)
            np.testing.assert_array_equal(got[tt, s], one)


def test_mul_mat_id_nine_tokens_take_the_grouped_path():
    """The boundary: 9 tokens go through grouping + grouped MMQ, with the same gates."""
    n_as, nrows, K, n_tokens, n_ids = 8, 256, 512, 9, 2
    ids = np.random.default_rng(3).integers(-1, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    _check("Q4_K", n_as, nrows, K, x, ids)


def test_mul_mat_id_grouping_chunks_expert_loops_and_unaligned_activations():
    """Grouping past one chunk of pairs (5600 pairs) and past one expert per
    grouping workgroup (300 experts), with out-of-range ids; the one-launch
    form (aligned activations) and the two-launch form (a row stride that is
    not a multiple of 4 floats) give identical outputs, and both pass the
    CPU and f64 gates."""
    import ctypes
    import ggml_hip as G
    n_as, nrows, K, n_tokens, n_ids = 300, 64, 256, 700, 8
    rng = np.random.default_rng(11)
    ids = rng.integers(-1, n_as + 2, size=(n_tokens, n_ids)).astype(np.int32)
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    t, wq, got = _run("Q4_K", n_as, nrows, K, x, ids)
    bad = (ids < 0) | (ids >= n_as)
    assert np.all(got[bad] == 0.0)
    ok_ids = np.where(bad, -1, ids).astype(np.int32)
    cpu = O.mul_mat_id(t, wq, n_as, nrows, K, x, ok_ids, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    y = G.quantize_q8_1(torch.from_numpy(x.reshape(-1, K)).cuda(), K).cpu().numpy()
    ideal = mul_mat_id_f64(t, wq, nrows, K, y, 1, ok_ids)
    assert max_err_scaled(got, ideal) < F64_TOL

    stride = K + 1
    xs = torch.zeros((n_tokens, stride), dtype=torch.float32, device="cuda")
    xs[:, :K] = torch.from_numpy(x.reshape(n_tokens, K)).cuda()
    w_d, ids_d = torch.from_numpy(wq).cuda(), torch.from_numpy(ids).cuda()
    out = torch.full((n_tokens, n_ids, nrows), float("nan"), device="cuda")
    need = int(G.lib().hip_qmm_mul_mat_id_workspace_size(t, K, n_as, 1, n_tokens, n_ids))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    p = lambda a: ctypes.c_void_p(a.data_ptr())  # noqa: E731
    rc = G.lib().hip_qmm_mul_mat_id(t, p(w_d), K, nrows, w_d.stride(1), w_d.stride(0), n_as, p(xs), 1, n_tokens,
                                    stride, p(ids_d), n_ids, n_ids, p(out), nrows, p(ws), need,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    np.testing.assert_array_equal(out.cpu().numpy(), got)


# The grouping kernel has two paths: up to 4 chunks of 4096 (token, slot) pairs
# and 256 experts it reads the ids once into registers (16 consecutive pairs
# per thread, 16-byte loads when the ids are dense and aligned, single loads
# otherwise); beyond either limit it re-reads them chunk by chunk.  Both must
# give every row its expert's product and -1 ids zero rows.
@pytest.mark.parametrize("n_as,n_tokens,n_ids,ids_layout", [
    (32, 1500, 4, "dense"),        # registers, 2 chunks
    (64, 2000, 8, "strided"),      # registers, 4 chunks, ids rows padded and misaligned
    (16, 2100, 8, "dense"),        # general path: 16800 pairs
    (300, 40, 4, "dense"),         # general path: more than 256 experts
])
def test_mul_mat_id_grouping_paths(n_as, n_tokens, n_ids, ids_layout):
    import ctypes
    import ggml_hip as G
    nrows, K = 64, 256
    t = O.TYPE_Q4_K
    rng = np.random.default_rng(n_as * 1000 + n_tokens)
    ids = rng.integers(-1, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    wq = _experts(t, n_as, nrows, K)
    w_d, x_d = torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda()
    if ids_layout == "strided":
        stride = n_ids + 3
        buf = torch.full((n_tokens * stride + 1,), n_as - 1, dtype=torch.int32, device="cuda")
        view = buf[1:1 + n_tokens * stride].view(n_tokens, stride)  # 4 bytes past 16-byte alignment
        view[:, :n_ids] = torch.from_numpy(ids).cuda()
        ids_ptr, ids_stride = view.data_ptr(), stride
    else:
        ids_d = torch.from_numpy(ids).cuda()
        ids_ptr, ids_stride = ids_d.data_ptr(), n_ids
    L = G.lib()
    need = int(L.hip_qmm_mul_mat_id_workspace_size(t, K, n_as, 1, n_tokens, n_ids))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.full((n_tokens, n_ids, nrows), float("nan"), device="cuda")
    vp = ctypes.c_void_p
    rc = L.hip_qmm_mul_mat_id(t, vp(w_d.data_ptr()), K, nrows, w_d.stride(1), w_d.stride(0), n_as,
                              vp(x_d.data_ptr()), 1, n_tokens, K, vp(ids_ptr), n_ids, ids_stride,
                              vp(out.data_ptr()), nrows, vp(ws.data_ptr()), ws.numel(),
                              vp(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, rc
    got = out.cpu().numpy()
    assert np.all(got[ids < 0] == 0.0)
    cpu = O.mul_mat_id(t, wq, n_as, nrows, K, x, ids, nth=8)
    assert nmse(got, cpu) < NMSE_GATE, nmse(got, cpu)
    y = G.quantize_q8_1(torch.from_numpy(x.reshape(-1, K)).cuda(), K).cpu().numpy()
    ideal = mul_mat_id_f64(t, wq, nrows, K, y, 1, ids)
    assert max_err_scaled(got, ideal) < F64_TOL, max_err_scaled(got, ideal)
