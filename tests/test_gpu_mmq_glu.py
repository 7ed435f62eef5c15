"""Gate/up/GLU fused into the MMQ (prefill): both weights' rows go through one
tile kernel and the tile writes glu(gate, up) (the reference's mul_mat_q with a
gate, src/ggml/cuda/mmq.zig:568-640, from its gate/up/GLU fusion,
src/ggml/cuda/fusion.zig:1226-1298, 1391).

Checks, per case:
  - hip_qmm_mmq_glu == hip_qmm_glu_f32 of two unsplit hip_qmm_mmq products bit
    for bit (each gate and up sum is the tile kernel's at the same K order),
    every type, ragged rows and columns, both tile widths, every GLU op;
  - the op (hip_qmm_mul_mat_glu) against the CPU path (x86 route products,
    then the CPU GLU op): NMSE < 5e-4, and on the column counts it leaves
    unfused (the GEMV's and the few-column kernel's) equal to the unfused ops;
  - MUL_MAT_ID: hip_qmm_mul_mat_id_glu == the GLU of two hip_qmm_mul_mat_id
    products bit for bit, on token counts that group (32- and 64-column tiles,
    so the persistent and the one-tile-per-workgroup loops), with invalid ids
    giving zero rows, and against the CPU path;
  - through the plugin: {MUL_MAT, MUL_MAT, GLU} at 64 columns and the MoE form
    at 64 tokens fuse (the intermediates, pre-filled with NaN, stay untouched)
    and equal the unfused graph."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from cases import acts, nmse, route_top_k, weights_f32, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
TYPES = {"Q4_K": O.TYPE_Q4_K, "Q5_K": O.TYPE_Q5_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0,
         "Q4_0": O.TYPE_Q4_0, "IQ4_XS": O.TYPE_IQ4_XS}
OPS = {"REGLU": O.GLU_REGLU, "GEGLU": O.GLU_GEGLU, "SWIGLU": O.GLU_SWIGLU, "SWIGLU_OAI": O.GLU_SWIGLU_OAI,
       "SWIGLU_CLAMP": O.GLU_SWIGLU_CLAMP}
ALPHA, LIMIT = 1.702, 7.0


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _mmq_unsplit(G, tname, w_d, K, qs, ds, n):
    """hip_qmm_mmq without a workspace: the tile kernel over the whole K."""
    t = G.TYPE_IDS[tname]
    nrows, rs = w_d.shape[0], w_d.stride(0)
    out = torch.empty((n, nrows), dtype=torch.float32, device="cuda")
    assert G.lib().hip_qmm_mmq(t, w_d.data_ptr(), K, nrows, rs, qs.data_ptr(), ds.data_ptr(), n, out.data_ptr(),
                               nrows, None, 0, torch.cuda.current_stream().cuda_stream) == 0
    return out


def _few_takes(G, tname, K, n):
    """Whether hip_qmm_mmq would send n columns to the few-column kernel."""
    return (n <= 32 and tname in ("Q4_K", "Q5_K", "Q8_0", "Q4_0")) or (n <= 16 and tname == "Q6_K" and K % 2048 == 0)


@pytest.mark.parametrize("tname", list(TYPES))
@pytest.mark.parametrize("nrows,K,ncols", [(256, 2048, 64), (200, 1024, 77), (70, 512, 33), (130, 768, 100)])
def test_mmq_glu_equals_unfused_tiles(tname, nrows, K, ncols):
    import ggml_hip as G
    t = TYPES[tname]
    w = _dev(weights_q(t, nrows, K, 0))
    wg = _dev(weights_q(t, nrows, K, 1))
    x_d = _dev(acts(ncols, K))
    qs, ds = G.quantize_q8_1_planar(x_d)
    assert not _few_takes(G, tname, K, ncols)
    g = _mmq_unsplit(G, tname, wg, K, qs, ds, ncols)
    u = _mmq_unsplit(G, tname, w, K, qs, ds, ncols)
    want = G.glu_f32(g, u, "SWIGLU").cpu().numpy()
    got = G.mmq_glu(tname, w, wg, K, qs, ds, "SWIGLU").cpu().numpy()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("opname", list(OPS))
def test_mmq_glu_every_op(opname):
    import ggml_hip as G
    nrows, K, ncols = 190, 1024, 48
    w = _dev(weights_q(O.TYPE_Q4_K, nrows, K, 0))
    wg = _dev(weights_q(O.TYPE_Q4_K, nrows, K, 1))
    x_d = _dev(acts(ncols, K) * 4)
    qs, ds = G.quantize_q8_1_planar(x_d)
    g = _mmq_unsplit(G, "Q4_K", wg, K, qs, ds, ncols)
    u = _mmq_unsplit(G, "Q4_K", w, K, qs, ds, ncols)
    want = G.glu_f32(g, u, opname, ALPHA, LIMIT).cpu().numpy()
    got = G.mmq_glu("Q4_K", w, wg, K, qs, ds, opname, ALPHA, LIMIT).cpu().numpy()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("tname", ["Q4_K", "Q8_0", "Q5_K"])
def test_mmq_glu_32_column_tiles_match_64(tname):
    """The 32-column tile (20 columns) gives the 64-column tile's bits on the
    same columns: per output the two tiles run the same sums in the same
    order.  Rows of 18 K-steps keep 40 columns on 64-column tiles (the
    grid-fill rule takes 32-column tiles on rows of at most 16)."""
    import ggml_hip as G
    t = TYPES[tname]
    nrows, K = 300, 4608
    w = _dev(weights_q(t, nrows, K, 0))
    wg = _dev(weights_q(t, nrows, K, 1))
    x_d = _dev(acts(40, K))
    qs, ds = G.quantize_q8_1_planar(x_d)
    a = G.mmq_glu(tname, w, wg, K, qs, ds).cpu().numpy()
    qs20, ds20 = G.quantize_q8_1_planar(x_d[:20].contiguous())
    b = G.mmq_glu(tname, w, wg, K, qs20, ds20).cpu().numpy()
    assert G.lib().hip_qmm_mmq_tile_n(20) == 32 and G.lib().hip_qmm_mmq_tile_n(40) == 64
    np.testing.assert_array_equal(b, a[:20])


def _cpu_glu(t, wq, wgq, nrows, K, x, op=O.GLU_SWIGLU):
    g = O.mul_mat_x86(t, wgq, nrows, K, x, nth=8)
    u = O.mul_mat_x86(t, wq, nrows, K, x, nth=8)
    return O.glu(op, g, u, ALPHA, LIMIT)


@pytest.mark.parametrize("tname,nrows,K,ncols", [("Q4_K", 14336, 4096, 512), ("Q4_K", 768, 2048, 128),
                                                 ("Q6_K", 1024, 4096, 64), ("Q8_0", 512, 4096, 40),
                                                 ("IQ4_XS", 300, 1024, 17)])
def test_mul_mat_glu_op_vs_cpu(tname, nrows, K, ncols):
    """The op at the config-2 shape (Llama-3-8B ffn_gate/up at T = 512, checked
    on a row subset) and smaller ones, against the CPU path."""
    import ggml_hip as G
    t = TYPES[tname]
    wq, wgq = weights_q(t, nrows, K, 0), weights_q(t, nrows, K, 1)
    x = acts(ncols, K)
    got = G.mul_mat_glu(tname, _dev(wq), _dev(wgq), _dev(x)).cpu().numpy()
    rows = np.r_[0:64, nrows // 2:nrows // 2 + 64, nrows - 64:nrows] if nrows > 256 else np.arange(nrows)
    rows = np.unique(rows)
    want = _cpu_glu(t, wq[rows], wgq[rows], len(rows), K, x)
    assert nmse(got[:, rows], want) < NMSE_GATE, nmse(got[:, rows], want)


@pytest.mark.parametrize("tname,ncols", [("Q4_K", 1), ("Q4_K", 3), ("Q4_K", 8), ("Q4_K", 24), ("Q8_0", 16),
                                         ("Q6_K", 12), ("Q5_K", 5)])
def test_mul_mat_glu_unfused_column_counts(tname, ncols):
    """Column counts the GEMV or the few-column kernel takes run the two
    products and the GLU kernel: equal to those ops run one by one."""
    import ggml_hip as G
    t = TYPES[tname]
    nrows, K = 4096, 2048
    w, wg = _dev(weights_q(t, nrows, K, 0)), _dev(weights_q(t, nrows, K, 1))
    x_d = _dev(acts(ncols, K))
    got = G.mul_mat_glu(tname, w, wg, x_d).cpu().numpy()
    if ncols == 1:
        want = G.mul_mat_vec_fused(tname, w, K, x_d, w_gate=wg).cpu().numpy()
    else:
        g = G.mul_mat(tname, wg, x_d)
        u = G.mul_mat(tname, w, x_d)
        want = G.glu_f32(g, u, "SWIGLU").cpu().numpy()
    np.testing.assert_array_equal(got, want)


def test_mul_mat_glu_rejects_bad_arguments():
    import ggml_hip as G
    L = G.lib()
    nrows, K, n = 128, 512, 64
    w = _dev(weights_q(O.TYPE_Q4_K, nrows, K, 0))
    x_d = _dev(acts(n, K))
    out = torch.empty((n, nrows), dtype=torch.float32, device="cuda")
    ws = torch.empty(int(L.hip_qmm_mul_mat_glu_workspace_size(O.TYPE_Q4_K, K, nrows, n)), dtype=torch.uint8,
                     device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    args = lambda wg, op, wsz: (O.TYPE_Q4_K, w.data_ptr(), wg, K, nrows, w.stride(0), x_d.data_ptr(), n, K,  # noqa
                                op, ALPHA, LIMIT, out.data_ptr(), nrows, ws.data_ptr(), wsz, s)
    assert L.hip_qmm_mul_mat_glu(*args(None, O.GLU_SWIGLU, ws.numel())) != 0          # no gate
    assert L.hip_qmm_mul_mat_glu(*args(w.data_ptr(), 5, ws.numel())) != 0            # not a GLU op
    assert L.hip_qmm_mul_mat_glu(*args(w.data_ptr(), O.GLU_SWIGLU, ws.numel() - 1)) != 0  # workspace short
    assert L.hip_qmm_mul_mat_glu(*args(w.data_ptr(), O.GLU_SWIGLU, ws.numel())) == 0


def _experts(t, n_as, nrows, K, idx):
    return O.quantize_rows(t, weights_f32(n_as * nrows, K, idx)).reshape(n_as, nrows, -1)


@pytest.mark.parametrize("tname,n_as,nrows,K,n_tokens,n_ids", [("Q4_K", 16, 192, 1024, 64, 4),
                                                               ("Q4_K", 4, 130, 512, 60, 4),
                                                               ("Q6_K", 8, 128, 512, 40, 2),
                                                               ("Q8_0", 8, 100, 1024, 33, 2),
                                                               ("Q8_0", 4, 200, 768, 70, 2),
                                                               ("Q4_0", 8, 100, 1024, 33, 2),
                                                               ("Q4_0", 4, 200, 768, 70, 2),
                                                               ("Q5_K", 8, 100, 1024, 33, 2),
                                                               ("Q5_K", 4, 200, 768, 70, 2),
                                                               ("IQ4_XS", 8, 100, 1024, 33, 2),
                                                               ("IQ4_XS", 4, 200, 1024, 70, 2)])
def test_mul_mat_id_glu_equals_unfused(tname, n_as, nrows, K, n_tokens, n_ids):
    """Grouped fused MMQ == the GLU of two grouped MMQs, bit for bit; 16
    experts x 16 routed columns run 32-column tiles (the persistent loop for
    Q4_K), 4 experts x 60 run 64-column tiles.  Every direct-transfer type
    takes both widths, partial row tiles and (Q4_0 at K = 768) an odd number
    of K-steps; both the fused and the unfused results pass the CPU gate."""
    import ggml_hip as G
    t = TYPES[tname]
    wq, wgq = _experts(t, n_as, nrows, K, 0), _experts(t, n_as, nrows, K, 1)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    ids[::5, 0] = -1
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    w_d, wg_d, x_d, ids_d = _dev(wq), _dev(wgq), _dev(x), _dev(ids)
    g = G.mul_mat_id(tname, wg_d, x_d, ids_d)
    u = G.mul_mat_id(tname, w_d, x_d, ids_d)
    want = G.glu_f32(g.reshape(-1, nrows), u.reshape(-1, nrows), "SWIGLU").reshape(g.shape).cpu().numpy()
    got = G.mul_mat_id_glu(tname, w_d, wg_d, x_d, ids_d).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    assert np.all(got[ids < 0] == 0.0)
    cg = O.mul_mat_id(t, wgq, n_as, nrows, K, x, ids, nth=8)
    cu = O.mul_mat_id(t, wq, n_as, nrows, K, x, ids, nth=8)
    cpu = O.glu(O.GLU_SWIGLU, cg, cu)
    assert nmse(got, cpu) < NMSE_GATE


def test_mul_mat_id_glu_config4_qwen3_moe_gate_up():
    """Config 4's gate/up projection (Qwen3-30B-A3B: 128 experts of 768 x
    2048, top-8 of 512 tokens) through the fused op, checked against the
    unfused ops bit for bit and against the CPU path on a token subset."""
    import ggml_hip as G
    n_as, nrows, K, n_tokens, k = 128, 768, 2048, 512, 8
    t = O.TYPE_Q4_K
    wq, wgq = _experts(t, n_as, nrows, K, 0), _experts(t, n_as, nrows, K, 1)
    ids, _ = route_top_k(n_tokens, n_as, k)
    x = np.array(acts(n_tokens, K)).reshape(n_tokens, 1, K)
    w_d, wg_d, x_d, ids_d = _dev(wq), _dev(wgq), _dev(x), _dev(ids)
    got = G.mul_mat_id_glu("Q4_K", w_d, wg_d, x_d, ids_d).cpu().numpy()
    g = G.mul_mat_id("Q4_K", wg_d, x_d, ids_d)
    u = G.mul_mat_id("Q4_K", w_d, x_d, ids_d)
    want = G.glu_f32(g.reshape(-1, nrows), u.reshape(-1, nrows), "SWIGLU").reshape(g.shape).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    tok = np.r_[0:24, 500:512]
    cg = O.mul_mat_id(t, wgq, n_as, nrows, K, x[tok], ids[tok], nth=8)
    cu = O.mul_mat_id(t, wq, n_as, nrows, K, x[tok], ids[tok], nth=8)
    assert nmse(got[tok], O.glu(O.GLU_SWIGLU, cg, cu)) < NMSE_GATE


@pytest.fixture(scope="module")
def hb():
    from ggml_hip.backend import HipBackend
    with HipBackend(0) as b:
        yield b


def test_plugin_fuses_prefill_gate_up_glu(hb):
    """{MUL_MAT gate, MUL_MAT up, GLU} at 64 columns: the fused MMQ runs (g and
    u stay NaN) and its output equals the fused op's."""
    import ggml_hip as G
    from ggml_hip import abi
    M, K, T = 512, 2048, 64
    wq, wgq = weights_q(O.TYPE_Q4_K, M, K, 0), weights_q(O.TYPE_Q4_K, M, K, 1)
    wu = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M], name=b"up_w")
    wgt = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M], name=b"gate_w")
    x = abi.make_tensor(abi.GGML_TYPE_F32, [K, T], name=b"x")
    g = abi.make_tensor(abi.GGML_TYPE_F32, [M, T], op=abi.GGML_OP_MUL_MAT, srcs=(wgt, x), name=b"g")
    u = abi.make_tensor(abi.GGML_TYPE_F32, [M, T], op=abi.GGML_OP_MUL_MAT, srcs=(wu, x), name=b"u")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [M, T])
    hb.alloc([wu, wgt], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([x, g, u, glu], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(wu, wq)
    hb.set(wgt, wgq)
    xv = acts(T, K)
    hb.set(x, xv)
    for n in (g, u, glu):
        hb.set(n, np.full(M * T, np.nan, dtype=np.float32))
    assert hb.compute([g, u, glu]) == abi.GGML_STATUS_SUCCESS
    assert np.isnan(hb.get(g, np.float32, (T, M))).all() and np.isnan(hb.get(u, np.float32, (T, M))).all()
    got = hb.get(glu, np.float32, (T, M))
    want = G.mul_mat_glu("Q4_K", _dev(wq), _dev(wgq), _dev(xv)).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    # unfused, each product splits K over workgroups: the same values up to
    # the fp32 rounding of the split sums
    assert hb.compute([g, u, glu], use_counts=False) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(g, np.float32, (T, M))).any()
    unfused = hb.get(glu, np.float32, (T, M))
    assert np.max(np.abs(unfused - got)) <= 1e-5 * np.max(np.abs(got))


def test_plugin_fuses_prefill_moe_gate_up_glu(hb):
    """{MUL_MAT_ID gate, MUL_MAT_ID up, GLU} at 64 tokens takes the grouped
    fused MMQ (the intermediates stay NaN)."""
    import ggml_hip as G
    from ggml_hip import abi
    n_as, M, K, T, k = 8, 256, 1024, 64, 2
    wq, wgq = _experts(O.TYPE_Q4_K, n_as, M, K, 0), _experts(O.TYPE_Q4_K, n_as, M, K, 1)
    ids, _ = route_top_k(T, n_as, k)
    wu = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M, n_as], name=b"up_exps")
    wgt = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M, n_as], name=b"gate_exps")
    x = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1, T], name=b"x")
    idt = abi.make_tensor(abi.GGML_TYPE_I32, [k, T], name=b"ids")
    g = abi.make_tensor(abi.GGML_TYPE_F32, [M, k, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(wgt, x, idt), name=b"g")
    u = abi.make_tensor(abi.GGML_TYPE_F32, [M, k, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(wu, x, idt), name=b"u")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [M, k, T])
    hb.alloc([wu, wgt], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([x, idt, g, u, glu], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(wu, wq)
    hb.set(wgt, wgq)
    xv = np.array(acts(T, K))
    hb.set(x, xv)
    hb.set(idt, ids)
    for n in (g, u, glu):
        hb.set(n, np.full(M * k * T, np.nan, dtype=np.float32))
    assert hb.compute([g, u, glu]) == abi.GGML_STATUS_SUCCESS
    assert np.isnan(hb.get(g, np.float32, (T * k, M))).all()
    got = hb.get(glu, np.float32, (T, k, M))
    want = G.mul_mat_id_glu("Q4_K", _dev(wq), _dev(wgq), _dev(xv.reshape(T, 1, K)), _dev(ids)).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    assert hb.compute([g, u, glu], use_counts=False) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(g, np.float32, (T * k, M))).any()
    np.testing.assert_array_equal(hb.get(glu, np.float32, (T, k, M)), got)


def _deps_want(C, nodes, last):
    """addAllocDeps (src/ggml/cuda/graph.zig:753-770): each node before `last`
    and each of its sources, kept allocated until `last`."""
    want = set()
    for n in nodes:
        want.add((C.addressof(n), C.addressof(last)))
        for s in n.src:
            if s:
                want.add((C.cast(s, C.c_void_p).value, C.addressof(last)))
    return want


def test_plugin_graph_optimize_keeps_fused_mmq_inputs_alive(hb):
    """graph_optimize keeps the nodes and sources (weights, activations, ids)
    of every gate / up / GLU run the fused MMQ takes allocated until the GLU
    (src/ggml/cuda/graph.zig:849-862), dense at 64 columns and grouped at 64
    tokens; a one-column run (the fused GEMV) gets none, as in the reference."""
    from ggml_hip import abi
    M, K, T, n_as, k = 512, 2048, 64, 8, 2
    q4 = abi.GGML_TYPE_Q4_K
    wu, wgt = abi.make_tensor(q4, [K, M], name=b"up_w"), abi.make_tensor(q4, [K, M], name=b"gate_w")
    x = abi.make_tensor(abi.GGML_TYPE_F32, [K, T], name=b"x")
    g = abi.make_tensor(abi.GGML_TYPE_F32, [M, T], op=abi.GGML_OP_MUL_MAT, srcs=(wgt, x), name=b"g")
    u = abi.make_tensor(abi.GGML_TYPE_F32, [M, T], op=abi.GGML_OP_MUL_MAT, srcs=(wu, x), name=b"u")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [M, T])
    order, deps = hb.optimized([g, u, glu])
    assert [C.addressof(n) for n in order] == [C.addressof(n) for n in (g, u, glu)]
    assert set(deps) == _deps_want(C, (g, u), glu)

    ewu, ewg = abi.make_tensor(q4, [K, M, n_as], name=b"up_exps"), abi.make_tensor(q4, [K, M, n_as], name=b"gate_exps")
    ex = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1, T], name=b"x")
    idt = abi.make_tensor(abi.GGML_TYPE_I32, [k, T], name=b"ids")
    eg = abi.make_tensor(abi.GGML_TYPE_F32, [M, k, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(ewg, ex, idt), name=b"g")
    eu = abi.make_tensor(abi.GGML_TYPE_F32, [M, k, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(ewu, ex, idt), name=b"u")
    eglu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, eg, eu, [M, k, T])
    _, edeps = hb.optimized([eu, eg, eglu])  # up first: either order pairs
    assert set(edeps) == _deps_want(C, (eu, eg), eglu)

    x1 = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1], name=b"x1")
    g1 = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_MUL_MAT, srcs=(wgt, x1), name=b"g1")
    u1 = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_MUL_MAT, srcs=(wu, x1), name=b"u1")
    glu1 = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g1, u1, [M, 1])
    assert hb.optimized([g1, u1, glu1])[1] == []


def test_plugin_fused_mmq_result_on_gate_weights_runs_unfused(hb):
    """Under op offload the weights are compute-buffer copies, and without
    the allocation dependencies the GLU's result could be placed on the gate
    weights once their MUL_MAT is past.  The fused kernel would then write
    tiles while other tiles still read those weights; the backend instead runs
    the three nodes unfused (g and u are written), and the result is the
    fused op's up to the split sums' rounding.  Dense at 64 columns and the
    grouped form at 64 tokens."""
    import ggml_hip as G
    from ggml_hip import abi
    M, K, T = 512, 2048, 64
    q4 = abi.GGML_TYPE_Q4_K
    wq, wgq = weights_q(O.TYPE_Q4_K, M, K, 0), weights_q(O.TYPE_Q4_K, M, K, 1)
    wu, wgt = abi.make_tensor(q4, [K, M], name=b"up_w"), abi.make_tensor(q4, [K, M], name=b"gate_w")
    x = abi.make_tensor(abi.GGML_TYPE_F32, [K, T], name=b"x")
    g = abi.make_tensor(abi.GGML_TYPE_F32, [M, T], op=abi.GGML_OP_MUL_MAT, srcs=(wgt, x), name=b"g")
    u = abi.make_tensor(abi.GGML_TYPE_F32, [M, T], op=abi.GGML_OP_MUL_MAT, srcs=(wu, x), name=b"u")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [M, T])
    hb.alloc([wu, wgt, x, g, u], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    glu.data, glu.buffer = wgt.data, wgt.buffer  # the result placed on the gate weights' copy
    hb.set(wu, wq)
    hb.set(wgt, wgq)
    xv = acts(T, K)
    hb.set(x, xv)
    for n in (g, u):
        hb.set(n, np.full(M * T, np.nan, dtype=np.float32))
    assert hb.compute([g, u, glu]) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(g, np.float32, (T, M))).any() and not np.isnan(hb.get(u, np.float32, (T, M))).any()
    got = hb.get(glu, np.float32, (T, M))
    want = G.mul_mat_glu("Q4_K", _dev(wq), _dev(wgq), _dev(xv)).cpu().numpy()
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))

    n_as, k = 8, 2
    ewq, ewgq = _experts(O.TYPE_Q4_K, n_as, M, K, 0), _experts(O.TYPE_Q4_K, n_as, M, K, 1)
    ids, _ = route_top_k(T, n_as, k)
    ewu, ewg = abi.make_tensor(q4, [K, M, n_as], name=b"up_exps"), abi.make_tensor(q4, [K, M, n_as], name=b"gate_exps")
    ex = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1, T], name=b"x")
    idt = abi.make_tensor(abi.GGML_TYPE_I32, [k, T], name=b"ids")
    eg = abi.make_tensor(abi.GGML_TYPE_F32, [M, k, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(ewg, ex, idt), name=b"g")
    eu = abi.make_tensor(abi.GGML_TYPE_F32, [M, k, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(ewu, ex, idt), name=b"u")
    eglu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, eg, eu, [M, k, T])
    hb.alloc([ewu, ewg, ex, idt, eg, eu], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    eglu.data, eglu.buffer = ewg.data, ewg.buffer
    hb.set(ewu, ewq)
    hb.set(ewg, ewgq)
    exv = np.array(acts(T, K))
    hb.set(ex, exv)
    hb.set(idt, ids)
    for n in (eg, eu):
        hb.set(n, np.full(M * k * T, np.nan, dtype=np.float32))
    assert hb.compute([eg, eu, eglu]) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(eg, np.float32, (T * k, M))).any()
    got = hb.get(eglu, np.float32, (T, k, M))
    want = G.mul_mat_id_glu("Q4_K", _dev(ewq), _dev(ewgq), _dev(exv.reshape(T, 1, K)), _dev(ids)).cpu().numpy()
    np.testing.assert_array_equal(got, want)
