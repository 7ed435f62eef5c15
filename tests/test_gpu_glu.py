"""The GEMV fusion epilogue on the GPU: gate + up GEMVs + GLU in one kernel,
GEMV + bias, and the standalone GLU / ADD kernels the backend runs when it
does not fuse.

Checks, per case:
  - fused output == the unfused composition on the GPU (GEMV per lane, bias
    add, GLU kernel) bit for bit: the same dots, the same combination order,
    the same glu_apply;
  - the lanes' GEMVs (no gate) == hip_qmm_mul_mat_vec_f32 bit for bit, and
    within 2e-6 of the f64 evaluation of the Q8_1 formula;
  - fused output vs the CPU ggml path (Q8_K vec_dot + f32 bias add + the CPU
    GLU op) within NMSE < 5e-4;
  - standalone GLU vs the CPU GLU op: REGLU exact; SWIGLU / SWIGLU_OAI /
    SWIGLU_CLAMP within 8 f32 ulp (the device and libm exp differ in the last
    bits); GEGLU exact but for rare one-f16-step moves of the gelu factor
    where 1 + tanh cancels (the device and libm tanhf differ in the last bit);
  - through the plugin: {MUL_MAT, MUL_MAT, GLU}, {MUL_MAT, ADD, MUL_MAT, ADD,
    GLU} and {MUL_MAT, ADD} fuse (their intermediates, pre-filled with NaN,
    stay untouched) unless a use count or an output flag forbids it, and the
    fused and unfused graphs agree."""
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
OPS = {"REGLU": O.GLU_REGLU, "GEGLU": O.GLU_GEGLU, "SWIGLU": O.GLU_SWIGLU, "SWIGLU_OAI": O.GLU_SWIGLU_OAI,
       "SWIGLU_CLAMP": O.GLU_SWIGLU_CLAMP}
ALPHA, LIMIT = 1.702, 7.0  # ggml_swiglu_oai's defaults as gpt-oss uses them


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def glu_matches(op, g, u, got, want):
    """The standalone and fused GLU against the CPU op, per element."""
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    g = np.asarray(g, np.float32).reshape(-1)
    u = np.asarray(u, np.float32).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    got, want, g, u = got[ok], want[ok], g[ok], u[ok]
    if op == O.GLU_REGLU:
        np.testing.assert_array_equal(got, want)
        return
    if op == O.GLU_GEGLU:
        diff = got != want
        assert diff.mean() < 2e-3, diff.mean()
        # one f16 step of the gelu factor, times |u|
        gl = np.abs(want / np.where(u == 0, 1, u)).astype(np.float16)
        step = np.spacing(gl).astype(np.float32) * np.abs(u)
        assert np.all(np.abs(got - want)[diff] <= step[diff] * 1.001 + 1e-30)
        return
    tol = 8 * np.spacing(np.abs(want).astype(np.float32)) + 1e-37
    bad = np.abs(got - want) > tol
    assert not bad.any(), (got[bad][:5], want[bad][:5])


def glu_inputs(n, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 4).astype(np.float32)
    special = np.float32([0.0, -0.0, 10.0, -10.0, 9.99, -9.99, LIMIT, -LIMIT, 30.0, -30.0, 90.0, -90.0])
    g[:special.size] = special
    u[:special.size] = special[::-1]
    return g, u


@pytest.mark.parametrize("opname", list(OPS))
def test_glu_kernel_vs_cpu(opname):
    import ggml_hip as G
    op = OPS[opname]
    g, u = glu_inputs(3 * 5000, 11 + op)
    gd, ud = _dev(g.reshape(3, 5000)), _dev(u.reshape(3, 5000))
    got = G.glu_f32(gd, ud, opname, ALPHA, LIMIT).cpu().numpy()
    glu_matches(op, g, u, got, O.glu(op, g, u, ALPHA, LIMIT))
    # strided rows: every other row of a [6, 5000] buffer, into a strided output
    big = torch.zeros((6, 5000), dtype=torch.float32, device="cuda")
    big[::2] = gd
    out = torch.full((3, 6000), float("nan"), dtype=torch.float32, device="cuda")
    G.glu_f32(big[::2], ud, opname, ALPHA, LIMIT, out=out[:, :5000])
    np.testing.assert_array_equal(out[:, :5000].cpu().numpy(), got)
    assert torch.isnan(out[:, 5000:]).all()


def test_add_kernel_exact():
    import ggml_hip as G
    rng = np.random.default_rng(5)
    a = rng.standard_normal((7, 1234)).astype(np.float32)
    b = rng.standard_normal((7, 1234)).astype(np.float32)
    np.testing.assert_array_equal(G.add_f32(_dev(a), _dev(b)).cpu().numpy(), a + b)


def _one_share(tname, M, K):
    """Whether the plain one-column GEMV runs M x K in one K share: rows of one
    K-step of 64 lanes, at least 8192 rows, or at most 4096 columns on more
    than 2048 rows (the gated kernel always does)."""
    nsteps = -(-K // (64 * (32 if tname in ("Q8_0", "Q4_0") else 64)))
    return nsteps < 2 or M >= 8192 or (K <= 4096 and M > 2048)


def _fused_case(tname, M, K, opname, with_bias):
    import ggml_hip as G
    t = TYPES[tname]
    wu, wg = weights_q(t, M, K, 0), weights_q(t, M, K, 1)
    x = acts(1, K)
    wu_d, wg_d, x_d = _dev(wu), _dev(wg), _dev(x)
    rng = np.random.default_rng(M + K)
    bu = (rng.standard_normal(M) * 0.5).astype(np.float32) if with_bias else None
    bg = (rng.standard_normal(M) * 0.5).astype(np.float32) if with_bias else None
    bu_d = _dev(bu) if with_bias else None
    bg_d = _dev(bg) if with_bias else None
    op = OPS[opname]
    fused = G.mul_mat_vec_fused(tname, wu_d, K, x_d, w_gate=wg_d, bias=bu_d, gate_bias=bg_d, glu=opname,
                                alpha=ALPHA, limit=LIMIT)
    u = G.mul_mat_vec_fused(tname, wu_d, K, x_d, bias=bu_d)
    g = G.mul_mat_vec_fused(tname, wg_d, K, x_d, bias=bg_d)
    unfused = G.glu_f32(g, u, opname, ALPHA, LIMIT)
    torch.cuda.synchronize()
    return t, wu, wg, x, bu, bg, op, fused.cpu().numpy(), u.cpu().numpy(), g.cpu().numpy(), unfused.cpu().numpy()


@pytest.mark.parametrize("tname,M,K", [("Q4_K", 14336, 4096), ("Q4_K", 768, 2048), ("Q4_K", 3000, 8192),
                                       ("Q6_K", 4100, 4096), ("Q6_K", 8200, 1024), ("Q8_0", 2048, 4096),
                                       ("Q8_0", 333, 96), ("Q5_K", 14336, 4096), ("Q5_K", 768, 2048),
                                       ("Q4_0", 14336, 4096), ("Q4_0", 333, 96), ("IQ4_XS", 14336, 4096),
                                       ("IQ4_XS", 768, 2048)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_fused_gate_up_swiglu(tname, M, K, with_bias):
    import ggml_hip as G
    t, wu, wg, x, bu, bg, op, fused, u, g, unfused = _fused_case(tname, M, K, "SWIGLU", with_bias)
    if _one_share(tname, M, K):
        np.testing.assert_array_equal(fused, unfused)
    else:
        # the plain lanes split their rows into K shares (another summation
        # order than the gated kernel's): the same values to fp32 rounding
        assert max_err_scaled(fused, unfused) < F64_TOL * 4, max_err_scaled(fused, unfused)
    x_d = _dev(x)
    y = G.quantize_q8_1(x_d, K).cpu().numpy()
    for wq, lane, b in ((wu, u, bu), (wg, g, bg)):
        plain = lane - b if b is not None else lane
        if b is None and K <= (2048 if tname in ("Q8_0", "Q4_0") else 4096):
            # the lanes' GEMV is the one-column fused GEMV's arithmetic
            ref = G.mul_mat_vec_f32(tname, _dev(wq), K, x_d[0]).cpu().numpy()
            np.testing.assert_array_equal(lane, ref)
        ideal = O.mul_mat_q8_1_f64(t, wq, M, K, y, 1)
        assert max_err_scaled(plain, ideal) < F64_TOL * 2, max_err_scaled(plain, ideal)
    cu = O.mul_mat(t, wu, M, K, x, nth=8)
    cg = O.mul_mat(t, wg, M, K, x, nth=8)
    if bu is not None:
        cu, cg = cu + bu, cg + bg
    cpu = O.glu(op, cg, cu, ALPHA, LIMIT)
    e = nmse(fused, cpu)
    assert e < NMSE_GATE, f"NMSE {e:.3g}, max rel {max_rel(fused, cpu):.3g}"


@pytest.mark.parametrize("opname", ["REGLU", "GEGLU", "SWIGLU_OAI", "SWIGLU_CLAMP"])
def test_fused_gate_up_other_glu(opname):
    t, wu, wg, x, bu, bg, op, fused, u, g, unfused = _fused_case("Q4_K", 768, 2048, opname, True)
    np.testing.assert_array_equal(fused, unfused)
    glu_matches(op, g, u, fused, O.glu(op, g, u, ALPHA, LIMIT))  # the epilogue on the GPU's own lanes
    cu = O.mul_mat(t, wu, 768, 2048, x, nth=8) + bu
    cg = O.mul_mat(t, wg, 768, 2048, x, nth=8) + bg
    assert nmse(fused, O.glu(op, cg, cu, ALPHA, LIMIT)) < NMSE_GATE


def test_fused_bias_only():
    import ggml_hip as G
    M, K = 5000, 4096
    wq = weights_q(O.TYPE_Q4_K, M, K)
    x = acts(1, K)
    b = np.linspace(-1, 1, M, dtype=np.float32)
    got = G.mul_mat_vec_fused("Q4_K", _dev(wq), K, _dev(x), bias=_dev(b)).cpu().numpy()
    plain = G.mul_mat_vec_f32("Q4_K", _dev(wq), K, _dev(x)[0]).cpu().numpy()
    np.testing.assert_array_equal(got, plain + b)
    assert nmse(got, O.mul_mat(O.TYPE_Q4_K, wq, M, K, x, nth=8) + b) < NMSE_GATE


# ---------------------------------------------------------------- through the plugin

@pytest.fixture(scope="module")
def hb():
    from ggml_hip.backend import HipBackend
    with HipBackend(0) as b:
        yield b


def _ffn_graph(hb, M, K, with_bias, opname="SWIGLU", gate_first=True):
    """x -> up/gate MUL_MATs (+ bias ADDs) -> GLU, as llama's FFN builds it."""
    from ggml_hip import abi
    t = abi.GGML_TYPE_Q4_K
    wu, wg = weights_q(O.TYPE_Q4_K, M, K, 0), weights_q(O.TYPE_Q4_K, M, K, 1)
    x = acts(1, K)
    tw_u = abi.make_tensor(t, [K, M], name=b"ffn_up")
    tw_g = abi.make_tensor(t, [K, M], name=b"ffn_gate")
    tx = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1], name=b"x")
    up = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_MUL_MAT, srcs=(tw_u, tx), name=b"up")
    gate = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_MUL_MAT, srcs=(tw_g, tx), name=b"gate")
    leaves, inter = [tw_u, tw_g], [up, gate]
    u_out, g_out, biases = up, gate, None
    if with_bias:
        tb_u = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], name=b"b_up")
        tb_g = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], name=b"b_gate")
        u_out = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_ADD, srcs=(up, tb_u), name=b"up_b")
        g_out = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_ADD, srcs=(tb_g, gate), name=b"gate_b")
        inter += [u_out, g_out]
        rng = np.random.default_rng(3)
        biases = (tb_u, tb_g, (rng.standard_normal(M) * 0.5).astype(np.float32),
                  (rng.standard_normal(M) * 0.5).astype(np.float32))
    glu = abi.make_glu(OPS[opname], g_out, u_out, [M, 1], ALPHA, LIMIT)
    hb.alloc(leaves, usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([tx] + inter + [glu] + ([biases[0], biases[1]] if biases else []),
             usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(tw_u, wu)
    hb.set(tw_g, wg)
    hb.set(tx, x)
    if biases:
        hb.set(biases[0], biases[2])
        hb.set(biases[1], biases[3])
    if with_bias:
        nodes = [gate, g_out, up, u_out, glu] if gate_first else [up, u_out, gate, g_out, glu]
    else:
        nodes = [gate, up, glu] if gate_first else [up, gate, glu]
    return nodes, inter, glu, (wu, wg, x, biases)


def _run(hb, nodes, inter, glu, M, use_counts=True):
    for t in inter + [glu]:
        hb.set(t, np.full(M, np.nan, dtype=np.float32))
    from ggml_hip import abi
    assert hb.compute(nodes, use_counts=use_counts) == abi.GGML_STATUS_SUCCESS
    return hb.get(glu, np.float32, (M,)), [hb.get(t, np.float32, (M,)) for t in inter]


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("gate_first", [True, False])
def test_plugin_fuses_ffn_gate_up_glu(hb, with_bias, gate_first):
    import ggml_hip as G
    M, K = 4096, 4096
    nodes, inter, glu, (wu, wg, x, biases) = _ffn_graph(hb, M, K, with_bias, gate_first=gate_first)
    out, mids = _run(hb, nodes, inter, glu, M)
    assert all(np.isnan(m).all() for m in mids)  # fused: no intermediate written
    want = G.mul_mat_vec_fused("Q4_K", _dev(wu), K, _dev(x), w_gate=_dev(wg),
                               bias=_dev(biases[2]) if biases else None,
                               gate_bias=_dev(biases[3]) if biases else None, glu="SWIGLU").cpu().numpy()
    np.testing.assert_array_equal(out, want.reshape(-1))
    # the same graph without use counts runs node by node: the intermediates
    # are written, and at 4096 rows the one-column MUL_MAT is the same GEMV
    out2, mids2 = _run(hb, nodes, inter, glu, M, use_counts=False)
    assert not any(np.isnan(m).any() for m in mids2)
    np.testing.assert_array_equal(out2, out)
    cu = O.mul_mat(O.TYPE_Q4_K, wu, M, K, x, nth=8).reshape(-1)
    cg = O.mul_mat(O.TYPE_Q4_K, wg, M, K, x, nth=8).reshape(-1)
    if biases:
        cu, cg = cu + biases[2], cg + biases[3]
    assert nmse(out, O.glu(O.GLU_SWIGLU, cg, cu)) < NMSE_GATE


def test_plugin_does_not_fuse_an_output_intermediate(hb):
    from ggml_hip import abi
    M, K = 4096, 4096
    nodes, inter, glu, _ = _ffn_graph(hb, M, K, False)
    up = nodes[1]
    up.flags |= abi.GGML_TENSOR_FLAG_OUTPUT
    try:
        out, mids = _run(hb, nodes, inter, glu, M)
    finally:
        up.flags &= ~abi.GGML_TENSOR_FLAG_OUTPUT
    assert not any(np.isnan(m).any() for m in mids)
    out_f, _ = _run(hb, nodes, inter, glu, M)
    np.testing.assert_array_equal(out, out_f)


def test_plugin_does_not_fuse_a_shared_intermediate(hb):
    """The up result is also read by a node outside the run: no fusion."""
    from ggml_hip import abi
    M, K = 4096, 4096
    nodes, inter, glu, _ = _ffn_graph(hb, M, K, False)
    up = nodes[1]
    extra = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_ADD, srcs=(up, up), name=b"reuse")
    hb.alloc([extra], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    out, mids = _run(hb, nodes + [extra], inter, glu, M)
    assert not any(np.isnan(m).any() for m in mids)
    np.testing.assert_array_equal(hb.get(extra, np.float32, (M,)), mids[0] + mids[0])


def test_plugin_fuses_mul_mat_bias_and_runs_glu_alone(hb):
    import ggml_hip as G
    from ggml_hip import abi
    M, K = 5000, 4096
    wq = weights_q(O.TYPE_Q4_K, M, K)
    x = acts(1, K)
    b = np.linspace(-1, 1, M, dtype=np.float32)
    tw = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M], name=b"w")
    tx = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1], name=b"x")
    tb = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], name=b"b")
    mm = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_MUL_MAT, srcs=(tw, tx), name=b"mm")
    add = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_ADD, srcs=(mm, tb), name=b"mm_b")
    # a one-tensor swapped GEGLU over [2*M/2 ...]: halves of `add`'s rows are
    # not a GLU shape, so use a fresh [2n, 3] input for the standalone node
    h = abi.make_tensor(abi.GGML_TYPE_F32, [64, 3], name=b"h")
    gl = abi.make_tensor(abi.GGML_TYPE_F32, [32, 3], op=abi.GGML_OP_GLU, srcs=(h,), name=b"geglu_swapped")
    gl.op_params[0] = abi.GGML_GLU_OP_GEGLU
    gl.op_params[1] = 1
    hb.alloc([tw], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([tx, tb, mm, add, h, gl], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(tw, wq)
    hb.set(tx, x)
    hb.set(tb, b)
    hb.set(mm, np.full(M, np.nan, dtype=np.float32))
    hv = np.random.default_rng(9).standard_normal((3, 64)).astype(np.float32) * 3
    hb.set(h, hv)
    assert hb.compute([mm, add, gl]) == abi.GGML_STATUS_SUCCESS
    assert np.isnan(hb.get(mm, np.float32, (M,))).all()
    got = hb.get(add, np.float32, (M,))
    plain = G.mul_mat_vec_f32("Q4_K", _dev(wq), K, _dev(x)[0]).cpu().numpy().reshape(-1)
    np.testing.assert_array_equal(got, plain + b)
    # swapped: the second half of each row gates
    want = O.glu(O.GLU_GEGLU, hv[:, 32:], hv[:, :32])
    glu_matches(O.GLU_GEGLU, hv[:, 32:], hv[:, :32], hb.get(gl, np.float32, (3, 32)), want)


def test_plugin_does_not_take_a_run_node_as_bias(hb):
    """ADD(mm, mm): the bias would be mm itself, which a fused launch never
    computes, so the pair runs node by node and the sum is 2 * mm."""
    import ggml_hip as G
    from ggml_hip import abi
    M, K = 4096, 4096
    wq = weights_q(O.TYPE_Q4_K, M, K)
    x = acts(1, K)
    tw = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M], name=b"w")
    tx = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1], name=b"x")
    mm = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_MUL_MAT, srcs=(tw, tx), name=b"mm")
    add = abi.make_tensor(abi.GGML_TYPE_F32, [M, 1], op=abi.GGML_OP_ADD, srcs=(mm, mm), name=b"mm_mm")
    hb.alloc([tw], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([tx, mm, add], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(tw, wq)
    hb.set(tx, x)
    hb.set(mm, np.full(M, np.nan, dtype=np.float32))
    hb.set(add, np.full(M, np.nan, dtype=np.float32))
    assert hb.compute([mm, add]) == abi.GGML_STATUS_SUCCESS
    plain = G.mul_mat_vec_f32("Q4_K", _dev(wq), K, _dev(x)[0]).cpu().numpy().reshape(-1)
    np.testing.assert_array_equal(hb.get(mm, np.float32, (M,)), plain)
    np.testing.assert_array_equal(hb.get(add, np.float32, (M,)), plain + plain)


# ---------------------------------------------------------------- MUL_MAT_ID (MoE decode)

def _moe(tname, n_as, M, K, n_tokens, n_ids, seed):
    t = TYPES[tname]
    wu = O.quantize_rows(t, O.fill_normal(100 + seed, n_as * M * K, 0.0, 0.02).reshape(n_as * M, K)).reshape(n_as, M, -1)
    wg = O.quantize_rows(t, O.fill_normal(200 + seed, n_as * M * K, 0.0, 0.02).reshape(n_as * M, K)).reshape(n_as, M, -1)
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    x = O.fill_normal(300 + seed, n_tokens * K).reshape(n_tokens, 1, K)
    return t, wu, wg, ids, x


@pytest.mark.parametrize("tname,n_tokens,opname", [("Q4_K", 1, "SWIGLU"), ("Q4_K", 5, "GEGLU"),
                                                    ("Q6_K", 2, "SWIGLU_OAI"), ("Q8_0", 8, "SWIGLU_CLAMP"),
                                                    ("Q5_K", 3, "SWIGLU"), ("Q4_0", 4, "GEGLU"),
                                                    ("IQ4_XS", 6, "SWIGLU")])
def test_fused_gate_up_glu_with_ids(tname, n_tokens, opname):
    """MoE decode's gate / up / GLU over the selected experts in one launch:
    every (token, slot) row equals the one-column fused kernel on its expert
    bit for bit, and the whole passes the CPU gate (mul_mat_id twice + GLU)."""
    import ggml_hip as G
    n_as, M, K, n_ids = 16, 768, 1024, 4
    t, wu, wg, ids, x = _moe(tname, n_as, M, K, n_tokens, n_ids, n_tokens)
    wu_d, wg_d, x_d, ids_d = _dev(wu), _dev(wg), _dev(x), _dev(ids)
    got = G.mul_mat_id_vec_fused(tname, wu_d, x_d, ids_d, w_gate=wg_d, glu=opname, alpha=ALPHA,
                                 limit=LIMIT).cpu().numpy()
    for tt in range(n_tokens):
        for s in range(n_ids):
            e = ids[tt, s]
            one = G.mul_mat_vec_fused(tname, wu_d[e], K, x_d[tt, 0], w_gate=wg_d[e], glu=opname, alpha=ALPHA,
                                      limit=LIMIT).cpu().numpy().reshape(-1)
            np.testing.assert_array_equal(got[tt, s], one)
    cu = O.mul_mat_id(t, wu, n_as, M, K, x, ids, nth=8)
    cg = O.mul_mat_id(t, wg, n_as, M, K, x, ids, nth=8)
    assert nmse(got, O.glu(OPS[opname], cg, cu, ALPHA, LIMIT)) < NMSE_GATE


def test_plugin_fuses_moe_gate_up_glu(hb):
    """{MUL_MAT_ID, MUL_MAT_ID, GLU} of one decode token fuses (intermediates
    stay NaN) and equals the kernel-level fused call; unfused, the same."""
    import ggml_hip as G
    from ggml_hip import abi
    n_as, M, K, n_tokens, n_ids = 16, 768, 1024, 1, 4
    t, wu, wg, ids, x = _moe("Q4_K", n_as, M, K, n_tokens, n_ids, 7)
    tw_u = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M, n_as], name=b"ffn_up_exps")
    tw_g = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M, n_as], name=b"ffn_gate_exps")
    tx = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1, n_tokens], name=b"x")
    tids = abi.make_tensor(abi.GGML_TYPE_I32, [n_ids, n_tokens], name=b"ids")
    up = abi.make_tensor(abi.GGML_TYPE_F32, [M, n_ids, n_tokens], op=abi.GGML_OP_MUL_MAT_ID, srcs=(tw_u, tx, tids),
                         name=b"up")
    gate = abi.make_tensor(abi.GGML_TYPE_F32, [M, n_ids, n_tokens], op=abi.GGML_OP_MUL_MAT_ID,
                           srcs=(tw_g, tx, tids), name=b"gate")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, gate, up, [M, n_ids, n_tokens])
    hb.alloc([tw_u, tw_g], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([tx, tids, up, gate, glu], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(tw_u, wu)
    hb.set(tw_g, wg)
    hb.set(tx, x)
    hb.set(tids, ids)
    shape = (n_tokens, n_ids, M)
    for tns in (up, gate, glu):
        hb.set(tns, np.full(shape, np.nan, dtype=np.float32))
    assert hb.compute([gate, up, glu]) == abi.GGML_STATUS_SUCCESS
    assert np.isnan(hb.get(up, np.float32, shape)).all() and np.isnan(hb.get(gate, np.float32, shape)).all()
    out = hb.get(glu, np.float32, shape)
    want = G.mul_mat_id_vec_fused("Q4_K", _dev(wu), _dev(x), _dev(ids), w_gate=_dev(wg), glu="SWIGLU").cpu().numpy()
    np.testing.assert_array_equal(out, want)
    assert hb.compute([gate, up, glu], use_counts=False) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(up, np.float32, shape)).any()
    np.testing.assert_array_equal(hb.get(glu, np.float32, shape), out)


# ---------------------------------------------------------------- shared expert (MoE decode)

def _shared(tname, M, K, seed):
    t = TYPES[tname]
    su = O.quantize_rows(t, O.fill_normal(400 + seed, M * K, 0.0, 0.02).reshape(M, K))
    sg = O.quantize_rows(t, O.fill_normal(500 + seed, M * K, 0.0, 0.02).reshape(M, K))
    return su, sg


@pytest.mark.parametrize("tname,n_tokens,opname", [("Q4_K", 1, "SWIGLU"), ("Q4_K", 3, "GEGLU"),
                                                    ("Q6_K", 2, "SWIGLU_OAI"), ("Q8_0", 8, "SWIGLU_CLAMP")])
def test_fused_gate_up_glu_with_ids_and_shared_expert(tname, n_tokens, opname):
    """Routed experts and a shared expert in one launch: the routed rows equal
    the launch without the shared expert, and each token's shared row equals
    the one-column fused gate / up / GLU on the shared weights, bit for bit;
    both pass the CPU gate."""
    import ggml_hip as G
    n_as, M, K, n_ids = 16, 768, 1024, 4
    t, wu, wg, ids, x = _moe(tname, n_as, M, K, n_tokens, n_ids, 20 + n_tokens)
    su, sg = _shared(tname, M, K, n_tokens)
    wu_d, wg_d, x_d, ids_d, su_d, sg_d = _dev(wu), _dev(wg), _dev(x), _dev(ids), _dev(su), _dev(sg)
    routed, shared = G.mul_mat_id_vec_fused_shared(tname, wu_d, wg_d, x_d, ids_d, su_d, sg_d, glu=opname,
                                                   alpha=ALPHA, limit=LIMIT)
    routed, shared = routed.cpu().numpy(), shared.cpu().numpy()
    alone = G.mul_mat_id_vec_fused(tname, wu_d, x_d, ids_d, w_gate=wg_d, glu=opname, alpha=ALPHA,
                                   limit=LIMIT).cpu().numpy()
    np.testing.assert_array_equal(routed, alone)
    for tt in range(n_tokens):
        one = G.mul_mat_vec_fused(tname, su_d, K, x_d[tt, 0], w_gate=sg_d, glu=opname, alpha=ALPHA,
                                  limit=LIMIT).cpu().numpy().reshape(-1)
        np.testing.assert_array_equal(shared[tt], one)
    xs = x.reshape(n_tokens, K)
    cu = O.mul_mat(t, su, M, K, xs, nth=8)
    cg = O.mul_mat(t, sg, M, K, xs, nth=8)
    assert nmse(shared, O.glu(OPS[opname], cg, cu, ALPHA, LIMIT)) < NMSE_GATE


def test_fused_shared_expert_rejects_bad_arguments():
    import ctypes
    import ggml_hip as G
    n_as, M, K, n_tokens, n_ids = 4, 256, 256, 2, 2
    t, wu, wg, ids, x = _moe("Q4_K", n_as, M, K, n_tokens, n_ids, 3)
    su, sg = _shared("Q4_K", M, K, 3)
    d = [_dev(a) for a in (wu, wg, x, ids, su, sg)]
    out = torch.empty((n_tokens, n_ids, M), device="cuda")
    sout = torch.empty((n_tokens, M), device="cuda")
    p = lambda a: ctypes.c_void_p(a.data_ptr()) if a is not None else None  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(w_gate=d[1], shared_up=d[4], shared_gate=d[5], shared_dst=sout, sstride=M):
        return G.lib().hip_qmm_mul_mat_id_vec_fused_shared(
            t, p(d[0]), p(w_gate), K, M, d[0].stride(1), d[0].stride(0), n_as, p(d[2]), n_tokens, K, p(d[3]),
            n_ids, n_ids, G.GLU_OPS["SWIGLU"], 1.702, 7.0, p(out), M, p(shared_up), p(shared_gate), p(shared_dst),
            sstride, s)

    assert call() == 0
    assert call(w_gate=None) != 0       # the shared lane is gated
    assert call(shared_up=None) != 0
    assert call(shared_dst=None) != 0
    assert call(sstride=M - 1) != 0     # overlapping shared rows
    torch.cuda.synchronize()


def test_plugin_groups_and_fuses_shared_expert(hb):
    """graph_optimize moves the shared expert's {MUL_MAT, MUL_MAT, GLU} up
    behind the routed {MUL_MAT_ID, MUL_MAT_ID, GLU} (an unrelated node between
    them moves after) and keeps the routed input and ids alive until the
    shared GLU; the six nodes then run as one launch (intermediates stay NaN)
    equal to the kernel-level call, and unfused graphs give the same values."""
    import ctypes as C
    import ggml_hip as G
    from ggml_hip import abi
    n_as, M, K, n_tokens, n_ids = 16, 768, 1024, 3, 4
    t, wu, wg, ids, x = _moe("Q4_K", n_as, M, K, n_tokens, n_ids, 9)
    su, sg = _shared("Q4_K", M, K, 9)
    wo = weights_q(O.TYPE_Q4_K, 512, K, 5)
    q4 = abi.GGML_TYPE_Q4_K
    tw_u = abi.make_tensor(q4, [K, M, n_as], name=b"ffn_up_exps")
    tw_g = abi.make_tensor(q4, [K, M, n_as], name=b"ffn_gate_exps")
    tw_su = abi.make_tensor(q4, [K, M], name=b"ffn_up_shexp")
    tw_sg = abi.make_tensor(q4, [K, M], name=b"ffn_gate_shexp")
    tw_o = abi.make_tensor(q4, [K, 512], name=b"other")
    tx = abi.make_tensor(abi.GGML_TYPE_F32, [K, n_tokens], name=b"x")
    tids = abi.make_tensor(abi.GGML_TYPE_I32, [n_ids, n_tokens], name=b"ids")
    xr = abi.make_tensor(abi.GGML_TYPE_F32, [K, 1, n_tokens], op=abi.GGML_OP_RESHAPE, srcs=(tx,), name=b"x_r")
    xr.view_src = C.pointer(tx)
    rs = [M, n_ids, n_tokens]
    up = abi.make_tensor(abi.GGML_TYPE_F32, rs, op=abi.GGML_OP_MUL_MAT_ID, srcs=(tw_u, xr, tids), name=b"up")
    gate = abi.make_tensor(abi.GGML_TYPE_F32, rs, op=abi.GGML_OP_MUL_MAT_ID, srcs=(tw_g, xr, tids), name=b"gate")
    glu_r = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, gate, up, rs, name=b"routed")
    other = abi.make_tensor(abi.GGML_TYPE_F32, [512, n_tokens], op=abi.GGML_OP_MUL_MAT, srcs=(tw_o, tx), name=b"o")
    sup = abi.make_tensor(abi.GGML_TYPE_F32, [M, n_tokens], op=abi.GGML_OP_MUL_MAT, srcs=(tw_su, tx), name=b"sup")
    sgate = abi.make_tensor(abi.GGML_TYPE_F32, [M, n_tokens], op=abi.GGML_OP_MUL_MAT, srcs=(tw_sg, tx), name=b"sgt")
    glu_s = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, sgate, sup, [M, n_tokens], name=b"shared")
    hb.alloc([tw_u, tw_g, tw_su, tw_sg, tw_o], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([tx, tids, up, gate, glu_r, other, sup, sgate, glu_s], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    xr.data, xr.buffer = tx.data, tx.buffer
    for tns, arr in ((tw_u, wu), (tw_g, wg), (tw_su, su), (tw_sg, sg), (tw_o, wo), (tx, x), (tids, ids)):
        hb.set(tns, arr)
    order = [xr, gate, up, glu_r, other, sgate, sup, glu_s]

    # graph_optimize through the backend's vtable; without use counts the
    # nodes cannot be shown closed, so nothing moves
    same, deps0 = hb.optimized(order, use_counts=False)
    assert [C.addressof(n) for n in same] == [C.addressof(n) for n in order] and deps0 == []
    ordered = hb.optimized(order)
    want_order = [C.addressof(n) for n in [xr, gate, up, glu_r, sgate, sup, glu_s, other]]
    assert [C.addressof(n) for n in ordered[0]] == want_order
    assert sorted(ordered[1]) == sorted([(C.addressof(xr), C.addressof(glu_s)), (C.addressof(tids), C.addressof(glu_s))])

    rsh, ssh = (n_tokens, n_ids, M), (n_tokens, M)
    for tns, sh in ((up, rsh), (gate, rsh), (glu_r, rsh), (sup, ssh), (sgate, ssh), (glu_s, ssh)):
        hb.set(tns, np.full(sh, np.nan, dtype=np.float32))
    assert hb.compute(ordered[0]) == abi.GGML_STATUS_SUCCESS
    for tns, sh in ((up, rsh), (gate, rsh), (sup, ssh), (sgate, ssh)):
        assert np.isnan(hb.get(tns, np.float32, sh)).all()
    r_out, s_out = hb.get(glu_r, np.float32, rsh), hb.get(glu_s, np.float32, ssh)
    want_r, want_s = G.mul_mat_id_vec_fused_shared("Q4_K", _dev(wu), _dev(wg), _dev(x.reshape(n_tokens, 1, K)),
                                                   _dev(ids), _dev(su), _dev(sg), glu="SWIGLU")
    np.testing.assert_array_equal(r_out, want_r.cpu().numpy())
    np.testing.assert_array_equal(s_out, want_s.cpu().numpy())
    # unfused (no use counts): every node on its own
    assert hb.compute(ordered[0], use_counts=False) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(sup, np.float32, ssh)).any()
    np.testing.assert_array_equal(hb.get(glu_r, np.float32, rsh), r_out)
    u2, g2 = hb.get(sup, np.float32, ssh), hb.get(sgate, np.float32, ssh)
    assert nmse(hb.get(glu_s, np.float32, ssh), s_out) < 1e-10
    assert nmse(O.glu(O.GLU_SWIGLU, g2, u2), s_out) < 1e-10


# ---------------------------------------------------------------- MUL_MAT_ID bias lanes (ADD_ID)

def test_add_id_kernel_exact():
    """ADD_ID rows equal a + b[id] in f32 exactly; -1 ids copy the row."""
    import ggml_hip as G
    rng = np.random.default_rng(12)
    T_, S, nc, n_b = 5, 8, 777, 16
    a = rng.standard_normal((T_, S, nc)).astype(np.float32)
    b = rng.standard_normal((n_b, nc)).astype(np.float32)
    ids = rng.integers(-1, n_b, size=(T_, S)).astype(np.int32)
    got = G.add_id_f32(_dev(a), _dev(b), _dev(ids)).cpu().numpy()
    want = np.where((ids >= 0)[:, :, None], a + b[np.maximum(ids, 0)], a)
    np.testing.assert_array_equal(got, want)


def _moe_bias(n_as, M, seed):
    rng = np.random.default_rng(900 + seed)
    return ((rng.standard_normal((n_as, M)) * 0.5).astype(np.float32),
            (rng.standard_normal((n_as, M)) * 0.5).astype(np.float32))


@pytest.mark.parametrize("tname,n_tokens,opname", [("Q4_K", 1, "SWIGLU_OAI"), ("Q8_0", 3, "SWIGLU"),
                                                    ("Q6_K", 8, "GEGLU")])
def test_fused_gate_up_glu_with_ids_and_biases(tname, n_tokens, opname):
    """gpt-oss style MoE FFN with per-expert biases in one launch: equal bit
    for bit to the unfused GPU sequence (ids GEMV, ADD_ID, GLU) and within the
    CPU gate; the one-lane form equals ids GEMV + ADD_ID."""
    import ggml_hip as G
    n_as, M, K, n_ids = 16, 768, 1024, 4
    t, wu, wg, ids, x = _moe(tname, n_as, M, K, n_tokens, n_ids, 30 + n_tokens)
    ids[0, 0] = -1
    bu, bg = _moe_bias(n_as, M, n_tokens)
    wu_d, wg_d, x_d, ids_d, bu_d, bg_d = _dev(wu), _dev(wg), _dev(x), _dev(ids), _dev(bu), _dev(bg)
    got = G.mul_mat_id_vec_fused_bias(tname, wu_d, x_d, ids_d, bu_d, w_gate=wg_d, gate_bias=bg_d, glu=opname,
                                      alpha=ALPHA, limit=LIMIT).cpu().numpy()
    u = G.add_id_f32(G.mul_mat_id_vec_fused(tname, wu_d, x_d, ids_d), bu_d, ids_d)
    g = G.add_id_f32(G.mul_mat_id_vec_fused(tname, wg_d, x_d, ids_d), bg_d, ids_d)
    want = G.glu_f32(g.view(-1, M), u.view(-1, M), opname, alpha=ALPHA, limit=LIMIT).view(n_tokens, n_ids, M)
    np.testing.assert_array_equal(got, want.cpu().numpy())
    assert np.all(got[0, 0] == 0.0)  # an id of -1: zero row, no bias
    one = G.mul_mat_id_vec_fused_bias(tname, wu_d, x_d, ids_d, bu_d).cpu().numpy()
    one[0, 0] = 0.0  # the fused lone lane leaves the -1 row zero; ADD_ID alone would copy its input (zero) too
    np.testing.assert_array_equal(one, u.cpu().numpy())
    ok = ids >= 0
    cu = O.mul_mat_id(t, wu, n_as, M, K, x, np.where(ok, ids, -1), nth=8) + np.where(ok[:, :, None], bu[np.maximum(ids, 0)], 0)
    cg = O.mul_mat_id(t, wg, n_as, M, K, x, np.where(ok, ids, -1), nth=8) + np.where(ok[:, :, None], bg[np.maximum(ids, 0)], 0)
    assert nmse(got[ok], O.glu(OPS[opname], cg, cu, ALPHA, LIMIT)[ok]) < NMSE_GATE


def test_plugin_fuses_moe_bias_lanes(hb):
    """{MUL_MAT_ID, ADD_ID, MUL_MAT_ID, ADD_ID, GLU} and {MUL_MAT_ID, ADD_ID}
    fuse (intermediates stay NaN) and equal the kernel-level calls; without
    use counts every node runs alone, with the same values."""
    import ggml_hip as G
    from ggml_hip import abi
    n_as, M, K, n_tokens, n_ids = 16, 768, 1024, 2, 4
    t, wu, wg, ids, x = _moe("Q4_K", n_as, M, K, n_tokens, n_ids, 17)
    bu, bg = _moe_bias(n_as, M, 17)
    q4, f32 = abi.GGML_TYPE_Q4_K, abi.GGML_TYPE_F32
    tw_u = abi.make_tensor(q4, [K, M, n_as], name=b"ffn_up_exps")
    tw_g = abi.make_tensor(q4, [K, M, n_as], name=b"ffn_gate_exps")
    tb_u = abi.make_tensor(f32, [M, n_as], name=b"ffn_up_exps_b")
    tb_g = abi.make_tensor(f32, [M, n_as], name=b"ffn_gate_exps_b")
    tx = abi.make_tensor(f32, [K, 1, n_tokens], name=b"x")
    tids = abi.make_tensor(abi.GGML_TYPE_I32, [n_ids, n_tokens], name=b"ids")
    rs = [M, n_ids, n_tokens]
    up = abi.make_tensor(f32, rs, op=abi.GGML_OP_MUL_MAT_ID, srcs=(tw_u, tx, tids), name=b"up")
    upb = abi.make_tensor(f32, rs, op=abi.GGML_OP_ADD_ID, srcs=(up, tb_u, tids), name=b"up_b")
    gate = abi.make_tensor(f32, rs, op=abi.GGML_OP_MUL_MAT_ID, srcs=(tw_g, tx, tids), name=b"gate")
    gateb = abi.make_tensor(f32, rs, op=abi.GGML_OP_ADD_ID, srcs=(gate, tb_g, tids), name=b"gate_b")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU_OAI, gateb, upb, rs, ALPHA, LIMIT)
    # a lone biased projection (the down projection's shape of use)
    lone = abi.make_tensor(f32, rs, op=abi.GGML_OP_MUL_MAT_ID, srcs=(tw_u, tx, tids), name=b"lone")
    loneb = abi.make_tensor(f32, rs, op=abi.GGML_OP_ADD_ID, srcs=(lone, tb_u, tids), name=b"lone_b")
    hb.alloc([tw_u, tw_g], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    inter = [up, upb, gate, gateb, lone]
    hb.alloc([tb_u, tb_g, tx, tids, glu, loneb] + inter, usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    for tns, arr in ((tw_u, wu), (tw_g, wg), (tb_u, bu), (tb_g, bg), (tx, x), (tids, ids)):
        hb.set(tns, arr)
    shape = (n_tokens, n_ids, M)
    nodes = [gate, gateb, up, upb, glu, lone, loneb]
    for tns in inter + [glu, loneb]:
        hb.set(tns, np.full(shape, np.nan, dtype=np.float32))
    assert hb.compute(nodes) == abi.GGML_STATUS_SUCCESS
    for tns in inter:
        assert np.isnan(hb.get(tns, np.float32, shape)).all()
    out, lout = hb.get(glu, np.float32, shape), hb.get(loneb, np.float32, shape)
    wu_d, wg_d, x_d, ids_d = _dev(wu), _dev(wg), _dev(x), _dev(ids)
    want = G.mul_mat_id_vec_fused_bias("Q4_K", wu_d, x_d, ids_d, _dev(bu), w_gate=wg_d, gate_bias=_dev(bg),
                                       glu="SWIGLU_OAI", alpha=ALPHA, limit=LIMIT).cpu().numpy()
    np.testing.assert_array_equal(out, want)
    np.testing.assert_array_equal(lout, G.mul_mat_id_vec_fused_bias("Q4_K", wu_d, x_d, ids_d, _dev(bu)).cpu().numpy())
    assert hb.compute(nodes, use_counts=False) == abi.GGML_STATUS_SUCCESS
    assert not np.isnan(hb.get(upb, np.float32, shape)).any()
    np.testing.assert_array_equal(hb.get(glu, np.float32, shape), out)
    np.testing.assert_array_equal(hb.get(loneb, np.float32, shape), lout)
