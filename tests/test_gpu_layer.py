"""A Llama-3-8B decode layer through the plugin, split as the scheduler
splits it (computeSplits, src/ggml/backend_sched.zig:1405-1500).

The layer's graph holds every node, the CPU-only ones too: RMS_NORM and
FLASH_ATTN_EXT are not ops this backend takes (supports_op answers false), so
the scheduler cuts the graph into three splits for the HIP backend, each run
with graph_compute on a view of the whole graph's node array that shares its
use counts (ggml_graph_view), and does the CPU nodes between them (here in
numpy, and one token's attention is the exact value v of its own position per
query head):

  [attn_norm] | q k v | [attention] | o h=x+o | [ffn_norm] | g u glu dn out=h+dn

Weights: Llama-3-8B's shapes in the Q4_K_M mix (attn_q/k/o, ffn_gate/up Q4_K;
attn_v, ffn_down Q6_K), synthetic N(0, 0.02) quantized by the oracle.  At one
token the o projection and the residual add fuse ({MUL_MAT, ADD}), gate / up /
GLU fuse, and ffn_down and the second residual add fuse, so o, g, u and dn are
never written (pre-filled with NaN); at four tokens nothing fuses and every
node is written.  Every result the layer hands on is checked against the
oracle's CPU path on the same inputs: NMSE < 5e-4, and within 2e-6 of the f64
Q8_1 evaluation for the projections."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, nmse, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
F64_TOL = 2e-6
GGML_OP_RMS_NORM, GGML_OP_FLASH_ATTN_EXT = 24, 71  # src/ggml/types.zig:24-48

D, KV, FF, HEADS, KV_HEADS, HD = 4096, 1024, 14336, 32, 8, 128


@pytest.fixture(scope="module")
def hb():
    from ggml_hip.backend import HipBackend
    with HipBackend(0) as b:
        yield b


@pytest.fixture(scope="module")
def layer_weights():
    q4, q6 = O.TYPE_Q4_K, O.TYPE_Q6_K
    return {"q": (q4, weights_q(q4, D, D, 0)), "k": (q4, weights_q(q4, KV, D, 1)), "v": (q6, weights_q(q6, KV, D, 2)),
            "o": (q4, weights_q(q4, D, D, 3)), "gate": (q4, weights_q(q4, FF, D, 4)),
            "up": (q4, weights_q(q4, FF, D, 5)), "down": (q6, weights_q(q6, D, FF, 6))}


def _rms_norm(x, eps=1e-5):
    x = x.astype(np.float64)
    return (x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)).astype(np.float32)


def _check_proj(t, wq, nrows, K, x, got):
    import ggml_hip as G
    y = G.quantize_q8_1(torch.from_numpy(np.ascontiguousarray(x)).cuda(), K).cpu().numpy()
    ideal = O.mul_mat_q8_1_f64(t, wq, nrows, K, y, x.shape[0])
    assert max_err_scaled(got, ideal) < F64_TOL
    assert nmse(got, O.mul_mat_x86(t, wq, nrows, K, x, nth=8)) < NMSE_GATE


@pytest.mark.parametrize("T", [1, 4])
def test_llama3_8b_decode_layer_in_splits(hb, layer_weights, T):
    from ggml_hip import abi
    W = layer_weights
    gt = {O.TYPE_Q4_K: abi.GGML_TYPE_Q4_K, O.TYPE_Q6_K: abi.GGML_TYPE_Q6_K}
    f32 = abi.GGML_TYPE_F32
    w = {k: abi.make_tensor(gt[t], [K, n], name=k.encode())
         for k, (t, _), (n, K) in zip(W, W.values(), [(D, D), (KV, D), (KV, D), (D, D), (FF, D), (FF, D), (D, FF)])}
    x = abi.make_tensor(f32, [D, T], name=b"x")
    attn_norm = abi.make_tensor(f32, [D, T], op=GGML_OP_RMS_NORM, srcs=(x,), name=b"attn_norm")
    q = abi.make_tensor(f32, [D, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["q"], attn_norm), name=b"q")
    k = abi.make_tensor(f32, [KV, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["k"], attn_norm), name=b"k")
    v = abi.make_tensor(f32, [KV, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["v"], attn_norm), name=b"v")
    attn = abi.make_tensor(f32, [D, T], op=GGML_OP_FLASH_ATTN_EXT, srcs=(q, k, v), name=b"attn")
    o = abi.make_tensor(f32, [D, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["o"], attn), name=b"o")
    h = abi.make_tensor(f32, [D, T], op=abi.GGML_OP_ADD, srcs=(x, o), name=b"h")
    ffn_norm = abi.make_tensor(f32, [D, T], op=GGML_OP_RMS_NORM, srcs=(h,), name=b"ffn_norm")
    g = abi.make_tensor(f32, [FF, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["gate"], ffn_norm), name=b"g")
    u = abi.make_tensor(f32, [FF, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["up"], ffn_norm), name=b"u")
    glu = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [FF, T])
    dn = abi.make_tensor(f32, [D, T], op=abi.GGML_OP_MUL_MAT, srcs=(w["down"], glu), name=b"dn")
    out = abi.make_tensor(f32, [D, T], op=abi.GGML_OP_ADD, srcs=(h, dn), name=b"out")
    out.flags |= abi.GGML_TENSOR_FLAG_OUTPUT
    nodes = [attn_norm, q, k, v, attn, o, h, ffn_norm, g, u, glu, dn, out]
    from ggml_hip.backend import lib as backend_lib
    ok = lambda t: bool(backend_lib().ggml_backend_hip_op_supported(C.pointer(t)))  # noqa: E731
    assert [ok(n) for n in nodes] == [False, True, True, True, False, True, True, False, True, True, True, True,
                                      True]

    hb.alloc(list(w.values()), usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([x] + nodes, usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    for name, (t, wq) in W.items():
        hb.set(w[name], wq)
    xv = acts(T, D, 7)
    hb.set(x, xv)
    for n in nodes:
        hb.set(n, np.full(abi.nbytes(n) // 4, np.nan, dtype=np.float32))
    get = lambda t, rows: hb.get(t, np.float32, (T, rows))  # noqa: E731

    # CPU: attn_norm; split 1: q k v
    an = _rms_norm(xv)
    hb.set(attn_norm, an)
    assert hb.compute_view(nodes, 1, 4) == abi.GGML_STATUS_SUCCESS
    qv, kv, vv = get(q, D), get(k, KV), get(v, KV)
    for name, got, rows in (("q", qv, D), ("k", kv, KV), ("v", vv, KV)):
        _check_proj(W[name][0], W[name][1], rows, D, an, got)
    # CPU: one position per token, so softmax over a single key is 1 and each
    # query head reads the v of its key-value head (grouped-query attention)
    av = np.repeat(vv.reshape(T, KV_HEADS, HD), HEADS // KV_HEADS, axis=1).reshape(T, D)
    hb.set(attn, av)
    # split 2: o, h = x + o
    assert hb.compute_view(nodes, 5, 7) == abi.GGML_STATUS_SUCCESS
    hv = get(h, D)
    ov_cpu = O.mul_mat_x86(W["o"][0], W["o"][1], D, D, av, nth=8)
    assert nmse(hv, xv + ov_cpu) < NMSE_GATE
    if T == 1:
        assert np.isnan(get(o, D)).all()  # fused with the residual add
    else:
        _check_proj(W["o"][0], W["o"][1], D, D, av, get(o, D))
        np.testing.assert_array_equal(hv, xv + get(o, D))
    # CPU: ffn_norm; split 3: g u glu dn out
    fn = _rms_norm(hv)
    hb.set(ffn_norm, fn)
    assert hb.compute_view(nodes, 8, 13) == abi.GGML_STATUS_SUCCESS
    outv = get(out, D)
    gc = O.mul_mat_x86(W["gate"][0], W["gate"][1], FF, D, fn, nth=8)
    uc = O.mul_mat_x86(W["up"][0], W["up"][1], FF, D, fn, nth=8)
    if T == 1:
        for t_ in (g, u, dn):
            assert np.isnan(get(t_, FF if t_ is not dn else D)).all()
        a_gpu = None
    else:
        a_gpu = get(glu, FF)
        assert nmse(a_gpu, O.glu(O.GLU_SWIGLU, gc, uc)) < NMSE_GATE
        _check_proj(W["down"][0], W["down"][1], D, FF, a_gpu, get(dn, D))
    a_cpu = O.glu(O.GLU_SWIGLU, gc, uc) if a_gpu is None else a_gpu
    dc = O.mul_mat_x86(W["down"][0], W["down"][1], D, FF, a_cpu, nth=8)
    assert nmse(outv, hv + dc) < NMSE_GATE
    assert np.all(np.isfinite(outv))


# ---------------------------------------------------------------- Qwen3-30B-A3B MoE FFN in splits

QN_EMBD, QN_FF, QN_EXPERTS, QN_TOP_K = 2048, 768, 128, 8
GGML_OP_MUL, GGML_OP_SOFT_MAX, GGML_OP_GET_ROWS, GGML_OP_TOP_K = 6, 43, 39, 67  # src/ggml/types.zig:24-48


@pytest.fixture(scope="module")
def moe_weights():
    """Qwen3-30B-A3B's routed experts (128 of them, gate/up 768x2048 and down
    2048x768 each, Q4_K), synthetic N(0, 0.02) quantized by the oracle."""
    q4 = O.TYPE_Q4_K
    from cases import weights_f32

    def experts(nrows, K, idx):
        return O.quantize_rows(q4, weights_f32(QN_EXPERTS * nrows, K, idx)).reshape(QN_EXPERTS, nrows, -1)
    return {"gate": experts(QN_FF, QN_EMBD, 20), "up": experts(QN_FF, QN_EMBD, 21),
            "down": experts(QN_EMBD, QN_FF, 22)}


@pytest.mark.parametrize("T", [1, 64])
def test_qwen3_moe_ffn_in_splits(hb, moe_weights, T):
    """The MoE FFN of llama's graph (build_moe_ffn, src/llama/graph.zig:3265-3400)
    as the scheduler splits it: the router (an f32 MUL_MAT), its softmax, top-k
    and weights stay on the CPU (supports_op false), then one split for the
    HIP backend:

      [norm, router, softmax, top-k, weights] | up gate glu down | [weighted sum]

    up / gate / GLU fuse into one launch (the ids GEMV at one token, the
    grouped fused MMQ at 64), so up and gate stay NaN; down runs the grouped
    MMQ or the ids GEMV.  The expert outputs are checked against the CPU path
    (mul_mat_id and the GLU op of the oracle) with NMSE < 5e-4, and so is the
    layer's weighted sum over the 8 slots."""
    from ggml_hip import abi
    from cases import nmse as _nmse
    W = moe_weights
    f32, i32, q4 = abi.GGML_TYPE_F32, abi.GGML_TYPE_I32, abi.GGML_TYPE_Q4_K
    x = abi.make_tensor(f32, [QN_EMBD, 1, T], name=b"x")
    norm = abi.make_tensor(f32, [QN_EMBD, 1, T], op=GGML_OP_RMS_NORM, srcs=(x,), name=b"ffn_norm")
    w_inp = abi.make_tensor(f32, [QN_EMBD, QN_EXPERTS], name=b"ffn_gate_inp")
    logits = abi.make_tensor(f32, [QN_EXPERTS, T], op=abi.GGML_OP_MUL_MAT, srcs=(w_inp, norm), name=b"logits")
    probs = abi.make_tensor(f32, [QN_EXPERTS, T], op=GGML_OP_SOFT_MAX, srcs=(logits,), name=b"probs")
    sel = abi.make_tensor(i32, [QN_TOP_K, T], op=GGML_OP_TOP_K, srcs=(probs,), name=b"selected")
    wts = abi.make_tensor(f32, [1, QN_TOP_K, T], op=GGML_OP_GET_ROWS, srcs=(probs, sel), name=b"weights")
    wg = abi.make_tensor(q4, [QN_EMBD, QN_FF, QN_EXPERTS], name=b"ffn_gate_exps")
    wu = abi.make_tensor(q4, [QN_EMBD, QN_FF, QN_EXPERTS], name=b"ffn_up_exps")
    wd = abi.make_tensor(q4, [QN_FF, QN_EMBD, QN_EXPERTS], name=b"ffn_down_exps")
    up = abi.make_tensor(f32, [QN_FF, QN_TOP_K, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(wu, norm, sel), name=b"up")
    gate = abi.make_tensor(f32, [QN_FF, QN_TOP_K, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(wg, norm, sel), name=b"gate")
    par = abi.make_glu(abi.GGML_GLU_OP_SWIGLU, gate, up, [QN_FF, QN_TOP_K, T], name=b"ffn_par")
    down = abi.make_tensor(f32, [QN_EMBD, QN_TOP_K, T], op=abi.GGML_OP_MUL_MAT_ID, srcs=(wd, par, sel), name=b"down")
    weighted = abi.make_tensor(f32, [QN_EMBD, QN_TOP_K, T], op=GGML_OP_MUL, srcs=(down, wts), name=b"weighted")
    weighted.flags |= abi.GGML_TENSOR_FLAG_OUTPUT
    nodes = [norm, logits, probs, sel, wts, up, gate, par, down, weighted]
    from ggml_hip.backend import lib as backend_lib
    ok = lambda t: bool(backend_lib().ggml_backend_hip_op_supported(C.pointer(t)))  # noqa: E731
    assert [ok(n) for n in nodes] == [False] * 5 + [True] * 4 + [False]

    hb.alloc([wg, wu, wd], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([norm, sel, up, gate, par, down], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    for t_, name in ((wg, "gate"), (wu, "up"), (wd, "down")):
        hb.set(t_, W[name])
    for n in (up, gate, par, down):
        hb.set(n, np.full(abi.nbytes(n) // 4, np.nan, dtype=np.float32))

    # CPU: norm, router, softmax, top-8, their weights (renormalised, Qwen3's norm_w)
    xv = acts(T, QN_EMBD, 9)
    nv = _rms_norm(xv)
    rng = np.random.default_rng(31)
    router = (rng.standard_normal((QN_EXPERTS, QN_EMBD)) * 0.02).astype(np.float32)
    lg = nv @ router.T
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :QN_TOP_K].astype(np.int32)
    wv = np.take_along_axis(p, ids, axis=1)
    wv /= wv.sum(axis=1, keepdims=True)
    hb.set(norm, nv)
    hb.set(sel, ids)
    # the HIP split: up gate glu down
    assert hb.compute_view(nodes, 5, 9) == abi.GGML_STATUS_SUCCESS
    shape_ff = (T, QN_TOP_K, QN_FF)
    assert np.isnan(hb.get(up, np.float32, shape_ff)).all() and np.isnan(hb.get(gate, np.float32, shape_ff)).all()
    par_gpu = hb.get(par, np.float32, shape_ff)
    dn_gpu = hb.get(down, np.float32, (T, QN_TOP_K, QN_EMBD))
    # the CPU path on the same inputs
    xr = nv.reshape(T, 1, QN_EMBD)
    cg = O.mul_mat_id(O.TYPE_Q4_K, W["gate"], QN_EXPERTS, QN_FF, QN_EMBD, xr, ids, nth=8)
    cu = O.mul_mat_id(O.TYPE_Q4_K, W["up"], QN_EXPERTS, QN_FF, QN_EMBD, xr, ids, nth=8)
    par_cpu = O.glu(O.GLU_SWIGLU, cg, cu)
    assert _nmse(par_gpu, par_cpu) < NMSE_GATE
    dn_cpu = O.mul_mat_id(O.TYPE_Q4_K, W["down"], QN_EXPERTS, QN_EMBD, QN_FF, par_cpu, ids, nth=8)
    assert _nmse(dn_gpu, dn_cpu) < NMSE_GATE
    # CPU: the weighted sum over the slots
    out_gpu = (dn_gpu * wv[:, :, None]).sum(axis=1)
    out_cpu = (dn_cpu * wv[:, :, None]).sum(axis=1)
    assert _nmse(out_gpu, out_cpu) < NMSE_GATE
    assert np.all(np.isfinite(out_gpu))
