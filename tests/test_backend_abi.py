"""CPU checks of the C ABI and the backend plugin layer: every function the
include/ headers declare is exported, the ctypes layouts agree with the
reference's layout facts, and the device-independent vtable answers
(supports_op, get_alloc_size, the registry without a device) behave as the
reference's CUDA backend does.  Nothing here launches GPU work."""
import ctypes as C
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions(path):
    text = re.sub(r"/\*.*?\*/", " ", path.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    text = re.sub(r"#[^\n]*", " ", text)
    # the extern "C" wrapper: its opening line and its lone closing brace
    text = text.replace('extern "C" {', " ")
    text = re.sub(r"(?m)^\s*\}\s*$", " ", text)
    # drop struct / enum bodies (function-pointer members live there)
    prev = None
    while prev != text:
        prev = text
        text = re.sub(r"\{[^{}]*\}", " ", text)
    names = []
    for stmt in text.split(";"):
        stmt = " ".join(stmt.split())
        if not stmt or "(*" in stmt or stmt.startswith(("typedef", "struct", "enum", "extern \"C\"")):
            continue
        m = re.match(r"^(?:const )?[A-Za-z_][\w ]*[\s\*]+([A-Za-z_]\w*)\s*\(", stmt)
        if m:
            names.append(m.group(1))
    return names


@pytest.fixture(scope="module")
def L():
    import ggml_hip.backend as B
    return B.lib()


def test_headers_declare_functions():
    names = {h.name: declared_functions(h) for h in HEADERS}
    assert len(names["ggml_hip_qmm.h"]) >= 14
    assert "ggml_backend_hip_reg" in names["ggml_hip_backend.h"]
    assert names["ggml_hip_ggml_abi.h"] == []


def test_every_declared_function_is_exported(L):
    missing = [n for h in HEADERS for n in declared_functions(h) if not hasattr(L, n)]
    assert not missing, missing


def test_ten_hip_exports_mirror_the_cuda_header(L):
    # cuda/backend.zig:1225-1236 with `cuda` -> `hip`, plus the dynamic-loading pair
    for n in ["ggml_backend_hip_reg", "ggml_backend_hip_init", "ggml_backend_is_hip", "ggml_backend_hip_buffer_type",
              "ggml_backend_hip_host_buffer_type", "ggml_backend_hip_get_device_count",
              "ggml_backend_hip_get_device_description", "ggml_backend_hip_get_device_memory",
              "ggml_backend_hip_register_host_buffer", "ggml_backend_hip_unregister_host_buffer",
              "ggml_backend_init", "ggml_backend_score"]:
        assert hasattr(L, n), n


def test_layouts():
    from ggml_hip import abi
    # the trailing 8-byte padding member ends the tensor (backend_meta.zig:3221-3222)
    assert C.sizeof(abi.ggml_tensor) - 8 == abi.ggml_tensor.padding.offset
    assert C.sizeof(abi.ggml_tensor) == 336
    assert abi.ggml_tensor.data.offset == 248 and abi.ggml_tensor.src.offset == 152
    # cgraph: three ints then the node array (impl.zig:469-485)
    assert abi.ggml_cgraph.nodes.offset == 16
    # vtables: one pointer per member in the CUDA backend's order
    assert C.sizeof(abi.buffer_i) == 14 * 8 and C.sizeof(abi.buffer_type_i) == 8 * 8
    assert C.sizeof(abi.backend_i) == 16 * 8 and C.sizeof(abi.device_i) == 15 * 8 and C.sizeof(abi.reg_i) == 4 * 8


def test_registry_answers(L):
    import ggml_hip.backend as B
    n = L.ggml_backend_hip_get_device_count()
    r = B.registry()
    rp = L.ggml_backend_hip_reg()
    assert r.api_version == 2
    assert r.iface.get_name(rp) == b"HIP"
    assert r.iface.get_device_count(rp) == n
    assert L.ggml_backend_init() == rp
    assert r.iface.get_proc_address(rp, b"no_such_symbol") is None
    assert r.iface.get_proc_address(rp, b"ggml_backend_register_host_buffer")
    assert L.ggml_backend_hip_register_host_buffer(None, 0) is False
    if n == 0:
        assert L.ggml_backend_score() == 0
        assert not L.ggml_backend_hip_init(0)
        assert not L.ggml_backend_hip_buffer_type(0)
        assert not L.ggml_backend_is_hip(None)
    assert not L.ggml_backend_hip_init(-1)
    assert not L.ggml_backend_hip_buffer_type(n)


def mm(a_type, K, M, N, batch=(1, 1, 1, 1)):
    from ggml_hip import abi
    a = abi.make_tensor(a_type, [K, M, batch[0], batch[1]])
    b = abi.make_tensor(abi.GGML_TYPE_F32, [K, N, batch[2], batch[3]])
    d = abi.make_tensor(abi.GGML_TYPE_F32, [M, N, batch[2], batch[3]], op=abi.GGML_OP_MUL_MAT, srcs=(a, b))
    return a, b, d


def mmid(a_type, K, M, n_as, n_used, n_tokens, ne11=None):
    from ggml_hip import abi
    ne11 = n_used if ne11 is None else ne11
    a = abi.make_tensor(a_type, [K, M, n_as])
    b = abi.make_tensor(abi.GGML_TYPE_F32, [K, ne11, n_tokens])
    ids = abi.make_tensor(abi.GGML_TYPE_I32, [n_used, n_tokens])
    d = abi.make_tensor(abi.GGML_TYPE_F32, [M, n_used, n_tokens], op=abi.GGML_OP_MUL_MAT_ID, srcs=(a, b, ids))
    return a, b, ids, d


def test_supports_op(L):
    from ggml_hip import abi
    ok = lambda t: L.ggml_backend_hip_op_supported(C.pointer(t))  # noqa: E731
    for t in (abi.GGML_TYPE_Q4_K, abi.GGML_TYPE_Q5_K, abi.GGML_TYPE_Q6_K, abi.GGML_TYPE_Q8_0, abi.GGML_TYPE_Q4_0,
              abi.GGML_TYPE_IQ4_XS):
        assert ok(mm(t, 4096, 4096, 1)[2])
        assert ok(mm(t, 4096, 1024, 512, batch=(2, 1, 4, 1))[2])  # broadcast over dim 2
        assert ok(mmid(t, 2048, 768, 128, 8, 512)[3])
    assert ok(mm(abi.GGML_TYPE_Q8_0, 96, 64, 3)[2])  # Q8_0 / Q4_0 rows need only whole 32-blocks
    assert ok(mm(abi.GGML_TYPE_Q4_0, 96, 64, 3)[2])
    assert not ok(mm(abi.GGML_TYPE_F16, 4096, 4096, 1)[2])  # only the quantized weight types
    assert not ok(mm(abi.GGML_TYPE_Q4_K, 4096, 4096, 1, batch=(3, 1, 4, 1))[2])  # 4 % 3: no broadcast
    a, b, d = mm(abi.GGML_TYPE_Q4_K, 4096, 4096, 2)
    b.nb[0] = 8  # strided elements
    assert not ok(d)
    a, b, d = mm(abi.GGML_TYPE_Q4_K, 4096, 4096, 2)
    d.type = abi.GGML_TYPE_F16
    assert not ok(d)
    assert not ok(mmid(abi.GGML_TYPE_Q8_0, 96, 64, 4, 2, 3)[3])  # grouped MMQ needs K % 256
    assert not ok(mmid(abi.GGML_TYPE_Q4_K, 256, 64, 2000, 2, 3)[3])  # more than 1024 experts
    assert ok(mmid(abi.GGML_TYPE_Q4_K, 256, 64, 16, 4, 3, ne11=1)[3])  # one row broadcast per token
    assert not ok(mmid(abi.GGML_TYPE_Q4_K, 256, 64, 16, 4, 3, ne11=2)[3])
    other = abi.make_tensor(abi.GGML_TYPE_F32, [8, 8], op=abi.GGML_OP_ADD)
    assert not ok(other)  # an ADD without sources
    # GLU: f32, the device's five ops, split (same shapes) or one tensor of two halves
    g = abi.make_tensor(abi.GGML_TYPE_F32, [14336, 1], name=b"g")
    u = abi.make_tensor(abi.GGML_TYPE_F32, [14336, 1], name=b"u")
    for op in (abi.GGML_GLU_OP_REGLU, abi.GGML_GLU_OP_GEGLU, abi.GGML_GLU_OP_SWIGLU, abi.GGML_GLU_OP_SWIGLU_OAI,
               abi.GGML_GLU_OP_SWIGLU_CLAMP):
        assert ok(abi.make_glu(op, g, u, [14336, 1]))
    for op in (abi.GGML_GLU_OP_GEGLU_ERF, abi.GGML_GLU_OP_GEGLU_QUICK, 7):
        assert not ok(abi.make_glu(op, g, u, [14336, 1]))
    assert not ok(abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [14336, 2]))  # dst shape differs
    half = abi.make_tensor(abi.GGML_TYPE_F32, [64, 3], name=b"gu")
    single = abi.make_tensor(abi.GGML_TYPE_F32, [32, 3], op=abi.GGML_OP_GLU, srcs=(half,))
    single.op_params[0] = abi.GGML_GLU_OP_SWIGLU
    assert ok(single)
    single.ne[0] = 31
    assert not ok(single)
    h16 = abi.make_tensor(abi.GGML_TYPE_F16, [14336, 1])
    assert not ok(abi.make_glu(abi.GGML_GLU_OP_SWIGLU, h16, h16, [14336, 1]))
    # ADD: same-shape f32 only (no broadcasting)
    assert ok(abi.make_tensor(abi.GGML_TYPE_F32, [14336, 1], op=abi.GGML_OP_ADD, srcs=(g, u)))
    row = abi.make_tensor(abi.GGML_TYPE_F32, [14336, 1])
    mat = abi.make_tensor(abi.GGML_TYPE_F32, [14336, 4])
    assert not ok(abi.make_tensor(abi.GGML_TYPE_F32, [14336, 4], op=abi.GGML_OP_ADD, srcs=(mat, row)))
    for op in (abi.GGML_OP_NONE, abi.GGML_OP_VIEW, abi.GGML_OP_RESHAPE, abi.GGML_OP_PERMUTE, abi.GGML_OP_TRANSPOSE):
        assert ok(abi.make_tensor(abi.GGML_TYPE_F32, [8, 8], op=op))


def test_alloc_size_pads_quantized_rows(L):
    from ggml_hip import abi
    size = lambda t: L.ggml_backend_hip_tensor_alloc_size(C.pointer(t))  # noqa: E731
    t = abi.make_tensor(abi.GGML_TYPE_Q4_K, [4096, 14336])
    assert size(t) == 14336 * 16 * 144  # rows already a multiple of 512
    t = abi.make_tensor(abi.GGML_TYPE_Q4_K, [4352, 3])  # 4352 % 512 = 256 -> one extra Q4_K block
    assert size(t) == 3 * 17 * 144 + 144
    t = abi.make_tensor(abi.GGML_TYPE_Q8_0, [544, 2])  # 32 past 512 -> 480 elements = 15 blocks
    assert size(t) == 2 * 17 * 34 + 15 * 34
    t = abi.make_tensor(abi.GGML_TYPE_F32, [100, 3])
    assert size(t) == 1200


def test_fused_and_elementwise_entry_points_reject_bad_arguments(L):
    """Argument checks of the fused-epilogue GEMV and the GLU / ADD entry
    points: each rejected call returns hipErrorInvalidValue (1) before any
    device work, so this runs without a GPU."""
    import ctypes as C
    vp, i64, f = C.c_void_p, C.c_int64, C.c_float
    L.hip_qmm_mul_mat_vec_fused.restype = C.c_int
    L.hip_qmm_mul_mat_vec_fused.argtypes = [C.c_int, vp, vp, i64, i64, i64, vp, vp, vp, C.c_int, f, f, vp, vp]
    L.hip_qmm_glu_f32.restype = C.c_int
    L.hip_qmm_glu_f32.argtypes = [C.c_int, f, f, i64, i64, vp, i64, vp, i64, vp, i64, vp]
    L.hip_qmm_add_f32.restype = C.c_int
    L.hip_qmm_add_f32.argtypes = [i64, i64, vp, i64, vp, i64, vp, i64, vp]
    Q4K, F16 = 12, 1
    w, x, d = 0x100000, 0x200000, 0x300000  # aligned placeholders, never dereferenced
    rs = 16 * 144

    def fused(**kw):
        a = dict(type=Q4K, w=w, wg=None, K=4096, M=64, rs=rs, x=x, b=None, gb=None, op=2, dst=d)
        a.update(kw)
        return L.hip_qmm_mul_mat_vec_fused(a["type"], a["w"], a["wg"], a["K"], a["M"], a["rs"], a["x"], a["b"],
                                           a["gb"], a["op"], 1.702, 7.0, a["dst"], None)

    assert fused(type=F16) == 1                      # not a weight type
    assert fused(K=4000) == 1                         # Q4_K rows are whole super-blocks
    assert fused(K=65536, rs=256 * 144) == 1          # beyond the 32768-element column
    assert fused(w=None) == 1 and fused(x=None) == 1 and fused(dst=None) == 1
    assert fused(x=x + 4) == 1                        # column not 16-byte aligned
    assert fused(w=w + 2) == 1                        # Q4_K blocks are read 16 bytes at a time
    assert fused(wg=w + 2) == 1
    assert fused(gb=x) == 1                           # a gate bias without a gate
    assert fused(wg=w, op=4) == 1 and fused(wg=w, op=5) == 1 and fused(wg=w, op=7) == 1  # no device op
    assert fused(rs=rs - 1) == 1                      # rows shorter than K
    assert L.hip_qmm_glu_f32(4, 0.0, 0.0, 8, 2, x, 8, x, 8, d, 8, None) == 1
    assert L.hip_qmm_glu_f32(2, 0.0, 0.0, -1, 2, x, 8, x, 8, d, 8, None) == 1
    assert L.hip_qmm_glu_f32(2, 0.0, 0.0, 8, 2, x, 4, x, 8, d, 8, None) == 1  # stride below the row
    assert L.hip_qmm_glu_f32(2, 0.0, 0.0, 8, 2, None, 8, x, 8, d, 8, None) == 1
    assert L.hip_qmm_glu_f32(2, 0.0, 0.0, 0, 2, x, 8, x, 8, d, 8, None) == 0   # nothing to do
    assert L.hip_qmm_add_f32(8, 2, x, 8, x, 8, None, 8, None) == 1
    assert L.hip_qmm_add_f32(8, 0, x, 8, x, 8, d, 8, None) == 0


@pytest.mark.parametrize("env_extra", [{}, {"GGML_HIP_FUSION": "0"},
                                 {"GGML_HIP_FUSION": "1", "GGML_HIP_DISABLE_FUSION": "1"}],
                         ids=["default", "fusion_0", "fusion_disabled"])
def test_default_supports_op_is_mul_mat_only(env_extra):
    """By default (and with the fusion turned off) the device keeps only
    MUL_MAT / MUL_MAT_ID and the no-op views: GLU, ADD and ADD_ID stay on the
    CPU, the strict boundary of the quantized-matmul path.  Runs in a fresh
    process, since the library reads the variables once."""
    import os
    import subprocess
    import sys
    code = r'''
import ctypes as C, sys
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[2])
import ggml_hip.backend as B
from ggml_hip import abi
import test_backend_abi as T
L = B.lib()
ok = lambda t: L.ggml_backend_hip_op_supported(C.pointer(t))
g = abi.make_tensor(abi.GGML_TYPE_F32, [64, 1]); u = abi.make_tensor(abi.GGML_TYPE_F32, [64, 1])
assert not ok(abi.make_glu(abi.GGML_GLU_OP_SWIGLU, g, u, [64, 1]))
assert not ok(abi.make_tensor(abi.GGML_TYPE_F32, [64, 1], op=abi.GGML_OP_ADD, srcs=(g, u)))
mm3 = abi.make_tensor(abi.GGML_TYPE_F32, [64, 2, 3]); b = abi.make_tensor(abi.GGML_TYPE_F32, [64, 4])
ids = abi.make_tensor(abi.GGML_TYPE_I32, [2, 3])
assert not ok(abi.make_tensor(abi.GGML_TYPE_F32, [64, 2, 3], op=abi.GGML_OP_ADD_ID, srcs=(mm3, b, ids)))
assert ok(T.mm(abi.GGML_TYPE_Q4_K, 4096, 4096, 1)[2])
assert ok(T.mmid(abi.GGML_TYPE_Q6_K, 2048, 768, 128, 8, 512)[3])
assert ok(abi.make_tensor(abi.GGML_TYPE_F32, [8, 8], op=abi.GGML_OP_VIEW))
print("strict ok")
'''
    env = {k: v for k, v in os.environ.items() if k not in ("GGML_HIP_FUSION", "GGML_HIP_DISABLE_FUSION")}
    env.update(env_extra)
    r = subprocess.run([sys.executable, "-c", code, str(ROOT / "llama.zig_amd"), str(ROOT / "tests")], env=env,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "strict ok" in r.stdout, r.stderr[-2000:]


def test_mul_mat_rejects_overlapping_columns_before_any_launch(L):
    """hip_qmm_mul_mat refuses column strides below the column length with
    hipErrorInvalidValue before it touches memory (placeholder pointers)."""
    import ctypes as C
    vp, i64 = C.c_void_p, C.c_int64
    L.hip_qmm_mul_mat.restype = C.c_int
    L.hip_qmm_mul_mat.argtypes = [C.c_int, vp, i64, i64, i64, vp, i64, i64, vp, i64, vp, C.c_size_t, vp]
    w, x, d, ws = 0x100000, 0x200000, 0x300000, 0x400000  # aligned placeholders, never dereferenced
    for ncols in (2, 3, 8, 64):
        assert L.hip_qmm_mul_mat(12, w, 4096, 1024, 16 * 144, x, ncols, 4096, d, 1023, ws, 1 << 30, None) == 1
        assert L.hip_qmm_mul_mat(12, w, 4096, 1024, 16 * 144, x, ncols, 4064, d, 1024, ws, 1 << 30, None) == 1


def test_scaled_gate_up_lane_is_not_taken(L):
    """The reference's x_scale / gate_scale lane ({MUL_MAT, MUL(scale), MUL_MAT,
    MUL(scale), GLU}) fuses only for NVFP4 and F8_E4M3 weights
    (getMulMatScale, src/ggml/cuda/mulmat.zig:474-486); for the quantized
    types this backend takes the scale MUL is an ordinary node, which stays
    on the CPU backend, so the MUL_MATs and the GLU run as they do unscaled."""
    from ggml_hip import abi
    ok = lambda t: L.ggml_backend_hip_op_supported(C.pointer(t))  # noqa: E731
    GGML_OP_MUL = 6  # src/ggml/types.zig:24-48
    for t in (abi.GGML_TYPE_Q4_K, abi.GGML_TYPE_Q6_K, abi.GGML_TYPE_Q8_0):
        a, b, d = mm(t, 4096, 4096, 1)
        assert ok(d)
        s = abi.make_tensor(abi.GGML_TYPE_F32, [1], name=b"scale")
        scaled = abi.make_tensor(abi.GGML_TYPE_F32, [4096, 1], op=GGML_OP_MUL, srcs=(d, s))
        assert not ok(scaled)


def test_supports_add_id(L):
    """ADD_ID (ggml_add_id, src/ggml/ops.zig:113-130): f32 rows plus the row
    of b the int32 ids pick, the per-expert bias of an MoE projection."""
    from ggml_hip import abi
    ok = lambda t: L.ggml_backend_hip_op_supported(C.pointer(t))  # noqa: E731
    a = abi.make_tensor(abi.GGML_TYPE_F32, [768, 8, 5], name=b"mm")
    b = abi.make_tensor(abi.GGML_TYPE_F32, [768, 128], name=b"bias")
    ids = abi.make_tensor(abi.GGML_TYPE_I32, [8, 5], name=b"ids")
    add = abi.make_tensor(abi.GGML_TYPE_F32, [768, 8, 5], op=abi.GGML_OP_ADD_ID, srcs=(a, b, ids))
    assert ok(add)
    bad_b = abi.make_tensor(abi.GGML_TYPE_F32, [512, 128], name=b"bias")
    assert not ok(abi.make_tensor(abi.GGML_TYPE_F32, [768, 8, 5], op=abi.GGML_OP_ADD_ID, srcs=(a, bad_b, ids)))
    bad_ids = abi.make_tensor(abi.GGML_TYPE_I32, [4, 5], name=b"ids")
    assert not ok(abi.make_tensor(abi.GGML_TYPE_F32, [768, 8, 5], op=abi.GGML_OP_ADD_ID, srcs=(a, b, bad_ids)))
    f16_ids = abi.make_tensor(abi.GGML_TYPE_F16, [8, 5], name=b"ids")
    assert not ok(abi.make_tensor(abi.GGML_TYPE_F32, [768, 8, 5], op=abi.GGML_OP_ADD_ID, srcs=(a, b, f16_ids)))


def test_mul_mat_route_query(L):
    """hip_qmm_mul_mat_uses_mmq answers the op's shape rules without a device:
    the GEMV for one column and for small matrices, the few-column GEMM for
    4-8 columns of large ones (per type), the MMQ from 9 columns on."""
    L.hip_qmm_mul_mat_uses_mmq.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int64]
    q4k, q6k, q8_0 = 12, 14, 8
    q = lambda t, K, rows, cols: L.hip_qmm_mul_mat_uses_mmq(t, K, rows, cols)  # noqa: E731
    assert q(q4k, 4096, 14336, 1) == 0 and q(q4k, 4096, 14336, 4) == 0
    assert q(q4k, 4096, 14336, 5) == 1 and q(q4k, 4096, 14336, 8) == 1
    assert q(q4k, 4096, 4096, 8) == 0 and q(q4k, 4096, 1024, 8) == 0
    assert q(q4k, 14336, 4096, 4) == 0 and q(q4k, 14336, 4096, 5) == 1
    assert q(q6k, 14336, 4096, 3) == 0 and q(q6k, 14336, 4096, 4) == 1 and q(q6k, 14336, 4096, 8) == 1
    assert q(q6k, 4096, 1024, 8) == 0
    assert q(q8_0, 4096, 14336, 3) == 0 and q(q8_0, 4096, 14336, 4) == 1
    assert all(q(t, 4096, 4096, 9) == 1 for t in (q4k, q6k, q8_0))
    assert q(q4k, 4000, 4096, 16) == 0  # K % 256 != 0: no MMQ
    assert q(q4k, 4096, 0, 8) == 0 and q(q4k, 0, 4096, 8) == 0
    # 2-8 columns of small matrices: the one-column kernel per column
    L.hip_qmm_mul_mat_per_column.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int64]
    pc = lambda t, K, rows, cols: L.hip_qmm_mul_mat_per_column(t, K, rows, cols)  # noqa: E731
    q5k, q4_0, iq4xs = 13, 2, 23
    assert all(pc(t, 4096, 1024, c) == 1 for t in (q4k, q5k, q6k, iq4xs) for c in range(2, 9))
    assert pc(q4k, 4096, 2048, 8) == 1 and pc(q4k, 4096, 2049, 2) == 0 and pc(q4k, 4352, 1024, 2) == 0
    assert pc(q4k, 4096, 1024, 1) == 0 and pc(q4k, 4096, 1024, 9) == 0
    assert pc(q8_0, 4096, 1024, 4) == 1 and pc(q8_0, 4096, 1024, 5) == 0 and pc(q8_0, 4096, 2048, 2) == 0
    assert pc(q4_0, 4096, 1024, 4) == 1 and pc(q4_0, 4096, 1024, 6) == 0 and pc(q4_0, 2048, 1024, 8) == 1
    assert pc(q8_0, 2048, 1024, 8) == 1 and pc(q4_0, 2048, 1025, 2) == 0
    assert pc(q4k, 4096, 0, 2) == 0 and pc(q4k, 0, 1024, 2) == 0
