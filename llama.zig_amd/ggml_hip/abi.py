"""ctypes restatement of include/ggml_hip_ggml_abi.h: the ggml tensor, graph
and backend vtable layouts the HIP backend layer fills, for Python hosts and
tests that drive the backend through the plugin interface.

Layout sources (reference paths): ggml_tensor as read throughout src/ggml and
checked at src/ggml/backend_meta.zig:3221-3222; ggml_cgraph and
ggml_hash_set at src/ggml/impl.zig:422-435, 469-485; vtable member order as
the CUDA backend fills them (src/ggml/cuda/backend.zig:250-265, 343-352,
714-731, 1032-1048, 1141-1146); op ids from op_name
(src/ggml/types.zig:25-51), GLU op ids from glu_op_name (types.zig:103-106).
"""
import ctypes as C
import struct

GGML_MAX_DIMS = 4
GGML_MAX_SRC = 10
GGML_MAX_OP_PARAMS = 64
GGML_MAX_NAME = 64

# ggml_type ids
GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q4_0, GGML_TYPE_Q8_0, GGML_TYPE_Q8_1 = 0, 1, 2, 8, 9
GGML_TYPE_Q4_K, GGML_TYPE_Q5_K, GGML_TYPE_Q6_K, GGML_TYPE_Q8_K, GGML_TYPE_I32 = 12, 13, 14, 15, 26
GGML_TYPE_IQ4_XS = 23
# ggml_op ids (position in op_name)
GGML_OP_NONE, GGML_OP_ADD, GGML_OP_ADD_ID, GGML_OP_MUL_MAT, GGML_OP_MUL_MAT_ID = 0, 2, 3, 28, 29
GGML_OP_RESHAPE, GGML_OP_VIEW, GGML_OP_PERMUTE, GGML_OP_TRANSPOSE = 35, 36, 37, 38
GGML_OP_GLU = 98
# ggml_glu_op ids
GGML_GLU_OP_REGLU, GGML_GLU_OP_GEGLU, GGML_GLU_OP_SWIGLU, GGML_GLU_OP_SWIGLU_OAI = 0, 1, 2, 3
GGML_GLU_OP_GEGLU_ERF, GGML_GLU_OP_GEGLU_QUICK, GGML_GLU_OP_SWIGLU_CLAMP = 4, 5, 6
GGML_TENSOR_FLAG_OUTPUT = 2
GGML_STATUS_SUCCESS, GGML_STATUS_FAILED = 0, -1
GGML_BACKEND_BUFFER_USAGE_ANY, GGML_BACKEND_BUFFER_USAGE_WEIGHTS, GGML_BACKEND_BUFFER_USAGE_COMPUTE = 0, 1, 2
GGML_BACKEND_DEVICE_TYPE_GPU = 1

# (block elements, block bytes) per type
TYPE_BLOCK = {GGML_TYPE_F32: (1, 4), GGML_TYPE_F16: (1, 2), GGML_TYPE_I32: (1, 4), GGML_TYPE_Q4_0: (32, 18),
              GGML_TYPE_Q8_0: (32, 34), GGML_TYPE_IQ4_XS: (256, 136),
              GGML_TYPE_Q8_1: (32, 36), GGML_TYPE_Q4_K: (256, 144), GGML_TYPE_Q5_K: (256, 176), GGML_TYPE_Q6_K: (256, 210),
              GGML_TYPE_Q8_K: (256, 292)}


class ggml_tensor(C.Structure):
    pass


ggml_tensor._fields_ = [
    ("type", C.c_int),
    ("buffer", C.c_void_p),
    ("ne", C.c_int64 * GGML_MAX_DIMS),
    ("nb", C.c_size_t * GGML_MAX_DIMS),
    ("op", C.c_int),
    ("op_params", C.c_int32 * (GGML_MAX_OP_PARAMS // 4)),
    ("flags", C.c_int32),
    ("src", C.POINTER(ggml_tensor) * GGML_MAX_SRC),
    ("view_src", C.POINTER(ggml_tensor)),
    ("view_offs", C.c_size_t),
    ("data", C.c_void_p),
    ("name", C.c_char * GGML_MAX_NAME),
    ("extra", C.c_void_p),
    ("padding", C.c_char * 8),
]


class ggml_cgraph(C.Structure):
    _fields_ = [
        ("size", C.c_int),
        ("n_nodes", C.c_int),
        ("n_leafs", C.c_int),
        ("nodes", C.POINTER(C.POINTER(ggml_tensor))),
        ("grads", C.c_void_p),
        ("grad_accs", C.c_void_p),
        ("leafs", C.POINTER(C.POINTER(ggml_tensor))),
        ("use_counts", C.c_void_p),
        ("hash_size", C.c_size_t),  # visited_hash_set
        ("hash_used", C.c_void_p),
        ("hash_keys", C.c_void_p),
        ("order", C.c_int),
    ]


PT = C.POINTER(ggml_tensor)
VP = C.c_void_p
SZ = C.c_size_t
FN = C.CFUNCTYPE


class buffer_type_i(C.Structure):
    _fields_ = [
        ("get_name", FN(C.c_char_p, VP)),
        ("alloc_buffer", FN(VP, VP, SZ)),
        ("alloc_buffer_n", VP),
        ("get_alignment", FN(SZ, VP)),
        ("get_max_size", VP),
        ("get_alloc_size", FN(SZ, VP, PT)),
        ("get_alloc_size_n", VP),
        ("is_host", VP),
    ]


class buffer_type(C.Structure):
    _fields_ = [("iface", buffer_type_i), ("device", VP), ("context", VP)]


class buffer_i(C.Structure):
    _fields_ = [
        ("free_buffer", FN(None, VP)),
        ("get_base", FN(VP, VP)),
        ("init_tensor", FN(C.c_int, VP, PT)),
        ("memset_tensor", FN(None, VP, PT, C.c_uint8, SZ, SZ)),
        ("set_tensor", FN(None, VP, PT, VP, SZ, SZ)),
        ("get_tensor", FN(None, VP, PT, VP, SZ, SZ)),
        ("set_tensor_2d", VP),
        ("get_tensor_2d", VP),
        ("cpy_tensor", FN(C.c_bool, VP, PT, PT)),
        ("clear", FN(None, VP, C.c_uint8)),
        ("reset", VP),
        ("set_tensor_n", VP),
        ("get_tensor_n", VP),
        ("cpy_tensor_n", VP),
    ]


class buffer(C.Structure):
    _fields_ = [("iface", buffer_i), ("buft", VP), ("context", VP), ("size", SZ), ("usage", C.c_int)]


ADD_ALLOC_DEP = FN(None, VP, VP, VP)


class graph_optimize_params(C.Structure):
    """struct ggml_backend_graph_optimize_params (src/ggml/backend_sched.zig:997-1000)."""
    _fields_ = [("add_alloc_dep", ADD_ALLOC_DEP), ("user_data", VP)]


class backend_i(C.Structure):
    _fields_ = [
        ("get_name", FN(C.c_char_p, VP)),
        ("free", FN(None, VP)),
        ("set_tensor_async", FN(None, VP, PT, VP, SZ, SZ)),
        ("get_tensor_async", FN(None, VP, PT, VP, SZ, SZ)),
        ("set_tensor_2d_async", VP),
        ("get_tensor_2d_async", VP),
        ("cpy_tensor_async", VP),
        ("synchronize", FN(None, VP)),
        ("graph_plan_create", VP),
        ("graph_plan_free", VP),
        ("graph_plan_update", VP),
        ("graph_plan_compute", VP),
        ("graph_compute", FN(C.c_int, VP, C.POINTER(ggml_cgraph))),
        ("event_record", FN(None, VP, VP)),
        ("event_wait", FN(None, VP, VP)),
        ("graph_optimize", FN(None, VP, C.POINTER(ggml_cgraph), VP)),
    ]


class backend(C.Structure):
    _fields_ = [("guid", VP), ("iface", backend_i), ("device", VP), ("context", VP)]


class dev_caps(C.Structure):
    _fields_ = [("async_", C.c_bool), ("host_buffer", C.c_bool), ("buffer_from_host_ptr", C.c_bool),
                ("events", C.c_bool), ("mmap_support", C.c_bool)]


class dev_props(C.Structure):
    _fields_ = [("name", C.c_char_p), ("description", C.c_char_p), ("memory_free", SZ), ("memory_total", SZ),
                ("type", C.c_int), ("device_id", C.c_char_p), ("caps", dev_caps)]


class device_i(C.Structure):
    _fields_ = [
        ("get_name", FN(C.c_char_p, VP)),
        ("get_description", FN(C.c_char_p, VP)),
        ("get_memory", FN(None, VP, C.POINTER(SZ), C.POINTER(SZ))),
        ("get_type", FN(C.c_int, VP)),
        ("get_props", FN(None, VP, C.POINTER(dev_props))),
        ("init_backend", FN(VP, VP, C.c_char_p)),
        ("get_buffer_type", FN(VP, VP)),
        ("get_host_buffer_type", FN(VP, VP)),
        ("buffer_from_host_ptr", VP),
        ("supports_op", FN(C.c_bool, VP, PT)),
        ("supports_buft", FN(C.c_bool, VP, VP)),
        ("offload_op", FN(C.c_bool, VP, PT)),
        ("event_new", FN(VP, VP)),
        ("event_free", FN(None, VP, VP)),
        ("event_synchronize", FN(None, VP, VP)),
    ]


class device(C.Structure):
    _fields_ = [("iface", device_i), ("reg", VP), ("context", VP)]


class reg_i(C.Structure):
    _fields_ = [
        ("get_name", FN(C.c_char_p, VP)),
        ("get_device_count", FN(SZ, VP)),
        ("get_device", FN(VP, VP, SZ)),
        ("get_proc_address", FN(VP, VP, C.c_char_p)),
    ]


class reg(C.Structure):
    _fields_ = [("api_version", C.c_int), ("iface", reg_i), ("context", VP)]


def deref(ptr, cls):
    """The struct a void pointer returned by the library points at."""
    return C.cast(ptr, C.POINTER(cls)).contents


def make_tensor(gtype, ne, name=b"", op=GGML_OP_NONE, srcs=(), data=None, nb=None):
    """A ggml_tensor with dense strides for `ne` (padded to 4 dims)."""
    t = ggml_tensor()
    ne = list(ne) + [1] * (GGML_MAX_DIMS - len(ne))
    blck, size = TYPE_BLOCK[gtype]
    t.type = gtype
    t.op = op
    for i, v in enumerate(ne):
        t.ne[i] = v
    if nb is None:
        nb = [size, size * (ne[0] // blck)]
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    for i, v in enumerate(nb):
        t.nb[i] = v
    for i, s in enumerate(srcs):
        t.src[i] = C.pointer(s)
    t.data = data
    t.name = name
    return t


def set_op_param_f32(t, i, v):
    t.op_params[i] = struct.unpack("<i", struct.pack("<f", v))[0]


def make_glu(op, gate, up, ne, alpha=0.0, limit=0.0, name=b"glu"):
    """ggml_glu_split(gate, up) with op params as ggml_swiglu_oai /
    ggml_swiglu_clamp write them (src/ggml/ops.zig:727-751, 3779-3798)."""
    t = make_tensor(GGML_TYPE_F32, ne, name=name, op=GGML_OP_GLU, srcs=(gate, up))
    t.op_params[0] = op
    t.op_params[1] = 0
    set_op_param_f32(t, 2, alpha)
    set_op_param_f32(t, 3, limit)
    return t


def nbytes(t):
    blck, size = TYPE_BLOCK[t.type]
    if any(t.ne[i] <= 0 for i in range(4)):
        return 0
    if blck == 1:
        return size + sum((t.ne[i] - 1) * t.nb[i] for i in range(4))
    return t.ne[0] * t.nb[0] // blck + sum((t.ne[i] - 1) * t.nb[i] for i in range(1, 4))
