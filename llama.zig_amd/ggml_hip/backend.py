"""Python host over the ggml backend plugin interface of libggml_hip_qmm.so.

It plays the part ggml's allocator and scheduler play for a HIP backend
(src/ggml/alloc.zig, src/ggml/backend_sched.zig:1405-1500): tensors are
placed in a buffer from the device's buffer type (alignment and
get_alloc_size honoured), filled with set_tensor, computed with the backend's
graph_compute and read back with get_tensor, all through the vtables of
ggml_hip_ggml_abi.h.  No torch here: device memory comes from the buffer type.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import abi
from . import lib as _lib

_configured = False


def lib():
    """The library with the backend-layer prototypes set."""
    global _configured
    L = _lib()
    if not _configured:
        vp = C.c_void_p
        for name in ("ggml_backend_hip_reg", "ggml_backend_init", "ggml_backend_hip_host_buffer_type"):
            getattr(L, name).restype = vp
            getattr(L, name).argtypes = []
        L.ggml_backend_hip_init.restype = vp
        L.ggml_backend_hip_init.argtypes = [C.c_int]
        L.ggml_backend_hip_buffer_type.restype = vp
        L.ggml_backend_hip_buffer_type.argtypes = [C.c_int]
        L.ggml_backend_is_hip.restype = C.c_bool
        L.ggml_backend_is_hip.argtypes = [vp]
        L.ggml_backend_hip_get_device_count.restype = C.c_int
        L.ggml_backend_hip_get_device_count.argtypes = []
        L.ggml_backend_hip_get_device_description.restype = None
        L.ggml_backend_hip_get_device_description.argtypes = [C.c_int, C.c_char_p, C.c_size_t]
        L.ggml_backend_hip_get_device_memory.restype = None
        L.ggml_backend_hip_get_device_memory.argtypes = [C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        L.ggml_backend_hip_register_host_buffer.restype = C.c_bool
        L.ggml_backend_hip_register_host_buffer.argtypes = [vp, C.c_size_t]
        L.ggml_backend_hip_unregister_host_buffer.restype = None
        L.ggml_backend_hip_unregister_host_buffer.argtypes = [vp]
        L.ggml_backend_score.restype = C.c_int
        L.ggml_backend_score.argtypes = []
        L.ggml_backend_hip_op_supported.restype = C.c_bool
        L.ggml_backend_hip_op_supported.argtypes = [abi.PT]
        L.ggml_backend_hip_tensor_alloc_size.restype = C.c_size_t
        L.ggml_backend_hip_tensor_alloc_size.argtypes = [abi.PT]
        _configured = True
    return L


def registry():
    return abi.deref(lib().ggml_backend_hip_reg(), abi.reg)


class HipBackend:
    """One backend (stream + workspace) on `device` and a bump allocator over
    buffers of the device's buffer type."""

    def __init__(self, device: int = 0):
        L = lib()
        r = registry()
        if device >= r.iface.get_device_count(L.ggml_backend_hip_reg()):
            raise RuntimeError(f"HIP device {device} not present")
        self.device = device
        self.be_ptr = L.ggml_backend_hip_init(device)
        if not self.be_ptr:
            raise RuntimeError("ggml_backend_hip_init failed")
        self.be = abi.deref(self.be_ptr, abi.backend)
        self.buft_ptr = L.ggml_backend_hip_buffer_type(device)
        self.buft = abi.deref(self.buft_ptr, abi.buffer_type)
        self.buffers = []
        self.keep = []  # tensors and host arrays the C side points at

    # -- allocation: one buffer per call, tensors placed at aligned offsets
    def alloc(self, tensors, usage=abi.GGML_BACKEND_BUFFER_USAGE_ANY):
        align = self.buft.iface.get_alignment(self.buft_ptr)
        sizes = [self.buft.iface.get_alloc_size(self.buft_ptr, C.pointer(t)) for t in tensors]
        offs, total = [], 0
        for s in sizes:
            total = (total + align - 1) // align * align
            offs.append(total)
            total += s
        bptr = self.buft.iface.alloc_buffer(self.buft_ptr, max(total, 1))
        if not bptr:
            raise MemoryError("HIP buffer allocation failed")
        buf = abi.deref(bptr, abi.buffer)
        buf.usage = usage
        base = buf.iface.get_base(bptr)
        for t, o in zip(tensors, offs):
            t.buffer = bptr
            t.data = base + o
            st = buf.iface.init_tensor(bptr, C.pointer(t))
            if st != abi.GGML_STATUS_SUCCESS:
                raise RuntimeError("init_tensor failed")
        self.buffers.append(bptr)
        self.keep.extend(tensors)
        return bptr

    def set(self, t, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        n = min(arr.nbytes, abi.nbytes(t))
        buf = abi.deref(t.buffer, abi.buffer)
        buf.iface.set_tensor(t.buffer, C.pointer(t), arr.ctypes.data, 0, n)

    def get(self, t, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        buf = abi.deref(t.buffer, abi.buffer)
        buf.iface.get_tensor(t.buffer, C.pointer(t), out.ctypes.data, 0, out.nbytes)
        return out

    @staticmethod
    def _graph(nodes, use_counts=True):
        """A ggml_cgraph over `nodes`, and the arrays it points at.  With
        use_counts, the graph carries the visited hash set and per-tensor use
        counts ggml_build_forward fills (every node and source keyed at
        (addr >> 4) % size with linear probing, src/ggml/impl.zig:509-557; the
        count of a tensor is the number of node source slots naming it,
        src/ggml/graph.zig:472-520), which the backend's fusion reads."""
        arr = (abi.PT * len(nodes))(*[C.pointer(n) for n in nodes])
        g = abi.ggml_cgraph()
        g.size = len(nodes)
        g.n_nodes = len(nodes)
        g.n_leafs = 0
        g.nodes = arr
        keep = [arr]
        if use_counts:
            tensors = []
            for n in nodes:
                tensors.append(C.addressof(n))
                for s in n.src:
                    if s:
                        tensors.append(C.addressof(s.contents))
            size = 2 * len(tensors) + 1
            used = (C.c_uint32 * ((size + 31) // 32))()
            keys = (C.c_void_p * size)()
            counts = (C.c_int32 * size)()

            def slot(a):
                i = (a >> 4) % size
                while used[i >> 5] >> (i & 31) & 1 and keys[i] != a:
                    i = (i + 1) % size
                return i

            for a in tensors:
                i = slot(a)
                used[i >> 5] |= 1 << (i & 31)
                keys[i] = a
            for n in nodes:
                for s in n.src:
                    if s:
                        counts[slot(C.addressof(s.contents))] += 1
            g.use_counts = C.cast(counts, C.c_void_p)
            g.hash_size = size
            g.hash_used = C.cast(used, C.c_void_p)
            g.hash_keys = C.cast(keys, C.c_void_p)
            keep += [used, keys, counts]
        return g, keep

    def compute(self, nodes, use_counts=True):
        """Run `nodes` as one graph (see _graph for the use counts)."""
        g, keep = self._graph(nodes, use_counts)
        st = self.be.iface.graph_compute(self.be_ptr, C.pointer(g))
        self.be.iface.synchronize(self.be_ptr)
        del keep
        return st

    def compute_view(self, nodes, i0, i1):
        """Run nodes[i0:i1] as the scheduler runs a split: a view of the whole
        graph's node array (ggml_graph_view, src/ggml/graph.zig) that shares
        its hash set and use counts, so uses by nodes outside the split count."""
        g, keep = self._graph(nodes, True)
        view = abi.ggml_cgraph()
        C.memmove(C.addressof(view), C.addressof(g), C.sizeof(g))
        view.size = view.n_nodes = i1 - i0
        view.nodes = C.cast(C.addressof(keep[0]) + i0 * C.sizeof(abi.PT), C.POINTER(abi.PT))
        st = self.be.iface.graph_compute(self.be_ptr, C.pointer(view))
        self.be.iface.synchronize(self.be_ptr)
        del keep
        return st

    def optimized(self, nodes, use_counts=True):
        """The backend's graph_optimize on a graph of `nodes`: the node order
        it leaves and the (tensor, until) allocation dependencies it adds,
        as addresses."""
        g, keep = self._graph(nodes, use_counts)
        deps = []
        cb = abi.ADD_ALLOC_DEP(lambda ud, tensor, until: deps.append((tensor, until)))
        params = abi.graph_optimize_params(cb, None)
        self.be.iface.graph_optimize(self.be_ptr, C.pointer(g), C.cast(C.pointer(params), C.c_void_p))
        by_addr = {C.addressof(n): n for n in nodes}
        order = [by_addr[C.addressof(keep[0][k].contents)] for k in range(len(nodes))]
        del keep
        return order, deps

    def close(self):
        for b in self.buffers:
            abi.deref(b, abi.buffer).iface.free_buffer(b)
        self.buffers = []
        if self.be_ptr:
            self.be.iface.free(self.be_ptr)
            self.be_ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
