"""The backend plugin path end to end on the GPU: tensors placed in a HIP
buffer through the buffer-type vtable, a graph of MUL_MAT / MUL_MAT_ID nodes
run by the backend's graph_compute, results read back with get_tensor and
checked against the CPU ggml path (NMSE gate) and against the kernel-level
entry points (same kernels, so the bytes must agree)."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from cases import acts, max_err_scaled, mul_mat_id_f64, nmse, weights_f32, weights_q

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NMSE_GATE = 5e-4
TYPES = {"Q4_K": O.TYPE_Q4_K, "Q5_K": O.TYPE_Q5_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0,
         "Q4_0": O.TYPE_Q4_0, "IQ4_XS": O.TYPE_IQ4_XS}


@pytest.fixture(scope="module")
def hb():
    from ggml_hip.backend import HipBackend
    with HipBackend(0) as b:
        yield b


def test_registry_and_device(hb):
    import ggml_hip.backend as B
    from ggml_hip import abi
    L = B.lib()
    rp = L.ggml_backend_hip_reg()
    r = B.registry()
    n = r.iface.get_device_count(rp)
    assert n >= 1 and n == L.ggml_backend_hip_get_device_count()
    assert L.ggml_backend_score() > 0
    dp = r.iface.get_device(rp, 0)
    dev = abi.deref(dp, abi.device)
    assert dev.iface.get_name(dp) == b"HIP0"
    props = abi.dev_props()
    dev.iface.get_props(dp, C.pointer(props))
    assert props.type == abi.GGML_BACKEND_DEVICE_TYPE_GPU and props.memory_total > props.memory_free > 0
    assert props.caps.async_ and props.caps.events
    desc = C.create_string_buffer(256)
    L.ggml_backend_hip_get_device_description(0, desc, 256)
    assert desc.value and desc.value == props.description
    assert L.ggml_backend_is_hip(hb.be_ptr)
    assert dev.iface.supports_buft(dp, hb.buft_ptr)
    assert not dev.iface.supports_buft(dp, L.ggml_backend_hip_host_buffer_type())
    # events: record on the backend stream, wait, synchronize
    ev = dev.iface.event_new(dp)
    hb.be.iface.event_record(hb.be_ptr, ev)
    hb.be.iface.event_wait(hb.be_ptr, ev)
    dev.iface.event_synchronize(dp, ev)
    dev.iface.event_free(dp, ev)


def _mul_mat_graph(hb, t, wq, K, M, x, batch_w=1, batch_x=1):
    from ggml_hip import abi
    N = x.shape[-2]
    a = abi.make_tensor(t, [K, M, batch_w], name=b"w")
    b = abi.make_tensor(abi.GGML_TYPE_F32, [K, N, batch_x], name=b"x")
    d = abi.make_tensor(abi.GGML_TYPE_F32, [M, N, batch_x], op=abi.GGML_OP_MUL_MAT, srcs=(a, b), name=b"out")
    hb.alloc([a], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([b, d], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(a, wq)
    hb.set(b, x.astype(np.float32))
    hb.set(d, np.full((batch_x, N, M), np.nan, dtype=np.float32))
    view = abi.make_tensor(abi.GGML_TYPE_F32, [M, N, batch_x], op=abi.GGML_OP_VIEW, srcs=(d,))
    assert hb.compute([d, view]) == abi.GGML_STATUS_SUCCESS
    return hb.get(d, np.float32, (batch_x, N, M))


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_XS"])
@pytest.mark.parametrize("N", [1, 5, 40])
def test_graph_mul_mat(hb, tname, N):
    import ggml_hip as G
    t = TYPES[tname]
    M, K = 256, 1024
    wq, x = weights_q(t, M, K), np.array(acts(N, K))
    got = _mul_mat_graph(hb, t, wq, K, M, x)[0]
    cpu = O.mul_mat(t, wq, M, K, x, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    direct = G.mul_mat(tname, torch.from_numpy(np.array(wq)).cuda(), torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(got, direct)


def test_graph_mul_mat_broadcast_and_padding(hb):
    """src0 broadcast over dim 2 (2 weight slices for 4 activation slices) with
    a Q8_0 row length that is not a multiple of 512 (init_tensor zero-fills
    the padding get_alloc_size adds)."""
    t, M, K, N = O.TYPE_Q8_0, 96, 544, 3
    w = np.stack([O.quantize_rows(t, weights_f32(M, K, idx=i)) for i in range(2)])
    x = np.stack([np.array(acts(N, K, idx=i)) for i in range(4)])
    got = _mul_mat_graph(hb, t, w, K, M, x, batch_w=2, batch_x=4)
    for i in range(4):
        cpu = O.mul_mat(t, w[i // 2], M, K, x[i], nth=8)
        assert nmse(got[i], cpu) < NMSE_GATE, i


@pytest.mark.parametrize("tname", ["Q4_K", "Q5_K", "Q6_K", "Q4_0", "IQ4_XS"])
def test_graph_mul_mat_id(hb, tname):
    import ggml_hip as G
    from ggml_hip import abi
    t = TYPES[tname]
    n_as, M, K, n_tokens, n_ids = 8, 128, 512, 21, 3
    wq = O.quantize_rows(t, weights_f32(n_as * M, K)).reshape(n_as, M, -1)
    rng = np.random.default_rng(11)
    ids = rng.integers(-1, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    x = np.array(acts(n_tokens * n_ids, K)).reshape(n_tokens, n_ids, K)
    a = abi.make_tensor(t, [K, M, n_as], name=b"experts")
    b = abi.make_tensor(abi.GGML_TYPE_F32, [K, n_ids, n_tokens], name=b"x")
    it = abi.make_tensor(abi.GGML_TYPE_I32, [n_ids, n_tokens], name=b"ids")
    d = abi.make_tensor(abi.GGML_TYPE_F32, [M, n_ids, n_tokens], op=abi.GGML_OP_MUL_MAT_ID, srcs=(a, b, it))
    hb.alloc([a], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([b, it, d], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(a, wq)
    hb.set(b, x.astype(np.float32))
    hb.set(it, ids)
    assert hb.compute([d]) == abi.GGML_STATUS_SUCCESS
    got = hb.get(d, np.float32, (n_tokens, n_ids, M))
    assert np.all(got[ids < 0] == 0.0)
    cpu = O.mul_mat_id(t, wq, n_as, M, K, x, ids, nth=8)
    assert nmse(got, cpu) < NMSE_GATE
    y = G.quantize_q8_1(torch.from_numpy(x.reshape(-1, K)).cuda(), K).cpu().numpy()
    assert max_err_scaled(got, mul_mat_id_f64(t, wq, M, K, y, n_ids, ids)) < 2e-6


def test_graph_rejects_unsupported_node(hb):
    from ggml_hip import abi
    a = abi.make_tensor(abi.GGML_TYPE_F32, [64, 4], name=b"a")
    hb.alloc([a])
    # a broadcasting ADD (a row added to every row) stays on the CPU
    row = abi.make_tensor(abi.GGML_TYPE_F32, [64, 1], name=b"row")
    hb.alloc([row])
    add = abi.make_tensor(abi.GGML_TYPE_F32, [64, 4], op=abi.GGML_OP_ADD, srcs=(a, row), name=b"add")
    hb.alloc([add])
    assert hb.compute([add]) == abi.GGML_STATUS_FAILED
    # so does a GLU the device has no kernel for (GEGLU_ERF)
    glu = abi.make_glu(abi.GGML_GLU_OP_GEGLU_ERF, a, a, [64, 4])
    hb.alloc([glu])
    assert hb.compute([glu]) == abi.GGML_STATUS_FAILED


def test_alloc_buffer_out_of_memory_returns_null(hb):
    """alloc_buffer answers NULL when hipMalloc fails (cuda/backend.zig:294-303),
    forced from the host with a size no device holds, and clears the error:
    the next allocation and a MUL_MAT on it succeed."""
    from ggml_hip import abi
    assert not hb.buft.iface.alloc_buffer(hb.buft_ptr, 1 << 52)  # 4 PiB
    K, M = 1024, 256
    wq = weights_q(O.TYPE_Q4_K, M, K)
    x = np.array(acts(2, K))
    got = _mul_mat_graph(hb, abi.GGML_TYPE_Q4_K, wq, K, M, x)
    assert nmse(got[0], O.mul_mat(O.TYPE_Q4_K, wq, M, K, x, nth=8)) < NMSE_GATE


@pytest.mark.parametrize("tname,N,bw,bx", [("Q4_K", 8, (2, 1), (4, 3)), ("Q6_K", 2, (1, 2), (2, 4)),
                                           ("IQ4_XS", 1, (3, 1), (3, 2)), ("Q8_0", 12, (2, 1), (4, 1))])
def test_graph_mul_mat_batched_dims_2_and_3(hb, tname, N, bw, bx):
    """A MUL_MAT batched over dims 2 and 3 with src0 broadcast over both: up to
    8 columns run as one AoS quantize + one hip_qmm_mul_mat_vec_q launch over
    channels and samples (the reference's mulMatVecQ); more columns run the op
    per slice.  Every slice against the CPU path on its weight matrix."""
    from ggml_hip import abi
    t = TYPES[tname]
    M, K = 320, 1024
    nw, nx = bw[0] * bw[1], bx[0] * bx[1]
    w = np.stack([O.quantize_rows(t, weights_f32(M, K, idx=i)) for i in range(nw)])
    x = np.array(acts(nx * N, K)).reshape(nx, N, K)
    a = abi.make_tensor(t, [K, M, bw[0], bw[1]], name=b"w")
    b = abi.make_tensor(abi.GGML_TYPE_F32, [K, N, bx[0], bx[1]], name=b"x")
    d = abi.make_tensor(abi.GGML_TYPE_F32, [M, N, bx[0], bx[1]], op=abi.GGML_OP_MUL_MAT, srcs=(a, b), name=b"out")
    hb.alloc([a], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.alloc([b, d], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(a, w)
    hb.set(b, x)
    hb.set(d, np.full((nx, N, M), np.nan, dtype=np.float32))
    assert hb.compute([d]) == abi.GGML_STATUS_SUCCESS
    got = hb.get(d, np.float32, (nx, N, M))
    r2, r3 = bx[0] // bw[0], bx[1] // bw[1]
    for i3 in range(bx[1]):
        for i2 in range(bx[0]):
            wi = (i3 // r3) * bw[0] + i2 // r2
            xi = i3 * bx[0] + i2
            cpu = O.mul_mat(t, w[wi], M, K, x[xi], nth=8)
            assert nmse(got[xi], cpu) < NMSE_GATE, (i2, i3)


def test_chunked_async_upload_as_the_loader_does(hb):
    """The loader's upload of a tensor from a GGUF file (src/llama/loader.zig:
    1601-1640): the file read at an aligned offset into a ring of pinned host
    buffers from the host buffer type, each chunk sent with the backend's
    set_tensor_async at its running offset, an event recorded per buffer and
    synchronized before the buffer is reused.  The uploaded weight equals a
    one-call set_tensor byte for byte, and a MUL_MAT on it equals the same
    MUL_MAT on the one-call copy."""
    import ggml_hip.backend as B
    from ggml_hip import abi
    L = B.lib()
    K, M = 4096, 2048
    wq = np.array(weights_q(O.TYPE_Q4_K, M, K, 3))
    rng = np.random.default_rng(8)
    head = 123_457  # the tensor's offset in the file: not a multiple of the read alignment
    blob = np.concatenate([rng.integers(0, 256, head, dtype=np.uint8), wq.reshape(-1),
                           rng.integers(0, 256, 999, dtype=np.uint8)])
    n_size = wq.nbytes
    a = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M], name=b"chunked")
    ref = abi.make_tensor(abi.GGML_TYPE_Q4_K, [K, M], name=b"one_call")
    hb.alloc([a, ref], usage=abi.GGML_BACKEND_BUFFER_USAGE_WEIGHTS)
    hb.set(ref, wq)
    # the ring: n_buffers pinned host buffers of buffer_size (+ alignment slack) and an event each
    hbt_ptr = L.ggml_backend_hip_host_buffer_type()
    hbt = abi.deref(hbt_ptr, abi.buffer_type)
    rp = L.ggml_backend_hip_reg()
    dp = B.registry().iface.get_device(rp, 0)
    dev = abi.deref(dp, abi.device)
    n_buffers, buffer_size, alignment = 4, 1 << 20, 4096
    bufs = [hbt.iface.alloc_buffer(hbt_ptr, buffer_size + alignment) for _ in range(n_buffers)]
    assert all(bufs)
    host = [abi.deref(b, abi.buffer).iface.get_base(b) for b in bufs]
    events = [dev.iface.event_new(dp) for _ in range(n_buffers)]
    try:
        aligned_offset = head & ~(alignment - 1)
        offset_from_alignment = head - aligned_offset
        read_end = (head + n_size + alignment - 1) & ~(alignment - 1)
        bytes_read = data_read = 0
        idx = 0
        while bytes_read < read_end - aligned_offset:
            read_size = min(buffer_size, read_end - aligned_offset - bytes_read)
            dst = (host[idx] + alignment - 1) & ~(alignment - 1)
            dev.iface.event_synchronize(dp, events[idx])
            src = blob[aligned_offset + bytes_read:aligned_offset + bytes_read + read_size]
            C.memmove(dst, src.ctypes.data, src.nbytes)  # the file read (short at the file's end)
            ptr, to_copy = dst, read_size
            if bytes_read == 0:
                ptr += offset_from_alignment
                to_copy -= offset_from_alignment
            if aligned_offset + bytes_read + read_size > head + n_size:
                to_copy -= read_end - (head + n_size)
            hb.be.iface.set_tensor_async(hb.be_ptr, C.pointer(a), ptr, data_read, to_copy)
            hb.be.iface.event_record(hb.be_ptr, events[idx])
            data_read += to_copy
            bytes_read += read_size
            idx = (idx + 1) % n_buffers
        assert data_read == n_size
        hb.be.iface.synchronize(hb.be_ptr)
    finally:
        for e in events:
            dev.iface.event_free(dp, e)
        for b in bufs:
            abi.deref(b, abi.buffer).iface.free_buffer(b)
    got = hb.get(a, np.uint8, (n_size,))
    np.testing.assert_array_equal(got, wq.reshape(-1))
    x = abi.make_tensor(abi.GGML_TYPE_F32, [K, 3], name=b"x")
    d1 = abi.make_tensor(abi.GGML_TYPE_F32, [M, 3], op=abi.GGML_OP_MUL_MAT, srcs=(a, x), name=b"d1")
    d2 = abi.make_tensor(abi.GGML_TYPE_F32, [M, 3], op=abi.GGML_OP_MUL_MAT, srcs=(ref, x), name=b"d2")
    hb.alloc([x, d1, d2], usage=abi.GGML_BACKEND_BUFFER_USAGE_COMPUTE)
    hb.set(x, acts(3, K))
    assert hb.compute([d1, d2]) == abi.GGML_STATUS_SUCCESS
    np.testing.assert_array_equal(hb.get(d1, np.float32, (3, M)), hb.get(d2, np.float32, (3, M)))
