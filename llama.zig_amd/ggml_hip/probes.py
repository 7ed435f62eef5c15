"""Measurement aids for bench.py, over libqmm_probe.so (built beside the
backend library from probes/probe.hip, not part of it): the streaming-read
floor the decode GEMV is compared against, and the MFMA / VALU overlap probe
the MMQ's ceiling rests on.  Neither has a counterpart in the reference."""
from __future__ import annotations

import ctypes

import torch

from . import PKG_DIR, HipQmmError, _check, _ptr, _require_cuda, _stream

PROBE_LIB_PATH = PKG_DIR / "libqmm_probe.so"
OV_THREADS = 512  # threads per workgroup of the overlap probe (8 waves, one workgroup per CU)
OV_MODES = {
    1: "MFMAs only",
    2: "FMAs only",
    3: "both, interleaved in every wave",
    4: "both, MFMA waves beside FMA waves",
    5: "both in every wave, MFMA accumulators in AGPRs",
    6: "MFMA waves beside FMA waves, accumulators in AGPRs",
}

_plib = None


def plib():
    global _plib
    if _plib is None:
        if not PROBE_LIB_PATH.exists():
            raise HipQmmError(f"{PROBE_LIB_PATH} not built: run `make -C {PKG_DIR}`")
        L = ctypes.CDLL(str(PROBE_LIB_PATH))
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        L.qmm_probe_sink_words.restype = ctypes.c_size_t
        L.qmm_probe_sink_words.argtypes = [ctypes.c_size_t]
        L.qmm_probe_stream_read.restype = i32
        L.qmm_probe_stream_read.argtypes = [vp, ctypes.c_size_t, vp, vp]
        L.qmm_probe_empty_launch.restype = i32
        L.qmm_probe_empty_launch.argtypes = [i32, vp, vp]
        L.qmm_probe_q4k_gemv_pattern.restype = i32
        L.qmm_probe_q4k_gemv_pattern.argtypes = [vp, ctypes.c_int64, ctypes.c_int64, vp, vp]
        L.qmm_probe_mfma_valu.restype = i32
        L.qmm_probe_mfma_valu.argtypes = [i32, i32, i32, vp, vp, vp]
        _plib = L
    return _plib


def sink_words(nbytes: int) -> int:
    return int(plib().qmm_probe_sink_words(nbytes))


def stream_read(buf: torch.Tensor, sink=None):
    """Streaming read of a device buffer (the GEMV's memory floor probe);
    returns the XOR-folded sink words."""
    _require_cuda(buf)
    nbytes = buf.numel() * buf.element_size()
    if sink is None:
        sink = torch.empty(max(sink_words(nbytes), 1), dtype=torch.int32, device=buf.device)
    _check(plib().qmm_probe_stream_read(_ptr(buf), nbytes, _ptr(sink), _stream()), "qmm_probe_stream_read")
    return sink


def empty_launch(nblocks: int, sink: torch.Tensor):
    """A launch of nblocks empty workgroups of the headline GEMV's shape: the
    fixed cost a launch's duration carries."""
    _require_cuda(sink)
    _check(plib().qmm_probe_empty_launch(nblocks, _ptr(sink), _stream()), "qmm_probe_empty_launch")


def q4k_gemv_pattern(w: torch.Tensor, sink: torch.Tensor):
    """The headline GEMV's loads over a Q4_K [nrows, 2304-byte] matrix, no
    arithmetic; sink holds one word per wave (ceil(nrows / 28) * 14)."""
    _require_cuda(w)
    _check(plib().qmm_probe_q4k_gemv_pattern(_ptr(w), w.shape[0], w.stride(0), _ptr(sink), _stream()),
           "qmm_probe_q4k_gemv_pattern")


def mfma_valu(mode: int, iters: int, nblocks: int = 256, sink=None, hwid=None):
    """MFMA / VALU overlap probe (modes in OV_MODES).  Returns (sink, hwid):
    sink = [MFMA sums of every thread, FMA sums of every thread], hwid = the
    HW_ID register of every wave (SIMD in bits 5:4)."""
    n = nblocks * OV_THREADS
    if sink is None:
        sink = torch.empty(2 * n, dtype=torch.float32, device="cuda")
    if hwid is None:
        hwid = torch.empty(nblocks * (OV_THREADS // 64), dtype=torch.int32, device="cuda")
    _check(plib().qmm_probe_mfma_valu(mode, iters, nblocks, _ptr(sink), _ptr(hwid), _stream()),
           "qmm_probe_mfma_valu")
    return sink, hwid
