#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (one GPU).

Metric: "Q4_K GEMV GB/s (% HBM peak) @14336x4096 b=1; MMQ
int8 TOPS @b=512".  A step is one ggml_mul_mat of the headline decode shape:
the Q4_K weight 14336x4096 times one f32 activation column; for one column
the op runs a single kernel, the GEMV with the Q8_1 quantization fused in.
Inputs are resident in HBM; the weight is rotated over enough distinct copies
(> 2x the 256 MB Infinity Cache) that every step streams it from HBM.  The
timed steps are replayed from one HIP graph of exactly --steps launches, so
the measurement is of the GPU, not of Python launch overhead.

Inputs: weights f32 N(0, 0.02) from seed 42 quantized with the reference's
quantize_row_q4_K_ref, activations f32 N(0, 1) from seed 43.  Generating them
takes the reference quantizer, which lives in the CPU checker (oracle/), so
they are made in the CPU-baseline leg, which also times the reference's CPU
path on the same bytes and checks the GPU results against it.  With --no-cpu
the weights are random valid blocks instead (same work per step).

Printed JSON (one line): value = whole-step GB/s (algorithmic bytes /
wall-clock per step); roofline = the step's kernel alone (algorithmic bytes /
its average duration from HIP events), with HBM traffic per launch measured
by a rocprofv3 counter pass of this script run as a child process; mmq = the
T=512 MMQ half of the metric with its own roofline, CPU baseline and parity;
cpu_baseline = the reference CPU path (restated AVX2 vec_dot_q4_K_q8_K in
ggml's mul_mat chunking) on a bounded sample, timed on this host; parity =
NMSE and maximum relative error of the GPU op against that CPU path.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import pathlib
import shutil
import statistics
import subprocess
import sys
import tempfile
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llama.zig_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
INFINITY_CACHE = 256 << 20
NMSE_GATE = 5e-4

M, K = 14336, 4096             # headline weight: Llama-3-8B ffn_gate/up
HEADLINE = (M, K)
T_MMQ = 512
CPU_SAMPLE_S = 10.0            # CPU work per baseline leg


BLOCKS = {"Q4_K": (256, 144), "Q5_K": (256, 176), "Q6_K": (256, 210), "Q8_0": (32, 34), "Q4_0": (32, 18),
          "IQ4_XS": (256, 136)}


def q4k_row_bytes(k):
    return k // 256 * 144


def row_bytes(qtype, k):
    bs, bb = BLOCKS[qtype]
    return k // bs * bb


def random_blocks(torch, qtype, nrows, k, gen, device):
    """Random but valid blocks of a weight type: random quant / scale bytes and
    f16 super-block scales at the magnitude N(0, 0.02) weights quantize to.
    Throughput does not depend on the values; parity tests use quantized
    N(0, 0.02) weights instead."""
    bs, bb = BLOCKS[qtype]
    nb = nrows * (k // bs)
    blocks = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, generator=gen, device="cpu")
    def f16(v):
        return torch.full((nb,), v, dtype=torch.float16).view(torch.uint8).view(nb, 2)
    if qtype in ("Q4_K", "Q5_K"):
        blocks[:, 0:2] = f16(2.5e-4 if qtype == "Q4_K" else 1.2e-4)
        blocks[:, 2:4] = f16(4.0e-4)
    elif qtype == "Q6_K":
        blocks[:, 208:210] = f16(2.5e-4)
    else:
        blocks[:, 0:2] = f16(5.0e-4)
    return blocks.view(nrows, row_bytes(qtype, k)).to(device)


def random_q4k(torch, nrows, k, gen, device):
    return random_blocks(torch, "Q4_K", nrows, k, gen, device)


def event_time_kernel(torch, launch, n):
    """Average device duration of `launch(i)` over n launches, from HIP event
    pairs on the launching stream.  A spin kernel first fills the queue so the
    events bracket back-to-back GPU work, not host launch gaps."""
    s = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    torch.cuda.synchronize()
    torch.cuda._sleep(20_000_000)
    for i in range(n):
        starts[i].record(s)
        launch(i)
        ends[i].record(s)
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in zip(starts, ends))
    return sum(ts) / len(ts), ts[len(ts) // 2]


def capture(torch, launch, n):
    """n launches captured into one HIP graph on a side stream."""
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        with torch.cuda.graph(g, stream=cs):
            for i in range(n):
                launch(i)
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    return g


def event_time_batch(torch, launch, n):
    """Average device time per launch of n back-to-back launches: the launches
    are captured into one HIP graph, and each replay is bracketed by two HIP
    events on the replaying stream, so host launch cost cannot starve the GPU.
    The mean of 3 timed replays after the warm-up (event_time_replays)."""
    return event_time_replays(torch, launch, n, warm=2, reps=3)[0]


WARM_S = 0.1  # untimed GPU work before a timed replay: the clocks ramp up over the first tens of ms of load


def warm_up(torch, g, min_replays):
    """Untimed replays of graph g: at least min_replays, and until WARM_S of
    wall time has passed (the first replays after an idle period or a switch
    of kernel run slower while the clocks settle)."""
    t0 = time.perf_counter()
    i = 0
    while i < min_replays or time.perf_counter() - t0 < WARM_S:
        g.replay()
        torch.cuda.synchronize()
        i += 1


def event_time_replays(torch, launch, n, warm=3, reps=5):
    """As event_time_batch, over `reps` timed replays of the graph after the
    warm-up (warm_up with `warm` replays at least): the mean per-launch time
    over the timed replays, and each replay's per-launch time."""
    g = capture(torch, launch, n)
    warm_up(torch, g, warm)
    s = torch.cuda.current_stream()
    per = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        g.replay()
        b.record(s)
        torch.cuda.synchronize()
        per.append(a.elapsed_time(b) / n)
    return sum(per) / len(per), per


# ---------------------------------------------------------------- the CPU-baseline leg

def _oracle():
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O  # noqa: E402  (test infrastructure: input generator, baseline and checker only)
    return O


def host_info(threads):
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = None
    return {"cpu_model": model, "host_logical_cpus": os.cpu_count(), "cpus_allowed": allowed, "threads": threads,
            "thread_cap": "16: the GPU box's CPU share for one GPU"}


def reference_inputs(T):
    """Seeded inputs quantized by the reference's own quantizer: weights f32
    N(0, 0.02) seed 42 -> quantize_row_q4_K_ref, activations f32 N(0, 1) seed
    43 (one column), and T columns for the MMQ leg (seed 43, index 1)."""
    O = _oracle()
    w = O.fill_normal(42, M * K, 0.0, 0.02).reshape(M, K)
    wq = O.quantize_rows(O.TYPE_Q4_K, w)
    x = O.fill_normal(43, K).reshape(1, K)
    xt = O.fill_normal(43 + 1000, T * K).reshape(T, K)
    return wq, x, xt


CPU_ROTATE_BYTES = 1 << 30      # weight copies the CPU legs cycle through: beyond any host L3


def cpu_copies(wq):
    """Copies of a host weight array totalling about CPU_ROTATE_BYTES (at least
    one, at most 64), so that each timed CPU run streams its weights from DRAM
    as a model larger than the host's caches does."""
    import numpy as np
    n = max(1, min(64, CPU_ROTATE_BYTES // max(1, wq.nbytes)))
    return [wq] + [np.array(wq, copy=True) for _ in range(n - 1)]


def time_cpu(fn, budget_s, min_runs=5):
    fn()  # warm-up
    times, t0 = [], time.perf_counter()
    while (time.perf_counter() - t0 < budget_s and len(times) < 2000) or len(times) < min_runs:
        t1 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t1)
    return statistics.median(times), len(times)


def parity(got, want):
    import numpy as np
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    nmse = float(np.sum((got - want) ** 2) / max(float(np.sum(want * want)), 1e-300))
    scale = np.maximum(np.abs(want), 1e-3 * float(np.max(np.abs(want))))
    return {"nmse_vs_cpu": nmse, "max_rel_vs_cpu": float(np.max(np.abs(got - want) / scale)),
            "max_rel_floor": "1e-3 x max|cpu|",
            "max_err_over_max_vs_cpu": float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-300)),
            "nmse_gate": NMSE_GATE, "pass": bool(nmse < NMSE_GATE)}


def cpu_gemv_leg(wq, x, gpu_out):
    """Reference CPU path at b=1 on a bounded sample: quantize_row_q8_K_ref
    staging, the restated AVX2 vec_dot_q4_K_q8_K, ggml's mul_mat chunking, on
    the host threads this process may use (at most 16); and the GPU op's
    result checked against that CPU result."""
    O = _oracle()
    nth = O.gen_threads()
    impl = O.IMPL_AVX2 if O.has_avx2() else O.IMPL_GENERIC
    out = {}
    wqs, it = cpu_copies(wq), [0]

    def run():
        out["y"] = O.mul_mat(O.TYPE_Q4_K, wqs[it[0] % len(wqs)], M, K, x, nth=nth, impl=impl)
        it[0] += 1

    med, runs = time_cpu(run, CPU_SAMPLE_S, 20)
    bytes_alg = M * q4k_row_bytes(K) + K * 4 + M * 4
    base = {"value": round(bytes_alg / med / 1e9, 3), "unit": "GB/s", "cores": nth, "kind": "port",
            "sample": f"Q4_K {M}x{K} b=1 mul_mat (seed-42 weights, {len(wqs)} host copies cycled), "
                      f"{'AVX2' if impl == O.IMPL_AVX2 else 'generic'} vec_dot path, persistent threads, "
                      f"median of {runs} runs ({med * 1e3:.3f} ms each)",
            **host_info(nth)}
    return base, parity(gpu_out, out["y"])


def cpu_mmq_leg(wq, xt, gpu_out):
    """Reference CPU path at T=512: what ggml's CPU mul_mat runs on x86 for 8
    or more columns, the tiled integer GEMM (restated AVX2 arm, Q8_K
    activations); the vec_dot path where the host lacks AVX2."""
    O = _oracle()
    nth = O.gen_threads()
    out = {}

    wqs, it = cpu_copies(wq), [0]

    def run():
        w_i = wqs[it[0] % len(wqs)]
        it[0] += 1
        y = O.mul_mat_tiled(O.TYPE_Q4_K, w_i, M, K, xt, nth=nth)
        out["y"] = y if y is not None else O.mul_mat(O.TYPE_Q4_K, w_i, M, K, xt, nth=nth)

    med, runs = time_cpu(run, CPU_SAMPLE_S, 3)
    tiled = O.has_avx2()
    ops = 2.0 * M * K * T_MMQ
    base = {"value": round(ops / med / 1e12, 4), "unit": "TOP/s", "cores": nth, "kind": "port",
            "sample": f"Q4_K {M}x{K} x T={T_MMQ} mul_mat (seed-42 weights, {len(wqs)} host copies cycled), "
                      f"{'x86 tiled GEMM (AVX2 arm)' if tiled else 'generic vec_dot path'}, "
                      f"median of {runs} runs ({med * 1e3:.1f} ms each)",
            **host_info(nth)}
    return base, parity(gpu_out, out["y"])


# ---------------------------------------------------------------- HBM traffic, measured live

PROBE_KERNELS = {"gemv": "gemv_fx_kernel", "mmq": "mmq_q4k_dma_kernel", "copy": "copyBuffer"}
COPY_BYTES = 64 << 20


def traffic_probe():
    """Child mode (run under rocprofv3 --pmc): a 64 MiB device copy for the
    counter calibration, then the headline GEMV and the T=512 MMQ kernels on
    rotated random weights."""
    import torch
    import ggml_hip as G
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(7)
    a = torch.randint(0, 255, (COPY_BYTES,), dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(8):
        b.copy_(a)
    ncopy = max(4, -(-2 * INFINITY_CACHE // (M * q4k_row_bytes(K))))
    ws = [random_q4k(torch, M, K, gen, dev) for _ in range(ncopy)]
    x = torch.randn((1, K), generator=gen).to(dev)
    out = torch.empty((1, M), device=dev)
    for i in range(4 * ncopy):
        G.mul_mat_vec_f32("Q4_K", ws[i % ncopy], K, x, out=out)
    xt = torch.randn((T_MMQ, K), generator=gen).to(dev)
    qs, ds = G.quantize_q8_1_planar(xt)
    outt = torch.empty((T_MMQ, M), device=dev)
    for i in range(2 * ncopy):
        G.mmq("Q4_K", ws[i % ncopy], K, qs, ds, out=outt)
    torch.cuda.synchronize()


def _counter_medians(csv_path):
    vals = {k: [] for k in PROBE_KERNELS}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            for key, pat in PROBE_KERNELS.items():
                if pat in r["Kernel_Name"]:
                    vals[key].append(float(r["Counter_Value"]))
    return {k: statistics.median(v) for k, v in vals.items() if v}


def measure_traffic():
    """HBM bytes per launch of the headline GEMV and the MMQ: two rocprofv3
    counter passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch) over this
    script's probe mode, each scaled by what the same counter reads for a
    64 MiB copy.  Returns ({kernel: bytes}, calibration) or (None, reason)."""
    prof = shutil.which("rocprofv3")
    if not prof:
        return None, "rocprofv3 not found"
    med = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="qmm_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "probe", "--",
               sys.executable, str(ROOT / "bench.py"), "--traffic-probe"]
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), capture_output=True, text=True,
                               timeout=180)
        except subprocess.TimeoutExpired:
            shutil.rmtree(d, ignore_errors=True)
            return None, f"rocprofv3 --pmc {counter} timed out"
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            shutil.rmtree(d, ignore_errors=True)
            return None, f"rocprofv3 --pmc {counter}: no counter file (rc {r.returncode}): {r.stderr[-300:]}"
        med[counter] = _counter_medians(files[0])
        shutil.rmtree(d, ignore_errors=True)
    try:
        f_scale = (COPY_BYTES / 1024) / med["FETCH_SIZE"]["copy"]
        w_scale = (COPY_BYTES / 1024) / med["WRITE_SIZE"]["copy"]
        out = {k: int(round((med["FETCH_SIZE"][k] * f_scale + med["WRITE_SIZE"][k] * w_scale) * 1024))
               for k in ("gemv", "mmq")}
    except (KeyError, ZeroDivisionError) as e:
        return None, f"counter pass incomplete: {e!r}"
    return out, {"fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
                 "calibration": "64 MiB device copy, same counters, same pass"}


CPU_SUITE_S = 0.3              # CPU work per suite case
CPU_SUITE_MACS = 2e10          # cases above this many MACs time a row sample on the CPU


def cpu_suite_case(qtype, w_dev, M, Kx, x_dev):
    """The reference CPU path for one suite case, through the route ggml's CPU
    mul_mat takes on an x86 AVX2 host (the tiled GEMM for the tiled K-quants
    from 8 columns, tinyBLAS for Q8_0 / Q4_0 from 2, else the AVX2 vec_dot;
    oracle_lib.mul_mat_x86), on this host's threads (at most 16).  The whole
    case where it has at most CPU_SUITE_MACS multiply-adds; above that a sample
    of the first rows (a multiple of 256, at least 4096) against all the
    case's columns, its time scaled by M / rows (each output row is
    independent work)."""
    O = _oracle()
    tid = {"Q4_K": O.TYPE_Q4_K, "Q6_K": O.TYPE_Q6_K, "Q8_0": O.TYPE_Q8_0, "Q5_K": O.TYPE_Q5_K,
           "Q4_0": O.TYPE_Q4_0, "IQ4_XS": O.TYPE_IQ4_XS}[qtype]
    T = x_dev.shape[0]
    macs = float(M) * Kx * T
    rows = M if macs <= CPU_SUITE_MACS else min(M, max(4096, int(M * CPU_SUITE_MACS / macs) // 256 * 256))
    wq = w_dev[:rows].cpu().numpy()
    x = x_dev.cpu().numpy().reshape(-1, Kx)
    nth = O.gen_threads()
    route = ("tiled GEMM" if T >= 8 and qtype in ("Q4_K", "Q5_K", "Q6_K", "IQ4_XS") and O.has_avx2() else
             "tinyBLAS" if T >= 2 and qtype in ("Q8_0", "Q4_0") and O.has_avx2() else
             "AVX2 vec_dot" if O.has_avx2() else "generic vec_dot")
    wqs, it = cpu_copies(wq), [0]

    def run():
        O.mul_mat_x86(tid, wqs[it[0] % len(wqs)], rows, Kx, x, nth=nth)
        it[0] += 1

    med, runs = time_cpu(run, CPU_SUITE_S, 2)
    return {"cpu_us": round(med * 1e6 * M / rows, 1), "cpu_rows_timed": rows, "cpu_runs": runs,
            "cpu_route": route, "cpu_threads": nth, "cpu_weight_copies": len(wqs)}


def run_suite(name, torch, G, dev, reps, cpu=True):
    """Kernel-level measurements over the configs of BASELINE.json, one JSON
    line per case (device time from a HIP graph of launches between events,
    weights rotated over > 2 x the Infinity Cache), with the reference CPU
    path's time for the same case beside it (cpu_us, see cpu_suite_case)."""
    gen = torch.Generator().manual_seed(42)
    xg = torch.Generator().manual_seed(43)
    if cpu and name not in ("floor", "overlap"):
        print(json.dumps({"suite": name, "cpu_host": host_info(_oracle().gen_threads())}), flush=True)

    def copies(qtype, nrows, k):
        wb = nrows * row_bytes(qtype, k)
        n = max(3, -(-2 * INFINITY_CACHE // wb))
        return [random_blocks(torch, qtype, nrows, k, gen, dev) for _ in range(n)], wb

    def emit(rec):
        print(json.dumps(rec), flush=True)

    if name in ("decode", "crossquant", "mmq", "few"):
        if name == "decode":
            shapes = [("Q4_K", 4096, 4096, "attn_q/o"), ("Q4_K", 1024, 4096, "attn_k"), ("Q6_K", 1024, 4096, "attn_v"),
                      ("Q4_K", 14336, 4096, "ffn_gate/up"), ("Q6_K", 4096, 14336, "ffn_down")]
            batches = (1, 2, 4, 8)
        elif name == "mmq":
            shapes = [("Q4_K", 14336, 4096, "ffn_gate/up")]
            batches = (128, 512, 2048)
        elif name == "few":
            # batched decode: the few-column GEMM against the GEMV (<= 8
            # columns) and the 128-row MMQ tile it replaced (9-32 columns;
            # for Q6_K / Q8_0 / Q4_0 / IQ4_XS the tile is timed on the same
            # weights at a base 2 (IQ4_XS: 8) bytes past 16-byte alignment,
            # which the few-column kernel does not take; Q5_K rows must be
            # 16-byte aligned for both, so it has no tile line)
            shapes = [("Q4_K", 14336, 4096, "ffn_gate/up"), ("Q4_K", 4096, 14336, "Q4_K 4096x14336"),
                      ("Q4_K", 4096, 4096, "attn_q/o"), ("Q6_K", 4096, 14336, "ffn_down"),
                      ("Q6_K", 4096, 4096, "Q6_K 4096x4096"), ("Q8_0", 4096, 4096, "Q8_0 4096x4096"),
                      ("Q8_0", 4096, 14336, "Q8_0 4096x14336"), ("Q5_K", 4096, 14336, "Q5_K 4096x14336"),
                      ("Q4_0", 4096, 14336, "Q4_0 4096x14336"), ("IQ4_XS", 4096, 14336, "IQ4_XS 4096x14336")]
            batches = (4, 6, 8, 9, 16, 24, 32)
        else:
            shapes = [(t, 4096, k, f"{t} 4096x{k}") for t in ("Q8_0", "Q6_K", "Q4_K", "Q5_K", "Q4_0", "IQ4_XS")
                      for k in (4096, 14336)]
            batches = (1, 32, 512)
        for qtype, M, Kx, label in shapes:
            ws, wb = copies(qtype, M, Kx)
            for T in batches:
                x = torch.randn((T, Kx), generator=xg, dtype=torch.float32).to(dev)
                qs, ds = G.quantize_q8_1_planar(x)
                out = torch.empty((T, M), dtype=torch.float32, device=dev)
                n = len(ws) * reps
                mmq_ws = torch.empty(max(1, int(G.lib().hip_qmm_mmq_workspace_size(G.TYPE_IDS[qtype], Kx, M, T))),
                                     dtype=torch.uint8, device=dev)
                # the kernel the op takes for these columns (the GEMV up to 8
                # columns except where the few-column GEMM measured faster)
                gemv_fn = lambda i: G.mul_mat_vec(qtype, ws[i % len(ws)], Kx, qs, ds, out=out)  # noqa: E731
                mmq_fn = lambda i: G.mmq(qtype, ws[i % len(ws)], Kx, qs, ds, out=out, workspace=mmq_ws)  # noqa: E731
                # the op on f32 activations (hip_qmm_mul_mat: quantizer + kernel,
                # or for one column the GEMV that quantizes in its prologue)
                wsp = torch.empty(int(G.lib().hip_qmm_mul_mat_workspace_size(G.TYPE_IDS[qtype], Kx, M, T)),
                                  dtype=torch.uint8, device=dev)
                op_fn = lambda i: G.mul_mat(qtype, ws[i % len(ws)], x, out=out, workspace=wsp)  # noqa: E731
                if 2 <= T <= 8 and G.lib().hip_qmm_mul_mat_per_column(G.TYPE_IDS[qtype], Kx, M, T):
                    # one launch: the one-column kernel per column, quantizing in the kernel
                    fn, kern = op_fn, "gemv one-column kernel per column"
                elif T <= 8 and not G.lib().hip_qmm_mul_mat_uses_mmq(G.TYPE_IDS[qtype], Kx, M, T):
                    fn, kern = gemv_fn, "gemv"
                else:
                    fn, kern = mmq_fn, ("mmq few-column" if T <= 8 else "mmq")
                ms = event_time_batch(torch, fn, n)
                extra = {}
                if T <= 8 and kern != "gemv":
                    extra["gemv_us"] = round(event_time_batch(torch, gemv_fn, n) * 1e3, 3)
                if name == "few":
                    # the few-column GEMM at every width (next to the GEMV up
                    # to 8 columns)
                    few_fn = lambda i: G.mmq(qtype, ws[i % len(ws)], Kx, qs, ds, out=out, workspace=mmq_ws)  # noqa: E731
                    extra["few_us"] = round(event_time_batch(torch, few_fn, n) * 1e3, 3)
                    extra["few_split"] = int(G.lib().hip_qmm_mmq_split_k(G.TYPE_IDS[qtype], Kx, M, T))
                    if qtype not in ("Q4_K", "Q5_K") and T > 8:
                        if T == 9:
                            off = []
                            sh = 8 if qtype == "IQ4_XS" else 2
                            for wt in ws:  # the same rows at a base sh bytes past 16-byte alignment
                                buf = torch.zeros(wt.numel() + 16, dtype=torch.uint8, device=dev)
                                off.append(buf[sh:sh + wt.numel()].view(wt.shape))
                                off[-1].copy_(wt)
                        tile_fn = lambda i: G.mmq(qtype, off[i % len(off)], Kx, qs, ds, out=out,  # noqa: E731
                                                  workspace=mmq_ws)
                        extra["tile128_us"] = round(event_time_batch(torch, tile_fn, n) * 1e3, 3)
                ms_op = event_time_batch(torch, op_fn, n)
                alg = wb + Kx * 4 * T + M * 4 * T
                ops = 2.0 * M * Kx * T
                if cpu:
                    extra.update(cpu_suite_case(qtype, ws[0], M, Kx, x))
                    extra["op_speedup_vs_cpu"] = round(extra["cpu_us"] / (ms_op * 1e3), 1)
                emit({"suite": name, "kernel": kern, "type": qtype, "shape": f"{M}x{Kx}", "label": label, "T": T,
                      "us": round(ms * 1e3, 3), "op_us": round(ms_op * 1e3, 3), "GB/s": round(alg / ms / 1e6, 1),
                      "hbm_frac": round(alg / ms / 1e6 / HBM_PEAK_GBS, 4), "TOPS": round(ops / ms / 1e9, 2),
                      "int8_frac": round(ops / ms / 1e9 / INT8_PEAK_TOPS, 4), **extra})
            del ws
            if name == "few" and qtype not in ("Q4_K", "Q5_K"):
                del off
            torch.cuda.empty_cache()
    elif name == "moe":
        n_as, n_tokens, k = 128, 512, 8
        logits = torch.randn((n_tokens, n_as), generator=torch.Generator().manual_seed(44))
        ids = torch.topk(torch.softmax(logits, dim=1), k, dim=1).indices.to(torch.int32).to(dev)
        for label, M, Kx, ne11 in (("gate/up", 768, 2048, 1), ("down", 2048, 768, k)):
            wb = n_as * M * row_bytes("Q4_K", Kx)
            n = max(2, -(-2 * INFINITY_CACHE // wb))
            ws = [random_blocks(torch, "Q4_K", n_as * M, Kx, gen, dev).view(n_as, M, -1) for _ in range(n)]
            x = torch.randn((n_tokens, ne11, Kx), generator=xg, dtype=torch.float32).to(dev)
            out = torch.empty((n_tokens, k, M), dtype=torch.float32, device=dev)
            wsp = torch.empty(int(G.lib().hip_qmm_mul_mat_id_workspace_size(12, Kx, n_as, ne11, n_tokens, k)),
                              dtype=torch.uint8, device=dev)
            fn = lambda i: G.mul_mat_id("Q4_K", ws[i % len(ws)], x, ids, out=out, workspace=wsp)  # noqa: E731
            ms = event_time_batch(torch, fn, n * reps)
            alg = wb + n_tokens * ne11 * Kx * 4 + n_tokens * k * M * 4
            ops = 2.0 * M * Kx * n_tokens * k
            extra = {}
            if cpu:
                # the reference CPU mul_mat_id (per-slot vec_dot rows over the
                # routed experts, AVX2 where the host has it) on the whole case
                O = _oracle()
                nth = O.gen_threads()
                wqs = cpu_copies(ws[0].cpu().numpy().reshape(n_as * M, -1))
                xh, idh = x.cpu().numpy(), ids.cpu().numpy()
                impl = O.IMPL_AVX2 if O.has_avx2() else O.IMPL_GENERIC
                it = [0]

                def run_id():
                    O.mul_mat_id(O.TYPE_Q4_K, wqs[it[0] % len(wqs)], n_as, M, Kx, xh, idh, nth=nth, impl=impl)
                    it[0] += 1

                med, runs = time_cpu(run_id, CPU_SUITE_S, 2)
                extra = {"cpu_us": round(med * 1e6, 1), "cpu_runs": runs, "cpu_threads": nth,
                         "cpu_route": "mul_mat_id, " + ("AVX2" if impl == O.IMPL_AVX2 else "generic") + " vec_dot",
                         "speedup_vs_cpu": round(med * 1e6 / (ms * 1e3), 1)}
            emit({"suite": name, "kernel": "mul_mat_id (quantize + group + grouped MMQ)", "type": "Q4_K",
                  "shape": f"{n_as}x{M}x{Kx}", "label": label, "tokens": n_tokens, "top_k": k,
                  "us": round(ms * 1e3, 3), "GB/s": round(alg / ms / 1e6, 1),
                  "hbm_frac": round(alg / ms / 1e6 / HBM_PEAK_GBS, 4), "TOPS": round(ops / ms / 1e9, 2), **extra})
            # decode: one token's 8 experts through the one-launch GEMV over
            # (token, slot) pairs; bytes = the 8 selected experts' weights
            x1 = torch.randn((1, ne11, Kx), generator=xg, dtype=torch.float32).to(dev)
            ids1 = ids[:1].contiguous()
            out1 = torch.empty((1, k, M), dtype=torch.float32, device=dev)
            fn1 = lambda i: G.mul_mat_id("Q4_K", ws[i % len(ws)], x1, ids1, out=out1, workspace=wsp)  # noqa: E731
            ms1 = event_time_batch(torch, fn1, n * reps * 4)
            alg1 = k * M * row_bytes("Q4_K", Kx) + ne11 * Kx * 4 + k * M * 4
            emit({"suite": name, "kernel": "mul_mat_id decode (GEMV over token/slot pairs)", "type": "Q4_K",
                  "shape": f"{n_as}x{M}x{Kx}", "label": label, "tokens": 1, "top_k": k,
                  "us": round(ms1 * 1e3, 3), "GB/s": round(alg1 / ms1 / 1e6, 1),
                  "hbm_frac": round(alg1 / ms1 / 1e6 / HBM_PEAK_GBS, 4)})
            if label == "gate/up":
                gs = [random_blocks(torch, "Q4_K", n_as * M, Kx, gen, dev).view(n_as, M, -1) for _ in range(n)]
                fz = lambda i: G.mul_mat_id_vec_fused("Q4_K", ws[i % n], x1, ids1, w_gate=gs[i % n],  # noqa: E731
                                                      glu="SWIGLU", out=out1)
                msf = event_time_batch(torch, fz, n * reps * 4)
                u1 = torch.empty_like(out1)
                g1 = torch.empty_like(out1)

                def unf(i):
                    G.mul_mat_id("Q4_K", ws[i % n], x1, ids1, out=u1, workspace=wsp)
                    G.mul_mat_id("Q4_K", gs[i % n], x1, ids1, out=g1, workspace=wsp)
                    G.glu_f32(g1.view(k, M), u1.view(k, M), "SWIGLU", out=out1.view(k, M))

                msu = event_time_batch(torch, unf, n * reps * 4)
                algf = 2 * k * M * row_bytes("Q4_K", Kx) + Kx * 4 + k * M * 4
                emit({"suite": name, "kernel": "mul_mat_id decode gate+up+swiglu fused", "type": "Q4_K",
                      "shape": f"{n_as}x{M}x{Kx}", "label": label, "tokens": 1, "top_k": k,
                      "us": round(msf * 1e3, 3), "GB/s": round(algf / msf / 1e6, 1),
                      "unfused_3_launches_us": round(msu * 1e3, 3)})
                # with a shared expert of the same shape in the same launch,
                # against the routed launch plus the shared expert's own one
                sus = [random_blocks(torch, "Q4_K", M, Kx, gen, dev) for _ in range(n)]
                sgs = [random_blocks(torch, "Q4_K", M, Kx, gen, dev) for _ in range(n)]
                sh_out = torch.empty((1, M), dtype=torch.float32, device=dev)
                fs = lambda i: G.mul_mat_id_vec_fused_shared("Q4_K", ws[i % n], gs[i % n], x1, ids1,  # noqa: E731
                                                             sus[i % n], sgs[i % n], glu="SWIGLU", out=out1,
                                                             shared_out=sh_out)

                def two(i):
                    fz(i)
                    G.mul_mat_vec_fused("Q4_K", sus[i % n], Kx, x1.view(1, Kx), w_gate=sgs[i % n], glu="SWIGLU",
                                        out=sh_out)

                mss = event_time_batch(torch, fs, n * reps * 4)
                ms2 = event_time_batch(torch, two, n * reps * 4)
                algs = algf + 2 * M * row_bytes("Q4_K", Kx) + M * 4
                emit({"suite": name, "kernel": "mul_mat_id decode gate+up+swiglu fused with a shared expert",
                      "type": "Q4_K", "shape": f"{n_as}x{M}x{Kx} + shared {M}x{Kx}", "label": label, "tokens": 1,
                      "top_k": k, "us": round(mss * 1e3, 3), "GB/s": round(algs / mss / 1e6, 1),
                      "routed_then_shared_2_launches_us": round(ms2 * 1e3, 3)})
                del sus, sgs
                del gs
            del ws
            torch.cuda.empty_cache()
    elif name == "ffn":
        # Decode FFN gate + up + SWIGLU on one f32 column: the fused kernel
        # (hip_qmm_mul_mat_vec_fused with a gate) against the unfused
        # sequence it replaces (two one-column quantizing GEMVs and the GLU
        # kernel), and the bias lane (GEMV + bias) against the plain GEMV.
        for M, Kx, label in ((14336, 4096, "llama3-8b ffn_gate/up"), (768, 2048, "qwen3-30b-a3b expert gate/up")):
            wb = M * row_bytes("Q4_K", Kx)
            n = max(3, -(-2 * INFINITY_CACHE // (2 * wb)))
            wu = [random_blocks(torch, "Q4_K", M, Kx, gen, dev) for _ in range(n)]
            wg = [random_blocks(torch, "Q4_K", M, Kx, gen, dev) for _ in range(n)]
            x = torch.randn((1, Kx), generator=xg, dtype=torch.float32).to(dev)
            bias = torch.randn((M,), generator=xg, dtype=torch.float32).to(dev)
            u = torch.empty((1, M), dtype=torch.float32, device=dev)
            g = torch.empty((1, M), dtype=torch.float32, device=dev)
            out = torch.empty((1, M), dtype=torch.float32, device=dev)
            reps_n = n * reps

            def fused(i):
                G.mul_mat_vec_fused("Q4_K", wu[i % n], Kx, x, w_gate=wg[i % n], glu="SWIGLU", out=out)

            def unfused(i):
                G.mul_mat_vec_f32("Q4_K", wu[i % n], Kx, x, out=u)
                G.mul_mat_vec_f32("Q4_K", wg[i % n], Kx, x, out=g)
                G.glu_f32(g, u, "SWIGLU", out=out)

            def lane_bias(i):
                G.mul_mat_vec_fused("Q4_K", wu[i % n], Kx, x, bias=bias, out=out)

            def lane_plain(i):
                G.mul_mat_vec_f32("Q4_K", wu[i % n], Kx, x, out=out)

            alg2 = 2 * wb + Kx * 4 + M * 4
            alg1 = wb + Kx * 4 + M * 4
            for kern, fn, alg in (("gate+up+swiglu fused", fused, alg2), ("gate+up+swiglu unfused (3 launches)",
                                                                         unfused, alg2),
                                  ("gemv+bias fused", lane_bias, alg1 + M * 4), ("gemv (one column)", lane_plain,
                                                                                  alg1)):
                ms = event_time_batch(torch, fn, reps_n)
                emit({"suite": name, "kernel": kern, "type": "Q4_K", "shape": f"{M}x{Kx}", "label": label, "T": 1,
                      "us": round(ms * 1e3, 3), "GB/s": round(alg / ms / 1e6, 1),
                      "hbm_frac": round(alg / ms / 1e6 / HBM_PEAK_GBS, 4)})
            del wu, wg
            torch.cuda.empty_cache()
    elif name == "prefill_ffn":
        # Prefill FFN gate + up + SWIGLU: the fused MMQ (hip_qmm_mul_mat_glu:
        # one quantization, one tile kernel over both weights, GLU in its
        # epilogue) against the unfused sequence (two hip_qmm_mul_mat and the
        # GLU kernel); then the MoE form at config 4 (hip_qmm_mul_mat_id_glu
        # against two hip_qmm_mul_mat_id and the GLU kernel).
        M, Kx = 14336, 4096
        wb = M * row_bytes("Q4_K", Kx)
        n = max(3, -(-2 * INFINITY_CACHE // (2 * wb)))
        wu = [random_blocks(torch, "Q4_K", M, Kx, gen, dev) for _ in range(n)]
        wg = [random_blocks(torch, "Q4_K", M, Kx, gen, dev) for _ in range(n)]
        for T in (64, 128, 512, 2048):
            x = torch.randn((T, Kx), generator=xg, dtype=torch.float32).to(dev)
            out = torch.empty((T, M), dtype=torch.float32, device=dev)
            u = torch.empty_like(out)
            g = torch.empty_like(out)
            t = G.TYPE_IDS["Q4_K"]
            wsf = torch.empty(max(1, int(G.lib().hip_qmm_mul_mat_glu_workspace_size(t, Kx, M, T))),
                              dtype=torch.uint8, device=dev)
            wsu = torch.empty(int(G.lib().hip_qmm_mul_mat_workspace_size(t, Kx, M, T)), dtype=torch.uint8, device=dev)

            def fused(i):
                G.mul_mat_glu("Q4_K", wu[i % n], wg[i % n], x, "SWIGLU", out=out, workspace=wsf)

            def unfused(i):
                G.mul_mat("Q4_K", wg[i % n], x, out=g, workspace=wsu)
                G.mul_mat("Q4_K", wu[i % n], x, out=u, workspace=wsu)
                G.glu_f32(g, u, "SWIGLU", out=out)

            msf = event_time_batch(torch, fused, n * reps)
            msu = event_time_batch(torch, unfused, n * reps)
            ops = 2.0 * 2 * M * Kx * T
            emit({"suite": name, "kernel": "gate+up+swiglu fused MMQ", "type": "Q4_K", "shape": f"2x{M}x{Kx}",
                  "label": "llama3-8b ffn_gate/up", "T": T, "fused": bool(G.lib().hip_qmm_mul_mat_glu_fused(
                      t, Kx, M, T)), "us": round(msf * 1e3, 3), "unfused_us": round(msu * 1e3, 3),
                  "TOPS": round(ops / msf / 1e9, 2), "int8_frac": round(ops / msf / 1e9 / INT8_PEAK_TOPS, 4)})
        del wu, wg
        torch.cuda.empty_cache()
        n_as, n_tokens, k, M, Kx = 128, 512, 8, 768, 2048
        logits = torch.randn((n_tokens, n_as), generator=torch.Generator().manual_seed(44))
        ids = torch.topk(torch.softmax(logits, dim=1), k, dim=1).indices.to(torch.int32).to(dev)
        wb = n_as * M * row_bytes("Q4_K", Kx)
        n = max(2, -(-2 * INFINITY_CACHE // (2 * wb)))
        wu = [random_blocks(torch, "Q4_K", n_as * M, Kx, gen, dev).view(n_as, M, -1) for _ in range(n)]
        wg = [random_blocks(torch, "Q4_K", n_as * M, Kx, gen, dev).view(n_as, M, -1) for _ in range(n)]
        x = torch.randn((n_tokens, 1, Kx), generator=xg, dtype=torch.float32).to(dev)
        out = torch.empty((n_tokens, k, M), dtype=torch.float32, device=dev)
        u = torch.empty_like(out)
        g = torch.empty_like(out)
        wsp = torch.empty(int(G.lib().hip_qmm_mul_mat_id_workspace_size(12, Kx, n_as, 1, n_tokens, k)),
                          dtype=torch.uint8, device=dev)

        def fused_id(i):
            G.mul_mat_id_glu("Q4_K", wu[i % n], wg[i % n], x, ids, "SWIGLU", out=out, workspace=wsp)

        def unfused_id(i):
            G.mul_mat_id("Q4_K", wg[i % n], x, ids, out=g, workspace=wsp)
            G.mul_mat_id("Q4_K", wu[i % n], x, ids, out=u, workspace=wsp)
            G.glu_f32(g.view(-1, M), u.view(-1, M), "SWIGLU", out=out.view(-1, M))

        msf = event_time_batch(torch, fused_id, n * reps)
        msu = event_time_batch(torch, unfused_id, n * reps)
        alg = 2 * wb + n_tokens * Kx * 4 + n_tokens * k * M * 4
        emit({"suite": name, "kernel": "mul_mat_id gate+up+swiglu fused (grouped MMQ)", "type": "Q4_K",
              "shape": f"2x{n_as}x{M}x{Kx}", "label": "qwen3-30b-a3b ffn_gate/up_exps", "tokens": n_tokens, "top_k": k,
              "us": round(msf * 1e3, 3), "unfused_us": round(msu * 1e3, 3), "GB/s": round(alg / msf / 1e6, 1)})
        del wu, wg
        torch.cuda.empty_cache()
    elif name == "floor":
        # The headline's weight stream against the memory floor: the same
        # rotated copies of the 14336x4096 Q4_K weight read by (1) the
        # streaming-read probe (the fastest plain read measured here), (2) the
        # GEMV on an already quantized column, (3) the headline op (GEMV with
        # the column's quantization fused in).  Bytes = the weight bytes.
        hm, hk = HEADLINE
        ws, wb = copies("Q4_K", hm, hk)
        x = torch.randn((1, hk), generator=xg, dtype=torch.float32).to(dev)
        qs, ds = G.quantize_q8_1_planar(x)
        out = torch.empty((1, hm), dtype=torch.float32, device=dev)
        from ggml_hip import probes as P
        sink = torch.empty(P.sink_words(wb), dtype=torch.int32, device=dev)
        n = len(ws) * reps
        gsink = torch.empty(max(P.sink_words(wb), -(-hm // 28) * 14), dtype=torch.int32, device=dev)
        cases = (("empty launch (512 workgroups of 896 threads)", lambda i: P.empty_launch(512, gsink)),
                 ("stream read probe", lambda i: P.stream_read(ws[i % len(ws)], sink=sink)),
                 ("the GEMV's own Q4_K loads, no arithmetic", lambda i: P.q4k_gemv_pattern(ws[i % len(ws)], gsink)),
                 ("gemv on a quantized column", lambda i: G.mul_mat_vec("Q4_K", ws[i % len(ws)], hk, qs, ds, out=out)),
                 ("op: gemv with fused quantization", lambda i: G.mul_mat("Q4_K", ws[i % len(ws)], x, out=out)))
        for kern, fn in cases:
            ms = event_time_batch(torch, fn, n)
            emit({"suite": name, "kernel": kern, "type": "Q4_K", "shape": f"{hm}x{hk}", "T": 1, "bytes": wb,
                  "weight_copies": len(ws), "us": round(ms * 1e3, 3), "GB/s": round(wb / ms / 1e6, 1),
                  "hbm_frac": round(wb / ms / 1e6 / HBM_PEAK_GBS, 4)})
        del ws
        torch.cuda.empty_cache()
    elif name == "overlap":
        # Whether MFMA and VALU work overlap on a SIMD (the MMQ ceiling rests on
        # it), from the overlap probe (probes/probe.hip): one 512-thread
        # workgroup per CU, so two waves per SIMD; SIMD cycles per substep from
        # HIP events around one launch, at the 2.4 GHz shader clock.  Modes 3-6
        # give every SIMD the same work per substep (two
        # v_mfma_f32_32x32x16_f16 and 32 wave64 FMAs); modes 4 and 6 split it
        # into MFMA waves (0-3) and FMA waves (4-7).  "mixed_simds" is the
        # share of SIMDs that held one wave of each half, from the waves' HW_ID.
        import numpy as np
        from ggml_hip import probes as P
        iters, nblocks = 4000, 256
        sink = torch.empty(2 * nblocks * P.OV_THREADS, dtype=torch.float32, device=dev)
        hwid = torch.empty(nblocks * P.OV_THREADS // 64, dtype=torch.int32, device=dev)
        for mode in sorted(P.OV_MODES):
            ms = event_time_batch(torch, lambda i: P.mfma_valu(mode, iters, nblocks, sink=sink, hwid=hwid), 3)
            ids = hwid.cpu().numpy().astype(np.int64).reshape(nblocks, P.OV_THREADS // 64)
            simd = (ids >> 4) & 3
            mixed = np.mean([len(set(simd[b, :4]) & set(simd[b, 4:])) / 4.0 for b in range(nblocks)])
            emit({"suite": name, "mode": mode, "work": P.OV_MODES[mode], "us": round(ms * 1e3, 3),
                  "simd_cycles_per_substep": round(ms * 1e-3 * 2.4e9 / (iters * 4), 1),
                  "mixed_simds": round(float(mixed), 3)})
    else:
        raise SystemExit(f"unknown suite {name}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs (headline: random weights, no parity; suites: no cpu_us)")
    ap.add_argument("--no-mmq", action="store_true", help="skip the MMQ leg")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 traffic passes")
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--suite", choices=["decode", "mmq", "crossquant", "moe", "ffn", "prefill_ffn", "few", "floor",
                                        "overlap"],
                    help="instead of the headline line, measure every case of one BASELINE config")
    ap.add_argument("--reps", type=int, default=4, help="passes over the weight copies per suite case")
    args = ap.parse_args()
    if args.traffic_probe:
        traffic_probe()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit("--steps must be >= 1 and --warmup >= 0")

    import numpy as np
    import torch
    import ggml_hip as G
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    G.lib()
    if args.suite:
        run_suite(args.suite, torch, G, dev, args.reps, cpu=not args.no_cpu)
        return

    w_bytes = M * q4k_row_bytes(K)
    ncopy = max(4, -(-2 * INFINITY_CACHE // w_bytes))
    gen = torch.Generator().manual_seed(42)
    xg = torch.Generator(device="cpu").manual_seed(43)
    if not args.no_cpu:
        wq_np, x_np, xt_np = reference_inputs(T_MMQ)
        w_host = torch.from_numpy(wq_np)
        weights = [w_host.to(dev) for _ in range(ncopy)]
        x = torch.from_numpy(x_np).to(dev)
        data = (f"synthetic: f32 N(0,0.02) weights from seed 42 quantized with quantize_row_q4_K_ref ({ncopy} "
                "HBM copies of the same bytes), f32 N(0,1) activations from seed 43")
    else:
        weights = [random_q4k(torch, M, K, gen, dev) for _ in range(ncopy)]
        x = torch.randn((1, K), generator=xg, dtype=torch.float32).to(dev)
        xt_np = None
        data = "synthetic: random valid Q4_K blocks (f16 d/dmin at N(0,0.02) scale), N(0,1) f32 activations"
    out = torch.empty((1, M), dtype=torch.float32, device=dev)
    ws = torch.empty(G.workspace_size("Q4_K", K, 1), dtype=torch.uint8, device=dev)
    qs = ws[: G.padded_k(K)].view(torch.int8).view(1, -1)
    ds = ws[G.padded_k(K):].view(torch.int32).view(1, -1)

    def step(i):
        G.mul_mat("Q4_K", weights[i % ncopy], x, out=out, workspace=ws)

    # W untimed warm-up steps, then exactly --steps steps in one HIP graph;
    # the graph is replayed once untimed first (its upload), then timed.
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    graph = capture(torch, step, args.steps)
    warm_up(torch, graph, 1)  # includes the graph's upload
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    del graph

    bytes_alg = w_bytes + K * 4 + M * 4
    value = bytes_alg / (ms_per_step * 1e-3) / 1e9

    # The step's kernel alone (the GEMV with the Q8_1 quantization fused in):
    # n back-to-back launches between two HIP events on the replaying stream
    # (agrees with rocprofv3's per-dispatch average); per-launch event pairs
    # carry ~2 us of event overhead and are reported beside it.  The unfused
    # pair (quantizer + GEMV on the quantized column) is timed for reference.
    n_ev = 8 * ncopy
    fused = lambda i: G.mul_mat_vec_f32("Q4_K", weights[i % ncopy], K, x, out=out)  # noqa: E731
    fused_batch_ms = event_time_batch(torch, fused, n_ev)
    fused_pair_ms, fused_pair_med_ms = event_time_kernel(torch, fused, n_ev)
    gemv = lambda i: G.mul_mat_vec("Q4_K", weights[i % ncopy], K, qs, ds, out=out)  # noqa: E731
    gemv_batch_ms = event_time_batch(torch, gemv, n_ev)
    quant_batch_ms = event_time_batch(
        torch, lambda i: G.lib().hip_qmm_quantize_q8_1_planar(
            G._ptr(x), K, 1, K, G._ptr(qs), G._ptr(ds), G._stream()), n_ev)
    achieved = bytes_alg / (fused_batch_ms * 1e-3) / 1e9
    gpu_out = G.mul_mat("Q4_K", weights[0], x).cpu().numpy()

    # The FFN's gate and up projections of the same shape fused with SWIGLU
    # into one kernel (the GEMV fusion epilogue), beside the three launches it
    # replaces: reported, not the headline metric.
    gates = [random_q4k(torch, M, K, gen, dev) for _ in range(ncopy)]
    g_out = torch.empty((1, M), dtype=torch.float32, device=dev)
    u_out = torch.empty((1, M), dtype=torch.float32, device=dev)

    def ffn_fused(i):
        G.mul_mat_vec_fused("Q4_K", weights[i % ncopy], K, x, w_gate=gates[i % ncopy], glu="SWIGLU", out=out)

    def ffn_unfused(i):
        G.mul_mat_vec_f32("Q4_K", weights[i % ncopy], K, x, out=u_out)
        G.mul_mat_vec_f32("Q4_K", gates[i % ncopy], K, x, out=g_out)
        G.glu_f32(g_out, u_out, "SWIGLU", out=out)

    ffn_fused_ms = event_time_batch(torch, ffn_fused, n_ev)
    ffn_unfused_ms = event_time_batch(torch, ffn_unfused, n_ev)
    ffn_bytes = 2 * w_bytes + K * 4 + M * 4
    del gates

    result = {
        "metric": "Q4_K GEMV GB/s (% HBM peak) @14336x4096 b=1; MMQ int8 TOPS @b=512",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot products, fp32 epilogue (Q4_K weights x Q8_1 activations)",
        "data": data,
        "config": {"workload": "Llama-3-8B ffn_gate/up Q4_K decode GEMV (config 1)", "rows": M, "K": K,
                   "batch": 1, "weight_copies": ncopy,
                   "step": "mul_mat: GEMV with the Q8_1 quantization fused (one kernel)",
                   "timed": f"one HIP-graph replay of exactly {args.steps} steps between synchronizes; untimed "
                            f"before it: {args.warmup} warm-up steps, then replays of the same graph (its upload "
                            f"first) for at least {WARM_S * 1e3:.0f} ms"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": bytes_alg,
                     "kernel": "gemv_fx_kernel<Q4_K, 14 waves (2 workgroups per CU), 2 rows per wave> (quantize-in-GEMV)",
                     "avg_us": round(fused_batch_ms * 1e3, 3),
                     "timing": f"HIP graph of {n_ev} launches, weights rotated over {ncopy} copies; untimed "
                               f"replays for at least {WARM_S * 1e3:.0f} ms, then the mean of 3 replays each between "
                               "HIP events",
                     "event_pair_avg_us": round(fused_pair_ms * 1e3, 3),
                     "event_pair_median_us": round(fused_pair_med_ms * 1e3, 3),
                     "unfused_gemv_avg_us": round(gemv_batch_ms * 1e3, 3),
                     "unfused_quantize_avg_us": round(quant_batch_ms * 1e3, 3)},
        "ffn_gate_up_swiglu": {"shape": f"2 x {M}x{K} Q4_K, b=1",
                               "fused_us": round(ffn_fused_ms * 1e3, 3),
                               "fused_GBps": round(ffn_bytes / (ffn_fused_ms * 1e-3) / 1e9, 1),
                               "unfused_3_launches_us": round(ffn_unfused_ms * 1e3, 3)},
    }

    gpu_mmq_out = None
    if not args.no_mmq:
        if xt_np is not None:
            xt = torch.from_numpy(xt_np).to(dev)
        else:
            xt = torch.randn((T_MMQ, K), generator=xg, dtype=torch.float32).to(dev)
        qst, dst_ = G.quantize_q8_1_planar(xt)
        outt = torch.empty((T_MMQ, M), dtype=torch.float32, device=dev)
        n_m = 2 * ncopy
        mmq = lambda i: G.mmq("Q4_K", weights[i % ncopy], K, qst, dst_, out=outt)  # noqa: E731
        mmq_avg_ms, mmq_reps = event_time_replays(torch, mmq, n_m)
        _, mmq_med_ms = event_time_kernel(torch, mmq, n_m)
        wst = torch.empty(G.workspace_size("Q4_K", K, T_MMQ, M), dtype=torch.uint8, device=dev)
        op = lambda i: G.mul_mat("Q4_K", weights[i % ncopy], xt, out=outt, workspace=wst)  # noqa: E731
        op_avg_ms, op_reps = event_time_replays(torch, op, n_m)
        gpu_mmq_out = G.mul_mat("Q4_K", weights[0], xt).cpu().numpy()
        ops = 2.0 * M * K * T_MMQ
        tops = ops / (mmq_avg_ms * 1e-3) / 1e12
        result["mmq"] = {
            "workload": f"Q4_K {M}x{K} x T={T_MMQ} (config 2)", "tops": round(tops, 2), "peak_tops": INT8_PEAK_TOPS,
            "frac": round(tops / INT8_PEAK_TOPS, 4), "avg_us": round(mmq_avg_ms * 1e3, 2),
            "event_pair_median_us": round(mmq_med_ms * 1e3, 2),
            "replays_us": [round(v * 1e3, 2) for v in mmq_reps],
            "op_avg_us": round(op_avg_ms * 1e3, 2),
            "op_replays_us": [round(v * 1e3, 2) for v in op_reps],
            "op": "mul_mat on f32 columns: Q8_1 quantizer + the MMQ",
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                         "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None,
                         "algorithmic_ops": ops, "algorithmic_bytes_read": w_bytes + T_MMQ * (G.padded_k(K) * 9 // 8),
                         "kernel": "mmq_q4k_dma_kernel (int8 MFMA, direct-to-LDS staging)",
                         "timing": f"HIP graph of {n_m} launches, weights rotated over {ncopy} copies; untimed "
                                   f"replays for at least {WARM_S * 1e3:.0f} ms, then the mean of 5 replays each "
                                   "between HIP events"},
        }

    if not args.no_traffic:
        traffic, cal = measure_traffic()
        if traffic:
            result["roofline"]["traffic"] = traffic["gemv"]
            result["roofline"]["traffic_ratio"] = round(traffic["gemv"] / bytes_alg, 4)
            result["roofline"]["traffic_source"] = {"method": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over "
                                                              "bench.py --traffic-probe, in this run", **cal}
            if "mmq" in result:
                rf = result["mmq"]["roofline"]
                rf["traffic"] = traffic["mmq"]
                rf["traffic_ratio_to_reads"] = round(traffic["mmq"] / (rf["algorithmic_bytes_read"] + T_MMQ * M * 4), 4)
        else:
            result["roofline"]["traffic_source"] = f"not measured: {cal}"

    if not args.no_cpu:
        base, par = cpu_gemv_leg(wq_np, x_np, gpu_out)
        result["cpu_baseline"] = base
        result["parity"] = {"op": f"mul_mat Q4_K {M}x{K} b=1, GPU against the CPU baseline's own result", **par}
        if gpu_mmq_out is not None:
            mbase, mpar = cpu_mmq_leg(wq_np, xt_np, gpu_mmq_out)
            result["mmq"]["cpu_baseline"] = mbase
            result["mmq"]["parity"] = {"op": f"mul_mat Q4_K {M}x{K} x T={T_MMQ}, GPU against the CPU baseline's "
                                             "own result", **mpar}

    print(json.dumps(result))


if __name__ == "__main__":
    main()
