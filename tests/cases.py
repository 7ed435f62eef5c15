"""Seeded synthetic cases shared by the GPU tests (test infrastructure).

Weights are f32 N(0, 0.02) quantized with the oracle's restatement of the
reference quantizers (quantize_row_*_ref); activations f32 N(0, 1); seeds:
weights 42, activations 43, router logits 44 (each tensor offset by an index).
"""
import functools

import numpy as np

import oracle_lib as O

SEED_W, SEED_X, SEED_ROUTER = 42, 43, 44


@functools.lru_cache(maxsize=16)
def weights_f32(nrows, K, idx=0):
    return O.fill_normal(SEED_W + 1000 * idx, nrows * K, 0.0, 0.02).reshape(nrows, K)


@functools.lru_cache(maxsize=16)
def weights_q(t, nrows, K, idx=0):
    q = O.quantize_rows(t, weights_f32(nrows, K, idx))
    q.setflags(write=False)
    return q


@functools.lru_cache(maxsize=16)
def acts(ncols, K, idx=0):
    x = O.fill_normal(SEED_X + 1000 * idx, ncols * K, 0.0, 1.0).reshape(ncols, K)
    x.setflags(write=False)
    return x


def nmse(got, want):
    """sum (got - want)^2 / sum want^2 (harness/blas_diff.c:341-350)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = float(np.sum(want * want))
    return float(np.sum((got - want) ** 2)) / (den if den > 0 else 1.0)


def max_rel(got, want, floor=1e-3):
    """Largest |got - want| / max(|want|, floor * max|want|): relative error,
    with outputs that cancel to near zero judged against the output scale."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = np.maximum(np.abs(want), floor * float(np.max(np.abs(want))))
    return float(np.max(np.abs(got - want) / scale))


def max_err_scaled(got, want):
    """max |got - want| / max |want|: the f64-agreement measure."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))


def route_top_k(n_tokens, n_experts, k, seed=SEED_ROUTER):
    """Softmax over seeded N(0,1) router logits, top-k experts per token
    (the ids of ggml's argsort_top_k, src/llama/graph.zig:3265-3318), and the
    renormalised weights (norm_w, graph.zig:3343-3362)."""
    logits = O.fill_normal(seed, n_tokens * n_experts).reshape(n_tokens, n_experts).astype(np.float64)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(p, ids, axis=1)
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def mul_mat_id_f64(t, wq_experts, nrows, K, y_q8_1_rows, ne11, ids):
    """f64 evaluation of the GPU's Q8_1 formula for mul_mat_id, expert by expert.
    y_q8_1_rows: AoS Q8_1 blocks of every activation row (n_tokens*ne11 rows)."""
    n_tokens, n_ids = ids.shape
    out = np.zeros((n_tokens, n_ids, nrows))
    rb = y_q8_1_rows.shape[1]
    for e in np.unique(ids[ids >= 0]):
        ts, ss = np.nonzero(ids == e)
        cols = np.stack([y_q8_1_rows[t * ne11 + s % ne11] for t, s in zip(ts, ss)]).reshape(len(ts), rb)
        res = O.mul_mat_q8_1_f64(t, wq_experts[e], nrows, K, cols, len(ts))
        out[ts, ss] = res
    return out
