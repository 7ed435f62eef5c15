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
