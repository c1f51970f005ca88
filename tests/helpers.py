"""Shared input generators and comparison helpers for the test suite."""

from __future__ import annotations

import numpy as np


def uniform_bins(rng, n, F, nb=256):
    return rng.integers(0, nb, size=(n, F)).astype(np.uint8)


def skewed_bins(rng, n, F, p_zero=0.9):
    """Each column: bin 0 with probability p_zero, else uniform on 1..255."""
    b = rng.integers(1, 256, size=(n, F)).astype(np.uint8)
    b[rng.random((n, F)) < p_zero] = 0
    return b


def grad_hess(rng, n, kind="normal"):
    if kind == "normal":
        g = rng.normal(size=n).astype(np.float32)
        h = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
    elif kind == "laplace":
        g = rng.laplace(size=n).astype(np.float32)
        h = np.ones(n, np.float32)
    elif kind == "logistic":
        y = (rng.random(n) < 0.5).astype(np.float32)
        p = np.full(n, 0.5, np.float32)
        g = (p - y).astype(np.float32)
        h = np.maximum(p * (1 - p), 1e-6).astype(np.float32)
    elif kind.startswith("outlier"):
        # N(0,1) gradients with one large value: "outlier" 50, "outlier1e3", "outlier1e5"
        g = rng.normal(size=n).astype(np.float32)
        g[n // 3] = float(kind[len("outlier"):] or 50)
        h = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
    elif kind.split("_")[0] in ("lognormal2", "lognormal3", "studentt", "cauchy"):
        # squared-loss gradients g = m - y at the mean (the base score) of a
        # heavy-tailed target (boosting.py:49-54), h = 1, or U(0.1, 1) with "_h"
        base = kind.split("_")[0]
        if base.startswith("lognormal"):
            y = rng.lognormal(0.0, float(base[-1]), size=n)
        elif base == "studentt":
            y = rng.standard_t(1.5, size=n)
        else:
            y = rng.standard_cauchy(size=n)
        y = y.astype(np.float32)
        g = (np.float32(y.astype(np.float64).mean()) - y).astype(np.float32)
        h = (rng.uniform(0.1, 1.0, size=n).astype(np.float32) if kind.endswith("_h")
             else np.ones(n, np.float32))
    else:
        raise ValueError(kind)
    return g, h


# Input kinds whose quantisation residual at the narrow shift selects the
# wide contract (tests check that the oracle agrees).
WIDE_KINDS = ("outlier", "outlier1e3", "outlier1e5", "lognormal2", "lognormal3", "studentt", "cauchy",
              "lognormal3_h", "studentt_h", "cauchy_h")


def normwise_rel(a, b):
    """max|a-b| / max|b|, the reference's histogram metric (test_cuda_hist.py:42-45)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def dequantise(qhist, sg, sh):
    """(3,F,256) int64 fixed point -> float64 (g, h, count)."""
    out = np.empty(qhist.shape, np.float64)
    out[0] = qhist[0].astype(np.float64) * 2.0 ** -sg
    out[1] = qhist[1].astype(np.float64) * 2.0 ** -sh
    out[2] = qhist[2]
    return out


def tree_arrays_equal(a: dict, b: dict, value_bits=True):
    """Exact equality of two trees' node arrays; returns the first mismatch name."""
    for k in ("feature", "thr_bin", "left", "right", "depth"):
        if not np.array_equal(np.asarray(a[k]), np.asarray(b[k])):
            return k
    va, vb = np.asarray(a["value"], np.float32), np.asarray(b["value"], np.float32)
    if value_bits and not np.array_equal(va.view(np.uint32), vb.view(np.uint32)):
        return "value"
    return None


def empty_between(counts_f, b1, b2):
    """True if bins (min(b1,b2), max(b1,b2)] hold no rows in a node whose
    per-bin counts of the split feature are counts_f."""
    lo, hi = sorted((int(b1), int(b2)))
    return int(np.asarray(counts_f)[lo + 1:hi + 1].sum()) == 0
