"""CPU oracle for the linear leaf models (TEST INFRASTRUCTURE ONLY).

Restates, in numpy float64, the per-leaf ridge fit of the reference's
`_fit_linear` (yabt/neural_leaves.py:42-90), the per-leaf counts and raw-input
envelopes of `fit_leaf_networks` (yabt/neural_leaves.py:157-176) and the fold
into raw space (yabt/neural_leaves.py:178-184).  Only tests/ use it, as the
reference the HIP kernels are compared against.

Pinned by tests/test_neural_oracle.py: the normal equations against an
independent least-squares solve of the same objective, eligibility rules,
envelopes against brute force, and the fold against direct evaluation.
"""

from __future__ import annotations

import numpy as np


def counts(leaf: np.ndarray, n_nodes: int) -> np.ndarray:
    return np.bincount(leaf, minlength=n_nodes).astype(np.int64)


def envelopes(Xs: np.ndarray, leaf: np.ndarray, n_nodes: int):
    """Per-node min / max of the raw inputs, +inf / -inf for empty nodes
    (scatter_reduce amin / amax with include_self, neural_leaves.py:170-176).
    Rows grouped by node (a stable sort), then one min and one max per run."""
    K = Xs.shape[1]
    lo = np.full((n_nodes, K), np.inf, np.float32)
    hi = np.full((n_nodes, K), -np.inf, np.float32)
    if leaf.size == 0:
        return lo, hi
    order = np.argsort(leaf, kind="stable")
    sl = leaf[order]
    starts = np.concatenate([[0], np.nonzero(np.diff(sl))[0] + 1])
    Xo = Xs.astype(np.float32)[order]
    lo[sl[starts]] = np.minimum.reduceat(Xo, starts, axis=0)
    hi[sl[starts]] = np.maximum.reduceat(Xo, starts, axis=0)
    return lo, hi


def moments(Xs: np.ndarray):
    """Mean and unbiased std clamped at 1e-6 (neural_leaves.py:152-154), in
    float64, rounded to float32."""
    X = Xs.astype(np.float64)
    mu = X.mean(axis=0)
    sd = X.std(axis=0, ddof=1)
    return mu.astype(np.float32), np.maximum(sd.astype(np.float32), np.float32(1e-6))


def standardise(Xs: np.ndarray, mu: np.ndarray, sd: np.ndarray) -> np.ndarray:
    """(Xs - mu) / sd in float32 (neural_leaves.py:152-155)."""
    return ((Xs.astype(np.float32) - mu.astype(np.float32)) / sd.astype(np.float32)).astype(np.float32)


def gram(Xn: np.ndarray, g: np.ndarray, h: np.ndarray, leaf: np.ndarray, n_nodes: int):
    """M[l] = sum h x1 x1^T, b[l] = -sum g x1 with x1 = [Xn, 1] in float64
    (neural_leaves.py:66-83)."""
    n, K = Xn.shape
    X1 = np.concatenate([Xn.astype(np.float64), np.ones((n, 1))], axis=1)
    Xh = X1 * h.astype(np.float64)[:, None]
    rhs = -(X1 * g.astype(np.float64)[:, None])
    M = np.zeros((n_nodes, K + 1, K + 1))
    b = np.zeros((n_nodes, K + 1))
    # every entry is a float64 sum over the node's rows in row order
    # (bincount adds its weights in input order)
    for i in range(K + 1):
        for j in range(i, K + 1):
            M[:, i, j] = np.bincount(leaf, weights=X1[:, i] * Xh[:, j], minlength=n_nodes)
            M[:, j, i] = M[:, i, j] if i == j else np.bincount(leaf, weights=X1[:, j] * Xh[:, i],
                                                                 minlength=n_nodes)
        b[:, i] = np.bincount(leaf, weights=rhs[:, i], minlength=n_nodes)
    return M, b


def fit_linear(Xn, g, h, leaf, eligible, n_nodes, lam):
    """(W (n_nodes, K), db (n_nodes)) float32, zero where not eligible
    (neural_leaves.py:42-90)."""
    K = Xn.shape[1]
    W = np.zeros((n_nodes, K), np.float32)
    db = np.zeros(n_nodes, np.float32)
    elig = np.nonzero(eligible)[0]
    if elig.size == 0:
        return W, db
    M, b = gram(Xn, g, h, leaf, n_nodes)
    reg = np.eye(K + 1) * lam
    reg[K, K] = 1e-8  # the bias is not penalised
    theta = np.linalg.solve(M[elig] + reg, b[elig][:, :, None])[:, :, 0].astype(np.float32)
    W[elig] = theta[:, :K]
    db[elig] = theta[:, K]
    return W, db


def eligible_nodes(feature: np.ndarray, cnt: np.ndarray, min_samples: int) -> np.ndarray:
    """Leaves with at least min_samples rows (neural_leaves.py:157-161)."""
    return (feature == -1) & (cnt >= min_samples)


def fold(value, W, db, mu, sd, lr):
    """value + lr (db - W . mu/sd) and lr W / sd in float32 (neural_leaves.py:181-184)."""
    mu, sd = mu.astype(np.float32), sd.astype(np.float32)
    value = (value.astype(np.float32) + np.float32(lr) * (db - (W * (mu / sd)).sum(axis=1))).astype(np.float32)
    return value, (np.float32(lr) * W / sd).astype(np.float32)
