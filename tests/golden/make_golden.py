"""Write the golden fixtures of tests/golden/ from the reference grow.c.

Runs the reference's own `cgrow` and `capply` (yabt/_cgrow/grow.c, compiled
from the reference sources into oracle/_ref/libgrow_ref.so by
``make -C oracle ref``) on small seeded inputs and stores inputs and outputs
as .npz files.  Needs the reference sources, so it runs only where they are
mounted; the fixtures it writes are what the test suite reads.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def sparse_layout(bins_nf: np.ndarray):
    """CSR of the cells that differ from their column's most frequent bin
    (lowest bin on ties), row-major; the layout cgrow's sparse path reads
    (grow.c:68-107)."""
    n, F = bins_nf.shape
    default = np.array([np.bincount(bins_nf[:, f], minlength=256).argmax() for f in range(F)],
                       dtype=np.int32)
    mask = bins_nf != default[None, :]
    indptr = np.concatenate([[0], np.cumsum(mask.sum(axis=1))]).astype(np.int64)
    r, c = np.nonzero(mask)
    return indptr, c.astype(np.int32), bins_nf[r, c].astype(np.int32), default


def quantile_bins(X: np.ndarray, max_bins: int):
    """Quantile edges and codes with the reference binner's semantics
    (binning.py:53-66, 97-112): float32 unique linear quantiles, bin = #{e < x}."""
    qs = np.linspace(0, 1, max_bins + 1)[1:-1]
    edges = [np.unique(np.quantile(X[:, f], qs).astype(np.float32)) for f in range(X.shape[1])]
    bins = np.stack([np.searchsorted(e, X[:, f], side="left") for f, e in enumerate(edges)], 1)
    nbins = np.array([min(len(e) + 1, 256) for e in edges], np.int32)
    return bins.astype(np.uint8), edges, nbins


def case(name, rng, n, F, *, source="uniform", nb=256, kind="regression", sparse=False,
         imat=False, fmask=False, **params):
    if source == "uniform":
        bins = rng.integers(0, nb, size=(n, F)).astype(np.uint8)
        nbins = np.full(F, nb, np.int32)
        X = None
    elif source == "quantile":
        X = rng.normal(size=(n, F)).astype(np.float32)
        bins, edges, nbins = quantile_bins(X, nb)
    elif source == "sparse_x":
        X = np.zeros((n, F), np.float32)
        m = rng.random((n, F)) < 0.1
        X[m] = rng.normal(size=int(m.sum())).astype(np.float32)
        bins, edges, nbins = quantile_bins(X, nb)
    elif source == "skewed":
        bins = rng.integers(1, 256, size=(n, F)).astype(np.uint8)
        bins[rng.random((n, F)) < 0.9] = 0
        nbins = np.full(F, 256, np.int32)
        X = None
    else:
        raise ValueError(source)
    if kind == "regression":
        y = rng.normal(size=n).astype(np.float32)
        if X is not None:
            y = (X[:, 0] + 0.5 * X[:, 1 % F] * X[:, 2 % F] + 0.1 * y).astype(np.float32)
        grad = (y - y.mean()).astype(np.float32)
        hess = np.ones(n, np.float32)
    elif kind == "logistic":
        p = 1 / (1 + np.exp(-rng.normal(size=n)))
        yb = (rng.random(n) < p).astype(np.float32)
        pr = np.full(n, 0.5, np.float32)
        grad = (pr - yb).astype(np.float32)
        hess = np.maximum(pr * (1 - pr), 1e-6).astype(np.float32)
    else:  # "random"
        grad = rng.normal(size=n).astype(np.float32)
        hess = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
    kw = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=31, max_depth=64)
    kw.update(params)
    extra = {}
    if imat:
        extra["imat"] = rng.random((F, F)).astype(np.float32)
        extra["ib"] = 0.5
    if fmask:
        extra["fmask"] = (rng.random(F) < 0.6).astype(np.uint8)
    sl = sparse_layout(bins) if sparse else None
    out = O.grow(bins.T, grad, hess, reference=True, sparse=sl, nbins=nbins, n_threads=2,
                 **extra, **kw)
    blob = dict(bins_fm=np.ascontiguousarray(bins.T), grad=grad, hess=hess, nbins=nbins,
                params=np.array([kw["lam"], kw["gamma"], kw["mcw"], kw["msl"], kw["lr"],
                                 kw["max_leaves"], kw["max_depth"]], np.float64))
    for k in ("imat", "fmask"):
        if k in extra:
            blob[k] = extra[k]
    if imat:
        blob["ib"] = np.float32(extra["ib"])
    if sl is not None:
        blob.update(sp_indptr=sl[0], sp_indices=sl[1], sp_data=sl[2], sp_default=sl[3])
    for k in ("feature", "thr_bin", "left", "right", "value", "depth"):
        blob["out_" + k] = out[k]
    if X is not None:
        # routing fixture: the reference capply on the raw features
        thr = np.zeros(out["n_nodes"], np.float32)
        for nid in np.nonzero(out["feature"] >= 0)[0]:
            e = edges[out["feature"][nid]]
            thr[nid] = e[min(out["thr_bin"][nid], len(e) - 1)]
        Xq = rng.normal(size=(min(n, 500), F)).astype(np.float32) * 1.5
        blob.update(apply_X=Xq, apply_threshold=thr,
                    apply_out=O.apply(Xq, out["feature"], thr, out["left"], out["right"],
                                      reference=True))
    np.savez_compressed(os.path.join(HERE, f"grow_{name}.npz"), **blob)
    print(f"{name}: n={n} F={F} nodes={out['n_nodes']}")


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libgrow_ref.so missing: run `make -C oracle ref` first")
    rng = np.random.default_rng(20260101)
    case("dense_regression", rng, 3000, 12, source="quantile")
    case("dense_random", rng, 4000, 9, kind="random")
    case("params", rng, 2500, 7, kind="random", nb=60, lam=0.0, gamma=0.05, mcw=0.5, msl=5,
         lr=0.3, max_leaves=40, max_depth=4)
    case("interaction", rng, 3000, 12, source="quantile", imat=True)
    case("feature_mask", rng, 2000, 10, source="quantile", fmask=True, max_leaves=16)
    case("sparse", rng, 3000, 40, source="sparse_x", sparse=True)
    case("logistic_depth8", rng, 5000, 8, source="quantile", nb=28, kind="logistic",
         max_leaves=256, max_depth=8, msl=1)
    case("skewed_depth6", rng, 6000, 25, source="skewed", kind="random", max_leaves=64,
         max_depth=6)
    case("one_leaf", rng, 500, 4, kind="random", max_leaves=1)
    case("two_leaves", rng, 500, 4, kind="random", max_leaves=2)
    case("tiny", rng, 5, 2, kind="random", msl=1, max_leaves=8)
    case("root_depth0", rng, 300, 3, kind="random", max_depth=0)


if __name__ == "__main__":
    main()
