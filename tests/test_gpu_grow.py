"""Whole-tree parity of yabt_grow and yabt_grow_batched (growth "rounds").

* against the oracle's fixed-point mode: bit-identical node arrays (feature,
  thr_bin, left, right, depth, value bits) and identical per-row leaf ids;
* against the reference arithmetic (oracle fp32 mode, itself pinned to the
  compiled reference grow.c by tests/golden): identical feature sequence and
  leaf membership; thr_bin equal or differing only across bins that are empty
  in that node; leaf values within 1e-5;
* with outliers and heavy-tailed squared-loss gradients, which select the wide
  contract: the same against the reference, its leaf values within
  1e-5 max(1, |ref|) of the reference's beyond the reference's own distance
  from the values of the exact (fp64) sums, and within 1e-6 max(1, |v|) of
  those.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import WIDE_KINDS, empty_between, grad_hess, skewed_bins, tree_arrays_equal, uniform_bins
from yabt_amd import IdentityBinner, TreeParams, grow_tree_hip
from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _grow_gpu(bins, g, h, nbins, **kw):
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    res = G.grow_device(lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV), nbins, **kw)
    out = {k: getattr(res, k).cpu().numpy() for k in
           ("feature", "thr_bin", "left", "right", "value", "depth")}
    leaf = G.leaf_ids(res, bins.shape[0], bins.shape[1], kw.get("max_leaves", 31)).cpu().numpy()
    res._keep = None
    return out, leaf


CASES = [
    dict(n=3000, F=12, nb=256, kind="normal", max_leaves=31),
    dict(n=20_000, F=20, nb=255, kind="normal", max_leaves=31, imat=True),
    dict(n=5000, F=9, nb=28, kind="logistic", max_leaves=256, max_depth=8, msl=1),
    dict(n=8000, F=40, nb=256, kind="laplace", max_leaves=64, max_depth=6, skew=True),
    dict(n=4000, F=17, nb=64, kind="normal", max_leaves=63, fmask=True, lam=0.0, gamma=0.05),
    dict(n=1, F=1, nb=256, kind="normal", max_leaves=31, msl=0),
    dict(n=100, F=3, nb=256, kind="normal", max_leaves=1),
    dict(n=50_000, F=30, nb=256, kind="normal", max_leaves=255, msl=20),
    # n > 2^18: packed root histogram, three channels and constant hessian
    dict(n=400_000, F=9, nb=256, kind="normal", max_leaves=63, msl=20),
    dict(n=400_000, F=9, nb=64, kind="laplace", max_leaves=63, msl=20),
    # a 4-feature tail tile of the root (F % 16 = 4), odd n, constant hessian
    dict(n=300_001, F=20, nb=256, kind="laplace", max_leaves=31, msl=20, skew=True),
]


@pytest.mark.parametrize("growth", ["sequential", "rounds"])
@pytest.mark.parametrize("dflt", ["auto", None, "modal"], ids=["skip-auto", "no-skip", "skip-every-feature"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"n{c['n']}F{c['F']}L{c['max_leaves']}")
def test_grow_matches_oracle(case, dflt, growth):
    print(f"case {case} default_bin {dflt} growth {growth}", flush=True)
    c = dict(case)
    n, F, nb = c.pop("n"), c.pop("F"), c.pop("nb")
    rng = np.random.default_rng(n * 31 + F)
    bins = skewed_bins(rng, n, F) if c.pop("skew", False) else uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n, c.pop("kind"))
    kw = dict(max_leaves=c.pop("max_leaves"), max_depth=c.pop("max_depth", 64),
              msl=c.pop("msl", 20), lam=c.pop("lam", 1.0), gamma=c.pop("gamma", 0.0),
              mcw=1e-3, lr=0.1)
    if c.pop("imat", False):
        kw["imat"] = rng.random((F, F)).astype(np.float32)
        kw["ib"] = 0.5
    if c.pop("fmask", False):
        kw["fmask"] = rng.random(F) < 0.7
    assert not c
    nbins = np.full(F, nb, np.int32)
    if dflt == "modal":   # skip each feature's most frequent bin, however rare
        dflt = np.array([np.bincount(bins[:, f], minlength=256).argmax() for f in range(F)], np.int32)
    got, leaf = _grow_gpu(bins, g, h, nbins, default_bin=dflt, growth=growth, **kw)
    ref = O.grow(bins.T, g, h, mode=O.MODE_FIXED, nbins=nbins, **kw)
    bad = tree_arrays_equal(got, ref)
    assert bad is None, f"{bad} differs from the fixed-point oracle"
    assert np.array_equal(leaf, O.leaf_of_rows(ref, n))

    # against the reference arithmetic
    r32 = O.grow(bins.T, g, h, mode=O.MODE_FP32, nbins=nbins, **kw)
    assert np.array_equal(got["feature"], r32["feature"])
    assert np.array_equal(leaf, O.leaf_of_rows(r32, n))
    assert np.abs(got["value"] - r32["value"]).max(initial=0) <= 1e-5
    for nid in np.nonzero(got["feature"] >= 0)[0]:
        if got["thr_bin"][nid] != r32["thr_bin"][nid]:
            rows = ref["rows"][ref["seg_lo"][nid]:ref["seg_hi"][nid]]
            f = got["feature"][nid]
            counts = np.bincount(bins[rows, f], minlength=256)
            assert empty_between(counts, got["thr_bin"][nid], r32["thr_bin"][nid])


def test_grow_tree_hip_dropin():
    """grow_tree_c's signature and Tree output (grow_c.py:336-452)."""
    rng = np.random.default_rng(5)
    n, F = 6000, 10
    bins = uniform_bins(rng, n, F, 100)
    g, h = grad_hess(rng, n)
    binner = IdentityBinner(F, 100)
    tp = TreeParams(max_leaves=24, min_samples_leaf=10)
    tree = grow_tree_hip(torch.from_numpy(bins), torch.from_numpy(g), torch.from_numpy(h),
                         binner, tp)
    assert tree.feature.device.type == "cpu"
    ref = O.grow(bins.T, g, h, mode=O.MODE_FIXED, nbins=np.full(F, 100, np.int32),
                 max_leaves=24, msl=10)
    assert np.array_equal(tree.feature.numpy(), ref["feature"])
    internal = ref["feature"] >= 0
    assert np.array_equal(tree.threshold.numpy()[internal], ref["thr_bin"][internal].astype(np.float32))
    assert tree.depth == int(ref["depth"].max()) + 1
    assert np.array_equal(tree.apply(torch.from_numpy(bins.astype(np.float32))).numpy(),
                          O.leaf_of_rows(ref, n))


@pytest.mark.parametrize("growth", ["sequential", "rounds"])
def test_grow_rejects_nonfinite(growth):
    rng = np.random.default_rng(1)
    n, F = 100, 3
    bins = uniform_bins(rng, n, F)
    g, h = grad_hess(rng, n)
    g[7] = np.nan
    with pytest.raises(ValueError):
        _grow_gpu(bins, g, h, np.full(F, 256, np.int32), max_leaves=4, growth=growth)


WIDE_TREES = [dict(n=200_000, F=10, kind=k, max_leaves=31) for k in
              ("outlier1e3", "outlier1e5", "lognormal2", "lognormal3", "studentt", "cauchy", "studentt_h",
               "cauchy_h")]
WIDE_TREES += [dict(n=50_000, F=24, kind="lognormal3_h", max_leaves=255),
               dict(n=600_000, F=20, kind="cauchy", max_leaves=64, max_depth=6)]


@pytest.mark.parametrize("growth", ["sequential", "rounds"])
@pytest.mark.parametrize("case", WIDE_TREES, ids=lambda c: f"{c['kind']}-n{c['n']}L{c['max_leaves']}")
def test_grow_wide_contract_vs_reference(case, growth):
    """Outliers and heavy-tailed squared-loss targets (boosting.py:52-54: g is
    unbounded) would make the narrow 19-bit quantum coarse against most rows;
    the per-call residual test selects the wide contract, and the tree is
    the fixed-point oracle's bit for bit and the reference's: same features,
    same leaf membership, thresholds equal or across empty bins, and leaf
    values that the reference's own fp32 rounding alone separates."""
    print(f"wide case {case} growth {growth}", flush=True)
    c = dict(case)
    n, F, kind = c.pop("n"), c.pop("F"), c.pop("kind")
    rng = np.random.default_rng(n + F + len(kind))
    bins = uniform_bins(rng, n, F)
    g, h = grad_hess(rng, n, kind)
    assert O.hist_contract(g, h)[2] == 1 and kind in WIDE_KINDS
    kw = dict(max_leaves=c.pop("max_leaves"), max_depth=c.pop("max_depth", 64), msl=20, lam=1.0, gamma=0.0,
              mcw=1e-3, lr=0.1)
    assert not c
    nbins = np.full(F, 256, np.int32)
    got, leaf = _grow_gpu(bins, g, h, nbins, default_bin="auto", growth=growth, **kw)
    ref = O.grow(bins.T, g, h, mode=O.MODE_FIXED, nbins=nbins, **kw)
    bad = tree_arrays_equal(got, ref)
    assert bad is None, f"{bad} differs from the fixed-point oracle"
    assert np.array_equal(leaf, O.leaf_of_rows(ref, n))

    r32 = O.grow(bins.T, g, h, mode=O.MODE_FP32, nbins=nbins, **kw)
    assert np.array_equal(got["feature"], r32["feature"])
    assert np.array_equal(leaf, O.leaf_of_rows(r32, n))
    for nid in np.nonzero(got["feature"] >= 0)[0]:
        if got["thr_bin"][nid] != r32["thr_bin"][nid]:
            rows = ref["rows"][ref["seg_lo"][nid]:ref["seg_hi"][nid]]
            counts = np.bincount(bins[rows, got["feature"][nid]], minlength=256)
            assert empty_between(counts, got["thr_bin"][nid], r32["thr_bin"][nid])
    # leaf values: the exact values of each leaf's rows (fp64 sums), the
    # reference's distance from them, and ours
    leaves = np.nonzero(got["feature"] == -1)[0]
    G64 = np.bincount(leaf, weights=g.astype(np.float64), minlength=len(got["feature"]))
    H64 = np.bincount(leaf, weights=h.astype(np.float64), minlength=len(got["feature"]))
    truth = (-np.float64(np.float32(0.1)) * G64 / (H64 + 1.0))[leaves]
    ours = got["value"][leaves].astype(np.float64)
    theirs = r32["value"][leaves].astype(np.float64)
    scale_t = np.maximum(1.0, np.abs(truth))
    assert (np.abs(ours - truth) <= 1e-6 * scale_t).all()
    assert (np.abs(ours - theirs) <= 1e-5 * np.maximum(1.0, np.abs(theirs)) + np.abs(theirs - truth)).all()
