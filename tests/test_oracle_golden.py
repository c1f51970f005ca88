"""The CPU oracle against the reference's own outputs (tests/golden/*.npz,
written by tests/golden/make_golden.py from the compiled reference grow.c).

* OR_MODE_FP32 must reproduce cgrow bit-for-bit (node arrays and value bits),
  including the sparse builder, interaction steering, feature masks, depth
  caps and the degenerate 1/2-leaf and tiny inputs.
* OR_MODE_FIXED (the HIP path's arithmetic) must agree with the reference on
  the split features and leaf membership, pick thresholds that differ only
  across bins that are empty in the node, and give values within 1e-5.
* The oracle's routing must reproduce the reference capply.
"""

import glob
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import empty_between, tree_arrays_equal

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "grow_*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _kwargs(d):
    lam, gamma, mcw, msl, lr, L, depth = d["params"]
    kw = dict(lam=float(lam), gamma=float(gamma), mcw=float(mcw), msl=int(msl), lr=float(lr),
              max_leaves=int(L), max_depth=int(depth), nbins=d["nbins"])
    if "imat" in d:
        kw["imat"] = d["imat"]
        kw["ib"] = float(d["ib"])
    if "fmask" in d:
        kw["fmask"] = d["fmask"]
    if "sp_indptr" in d:
        kw["sparse"] = (d["sp_indptr"], d["sp_indices"], d["sp_data"], d["sp_default"])
    return kw


def _expected(d):
    return {k[4:]: d[k] for k in d if k.startswith("out_")}


def test_fixtures_present():
    assert len(FIXTURES) >= 10


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
@pytest.mark.parametrize("threads", [1, 3])
def test_fp32_oracle_is_the_reference(path, threads):
    d = _load(path)
    got = O.grow(d["bins_fm"], d["grad"], d["hess"], mode=O.MODE_FP32, n_threads=threads, **_kwargs(d))
    assert tree_arrays_equal(got, _expected(d)) is None


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_fixed_oracle_vs_reference(path):
    d = _load(path)
    kw = _kwargs(d)
    ref = _expected(d)
    fx = O.grow(d["bins_fm"], d["grad"], d["hess"], mode=O.MODE_FIXED, **kw)
    f32 = O.grow(d["bins_fm"], d["grad"], d["hess"], mode=O.MODE_FP32, **kw)
    n = d["grad"].shape[0]
    assert np.array_equal(fx["feature"], ref["feature"])
    assert np.array_equal(fx["left"], ref["left"]) and np.array_equal(fx["right"], ref["right"])
    assert np.array_equal(fx["depth"], ref["depth"])
    assert np.array_equal(O.leaf_of_rows(fx, n), O.leaf_of_rows(f32, n))
    assert np.abs(fx["value"] - ref["value"]).max() <= 1e-5
    bins = d["bins_fm"]
    for nid in np.nonzero(fx["feature"] >= 0)[0]:
        if fx["thr_bin"][nid] != ref["thr_bin"][nid]:
            rows = fx["rows"][fx["seg_lo"][nid]:fx["seg_hi"][nid]]
            counts = np.bincount(bins[fx["feature"][nid], rows], minlength=256)
            assert empty_between(counts, fx["thr_bin"][nid], ref["thr_bin"][nid])


@pytest.mark.parametrize("path", [p for p in FIXTURES if "sparse" in p], ids=os.path.basename)
def test_fixed_sparse_equals_dense(path):
    """Exact sums: the sparse default-bin fill (grow.c:101-106) is exact, so
    the sparse and dense builders give the same tree bit for bit."""
    d = _load(path)
    kw = _kwargs(d)
    sp = O.grow(d["bins_fm"], d["grad"], d["hess"], mode=O.MODE_FIXED, **kw)
    kw.pop("sparse")
    de = O.grow(d["bins_fm"], d["grad"], d["hess"], mode=O.MODE_FIXED, **kw)
    assert tree_arrays_equal(sp, de) is None


@pytest.mark.parametrize("path", [p for p in FIXTURES if "apply_X" in np.load(p).files],
                         ids=os.path.basename)
def test_apply_is_the_reference(path):
    d = _load(path)
    ref = _expected(d)
    got = O.apply(d["apply_X"], ref["feature"], d["apply_threshold"], ref["left"], ref["right"])
    assert np.array_equal(got, d["apply_out"])
