"""The headline workload at its full size: one best-first tree over 10M rows x
100 features of uint8 bins uniform on 0..255, g ~ N(0,1), h ~ U(0.1, 1),
255 leaves, min_samples_leaf 20 (numpy default_rng(0), bins feature-major).

* reference arithmetic (yabt_grow_ref) against the compiled reference grow.c
  (oracle/_ref, built from the reference sources) on the same inputs: node
  arrays and value bits equal;
* exact arithmetic (yabt_grow), through properties that do not depend on the
  size: per-row leaf ids equal the raw-space routing of float(bins) (the
  partition/apply equivalence of test_splits.py:58-68), node sizes add up
  from the leaves to the root, every leaf holds at least min_samples_leaf
  rows, the leaf budget is used; and its split sequence against the
  reference's: the same features, and the same bins except at two small
  nodes where an empty bin separates two splits of equal gain (the same
  rows go left either way) and the reference's fp32 subtraction residue in
  that bin picks the later one.
"""

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import tree_arrays_equal
from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None
N, F = 10_000_000, 100
PARAMS = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=255, max_depth=64)
NBINS = np.full(F, 256, np.int32)


@pytest.fixture(scope="module")
def inputs():
    print("generating 10M x 100 inputs", flush=True)
    rng = np.random.default_rng(0)
    bins_fm = rng.integers(0, 256, size=(F, N), dtype=np.uint8)
    g = rng.standard_normal(N, dtype=np.float32)
    h = rng.uniform(0.1, 1.0, N).astype(np.float32)
    lay = G.make_layouts(torch.from_numpy(bins_fm).t(), DEV, binned_fmajor=bins_fm)
    return bins_fm, g, h, lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV)


@pytest.fixture(scope="module")
def reference_tree(inputs):
    if not O.ref_available():
        pytest.skip("oracle/_ref/libgrow_ref.so not built (make -C oracle ref)")
    bins_fm, g, h = inputs[:3]
    print("reference grow.c, 10M x 100", flush=True)
    return O.grow(bins_fm, g, h, reference=True, nbins=NBINS, n_threads=min(os.cpu_count() or 1, 16), **PARAMS)


def _arrays(res):
    return {k: getattr(res, k).cpu().numpy() for k in ("feature", "thr_bin", "left", "right", "value", "depth")}


def test_reference_arithmetic_equals_grow_c(inputs, reference_tree):
    lay, gd, hd = inputs[3:]
    print("yabt_grow_ref, 10M x 100", flush=True)
    got = _arrays(G.grow_device(lay, gd, hd, NBINS, arithmetic="reference", **PARAMS))
    assert (got["feature"] >= 0).sum() == 254
    assert tree_arrays_equal(got, reference_tree) is None


def test_exact_arithmetic_properties(inputs, reference_tree):
    lay, gd, hd = inputs[3:]
    print("yabt_grow, 10M x 100", flush=True)
    res = G.grow_device(lay, gd, hd, NBINS, **PARAMS)
    t = _arrays(res)
    feat, left, right = t["feature"], t["left"], t["right"]
    internal = feat >= 0
    assert internal.sum() == 254 and feat.size == 509
    leaf = G.leaf_ids(res, N, F, PARAMS["max_leaves"])
    # partition == routing of the raw features x = float(bin) by x <= thr_bin
    X = lay.rm[:N, :F].float()
    routed = G.apply_hip(X, res.feature, res.thr_bin.float(), res.left, res.right)
    del X
    assert torch.equal(routed, leaf)
    size = np.bincount(leaf.cpu().numpy(), minlength=feat.size).astype(np.int64)
    assert (size[internal] == 0).all()
    assert (size[~internal] >= PARAMS["msl"]).all()
    for nid in range(feat.size - 1, -1, -1):
        if internal[nid]:
            size[nid] = size[left[nid]] + size[right[nid]]
    assert size[0] == N
    # the split sequence against the reference's: the same features, and the
    # same bins except where the reference's fp32 sums decide a near-tie the
    # other way -- there the two bins' gains, from the node's rows summed in
    # float64, agree to fp32 rounding
    ref = reference_tree
    assert np.array_equal(feat, ref["feature"])
    differ = np.nonzero(internal & (t["thr_bin"] != ref["thr_bin"]))[0]
    print(f"exact vs reference: {len(differ)} of 254 split bins differ", flush=True)
    assert len(differ) <= 5
    bins_fm, g, h = inputs[:3]
    leaf_np = leaf.cpu().numpy()
    for nid in differ:
        below = np.zeros(feat.size, bool)
        stack = [nid]
        while stack:
            k = stack.pop()
            below[k] = True
            if internal[k]:
                stack += [left[k], right[k]]
        rows = np.nonzero(below[leaf_np])[0]
        f = feat[nid]
        b = bins_fm[f, rows]
        GL = np.cumsum(np.bincount(b, weights=g[rows].astype(np.float64), minlength=256))
        HL = np.cumsum(np.bincount(b, weights=h[rows].astype(np.float64), minlength=256))
        Gt, Ht = GL[-1], HL[-1]
        gain = lambda k: 0.5 * (GL[k] ** 2 / (HL[k] + 1) + (Gt - GL[k]) ** 2 / (Ht - HL[k] + 1) - Gt ** 2 / (Ht + 1))
        ge, gr = gain(t["thr_bin"][nid]), gain(ref["thr_bin"][nid])
        print(f"node {nid} ({rows.size} rows, feature {f}): bin {t['thr_bin'][nid]} gain {ge:.9g}, "
              f"reference bin {ref['thr_bin'][nid]} gain {gr:.9g}", flush=True)
        assert abs(ge - gr) <= 1e-6 * abs(ge)
        # here the node holds no row between the two bins: both splits send
        # the same rows left (the reference's fp32 subtraction leaves a
        # residue in the empty bin that the exact sums do not)
        lo, hi = sorted((t["thr_bin"][nid], ref["thr_bin"][nid]))
        assert not ((b > lo) & (b <= hi)).any()


def test_rounds_equal_split_by_split(inputs):
    """The exact grower with up to 16 splits per round: yabt_grow's tree bit
    for bit, and the same per-row leaf ids."""
    lay, gd, hd = inputs[3:]
    print("yabt_grow_batched and yabt_grow, 10M x 100", flush=True)
    rr = G.grow_device(lay, gd, hd, NBINS, growth="rounds", **PARAMS)
    rs = G.grow_device(lay, gd, hd, NBINS, growth="sequential", **PARAMS)
    assert tree_arrays_equal(_arrays(rr), _arrays(rs)) is None
    assert torch.equal(G.leaf_ids(rr, N, F, PARAMS["max_leaves"]), G.leaf_ids(rs, N, F, PARAMS["max_leaves"]))


# ---------------------------------------------------------------------------
# depth 6 over 4M rows x 500 features, each bin 0 with probability 0.9 else
# uniform on 1..255, g ~ Laplace(0, 1), h = 1, 64 leaves
# ---------------------------------------------------------------------------

N4, F4 = 4_000_000, 500
PARAMS4 = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=64, max_depth=6)


@pytest.fixture(scope="module")
def sparse_inputs():
    print("generating 4M x 500 mostly-zero inputs", flush=True)
    rng = np.random.default_rng(4)
    bins = rng.integers(1, 256, size=(N4, F4), dtype=np.uint8)
    bins[rng.random((N4, F4), dtype=np.float32) < 0.9] = 0
    g = rng.laplace(size=N4).astype(np.float32)
    h = np.ones(N4, np.float32)
    bins_fm = np.ascontiguousarray(bins.T)
    lay = G.make_layouts(torch.from_numpy(bins), DEV, binned_fmajor=bins_fm)
    return bins, bins_fm, g, h, lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV)


def test_sparse_reference_arithmetic_equals_grow_c(sparse_inputs):
    """cgrow's sparse builder (grow.c:68-107) with bin 0 as every feature's
    default, the layout the reference builds for these bins."""
    if not O.ref_available():
        pytest.skip("oracle/_ref/libgrow_ref.so not built (make -C oracle ref)")
    bins, bins_fm, g, h, lay, gd, hd = sparse_inputs
    print("CSR layout", flush=True)
    nondef = bins != 0
    indptr = np.zeros(N4 + 1, np.int64)
    np.cumsum(nondef.sum(axis=1), out=indptr[1:])
    r, c = np.nonzero(nondef)
    del nondef
    layout = (indptr, c.astype(np.int32), bins[r, c].astype(np.int32), np.zeros(F4, np.int32))
    del r, c
    nb = np.full(F4, 256, np.int32)
    print("reference grow.c (sparse builder), 4M x 500", flush=True)
    want = O.grow(bins_fm, g, h, reference=True, sparse=layout, nbins=nb,
                  n_threads=min(os.cpu_count() or 1, 16), **PARAMS4)
    del layout
    print("yabt_grow_ref (sparse builder), 4M x 500", flush=True)
    got = _arrays(G.grow_device(lay, gd, hd, nb, arithmetic="reference", default_bin=np.zeros(F4, np.int32),
                                **PARAMS4))
    print(f"{(got['feature'] >= 0).sum()} splits", flush=True)
    assert tree_arrays_equal(got, want) is None


def test_depth_batched_equals_split_by_split(sparse_inputs):
    """The exact grower grown depth by depth and split by split: the same tree
    bit for bit, and per-row leaf ids equal to raw-space routing."""
    bins, bins_fm, g, h, lay, gd, hd = sparse_inputs
    nb = np.full(F4, 256, np.int32)
    print("yabt_grow_levelwise and yabt_grow, 4M x 500", flush=True)
    rb = G.grow_device(lay, gd, hd, nb, batched=True, **PARAMS4)
    rs = G.grow_device(lay, gd, hd, nb, batched=False, **PARAMS4)
    assert tree_arrays_equal(_arrays(rb), _arrays(rs)) is None
    leaf = G.leaf_ids(rb, N4, F4, PARAMS4["max_leaves"])
    assert torch.equal(leaf, G.leaf_ids(rs, N4, F4, PARAMS4["max_leaves"]))
    X = lay.rm[:N4, :F4].float()
    routed = G.apply_hip(X, rb.feature, rb.thr_bin.float(), rb.left, rb.right)
    del X
    assert torch.equal(routed, leaf)
