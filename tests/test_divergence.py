"""yabt_amd.divergence on the CPU, against the oracle's own node histograms.

* The fp32 bounds hold: for every node of a reference-arithmetic tree, each
  bin of the histogram cgrow scanned there (oracle fp32 mode, keep_hist) is
  within the bound of the float64 sum of its rows -- built and subtracted
  nodes alike; so do the exact arithmetic's (oracle fixed-point mode).
* The bounds are not vacuous: at the root (row-order sums, no subtraction)
  the fp32 bound is within a few times the worst error actually seen, times
  the row count.
* first_difference / canonical_first_difference locate planted differences,
  and node_rows gives the oracle's own node membership.
* decision_gap's float64 gains equal a direct evaluation of grow.c's gain
  expression on the node's rows.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import grad_hess, uniform_bins
from yabt_amd import divergence as D

KW = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1)


def _tree(seed, n=20_000, F=6, nb=32, max_leaves=31, mode=O.MODE_FP32, kind="normal"):
    rng = np.random.default_rng(seed)
    bins = uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n, kind)
    t = O.grow(bins.T, g, h, mode=mode, nbins=np.full(F, nb, np.int32), max_leaves=max_leaves,
               keep_hist=True, **KW)
    return bins, g, h, t


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_fp32_bounds_hold_at_every_node(seed):
    bins, g, h, t = _tree(seed)
    bfm = torch.from_numpy(np.ascontiguousarray(bins.T))
    gt, ht = torch.from_numpy(g), torch.from_numpy(h)
    F = bins.shape[1]
    worst = 0.0
    for node in range(t["n_nodes"]):
        err, stats = D.fp32_bin_error_bounds(t, bfm, gt, ht, node, F)
        actual = np.abs(t["hist"][node, :2].astype(np.float64) - stats[:2].numpy())
        assert (actual <= err.numpy() + 1e-300).all(), f"node {node}"
        worst = max(worst, float((actual / np.maximum(err.numpy(), 1e-300)).max()))
        rows = D.node_rows(t["feature"], t["thr_bin"], t["left"], t["right"], bfm, node).numpy()
        assert np.array_equal(np.sort(rows), np.sort(t["rows"][t["seg_lo"][node]:t["seg_hi"][node]]))
    assert worst > 1e-4   # the bounds are met by errors that exist, not only by zeros


def test_fp32_root_bound_is_tight_enough():
    """At the root, the bound is (c - 1) u sum|x| per bin; the actual row-order
    error is a random walk, so the largest bound stays below c times the
    largest error seen."""
    bins, g, h, t = _tree(4, n=50_000, nb=16)
    bfm = torch.from_numpy(np.ascontiguousarray(bins.T))
    err, stats = D.fp32_bin_error_bounds(t, bfm, torch.from_numpy(g), torch.from_numpy(h), 0, bins.shape[1])
    actual = np.abs(t["hist"][0, 0].astype(np.float64) - stats[0].numpy())
    c = np.bincount(bins[:, 0], minlength=256)
    assert actual.max() > 0
    assert err[0, 0].numpy().max() / actual.max() < c[c > 0].min()


def test_exact_bounds_hold():
    bins, g, h, t = _tree(5, mode=O.MODE_FIXED)
    sg, sh = O.quant_shifts(g, h)
    bfm = torch.from_numpy(np.ascontiguousarray(bins.T))
    for node in range(t["n_nodes"]):
        rows = D.node_rows(t["feature"], t["thr_bin"], t["left"], t["right"], bfm, node)
        stats, cnt = D._bin_stats(bfm, torch.from_numpy(g), torch.from_numpy(h), rows, bins.shape[1])
        for c, s in ((0, sg), (1, sh)):
            got = t["hist"][node, c].astype(np.float64) * 2.0 ** -s
            assert (np.abs(got - stats[c].numpy()) <= cnt.numpy() * 2.0 ** (-s - 1) + 1e-12).all()


def test_differences_are_located():
    bins, g, h, t = _tree(6)
    assert D.first_difference(t, t) is None and D.canonical_first_difference(t, t) is None
    u = {k: np.array(t[k]) for k in ("feature", "thr_bin", "left", "right")}
    ev = D.split_events(u["feature"], u["left"])
    k = ev[5][0]
    u["thr_bin"][k] += 1
    d = D.first_difference(u, t)
    assert d["event"] == 5 and d["a"][:2] == d["b"][:2] and d["a"][2] == d["b"][2] + 1
    c = D.canonical_first_difference(u, t)
    assert c["node_a"] == c["node_b"] == k and c["a"] == (d["a"][1], d["a"][2])


def test_decision_gap_gains_are_grow_c_gains():
    bins, g, h, t = _tree(7, nb=24)
    bfm = torch.from_numpy(np.ascontiguousarray(bins.T))
    k = D.split_events(t["feature"], t["left"])[3][0]
    f = int(t["feature"][k])
    other = (f + 1) % bins.shape[1]
    diff = {"a": (k, other, 7), "b": (k, f, int(t["thr_bin"][k]))}
    sg, sh = O.quant_shifts(g, h)
    out = D.decision_gap(t, diff, bfm, torch.from_numpy(g), torch.from_numpy(h), np.full(6, 24), (sg, sh))
    rows = t["rows"][t["seg_lo"][k]:t["seg_hi"][k]]
    for side, (ff, bb) in (("exact", (other, 7)), ("reference", (f, int(t["thr_bin"][k])))):
        left = bins[rows, ff] <= bb
        GL, HL = g[rows][left].astype(np.float64).sum(), h[rows][left].astype(np.float64).sum()
        G, H = g[rows].astype(np.float64).sum(), h[rows].astype(np.float64).sum()
        GR, HR = G - GL, H - HL
        want = 0.5 * (GL * GL / (HL + 1) + GR * GR / (HR + 1) - G * G / (H + 1))
        assert out[side]["gain"] == pytest.approx(want, rel=1e-12, abs=1e-12)
    assert out["gap"] == pytest.approx(abs(out["exact"]["gain"] - out["reference"]["gain"]))
