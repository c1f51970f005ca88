"""yabt_grow_batched (growth "rounds": several best-first splits per round)
against yabt_grow and the oracle where the leaf budget binds.

The batched grower computes splits ahead of cgrow's best-first order and
commits them in that order (grow.c:321-408), so its trees must equal
yabt_grow's bit for bit -- node arrays in best-first numbering, value bits,
per-row leaf ids -- and the oracle's fixed-point mode, also when the budget
runs out with computed splits left uncommitted, at the depth cap, with
interaction constraints, feature masks and gamma stopping growth early.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import grad_hess, skewed_bins, tree_arrays_equal, uniform_bins
from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None

CASES = [
    dict(n=200_000, F=10, nb=256, kind="normal", max_leaves=1000, msl=5),
    dict(n=300_000, F=6, nb=64, kind="logistic", max_leaves=1024, msl=1),
    dict(n=50_000, F=30, nb=256, kind="normal", max_leaves=255, max_depth=6, msl=20),
    dict(n=20_000, F=20, nb=255, kind="normal", max_leaves=100, imat=True),
    dict(n=8000, F=40, nb=256, kind="laplace", max_leaves=200, msl=1, skew=True),
    dict(n=4000, F=17, nb=64, kind="normal", max_leaves=63, fmask=True, lam=0.0, gamma=0.05),
    dict(n=10_000, F=5, nb=256, kind="normal", max_leaves=500, gamma=20.0),
    dict(n=30_000, F=500, nb=256, kind="laplace", max_leaves=128, skew=True),
    dict(n=1_000_000, F=16, nb=256, kind="normal", max_leaves=255, msl=20),
    dict(n=5, F=2, nb=256, kind="normal", max_leaves=16, msl=0),
    dict(n=3000, F=5, nb=256, kind="normal", max_leaves=2),
    dict(n=100, F=3, nb=256, kind="normal", max_leaves=1),
    dict(n=2000, F=3, nb=256, kind="normal", max_leaves=31, gamma=1e6),
    dict(n=2_000_000, F=8, nb=256, kind="normal", max_leaves=511, msl=50, max_depth=12),
]


def _inputs(case):
    c = dict(case)
    rng = np.random.default_rng(c["n"] * 13 + c["F"])
    n, F, nb = c.pop("n"), c.pop("F"), c.pop("nb")
    bins = skewed_bins(rng, n, F) if c.pop("skew", False) else uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n, c.pop("kind"))
    kw = dict(max_leaves=c.pop("max_leaves"), max_depth=c.pop("max_depth", 64), msl=c.pop("msl", 20),
              lam=c.pop("lam", 1.0), gamma=c.pop("gamma", 0.0), mcw=1e-3, lr=0.1)
    if c.pop("imat", False):
        im = rng.random((F, F)).astype(np.float32)
        kw.update(imat=(im + im.T) / 2, ib=0.5)
    if c.pop("fmask", False):
        kw["fmask"] = rng.random(F) < 0.7
    assert not c
    return bins, g, h, np.full(F, nb, np.int32), kw


def _run(lay, g, h, nbins, growth, kw):
    res = G.grow_device(lay, g, h, nbins, growth=growth, **kw)
    out = {k: getattr(res, k).cpu().numpy() for k in ("feature", "thr_bin", "left", "right", "value", "depth")}
    leaf = G.leaf_ids(res, lay.n, lay.F, kw["max_leaves"]).cpu().numpy()
    return out, leaf


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"n{c['n']}_F{c['F']}_L{c['max_leaves']}")
def test_rounds_equal_sequential_and_oracle(case):
    print(f"case {case}", flush=True)
    bins, g, h, nbins, kw = _inputs(case)
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    gd, hd = torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV)
    got, leaf = _run(lay, gd, hd, nbins, "rounds", kw)
    seq, leaf_seq = _run(lay, gd, hd, nbins, "sequential", kw)
    assert tree_arrays_equal(got, seq) is None
    assert np.array_equal(leaf, leaf_seq)
    want = O.grow(np.ascontiguousarray(bins.T), g, h, mode=O.MODE_FIXED, nbins=nbins, **kw)
    assert tree_arrays_equal(got, want) is None
    assert np.array_equal(leaf, O.leaf_of_rows(want, bins.shape[0]))


def test_rounds_repeat_and_shrink():
    """Two calls in a row share the workspace: the second, smaller one gives
    its own tree, and a repeat of the first gives the first's bits."""
    out = []
    for case in (CASES[0], CASES[4], CASES[0]):
        bins, g, h, nbins, kw = _inputs(case)
        lay = G.make_layouts(torch.from_numpy(bins), DEV)
        out.append(_run(lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV), nbins, "rounds", kw))
        want = O.grow(np.ascontiguousarray(bins.T), g, h, mode=O.MODE_FIXED, nbins=nbins, **kw)
        assert tree_arrays_equal(out[-1][0], want) is None
    assert tree_arrays_equal(out[0][0], out[2][0]) is None
    assert np.array_equal(out[0][1], out[2][1])


def test_rounds_reject_too_many_leaves():
    bins, g, h, nbins, kw = _inputs(dict(n=1000, F=4, nb=256, kind="normal", max_leaves=1025))
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    with pytest.raises(ValueError):
        G.grow_device(lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV), nbins, growth="rounds", **kw)
