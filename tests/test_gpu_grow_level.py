"""yabt_grow_levelwise (depth-batched growth) against yabt_grow and the oracle.

Whenever the leaf budget cannot bind (max_leaves >= 2^max_depth) the batched
grower must give yabt_grow's tree bit for bit -- node arrays in cgrow's
best-first numbering, value bits, per-row leaf ids -- and so the oracle's
fixed-point mode too.
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
    dict(n=5000, F=9, nb=28, kind="logistic", max_leaves=256, max_depth=8, msl=1),
    dict(n=20_000, F=20, nb=255, kind="normal", max_leaves=64, max_depth=6, imat=True),
    dict(n=8000, F=40, nb=256, kind="laplace", max_leaves=64, max_depth=6, skew=True),
    dict(n=4000, F=17, nb=64, kind="normal", max_leaves=32, max_depth=5, fmask=True, lam=0.0, gamma=0.05),
    dict(n=30_000, F=500, nb=256, kind="laplace", max_leaves=64, max_depth=6, skew=True),
    dict(n=1, F=1, nb=256, kind="normal", max_leaves=4, max_depth=2, msl=0),
    dict(n=100, F=3, nb=256, kind="normal", max_leaves=1, max_depth=0),
    dict(n=3000, F=5, nb=256, kind="normal", max_leaves=2, max_depth=1),
    dict(n=300_000, F=28, nb=28, kind="logistic", max_leaves=256, max_depth=8, msl=20),
    dict(n=400_000, F=12, nb=256, kind="normal", max_leaves=1024, max_depth=10, msl=20, imat=True),
    dict(n=60_000, F=8, nb=256, kind="normal", max_leaves=300, max_depth=8, msl=1000),
]


def _inputs(case):
    c = dict(case)
    rng = np.random.default_rng(c["n"] * 7 + c["F"])
    n, F, nb = c.pop("n"), c.pop("F"), c.pop("nb")
    bins = skewed_bins(rng, n, F) if c.pop("skew", False) else uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n, c.pop("kind"))
    kw = dict(max_leaves=c.pop("max_leaves"), max_depth=c.pop("max_depth"), msl=c.pop("msl", 20),
              lam=c.pop("lam", 1.0), gamma=c.pop("gamma", 0.0))
    if c.pop("imat", False):
        im = rng.random((F, F)).astype(np.float32)
        kw.update(imat=(im + im.T) / 2, ib=0.5)
    if c.pop("fmask", False):
        kw["fmask"] = rng.random(F) < 0.7
    return bins, g, h, np.full(F, nb, np.int32), kw


def _run(lay, g, h, nbins, batched, kw):
    res = G.grow_device(lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV), nbins, batched=batched,
                        **kw)
    out = {k: getattr(res, k).cpu().numpy() for k in ("feature", "thr_bin", "left", "right", "value", "depth")}
    leaf = G.leaf_ids(res, lay.n, lay.F, kw["max_leaves"]).cpu().numpy()
    return out, leaf


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"n{c['n']}_F{c['F']}_L{c['max_leaves']}_D{c['max_depth']}")
def test_batched_equals_sequential_and_oracle(case):
    print(f"case {case}", flush=True)
    bins, g, h, nbins, kw = _inputs(case)
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    got, leaf = _run(lay, g, h, nbins, True, kw)
    seq, leaf_seq = _run(lay, g, h, nbins, False, kw)
    assert tree_arrays_equal(got, seq) is None
    assert np.array_equal(leaf, leaf_seq)
    want = O.grow(np.ascontiguousarray(bins.T), g, h, mode=O.MODE_FIXED, nbins=nbins, **kw)
    assert tree_arrays_equal(got, want) is None
    assert np.array_equal(leaf, O.leaf_of_rows(want, bins.shape[0]))


def test_batched_rejects_a_binding_budget():
    bins, g, h, nbins, kw = _inputs(dict(n=1000, F=4, nb=256, kind="normal", max_leaves=8, max_depth=6))
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    with pytest.raises(ValueError):
        G.grow_device(lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV), nbins, batched=True, **kw)
