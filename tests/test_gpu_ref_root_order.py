"""The reference-arithmetic grower's per-fit root rank table
(yabt_ref_root_order + k_rank_chain) against the per-tree bucketing of the
root (k_walk_sort + k_walk_chain): identical trees, rows[] and leaf ids, bit
for bit, on ragged tiles, a single partial tile, bins skewed enough that a
tile's run of one bin exceeds both the chain's 32-rank LDS window and 255,
and features of few bins (the window widened to 128 .. 4096 ranks).

Both paths restate cgrow's row-order fp32 histogram chains
(yabt/_cgrow/grow.c:37-62); their agreement with grow.c itself is checked by
tests/test_gpu_grow_ref.py and tests/test_gpu_full_size.py, which grow through
the rank table now.
"""

import numpy as np
import pytest
import torch

from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _bins(kind, n, F, rng):
    if kind == "uniform":
        return rng.integers(0, 256, size=(n, F)).astype(np.uint8)
    if kind == "few":
        # per feature a different span of bins: 28 (a window of 256 ranks),
        # 2, 1 (all zero: a window of the whole tile), 33 (bins 0..31 and a
        # single row of bin 32 in one tile: a window of 128 ranks for every
        # tile), 32, and 20 with 90% of rows in bin 3 (runs of ~3700 per tile,
        # past the 256-rank window)
        spans = [28, 2, 1, 32, 32, 20]
        b = np.stack([rng.integers(0, spans[f % len(spans)], size=n) for f in range(F)], axis=1)
        sk = [f for f in range(F) if f % len(spans) == len(spans) - 1]
        b[:, sk] = np.where(rng.random((n, len(sk))) < 0.9, 3, b[:, sk])
        if F > 3:
            b[n // 2, 3] = 32     # the span-33 feature's largest bin in one row only
        return b.astype(np.uint8)
    # skewed: 90% of rows in bin 7, the rest spread (runs of ~3700 per tile)
    b = rng.integers(0, 256, size=(n, F)).astype(np.uint8)
    b[rng.random((n, F)) < 0.9] = 7
    return b


@pytest.mark.parametrize("kind,n,F,leaves", [
    ("uniform", 50_000, 12, 31),     # 13 tiles, the last one partial
    ("uniform", 100, 5, 8),          # one partial tile
    ("skewed", 30_000, 6, 24),       # runs longer than 32 and than 255 ranks
    ("few", 60_000, 6, 31),          # spans of 1..33 bins: windows of 256..4096 ranks
])
def test_rank_table_root_equals_bucketed_root(kind, n, F, leaves):
    rng = np.random.default_rng(11)
    bins = _bins(kind, n, F, rng)
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    g = torch.from_numpy(rng.normal(size=n).astype(np.float32)).to(DEV)
    h = torch.from_numpy(rng.uniform(0.05, 1.0, size=n).astype(np.float32)).to(DEV)
    nbins = np.full(F, 256, np.int32)
    kw = dict(fmask=None, imat=None, ib=0.0, lam=1.0, gamma=0.0, mcw=1e-3, msl=5, lr=0.1,
              max_leaves=leaves, max_depth=64)
    print(f"reference root: {kind} n={n} F={F}", flush=True)
    a = G._grow_device_ref(lay, g, h, nbins, root_order=True, **kw)
    b = G._grow_device_ref(lay, g, h, nbins, root_order=False, **kw)
    torch.cuda.synchronize()
    assert a.n_nodes == b.n_nodes and a.n_nodes > 1
    for name in ("feature", "thr_bin", "left", "right", "depth"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert torch.equal(a.value.view(torch.int32), b.value.view(torch.int32))
    assert torch.equal(a.rows, b.rows)
    assert torch.equal(a.leaf_of_row, b.leaf_of_row)


@pytest.mark.parametrize("kind,n,F", [("uniform", 70_001, 9), ("skewed", 20_000, 4), ("few", 50_003, 12)])
def test_reference_root_histogram_equals_oracle(kind, n, F):
    """yabt_ref_root_hist bit for bit against the oracle's row-order fp32
    build_hist (oracle/grow_oracle.c, grow.c:37-62)."""
    from oracle import oracle as O
    rng = np.random.default_rng(5)
    bins = _bins(kind, n, F, rng)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.05, 1.0, size=n).astype(np.float32)
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    print(f"reference root histogram: {kind} n={n} F={F}", flush=True)
    got = G.ref_root_hist(lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV)).cpu().numpy()
    want = O.hist_f32(np.ascontiguousarray(bins.T), g, h)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
