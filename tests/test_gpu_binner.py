"""The device binner (yabt_bin_fit / yabt_bin_transform) against the
reference's numpy path (oracle/boost_oracle.Binner, the reference's own numpy
calls): edges bit for bit, edge counts, scales (IQR and numpy's float32 std
fallback), NaN-ignoring medians of all rows, codes, imputed matrix and the
grower's two layouts."""

import numpy as np
import pytest
import torch

from oracle import boost_oracle as BO
from yabt_amd import Binner
from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _data(kind, n, F, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        X = rng.normal(size=(n, F)).astype(np.float32)
    elif kind == "ties":           # few distinct values: repeated quantiles, zero IQR columns
        X = rng.integers(0, 5, size=(n, F)).astype(np.float32)
        X[:, 0] = 7.0
    elif kind == "sparse":         # 90% zeros (zero IQR, std fallback)
        X = np.where(rng.random((n, F)) < 0.9, 0.0, rng.normal(size=(n, F))).astype(np.float32)
    elif kind == "nan":            # NaNs, an all-NaN column, signed and huge values
        X = (rng.normal(size=(n, F)) * np.exp(rng.normal(size=(n, F)) * 3)).astype(np.float32)
        X[rng.random((n, F)) < 0.2] = np.nan
        X[:, 1] = np.nan
        X[:5, 2] = [np.inf, -np.inf, 3e38, -3e38, 1e-40]
    else:
        raise ValueError(kind)
    return X


CASES = [
    ("normal", 20_000, 20, 255),
    ("normal", 5_000, 3, 256),
    ("normal", 999, 17, 28),
    ("ties", 3_000, 5, 64),
    ("sparse", 40_000, 9, 256),
    ("nan", 10_000, 6, 32),
    ("normal", 1, 2, 256),
    ("normal", 350_000, 4, 255),     # > 200 000 rows: the seeded subsample
    ("sparse", 250_001, 3, 2),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}_n{c[1]}_F{c[2]}_B{c[3]}")
def test_fit_and_transform_match_numpy_path(case):
    kind, n, F, B = case
    print(f"binner {case}", flush=True)
    X = _data(kind, n, F, n + F)
    ref = BO.Binner(B).fit(X)
    b = Binner(B).fit(X)
    for f in range(F):
        got = b.edges_[f].numpy()
        want = ref.edges_[f]
        assert got.shape == want.shape, f"feature {f}: {got.size} edges, numpy {want.size}"
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), f"feature {f} edges"
    assert np.array_equal(b.scales_.numpy().view(np.uint32), ref.scales_.view(np.uint32)), "scales"
    med = np.where(np.isnan(np.nanmedian(X, axis=0)), 0.0, np.nanmedian(X, axis=0)).astype(np.float32) \
        if n else np.zeros(F, np.float32)
    assert np.array_equal(b.medians_.view(np.uint32), med.view(np.uint32)), "medians"
    # codes: the device transform, torch.searchsorted on the same edges, the oracle
    codes = b.transform(X).cpu().numpy()
    assert np.array_equal(codes, ref.transform(X))
    Xi = ref.impute(X)
    ts = np.stack([torch.searchsorted(b.edges_[f], torch.from_numpy(np.ascontiguousarray(Xi[:, f]))).numpy()
                   for f in range(F)], axis=1).astype(np.uint8)
    assert np.array_equal(codes, ts)
    # both layouts and the imputed matrix in one pass
    lay, imp = b.layouts(X)
    assert np.array_equal(lay.fm[:, :n].cpu().numpy(), codes.T)
    assert np.array_equal(lay.rm[:n, :F].cpu().numpy(), codes)
    assert np.array_equal(imp.cpu().numpy().view(np.uint32), Xi.view(np.uint32))
    ref_lay = G.make_layouts(torch.from_numpy(codes).to(DEV), DEV)
    assert torch.equal(ref_lay.fm, lay.fm) and torch.equal(ref_lay.rm, lay.rm)


def test_split_equivalence_on_device_bins():
    """bin(x) <= b  <=>  x <= edge_value(f, b) (test_splits.py:58-68)."""
    rng = np.random.default_rng(1)
    X = rng.normal(size=(5000, 3)).astype(np.float32)
    b = Binner(max_bins=16).fit(torch.from_numpy(X).to(DEV))
    codes = b.transform(X).cpu().numpy()
    for f in range(3):
        for k in range(len(b.edges_[f])):
            assert ((codes[:, f] <= k) == (X[:, f] <= b.edge_value(f, k))).all()
