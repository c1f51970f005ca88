"""Host-side pieces: the oracle binner's semantics (the reference's numpy
path, which the device binner is compared against on the GPU), the Tree
type's path pairs (and that its routing has no CPU path), the identity
binner."""

import numpy as np
import pytest
import torch

from oracle.boost_oracle import Binner
from yabt_amd import IdentityBinner, Tree


def test_binner_split_equivalence():
    """bin(x) <= b  <=>  x <= edge_value(f, b) (test_splits.py:58-68)."""
    rng = np.random.default_rng(1)
    X = rng.normal(size=(1000, 3)).astype(np.float32)
    binner = Binner(max_bins=16).fit(X)
    binned = binner.transform(X)
    for f in range(3):
        for b in range(len(binner.edges_[f])):
            assert ((binned[:, f] <= b) == (X[:, f] <= binner.edge_value(f, b))).all()


def test_binner_edges_closed_form():
    X = np.arange(1, 101, dtype=np.float32).reshape(100, 1)
    b = Binner(max_bins=4).fit(X)
    assert np.allclose(b.edges_[0], np.quantile(X[:, 0], [0.25, 0.5, 0.75]))
    assert float(b.scales_[0]) == np.float32(np.quantile(X[:, 0], 0.75) - np.quantile(X[:, 0], 0.25))
    codes = b.transform(X)[:, 0]
    assert codes.min() == 0 and codes.max() == 3
    # constant column: one edge, zero IQR -> std -> 1.0
    c = Binner().fit(np.ones((50, 1), np.float32))
    assert len(c.edges_[0]) == 1 and float(c.scales_[0]) == 1.0


def test_binner_imputes_nan_with_median():
    X = np.array([[1.0], [np.nan], [3.0], [5.0]], np.float32)
    b = Binner(max_bins=4).fit(X)
    assert b.medians_[0] == 3.0
    assert b.impute(X)[1, 0] == 3.0


def test_tree_routing_has_no_cpu_path():
    """Tree.apply / Tree.predict run the HIP kernels only: without a device
    they raise instead of routing on the CPU."""
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present; routing is covered by the GPU tests")
    tree = Tree(feature=torch.tensor([0, -1, -1]), threshold=torch.tensor([0.5, 0.0, 0.0]),
                left=torch.tensor([1, -1, -1]), right=torch.tensor([2, -1, -1]),
                value=torch.tensor([0.0, 1.0, 2.0]), depth=2)
    X = torch.zeros(4, 2)
    with pytest.raises(RuntimeError):
        tree.apply(X)
    with pytest.raises(RuntimeError):
        tree.predict(X)


def test_path_feature_pairs():
    # root(f0) -> [leaf, node(f2) -> [leaf, leaf]]  (test_interaction_aware.py:44-56)
    tree = Tree(feature=torch.tensor([0, -1, 2, -1, -1]), threshold=torch.zeros(5),
                left=torch.tensor([1, -1, 3, -1, -1]), right=torch.tensor([2, -1, 4, -1, -1]),
                value=torch.zeros(5), depth=3)
    assert tree.path_feature_pairs() == [(0, 2)]
    # deeper: 0 -> (1 -> (3, 4), 2:f5 -> (5:f0 -> ...)): every ancestor pairs with each split below
    tree = Tree(feature=torch.tensor([0, 1, 5, -1, -1, 0, -1, -1, -1]), threshold=torch.zeros(9),
                left=torch.tensor([1, 3, 5, -1, -1, 7, -1, -1, -1]),
                right=torch.tensor([2, 4, 6, -1, -1, 8, -1, -1, -1]), value=torch.zeros(9), depth=4)
    assert sorted(tree.path_feature_pairs()) == sorted([(0, 1), (0, 5), (0, 0), (5, 0)])


def test_identity_binner():
    b = IdentityBinner(3, 256)
    assert b.edge_value(1, 17) == 17.0
    assert b.edge_value(1, 300) == 254.0
    assert len(b.edges_[0]) == 255


def test_layout_cache_reuses_per_tensor_and_forgets_dead_tensors(monkeypatch):
    """layouts_for caches one layout pair per binned tensor: the same tensor
    again hits (a second call once failed on tensor key comparison), an
    in-place change rebuilds, and the entry goes when the tensor dies."""
    import gc

    from yabt_amd import grow_hip as G
    built = []
    monkeypatch.setattr(G, "make_layouts", lambda b, d, f=None: built.append(object()) or built[-1])
    monkeypatch.setattr(G, "_LAYOUTS", {})
    t = torch.zeros(5, 3, dtype=torch.uint8)
    a = G.layouts_for(t, "dev")
    assert G.layouts_for(t, "dev") is a and len(built) == 1
    t.add_(1)
    assert G.layouts_for(t, "dev") is not a and len(built) == 2
    u = torch.zeros(5, 3, dtype=torch.uint8)
    G.layouts_for(u, "dev")
    assert len(G._LAYOUTS) == 2
    del t
    gc.collect()
    assert list(G._LAYOUTS) == [id(u)]
