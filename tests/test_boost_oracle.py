"""Pins of the boosting-loop oracle (oracle/boost_oracle.py) on the CPU:
closed forms of the losses, the interaction detector on hand-counted trees,
routing against a per-row walk, partition/routing equivalence of the
training leaf ids, properties of the leaf output, and monotone training loss."""

import numpy as np
import pytest

from oracle import boost_oracle as BO
from oracle import oracle as O


def test_mse_grad_hess_closed_form():
    rng = np.random.default_rng(0)
    m = rng.normal(size=1000).astype(np.float32)
    y = rng.normal(size=1000).astype(np.float32)
    g, h = BO.grad_hess("mse", m, y)
    assert np.array_equal(g, m - y) and np.array_equal(h, np.ones(1000, np.float32))
    assert BO.base_score("mse", y) == pytest.approx(float(y.astype(np.float64).mean()), abs=1e-6)


def test_logloss_grad_hess_closed_form():
    m = np.array([-40.0, -5.0, -1.0, 0.0, 0.5, 3.0, 40.0], np.float32)
    y = np.array([0, 1, 0, 1, 1, 0, 1], np.float32)
    g, h = BO.grad_hess("log", m, y)
    p = 1.0 / (1.0 + np.exp(-m.astype(np.float64)))
    assert np.allclose(g, p - y, rtol=0, atol=1e-7)
    assert np.allclose(h, np.maximum(p * (1 - p), 1e-6), rtol=2e-6, atol=0)
    # saturated margins hit the hessian floor; p = 0.5 gives the maximum 1/4
    assert h[0] == np.float32(1e-6) and h[-1] == np.float32(1e-6) and h[3] == np.float32(0.25)
    yb = np.array([1, 1, 1, 0], np.float32)
    assert BO.base_score("log", yb) == pytest.approx(np.log(3.0), rel=1e-6)
    # all-positive labels: the mean is clamped to 1 - 1e-6 in float32 before the logit
    p1 = float(np.float32(1 - 1e-6))
    assert BO.base_score("log", np.ones(4, np.float32)) == pytest.approx(np.log(p1 / (1 - p1)), rel=1e-12)


def test_path_pairs_and_detector():
    # root(f0) -> [leaf, node(f2) -> [node(f0) -> [leaf, leaf], leaf]]
    feature = np.array([0, -1, 2, 0, -1, -1, -1])
    left = np.array([1, -1, 3, 5, -1, -1, -1])
    right = np.array([2, -1, 4, 6, -1, -1, -1])
    pairs = sorted(BO.path_pairs(feature, left, right))
    assert pairs == sorted([(0, 2), (0, 0), (2, 0)])
    det = BO.Interactions(3)
    assert np.array_equal(det.normalized(), np.zeros((3, 3), np.float32))  # all-zero counts pass through
    det.update(pairs)  # (0,0) is dropped, (0,2) and (2,0) each add to both cells
    assert det.m[0, 2] == 2 and det.m[2, 0] == 2 and det.m.sum() == 4
    # uniform nonzero counts normalise to zero (no pair stands out)
    assert np.array_equal(det.normalized(), np.zeros((3, 3), np.float32))
    det.update([(0, 1)])
    nm = det.normalized()
    bg = np.float32((2 + 2 + 1 + 1) / 4)
    assert nm[0, 2] == pytest.approx((2 - bg) / (2 - bg + 1e-8)) and nm[0, 1] == 0.0
    assert nm[0, 2] == nm[2, 0] and nm.min() == 0.0


def _walk(x, feature, threshold, left, right):
    node = 0
    while feature[node] >= 0:
        node = left[node] if x[feature[node]] <= threshold[node] else right[node]
    return node


def test_route_matches_per_row_walk():
    rng = np.random.default_rng(3)
    n, F = 3000, 5
    bins = rng.integers(0, 32, size=(F, n), dtype=np.uint8)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.5, 1, size=n).astype(np.float32)
    t = O.grow(bins, g, h, mode=O.MODE_FIXED, max_leaves=20, msl=5)
    thr = t["thr_bin"].astype(np.float32) + 0.5
    X = rng.uniform(-2, 34, size=(200, F)).astype(np.float32)
    got = BO.route(X, t["feature"], thr, t["left"], t["right"])
    want = [_walk(X[i], t["feature"], thr, t["left"], t["right"]) for i in range(200)]
    assert got.tolist() == want


def _cfg1(n, seed=0):
    """X ~ N(0,1) (n, 20); y = sin x0 + 0.5 x1 x2 + x3^2 + 0.3 sum x4..x9 + N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, 20)).astype(np.float32)
    y = (np.sin(X[:, 0]) + 0.5 * X[:, 1] * X[:, 2] + X[:, 3] ** 2 + 0.3 * X[:, 4:10].sum(axis=1)
         + rng.normal(scale=0.1, size=n)).astype(np.float32)
    return X, y


def test_training_leaf_ids_equal_routing_and_loss_decreases():
    X, y = _cfg1(3000)
    model = BO.fit(X, y, n_estimators=6, max_leaves=15, max_bins=63)
    # the training margin (leaf ids from the partition) equals routing the raw rows
    assert np.array_equal(BO.predict_margin(model, X), model["margin"])
    tl = model["train_loss"]
    assert all(b < a for a, b in zip(tl, tl[1:]))
    assert all(t.get("feats") is not None for t in model["trees"])


def test_loss_decreases_without_leaf_models_and_with_sampling():
    X, y = _cfg1(2500, seed=1)
    model = BO.fit(X, y, n_estimators=5, max_leaves=8, neural_leaves=False, subsample=0.7, colsample=0.5)
    tl = model["train_loss"]
    assert all(b < a for a, b in zip(tl, tl[1:]))
    for t in model["trees"]:
        assert len(set(t["feature"][t["feature"] >= 0].tolist())) <= 10
    assert np.array_equal(BO.predict_margin(model, X), model["margin"])


def test_tree_output_properties():
    rng = np.random.default_rng(5)
    n, K = 500, 3
    X = rng.normal(size=(n, 6)).astype(np.float32)
    node = rng.integers(0, 4, size=n)
    tree = {"value": rng.normal(size=4).astype(np.float32), "feats": np.array([4, 0, 2]),
            "linear": np.zeros((4, K), np.float32),
            "lo": np.full((4, K), -np.inf, np.float32), "hi": np.full((4, K), np.inf, np.float32)}
    assert np.array_equal(BO.tree_output(tree, X, node), tree["value"][node])
    tree["linear"] = rng.normal(size=(4, K)).astype(np.float32)
    base = BO.tree_output(tree, X, node) - tree["value"][node]
    lin_direct = (tree["linear"][node] * X[:, [4, 0, 2]]).astype(np.float64).sum(axis=1)
    assert np.allclose(base, lin_direct, atol=1e-5)
    # clamping: inputs beyond the envelope act as the envelope's edge
    tree["lo"] = np.full((4, K), -0.5, np.float32)
    tree["hi"] = np.full((4, K), 0.5, np.float32)
    Xc = np.clip(X, -0.5, 0.5)
    assert np.array_equal(BO.tree_output(tree, X, node), BO.tree_output(tree, Xc, node))


def test_select_features_pads_by_gradient_correlation():
    rng = np.random.default_rng(7)
    X = rng.normal(size=(4000, 6)).astype(np.float32)
    g = (3 * X[:, 4] - X[:, 1] + 0.01 * rng.normal(size=4000)).astype(np.float32)
    feature = np.array([2, 2, 5, -1, -1, -1, -1])
    f = BO.select_features(feature, X, g, 4)
    # split features by use count first, then the two most gradient-correlated
    assert f.tolist() == [2, 5, 4, 1]
    assert BO.select_features(feature, X, g, 1).tolist() == [2]


def _golden(name):
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _logistic(n, F, seed):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, F)).astype(np.float32)
    w = rng.normal(size=F)
    y = (rng.random(n) < 1 / (1 + np.exp(-(X @ w)))).astype(np.float32)
    return X, y


def _same_trees(model, d):
    off = d["node_off"]
    assert len(model["trees"]) == off.size - 1
    for t, tr in enumerate(model["trees"]):
        a, b = off[t], off[t + 1]
        assert np.array_equal(tr["feature"], d["feature"][a:b]), f"tree {t}"
        assert np.array_equal(tr["threshold"], d["threshold"][a:b]), f"tree {t}"
        assert np.array_equal(tr["left"], d["left"][a:b]) and np.array_equal(tr["right"], d["right"][a:b])
        assert np.abs(tr["value"] - d["value"][a:b]).max() <= 1e-6


def test_fp32_oracle_reproduces_reference_regression_fit():
    """The reference's estimator fit on 20 000 x 20 (25 trees, 31 leaves,
    linear leaves, interaction steering, 255 bins, y standardised)."""
    d = _golden("booster_regression_20kx20.npz")
    X, y = _cfg1(20_000, 0)
    Xt, _ = _cfg1(4_000, 11)
    mean, std = float(y.mean()), float(y.std()) or 1.0
    assert float(d["y_mean"]) == mean and float(d["y_std"]) == std
    model = BO.fit(X, (y - mean) / std, loss="mse", n_estimators=25, max_leaves=31, max_bins=255,
                   mode=O.MODE_FP32)
    assert model["base"] == pytest.approx(float(d["base"]), abs=1e-12)
    _same_trees(model, d)
    assert np.abs(BO.predict_margin(model, Xt) * std + mean - d["pred"]).max() <= 1e-5


def test_fp32_oracle_reproduces_reference_logistic_fit():
    """The reference's binary fit on 50 000 x 28 (10 depth-8 trees, 28 bins)."""
    d = _golden("booster_logistic_50kx28.npz")
    X, y = _logistic(50_000, 28, 1)
    Xt, _ = _logistic(4_000, 28, 2)
    model = BO.fit(X, y, loss="log", n_estimators=10, max_leaves=256, max_depth=8, max_bins=28,
                   neural_leaves=False, mode=O.MODE_FP32)
    assert model["base"] == pytest.approx(float(d["base"]), abs=1e-12)
    _same_trees(model, d)
    p = 1 / (1 + np.exp(-BO.predict_margin(model, Xt).astype(np.float64)))
    assert np.abs(p - d["proba"]).max() <= 1e-6


def _sparse_regression(n, F, seed):
    rng = np.random.default_rng(seed)
    X = np.where(rng.random((n, F)) < 0.1, rng.normal(size=(n, F)), 0.0).astype(np.float32)
    y = (X[:, 0] + 2 * X[:, 5] - X[:, 7] * X[:, 9] + rng.normal(scale=0.1, size=n)).astype(np.float32)
    return X, y


def test_fp32_oracle_reproduces_reference_sparse_fit():
    """The reference's fit on 30 000 x 60 with 90% zeros (10 depth-6 trees):
    sparse_hist "auto" estimates the density at about 0.1 and grows every tree
    with cgrow's sparse builder, whose default-bin cells are fp32 roundings of
    double sums (grow.c:68-107)."""
    d = _golden("booster_sparse_30kx60.npz")
    X, y = _sparse_regression(30_000, 60, 3)
    Xt, _ = _sparse_regression(4_000, 60, 4)
    mean, std = float(y.mean()), float(y.std()) or 1.0
    assert float(d["y_mean"]) == mean and float(d["y_std"]) == std
    kw = dict(loss="mse", n_estimators=10, max_leaves=64, max_depth=6, max_bins=255, neural_leaves=False,
              mode=O.MODE_FP32)
    model = BO.fit(X, (y - mean) / std, **kw)
    assert model["base"] == pytest.approx(float(d["base"]), abs=1e-12)
    _same_trees(model, d)
    # without leaf models the node values are cgrow's own: equal bit for bit,
    # which the dense builder's sums miss by up to ~2e-6 on this data
    v = np.concatenate([t["value"] for t in model["trees"]])
    assert np.array_equal(v.view(np.uint32), d["value"].view(np.uint32))
    dense = np.concatenate([t["value"] for t in BO.fit(X, (y - mean) / std, sparse_hist=False, **kw)["trees"]])
    assert not np.array_equal(dense.view(np.uint32), d["value"].view(np.uint32))
    assert np.abs(BO.predict_margin(model, Xt) * std + mean - d["pred"]).max() <= 1e-5


def test_sparse_layout_and_density():
    """The layout's default bin is the most frequent (lowest on ties), its CSR
    lists exactly the other cells row by row, and the density estimate counts
    the non-modal cells of the linspace-sampled rows (brute force with
    collections.Counter)."""
    import collections
    rng = np.random.default_rng(5)
    n, F = 9000, 7
    bins = np.where(rng.random((n, F)) < 0.8, 3, rng.integers(0, 256, (n, F))).astype(np.uint8)
    bins[:, 1] = np.arange(n) % 4                   # ties: 0..3 equally often
    bins[:, 2] = 200
    indptr, indices, data, default = BO.sparse_layout(bins)
    assert default.tolist() == [3, 0, 200, 3, 3, 3, 3]
    rebuilt = np.repeat(default[None, :], n, 0)
    for r in range(n):
        for k in range(indptr[r], indptr[r + 1]):
            assert data[k] != default[indices[k]]
            rebuilt[r, indices[k]] = data[k]
        assert np.all(np.diff(indices[indptr[r]:indptr[r + 1]]) > 0)
    assert np.array_equal(rebuilt, bins)
    idx = [int(i) for i in np.linspace(0, n - 1, 4096)]
    modal = sum(collections.Counter(bins[i, f] for i in idx).most_common(1)[0][1] for f in range(F))
    assert BO.estimate_density(bins) == pytest.approx(1 - modal / (4096 * F), abs=1e-15)
    assert BO.estimate_density(bins[:100]) == pytest.approx(
        1 - sum(collections.Counter(bins[:100, f]).most_common(1)[0][1] for f in range(F)) / (100 * F), abs=1e-15)
