"""The boosting step on the GPU (csrc/boost.hip through the C ABI) and the
booster / estimators built on it, against the boosting oracle
(oracle/boost_oracle.py).

* g, h: bit-exact for squared error; logistic within 3e-7 absolute (one
  fp32 exp evaluated by two libraries);
* margin update and forest prediction: bit-exact (same fp32 operations in
  the same order);
* whole fits: the oracle grows its trees with the fixed-point C oracle,
  whose split decisions equal the HIP grower's; split (feature, bin)
  sequences must be identical and predictions within 1e-5 (absolute, on
  targets of unit scale) -- leaf models solved in fp64 by two solvers differ
  in the last fp32 bits, so margins agree to rounding, not bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import boost_oracle as BO
from oracle import oracle as O
from yabt_amd import Booster, BoostParams, Tree, YABTClassifier, YABTRegressor
from yabt_amd import boost_ops
from yabt_amd.losses import LogLoss, MSELoss

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _cfg1(n, seed=0):
    """X ~ N(0,1) (n, 20); y = sin x0 + 0.5 x1 x2 + x3^2 + 0.3 sum x4..x9 + N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, 20)).astype(np.float32)
    y = (np.sin(X[:, 0]) + 0.5 * X[:, 1] * X[:, 2] + X[:, 3] ** 2 + 0.3 * X[:, 4:10].sum(axis=1)
         + rng.normal(scale=0.1, size=n)).astype(np.float32)
    return X, y


def _logistic(n, F, seed=0):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, F)).astype(np.float32)
    w = rng.normal(size=F)
    y = (rng.random(n) < 1 / (1 + np.exp(-(X @ w)))).astype(np.float32)
    return X, y


def _tree_of(d: dict) -> Tree:
    """Oracle tree dict -> Tree."""
    kw = {}
    if d.get("feats") is not None:
        kw = dict(leaf_net_feats=torch.from_numpy(np.asarray(d["feats"], np.int64)),
                  leaf_net_linear=torch.from_numpy(d["linear"]), leaf_net_lo=torch.from_numpy(d["lo"]),
                  leaf_net_hi=torch.from_numpy(d["hi"]))
    return Tree(feature=torch.from_numpy(d["feature"]), threshold=torch.from_numpy(d["threshold"]),
                left=torch.from_numpy(d["left"]), right=torch.from_numpy(d["right"]),
                value=torch.from_numpy(d["value"]), depth=64, **kw)


# --------------------------------------------------------------------------
# kernels
# --------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 1000, 100_003])
def test_grad_hess_mse_bit_exact(n):
    print(f"grad_hess mse n={n}", flush=True)
    rng = np.random.default_rng(n)
    m = rng.normal(size=n).astype(np.float32)
    y = rng.normal(size=n).astype(np.float32)
    g, h = boost_ops.grad_hess(MSELoss(), _t(m), _t(y))
    go, ho = BO.grad_hess("mse", m, y)
    assert np.array_equal(g.cpu().numpy(), go) and np.array_equal(h.cpu().numpy(), ho)
    # at margin + value[leaf] (the leaf-model targets)
    value = rng.normal(size=7).astype(np.float32)
    leaf = rng.integers(0, 7, size=n)
    g2, h2 = boost_ops.grad_hess(MSELoss(), _t(m), _t(y), _t(leaf), _t(value))
    go2, _ = BO.grad_hess("mse", (m + value[leaf]).astype(np.float32), y)
    assert np.array_equal(g2.cpu().numpy(), go2)


def test_grad_hess_logloss():
    print("grad_hess logloss", flush=True)
    rng = np.random.default_rng(1)
    n = 200_000
    m = (rng.normal(size=n) * 6).astype(np.float32)
    m[:4] = [-100.0, 100.0, 0.0, -0.0]
    y = (rng.random(n) < 0.4).astype(np.float32)
    g, h = boost_ops.grad_hess(LogLoss(), _t(m), _t(y))
    go, ho = BO.grad_hess("log", m, y)
    g, h = g.cpu().numpy(), h.cpu().numpy()
    assert np.abs(g - go).max() <= 3e-7
    assert np.abs(h - ho).max() <= 3e-7
    assert h.min() >= np.float32(1e-6) and h[0] == np.float32(1e-6) and h[2] == np.float32(0.25)
    value = rng.normal(size=5).astype(np.float32)
    leaf = rng.integers(0, 5, size=n)
    g2, _ = boost_ops.grad_hess(LogLoss(), _t(m), _t(y), _t(leaf), _t(value))
    go2, _ = BO.grad_hess("log", (m + value[leaf]).astype(np.float32), y)
    assert np.abs(g2.cpu().numpy() - go2).max() <= 3e-7


def _random_leaf_tree(rng, n_nodes, K, F):
    feats = rng.permutation(F)[:K]
    d = {"feature": np.full(n_nodes, -1, np.int64), "threshold": np.zeros(n_nodes, np.float32),
         "left": np.full(n_nodes, -1, np.int64), "right": np.full(n_nodes, -1, np.int64),
         "value": rng.normal(size=n_nodes).astype(np.float32)}
    if K:
        d.update(feats=feats, linear=rng.normal(size=(n_nodes, K)).astype(np.float32),
                 lo=np.full((n_nodes, K), -1.0, np.float32), hi=np.full((n_nodes, K), 1.5, np.float32))
    return d


@pytest.mark.parametrize("K", [0, 1, 3, 8])
def test_margin_update_bit_exact(K):
    print(f"margin_update K={K}", flush=True)
    rng = np.random.default_rng(10 + K)
    n, F, N = 50_001, 11, 9
    d = _random_leaf_tree(rng, N, K, F)
    leaf = rng.integers(0, N, size=n)
    margin = rng.normal(size=n).astype(np.float32)
    # fp32 row-major inputs with a padded leading dimension
    Xpad = rng.normal(size=(n, F + 5)).astype(np.float32) * 2
    X = Xpad[:, :F]
    out = _t(margin)
    boost_ops.margin_update(out, _t(leaf), _tree_of(d), _t(Xpad)[:, :F], x_kind=0)
    want = (margin + BO.tree_output(d, X, leaf)).astype(np.float32)
    assert np.array_equal(out.cpu().numpy(), want)
    # the same inputs fp32 feature-major (the estimators' per-fit copy)
    Xfm = np.zeros((F, n + 3), np.float32)
    Xfm[:, :n] = X.T
    out = _t(margin)
    boost_ops.margin_update(out, _t(leaf), _tree_of(d), _t(Xfm), x_kind=2)
    assert np.array_equal(out.cpu().numpy(), want)
    # uint8 feature-major inputs, x = float(bin)
    bins = rng.integers(0, 256, size=(F, n + 13), dtype=np.uint8)
    if K:
        d["lo"][:] = 10.0
        d["hi"][:] = 200.0
    out = _t(margin)
    boost_ops.margin_update(out, _t(leaf), _tree_of(d), _t(bins), x_kind=1)
    want = (margin + BO.tree_output(d, bins[:, :n].T.astype(np.float32), leaf)).astype(np.float32)
    assert np.array_equal(out.cpu().numpy(), want)


def test_predict_forest_bit_exact():
    print("predict forest", flush=True)
    X, y = _cfg1(4000, seed=2)
    model = BO.fit(X, y, n_estimators=6, max_leaves=15, max_bins=63)
    trees = [_tree_of(t) for t in model["trees"]]
    Xt, _ = _cfg1(3001, seed=3)
    Xt[:5] *= 40  # far outside the leaf envelopes: clamping decides
    forest = boost_ops.Forest(trees, DEV)
    got = boost_ops.predict(forest, _t(Xt), model["base"]).cpu().numpy()
    assert np.array_equal(got, BO.predict_margin(model, Xt))
    # the first k trees, accumulated one tree at a time
    acc = torch.full((Xt.shape[0],), model["base"], device=DEV)
    for tr in trees[:4]:
        boost_ops.predict(boost_ops.Forest([tr], DEV), _t(Xt), out=acc, accumulate=True)
    assert np.array_equal(acc.cpu().numpy(), BO.predict_margin(model, Xt, n_trees=4))
    # Tree.predict / Tree.apply on CPU inputs run on the device
    tr = trees[0]
    node = BO.route(Xt, model["trees"][0]["feature"], model["trees"][0]["threshold"],
                    model["trees"][0]["left"], model["trees"][0]["right"])
    assert np.array_equal(tr.apply(torch.from_numpy(Xt)).numpy(), node)
    assert np.array_equal(tr.predict(torch.from_numpy(Xt)).numpy(),
                          BO.tree_output(model["trees"][0], Xt, node))


def test_predict_empty_forest_and_rows():
    forest = boost_ops.Forest([], DEV)
    X = torch.randn(100, 4, device=DEV)
    assert torch.all(boost_ops.predict(forest, X, 0.25) == 0.25)
    assert boost_ops.predict(forest, X[:0], 0.25).numel() == 0


# --------------------------------------------------------------------------
# fits
# --------------------------------------------------------------------------

def _same_splits(trees, otrees):
    for i, (t, o) in enumerate(zip(trees, otrees)):
        f = t.feature.cpu().numpy()
        assert np.array_equal(f, o["feature"]), f"tree {i}: split features differ"
        thr = t.threshold.cpu().numpy()
        assert np.array_equal(thr[f >= 0], o["threshold"][o["feature"] >= 0]), f"tree {i}: thresholds differ"
        assert np.array_equal(t.left.cpu().numpy(), o["left"]) and np.array_equal(t.right.cpu().numpy(), o["right"])


@pytest.mark.parametrize("neural", [False, True])
def test_booster_mse_matches_oracle(neural):
    print(f"booster mse neural={neural}", flush=True)
    X, y = _cfg1(20_000)
    kw = dict(n_estimators=8, learning_rate=0.1, max_leaves=31, max_bins=255, neural_leaves=neural)
    b = Booster(BoostParams(**kw), MSELoss()).fit(X, y)
    model = BO.fit(X, y, loss="mse", **kw)
    assert len(b.trees) == 8
    _same_splits(b.trees, model["trees"])
    assert b.base_score == pytest.approx(model["base"], abs=1e-7)
    Xt, _ = _cfg1(5000, seed=9)
    got = b.predict_margin(Xt)
    want = BO.predict_margin(model, Xt)
    assert np.abs(got - want).max() <= 1e-5
    if not neural:
        assert np.array_equal(got, want)  # no leaf models: every step is bit-exact


def test_regressor_config1_matches_oracle():
    """The estimator on 20 000 x 20, 25 trees, 31 leaves, lr 0.1, linear leaves,
    255 bins: identical splits, predictions within 1e-5 of the target scale."""
    print("regressor config 1", flush=True)
    X, y = _cfg1(20_000)
    est = YABTRegressor(n_estimators=25, max_leaves=31, learning_rate=0.1, max_bins=255,
                        neural_leaves=True, refine_steps=0)
    est.fit(X, y)
    mean, std = float(y.mean()), float(y.std()) or 1.0
    model = BO.fit(X, (y - mean) / std, loss="mse", n_estimators=25, max_leaves=31, max_bins=255)
    _same_splits(est.booster_.trees, model["trees"])
    Xt, yt = _cfg1(4000, seed=11)
    got = est.predict(Xt)
    want = BO.predict_margin(model, Xt) * std + mean
    assert np.abs(got - want).max() <= 1e-5 * std
    r2 = 1 - np.mean((got - yt) ** 2) / np.var(yt)
    assert r2 > 0.6


def test_classifier_binary_matches_oracle():
    print("classifier binary", flush=True)
    X, y = _logistic(30_000, 10, seed=4)
    labels = np.where(y > 0, 7.0, -2.0)
    est = YABTClassifier(n_estimators=6, max_leaves=16, max_depth=4, max_bins=28, neural_leaves=False)
    est.fit(X, labels)
    assert est.classes_.tolist() == [-2.0, 7.0]
    model = BO.fit(X, y, loss="log", n_estimators=6, max_leaves=16, max_depth=4, max_bins=28,
                   neural_leaves=False)
    _same_splits(est.booster_.trees, model["trees"])
    Xt, _ = _logistic(3000, 10, seed=5)
    p = est.predict_proba(Xt)
    po = 1 / (1 + np.exp(-BO.predict_margin(model, Xt).astype(np.float64)))
    assert np.abs(p[:, 1] - po).max() <= 1e-5
    assert np.allclose(p.sum(axis=1), 1.0)
    assert set(np.unique(est.predict(Xt)).tolist()) <= {-2.0, 7.0}


def test_multiclass_one_vs_rest():
    print("multiclass", flush=True)
    rng = np.random.default_rng(6)
    X = rng.normal(size=(9000, 6)).astype(np.float32)
    y = np.digitize(X[:, 0] + 0.5 * X[:, 1], [-0.7, 0.7]).astype(np.float32)  # 3 classes
    est = YABTClassifier(n_estimators=4, max_leaves=8, max_bins=64, neural_leaves=True)
    est.fit(X, y)
    Xt = rng.normal(size=(1000, 6)).astype(np.float32)
    P = est.predict_proba(Xt)
    margins = []
    for c in range(3):
        m = BO.fit(X, (y == c).astype(np.float32), loss="log", n_estimators=4, max_leaves=8, max_bins=64)
        _same_splits(est.booster_.boosters_[c].trees, m["trees"])
        margins.append(BO.predict_margin(m, Xt).astype(np.float64))
    M = np.stack(margins, axis=1)
    Po = np.exp(M - M.max(axis=1, keepdims=True))
    Po /= Po.sum(axis=1, keepdims=True)
    assert np.abs(P - Po).max() <= 1e-5
    assert (est.predict(Xt) == np.argmax(Po, axis=1)).mean() > 0.999


def test_sampling_matches_oracle():
    print("subsample/colsample", flush=True)
    X, y = _cfg1(12_000, seed=12)
    kw = dict(n_estimators=5, max_leaves=12, max_bins=64, subsample=0.8, colsample=0.5, seed=3)
    b = Booster(BoostParams(neural_leaves=True, **kw), MSELoss()).fit(X, y)
    model = BO.fit(X, y, loss="mse", neural_leaves=True, **kw)
    _same_splits(b.trees, model["trees"])
    Xt, _ = _cfg1(2000, seed=13)
    assert np.abs(b.predict_margin(Xt) - BO.predict_margin(model, Xt)).max() <= 1e-5


def test_eval_set_early_stopping():
    """The early-stopping bookkeeping of boosting.py:512-532: best_iter is the
    first eval loss that beats the best so far by 1e-7, the fit stops after
    early_stopping_rounds rounds without one, and predict_margin uses the
    first best_iter + 1 trees.  The eval losses are recomputed from the
    forest prediction (bit-exact with the per-round margin update) with the
    loss's own torch expression."""
    print("eval set", flush=True)
    X, y = _cfg1(6000, seed=14)
    Xv, yv = _cfg1(2000, seed=15)
    yv = yv + np.random.default_rng(0).normal(scale=3.0, size=yv.size).astype(np.float32)  # noisy: stops early
    p = BoostParams(n_estimators=40, max_leaves=31, max_bins=64, learning_rate=0.5, early_stopping_rounds=3,
                    neural_leaves=False)
    b = Booster(p, MSELoss()).fit(X, y, eval_set=(Xv, yv))
    model = BO.fit(X, y, loss="mse", n_estimators=len(b.trees), max_leaves=31, max_bins=64, learning_rate=0.5,
                   neural_leaves=False)
    _same_splits(b.trees, model["trees"])
    Xvt, yvt = _t(Xv), _t(yv)
    losses = [float(MSELoss.loss(b._margin(Xvt, k + 1), yvt)) for k in range(len(b.trees))]
    best, best_i, since = float("inf"), None, 0
    for i, v in enumerate(losses):
        if v < best - 1e-7:
            best, best_i, since = v, i, 0
        else:
            since += 1
    assert b.best_iter == best_i
    assert len(b.trees) < 40 and since == 3
    assert np.array_equal(b.predict_margin(Xv), BO.predict_margin(model, Xv, n_trees=best_i + 1))
    assert np.array_equal(b.predict_margin(Xv, use_best_iter=False), BO.predict_margin(model, Xv))
