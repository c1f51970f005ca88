"""The 10-class linear-leaf workload (2M x 50 in the benchmark) at reduced
rows, through the estimator, against the boosting oracle.

The reference has no softmax booster: more than two classes are one-vs-rest,
one LogLoss ``Booster`` per class over the same binned X
(yabt/multiclass.py:18-48), and the probabilities are the softmax of the
per-class margins.  Parameters are the benchmark's: 50 features, 256 bins, 63
leaves, linear leaf models over K = 8 inputs with ridge ``leaf_net_l2`` = 1e-3
and the bias penalty 1e-8 (yabt/neural_leaves.py:76-87).

Per class, every tree must have the oracle's split features, thresholds and
children, and the oracle's leaf-model inputs; the softmax probabilities must
agree within 1e-5.  A second fit with 6 leaves (at most 5 distinct split
features) makes the input selection pad with features ranked by gradient
correlation (yabt/neural_leaves.py:27-39), which 63-leaf trees never need.
"""

import numpy as np
import pytest
import torch

from oracle import boost_oracle as BO
from yabt_amd import YABTClassifier

pytestmark = pytest.mark.gpu


def _softmax_classes(n, F, C, seed):
    """X ~ N(0,1) (n, F); y = argmax(X W + Gumbel noise), W ~ N(0,1) (F, C)
    -- the benchmark's generator."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, F)).astype(np.float32)
    W = rng.normal(size=(F, C)).astype(np.float32)
    y = np.argmax(X @ W + rng.gumbel(size=(n, C)).astype(np.float32), axis=1).astype(np.float32)
    return X, y


def _check_class(booster, model, c):
    assert len(booster.trees) == len(model["trees"])
    for i, (t, o) in enumerate(zip(booster.trees, model["trees"])):
        f = t.feature.cpu().numpy()
        assert np.array_equal(f, o["feature"]), f"class {c} tree {i}: split features differ"
        thr = t.threshold.cpu().numpy()
        assert np.array_equal(thr[f >= 0], o["threshold"][o["feature"] >= 0]), \
            f"class {c} tree {i}: thresholds differ"
        assert np.array_equal(t.left.cpu().numpy(), o["left"])
        assert np.array_equal(t.right.cpu().numpy(), o["right"])
        feats = None if t.leaf_net_feats is None else t.leaf_net_feats.cpu().numpy()
        want = o.get("feats")
        assert (feats is None) == (want is None), f"class {c} tree {i}: leaf models present on one side only"
        if want is not None:
            assert np.array_equal(feats, np.asarray(want, np.int64)), f"class {c} tree {i}: leaf inputs differ"


def _oracle_proba(models, Xt):
    M = np.stack([BO.predict_margin(m, Xt).astype(np.float64) for m in models], axis=1)
    P = np.exp(M - M.max(axis=1, keepdims=True))
    return P / P.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("max_leaves,n_trees,K_padded", [(63, 3, False), (6, 2, True)])
def test_ten_class_linear_leaves(max_leaves, n_trees, K_padded):
    print(f"10-class one-vs-rest, 100000 x 50, {max_leaves} leaves, {n_trees} trees, K=8, l2 1e-3",
          flush=True)
    n, F, C = 100_000, 50, 10
    X, y = _softmax_classes(n, F, C, seed=21)
    kw = dict(n_estimators=n_trees, max_leaves=max_leaves, learning_rate=0.1, max_bins=256,
              neural_leaves=True, leaf_net_features=8, leaf_net_l2=1e-3)
    est = YABTClassifier(**kw)
    est.fit(X, y)
    assert est.classes_.tolist() == list(range(C))
    Xt, _ = _softmax_classes(5000, F, C, seed=22)
    P = est.predict_proba(Xt)
    models = []
    for c in range(C):
        m = BO.fit(X, (y == c).astype(np.float32), loss="log", **kw)
        _check_class(est.booster_.boosters_[c], m, c)
        models.append(m)
        if K_padded:
            # 6 leaves: at most 5 split features, the rest of the 8 inputs come
            # from the gradient-correlation ranking
            t0 = est.booster_.boosters_[c].trees[0]
            n_split = np.unique(t0.feature.cpu().numpy()[t0.feature.cpu().numpy() >= 0]).size
            assert n_split < 8 and t0.leaf_net_feats.numel() == 8
    Po = _oracle_proba(models, Xt)
    assert np.abs(P - Po).max() <= 1e-5
    assert np.allclose(P.sum(axis=1), 1.0)
    assert (est.predict(Xt) == np.argmax(Po, axis=1)).mean() > 0.999


def test_concurrent_class_fits_equal_sequential():
    """The class boosters fitted on concurrent streams (4 threads) are the
    sequential fit's, bit for bit: node arrays, values, leaf models and the
    training margins."""
    from yabt_amd.boosting import BoostParams, MulticlassBooster
    print("10-class one-vs-rest, concurrent vs sequential class fits, 60000 x 30", flush=True)
    X, y = _softmax_classes(60_000, 30, 10, seed=23)
    p = BoostParams(n_estimators=4, max_leaves=31, learning_rate=0.1, max_bins=256, neural_leaves=True,
                    leaf_net_features=8, leaf_net_l2=1e-3)
    seq = MulticlassBooster(p, concurrency=1).fit(X, y)
    con = MulticlassBooster(p, concurrency=4).fit(X, y)
    assert len(seq.boosters_) == len(con.boosters_) == 10
    for a, b in zip(seq.boosters_, con.boosters_):
        assert np.array_equal(a.margin_.cpu().numpy().view(np.uint32), b.margin_.cpu().numpy().view(np.uint32))
        for ta, tb in zip(a.trees, b.trees):
            for k in ("feature", "threshold", "left", "right", "value", "leaf_net_feats", "leaf_net_linear",
                      "leaf_net_lo", "leaf_net_hi"):
                u, v = getattr(ta, k), getattr(tb, k)
                assert (u is None) == (v is None)
                if u is not None:
                    assert np.array_equal(u.cpu().numpy(), v.cpu().numpy()), k
    Xt, _ = _softmax_classes(2000, 30, 10, seed=24)
    assert np.array_equal(seq.predict_proba(Xt), con.predict_proba(Xt))
