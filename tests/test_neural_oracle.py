"""The linear-leaf oracle against independent formulations (CPU only).

* fit_linear: the ridge normal equations against a least-squares solve of the
  same objective, sum h (x1 . theta + g / h)^2 + lam |w|^2 + 1e-8 b^2, written
  as an augmented system (numpy.linalg.lstsq, a different algorithm);
* eligibility: internal nodes and leaves under min_samples keep zeros;
* envelopes: per-node min / max by brute force;
* fold: the raw-space model equals lr (w . (x - mu) / sd + b) + value.
"""

import numpy as np
import pytest

from oracle import neural_oracle as NO


def _problem(seed, n=3000, K=5, n_nodes=9):
    rng = np.random.default_rng(seed)
    Xs = rng.normal(size=(n, K)).astype(np.float32) * np.float32(3) + np.float32(1)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
    feature = np.full(n_nodes, -1, np.int64)
    feature[[0, 1, 3]] = [2, 0, 1]          # internal nodes
    leaves = np.nonzero(feature == -1)[0]
    leaf = rng.choice(leaves, size=n, p=np.linspace(1, 3, leaves.size) / np.linspace(1, 3, leaves.size).sum())
    mu = Xs.mean(axis=0).astype(np.float32)
    sd = Xs.std(axis=0, ddof=1).astype(np.float32)
    return Xs, g, h, leaf.astype(np.int64), feature, mu, sd


@pytest.mark.parametrize("lam", [1.0, 1e-3, 0.0])
def test_fit_linear_against_lstsq(lam):
    Xs, g, h, leaf, feature, mu, sd = _problem(1)
    n_nodes, K = feature.size, Xs.shape[1]
    Xn = NO.standardise(Xs, mu, sd)
    cnt = NO.counts(leaf, n_nodes)
    elig = NO.eligible_nodes(feature, cnt, 50)
    W, db = NO.fit_linear(Xn, g, h, leaf, elig, n_nodes, lam)
    for l in np.nonzero(elig)[0]:
        r = leaf == l
        X1 = np.concatenate([Xn[r].astype(np.float64), np.ones((r.sum(), 1))], axis=1)
        sw = np.sqrt(h[r].astype(np.float64))
        A = X1 * sw[:, None]
        t = -g[r].astype(np.float64) / sw
        pen = np.sqrt(np.r_[np.full(K, lam), 1e-8])
        A = np.vstack([A, np.diag(pen)])
        t = np.r_[t, np.zeros(K + 1)]
        theta = np.linalg.lstsq(A, t, rcond=None)[0]
        np.testing.assert_allclose(W[l], theta[:K].astype(np.float32), rtol=2e-5, atol=1e-6)
        np.testing.assert_allclose(db[l], np.float32(theta[K]), rtol=2e-5, atol=1e-6)


def test_ineligible_nodes_keep_zeros():
    Xs, g, h, leaf, feature, mu, sd = _problem(2, n=400)
    n_nodes = feature.size
    cnt = NO.counts(leaf, n_nodes)
    ms = int(np.sort(cnt[feature == -1])[2]) + 1   # the two smallest leaves fall below it
    elig = NO.eligible_nodes(feature, cnt, ms)
    assert (~elig[feature >= 0]).all()
    W, db = NO.fit_linear(NO.standardise(Xs, mu, sd), g, h, leaf, elig, n_nodes, 1.0)
    assert (W[~elig] == 0).all() and (db[~elig] == 0).all()
    assert (np.abs(W[elig]).sum(axis=1) > 0).all()


def test_envelopes_brute_force():
    Xs, g, h, leaf, feature, mu, sd = _problem(3, n=500)
    lo, hi = NO.envelopes(Xs, leaf, feature.size)
    for l in range(feature.size):
        r = leaf == l
        if r.any():
            assert (lo[l] == Xs[r].min(axis=0)).all() and (hi[l] == Xs[r].max(axis=0)).all()
        else:
            assert np.isinf(lo[l]).all() and (lo[l] > 0).all() and (hi[l] < 0).all()


def test_fold_is_the_standardised_model():
    Xs, g, h, leaf, feature, mu, sd = _problem(4)
    n_nodes = feature.size
    Xn = NO.standardise(Xs, mu, sd)
    elig = NO.eligible_nodes(feature, NO.counts(leaf, n_nodes), 50)
    W, db = NO.fit_linear(Xn, g, h, leaf, elig, n_nodes, 1.0)
    value = np.linspace(-1, 1, n_nodes).astype(np.float32)
    lr = 0.1
    v2, lin = NO.fold(value, W, db, mu, sd, lr)
    raw = v2[leaf] + (lin[leaf] * Xs).sum(axis=1)
    direct = value[leaf] + lr * ((W[leaf] * Xn).sum(axis=1) + db[leaf])
    np.testing.assert_allclose(raw, direct, rtol=1e-4, atol=1e-5)
