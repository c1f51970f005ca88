"""Linear leaf models (yabt_leaf_fit) against the oracle, through the C ABI.

Counts and envelopes must be identical; weights and biases, solved in fp64 on
exact fixed-point sums of the reference's fp64 products, within 1e-5 relative
of the oracle's fp64 normal equations (the fp32 outputs of two fp64 solves).
Two calls give identical bits, and the uint8 input path equals the fp32 path
on the same values.
"""

from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import neural_oracle as NO
from tests.helpers import grad_hess, uniform_bins
from yabt_amd import IdentityBinner, TreeParams, grow_tree_hip
from yabt_amd import grow_hip as G
from yabt_amd.losses import MSELoss
from yabt_amd.neural_leaves import fit_leaf_networks, fold, leaf_fit, leaf_moments
from yabt_amd.tree import Tree

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _problem(seed, n, K, n_nodes, bins=False):
    rng = np.random.default_rng(seed)
    F = K + 3
    if bins:
        X = uniform_bins(rng, n, F)                      # (n, F) u8
        Xf = X.astype(np.float32)
    else:
        Xf = (rng.normal(size=(n, F)) * 2 + 0.5).astype(np.float32)
        X = Xf
    feats = rng.permutation(F)[:K].astype(np.int32)
    g, h = grad_hess(rng, n)
    feature = np.full(n_nodes, -1, np.int64)
    feature[: n_nodes // 2] = rng.integers(0, F, n_nodes // 2)   # the first half are internal
    leaves = np.nonzero(feature == -1)[0]
    leaf = rng.choice(leaves, size=n).astype(np.int64)
    Xs = Xf[:, feats]
    mu = Xs.mean(axis=0).astype(np.float32)
    sd = np.maximum(Xs.std(axis=0, ddof=1), 1e-6).astype(np.float32)
    return X, Xf, feats, g, h, feature, leaf, mu, sd


def _oracle(Xf, feats, g, h, feature, leaf, mu, sd, min_samples, lam):
    n_nodes = feature.size
    Xs = Xf[:, feats]
    cnt = NO.counts(leaf, n_nodes)
    lo, hi = NO.envelopes(Xs, leaf, n_nodes)
    W, db = NO.fit_linear(NO.standardise(Xs, mu, sd), g, h, leaf, NO.eligible_nodes(feature, cnt, min_samples),
                          n_nodes, lam)
    return W, db, lo, hi, cnt


def _gpu(X, x_kind, feats, g, h, feature, leaf, mu, sd, min_samples, lam, gram="exact", pad=False):
    """pad: uint8 inputs as (F, ld) with ld a multiple of 16 above n (the
    grower's feature-major layout), so the 4-row vector loads apply."""
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    if x_kind == 0:
        Xd = t(X)
    elif pad:
        n = X.shape[0]
        Xp = np.zeros((X.shape[1], (n + 15) // 16 * 16 + 16), np.uint8)
        Xp[:, :n] = X.T
        Xd = t(Xp)
    else:
        Xd = t(np.ascontiguousarray(X.T))
    out = leaf_fit(Xd, x_kind, t(feats), t(mu), t(sd), t(g), t(h), t(leaf), t(feature), min_samples, lam,
                   gram=gram)
    return [o.cpu().numpy() for o in out]


@pytest.mark.parametrize("gram", ["exact", "mfma"])
@pytest.mark.parametrize("n,K,n_nodes,x_kind,lam", [
    (5000, 8, 61, 0, 1.0), (20_000, 5, 31, 1, 1e-3), (777, 1, 7, 0, 1.0), (300_000, 8, 511, 1, 1.0),
    (40_000, 3, 1501, 0, 0.5),   # more nodes than the LDS tables hold
    (2_000_000, 8, 63, 1, 1e-3),   # leaves of ~60 000 rows: many Gram chunks per leaf
])
def test_leaf_fit_matches_oracle(n, K, n_nodes, x_kind, lam, gram):
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(n + K, n, K, n_nodes, bins=x_kind == 1)
    W, b, lo, hi, cnt = _gpu(X, x_kind, feats, g, h, feature, leaf, mu, sd, 50, lam, gram)
    rW, rb, rlo, rhi, rcnt = _oracle(Xf, feats, g, h, feature, leaf, mu, sd, 50, lam)
    assert np.array_equal(cnt, rcnt)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    np.testing.assert_allclose(W, rW, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(b, rb, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n,K,n_nodes", [(20_003, 5, 31), (4_097, 8, 15), (1_000_001, 7, 255)])
def test_leaf_fit_vector_rows_match_oracle(n, K, n_nodes):
    """uint8 inputs in the padded feature-major layout: four rows per thread
    in the stats and scatter passes, the last n % 4 rows one by one."""
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(n + 7, n, K, n_nodes, bins=True)
    W, b, lo, hi, cnt = _gpu(X, 1, feats, g, h, feature, leaf, mu, sd, 50, 1e-3, pad=True)
    rW, rb, rlo, rhi, rcnt = _oracle(Xf, feats, g, h, feature, leaf, mu, sd, 50, 1e-3)
    assert np.array_equal(cnt, rcnt)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    np.testing.assert_allclose(W, rW, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(b, rb, rtol=1e-5, atol=1e-6)
    # the same bits as the unpadded (one row at a time) layout
    u = _gpu(X, 1, feats, g, h, feature, leaf, mu, sd, 50, 1e-3)
    for x, y in zip((W, b, lo, hi, cnt), u):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("n,K,x_kind", [(1, 1, 0), (1000, 3, 0), (100_003, 8, 1), (2_000_000, 5, 1)])
def test_leaf_moments(n, K, x_kind):
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(n, n, K, 5, bins=x_kind == 1)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    Xd = t(X) if x_kind == 0 else t(np.ascontiguousarray(X.T))
    m, s = (v.cpu().numpy() for v in leaf_moments(Xd, x_kind, t(feats), n))
    rm, rs = NO.moments(Xf[:, feats])
    np.testing.assert_allclose(m, rm, rtol=2e-7, atol=0)
    if n > 1:
        np.testing.assert_allclose(s, rs, rtol=2e-7, atol=0)
    a = [v.cpu().numpy() for v in leaf_moments(Xd, x_kind, t(feats), n)]
    assert np.array_equal(a[0], m) and np.array_equal(a[1], s)


@pytest.mark.parametrize("gram", ["exact", "mfma"])
def test_leaf_fit_deterministic_and_u8_equals_f32(gram):
    """Exact sums: identical bits on every call and for either input path.
    The fp64 MFMA sums depend on the order of a leaf's rows, which the scatter
    does not fix: equal to 1e-12 there."""
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(9, 50_000, 6, 63, bins=True)
    a = _gpu(X, 1, feats, g, h, feature, leaf, mu, sd, 50, 1.0, gram)
    b = _gpu(X, 1, feats, g, h, feature, leaf, mu, sd, 50, 1.0, gram)
    c = _gpu(Xf, 0, feats, g, h, feature, leaf, mu, sd, 50, 1.0, gram)
    for u, v, w in zip(a, b, c):
        if gram == "exact":
            assert np.array_equal(u, v)
            assert np.array_equal(u, w)
        else:
            np.testing.assert_allclose(u, v, rtol=1e-6, atol=1e-9)
            np.testing.assert_allclose(u, w, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("n,K,n_nodes,ld_pad", [(50_000, 6, 63, 0), (20_003, 8, 31, 1), (777, 1, 7, 3),
                                                 (1_000_001, 7, 255, 0), (40_000, 3, 1501, 1)])
def test_leaf_fit_f32_feature_major_equals_row_major(n, K, n_nodes, ld_pad):
    """fp32 inputs feature-major (x_kind 2, the estimators' per-fit copy):
    the same bits as row-major (x_kind 0), fit and moments, with the 4-row
    vector loads (ld a multiple of 4, ld_pad 0) and without them (odd ld)."""
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(n + 11, n, K, n_nodes)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    ld = (n + 3) // 4 * 4 + ld_pad
    Xp = np.zeros((Xf.shape[1], ld), np.float32)
    Xp[:, :n] = Xf.T
    row = leaf_fit(t(Xf), 0, t(feats), t(mu), t(sd), t(g), t(h), t(leaf), t(feature), 50, 1e-3)
    col = leaf_fit(t(Xp), 2, t(feats), t(mu), t(sd), t(g), t(h), t(leaf), t(feature), 50, 1e-3)
    for u, v in zip(row, col):
        assert np.array_equal(u.cpu().numpy(), v.cpu().numpy())
    m0 = [v.cpu().numpy() for v in leaf_moments(t(Xf), 0, t(feats), n)]
    m2 = [v.cpu().numpy() for v in leaf_moments(t(Xp), 2, t(feats), n)]
    assert np.array_equal(m0[0], m2[0]) and np.array_equal(m0[1], m2[1])
    rW, rb, rlo, rhi, rcnt = _oracle(Xf, feats, g, h, feature, leaf, mu, sd, 50, 1e-3)
    np.testing.assert_allclose(col[0].cpu().numpy(), rW, rtol=1e-5, atol=1e-6)
    assert np.array_equal(col[4].cpu().numpy(), rcnt)


@pytest.mark.parametrize("K", [1, 5, 8])
def test_leaf_fold_equals_torch_expressions(K):
    """yabt_leaf_fold bit for bit against the reference's own torch fold
    (neural_leaves.py:178-184) evaluated on the device."""
    rng = np.random.default_rng(K)
    N = 301
    W = torch.from_numpy(rng.normal(size=(N, K)).astype(np.float32)).to(DEV)
    db = torch.from_numpy(rng.normal(size=N).astype(np.float32)).to(DEV)
    mu = torch.from_numpy((rng.normal(size=K) * 3).astype(np.float32)).to(DEV)
    sd = torch.from_numpy(rng.uniform(0.1, 5.0, size=K).astype(np.float32)).to(DEV)
    value = torch.from_numpy(rng.normal(size=N).astype(np.float32)).to(DEV)
    W[::7] = 0.0
    db[::7] = 0.0
    lr = 0.1
    tree = Tree(torch.full((N,), -1, dtype=torch.int64), torch.zeros(N), torch.zeros(N, dtype=torch.int64),
                torch.zeros(N, dtype=torch.int64), value, 0)
    out = fold(tree, W, db, mu, sd, lr, torch.arange(K), None, None)
    prod = W * (mu / sd)
    acc = prod[:, 0].clone()
    for j in range(1, K):
        acc = acc + prod[:, j]
    ref_value = value + lr * (db - acc)
    ref_linear = lr * W / sd
    assert torch.equal(out.value, ref_value)
    assert torch.equal(out.leaf_net_linear, ref_linear)


def test_leaf_fit_rejects_bad_leaf_ids():
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(3, 1000, 2, 9)
    leaf[17] = 9
    with pytest.raises(ValueError):
        _gpu(X, 0, feats, g, h, feature, leaf, mu, sd, 50, 1.0)


def test_leaf_fit_rejects_bad_leaf_ids_vector_rows():
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(5, 10_001, 4, 9, bins=True)
    leaf[4_001] = -3
    with pytest.raises(ValueError):
        _gpu(X, 1, feats, g, h, feature, leaf, mu, sd, 50, 1.0, pad=True)


def test_leaf_fit_rejects_nonfinite_inputs():
    X, Xf, feats, g, h, feature, leaf, mu, sd = _problem(4, 1000, 3, 9)
    X = X.copy()
    X[5, feats[1]] = np.nan
    with pytest.raises(ValueError):
        _gpu(X, 0, feats, g, h, feature, leaf, mu, sd, 50, 1.0)


@dataclass
class _P:
    learning_rate: float = 0.1
    leaf_net_features: int = 8
    leaf_net_min_samples: int = 50
    leaf_net_l2: float = 1.0
    leaf_net_hidden: int = 0


def test_fit_leaf_networks_end_to_end():
    """grow_tree_hip + fit_leaf_networks against the oracle on the same
    selected features and standardisation (neural_leaves.py:131-184)."""
    rng = np.random.default_rng(11)
    n, F = 30_000, 12
    Xf = rng.normal(size=(n, F)).astype(np.float32)
    y = (np.sin(Xf[:, 0]) + 0.5 * Xf[:, 1] * Xf[:, 2] + Xf[:, 3] ** 2).astype(np.float32)
    binner = IdentityBinner(F, 256)
    bins = np.clip(np.floor((Xf + 4) * 32), 0, 255).astype(np.uint8)
    Xraw = bins.astype(np.float32)
    margin = np.zeros(n, np.float32)
    g, h = MSELoss.grad_hess(torch.from_numpy(margin), torch.from_numpy(y))
    tree = grow_tree_hip(torch.from_numpy(bins).to(DEV), g.to(DEV), h.to(DEV), binner, TreeParams(max_leaves=31))
    Xd, yd, md = (torch.from_numpy(a).to(DEV) for a in (Xraw, y, margin))
    out = fit_leaf_networks(tree, Xd, yd, md, MSELoss, _P())
    feats = out.leaf_net_feats.cpu().numpy()
    used = tree.feature.cpu().numpy()
    used = used[used >= 0]
    # the most used split features come first
    counts = np.bincount(used, minlength=F)
    m = min(8, len(set(used.tolist())))
    assert (np.diff(counts[feats[:m]]) <= 0).all() and (counts[feats[:m]] > 0).all()
    mu, sd = (torch.from_numpy(v) for v in NO.moments(Xraw[:, feats]))
    leaf = tree.apply(Xd).cpu().numpy()
    value = tree.value.cpu().numpy()
    g2 = (margin + value[leaf] - y).astype(np.float32)
    h2 = np.ones(n, np.float32)
    feature = tree.feature.cpu().numpy()
    W, db, lo, hi, cnt = _oracle(Xraw, feats.astype(np.int32), g2, h2, feature, leaf, mu.cpu().numpy(),
                                 sd.cpu().numpy(), 50, 1.0)
    v2, lin = NO.fold(value, W, db, mu.cpu().numpy(), sd.cpu().numpy(), 0.1)
    np.testing.assert_allclose(out.value.cpu().numpy(), v2, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out.leaf_net_linear.cpu().numpy(), lin, rtol=1e-5, atol=1e-7)
    assert np.array_equal(out.leaf_net_lo.cpu().numpy(), lo)
    assert np.array_equal(out.leaf_net_hi.cpu().numpy(), hi)
    # the fitted model lowers the squared loss of the constant tree on its rows
    pred0 = value[leaf]
    pred1 = out.predict(Xd).cpu().numpy()
    assert ((pred1 - (y - margin)) ** 2).mean() < ((pred0 - (y - margin)) ** 2).mean()


def _rank_device(feature, F, k):
    """yabt_leaf_rank_features through the C ABI: (feats[:k] int64, n used)."""
    from yabt_amd import _lib
    lib = _lib.load()
    ft = torch.as_tensor(feature, dtype=torch.int64, device=DEV)
    out = torch.full((k,), -7, dtype=torch.int64, device=DEV)
    out32 = torch.full((k,), -7, dtype=torch.int32, device=DEV)
    m = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    st = torch.cuda.current_stream(DEV).cuda_stream
    _lib.check(lib.yabt_leaf_rank_features(ft.data_ptr(), int(ft.numel()), F, k, out.data_ptr(), out32.data_ptr(),
                                           m.data_ptr(), st), "yabt_leaf_rank_features")
    torch.cuda.synchronize()
    assert torch.equal(out.to(torch.int32), out32)
    return out.cpu(), int(m.item())


def _rank_cases():
    rng = np.random.default_rng(11)
    cases = []
    for trial in range(160):
        F = int(rng.choice([1, 3, 8, 28, 100, 500, 4096]))
        N = int(rng.choice([1, 3, 31, 255, 511, 2047, 2049]))
        spread = int(rng.integers(1, F + 1))
        feature = rng.integers(0, spread, N)
        if trial % 4 == 1:
            feature = np.sort(feature)                     # ties met in sorted runs
        if trial % 4 == 2:
            feature[:N // 2] = rng.integers(0, max(1, spread // 8), N // 2)   # a few dominant features
        feature[rng.random(N) < 0.5] = -1                  # leaves
        cases.append((feature, F, int(rng.integers(1, 9))))
    cases.append((np.full(7, -1, np.int64), 10, 8))        # no internal node
    cases.append((np.arange(40, dtype=np.int64) % 20, 20, 8))   # 20 features, all counts equal
    return cases


def test_leaf_rank_features_equals_torch_cpu_argsort():
    """The device ranking gives torch's unique + CPU argsort order (the
    reference's _used_features), ties included, for trees using more or fewer
    features than k."""
    from yabt_amd.neural_leaves import _used_features
    for feature, F, k in _rank_cases():
        got, m = _rank_device(feature, F, k)
        want = _used_features(torch.as_tensor(feature), k)
        f = feature[feature >= 0]
        assert m == len(np.unique(f))
        assert got[:want.numel()].tolist() == want.tolist(), (F, k, m)
        assert (got[want.numel():] == 0).all()


def test_leaf_rank_features_flags_feature_out_of_range():
    got, m = _rank_device(np.array([0, 5, -1, 2], np.int64), 5, 3)
    assert m == -1


def test_fit_binned_device_ranking_equals_host_ranking():
    """fit_leaf_networks_binned with the device ranking (the default: one
    yabt_leaf_step call) gives the same tree, bit for bit, as the host
    ranking path (separate yabt_leaf_moments, yabt_leaf_fit and
    yabt_leaf_fold calls)."""
    from yabt_amd import neural_leaves as NL
    rng = np.random.default_rng(5)
    n, F = 50_000, 30
    X = uniform_bins(rng, n, F)
    fm = torch.as_tensor(np.ascontiguousarray(X.T), device=DEV)
    g, h = grad_hess(rng, n)
    gd, hd = torch.as_tensor(g, device=DEV), torch.as_tensor(h, device=DEV)
    # a tree with many tied feature counts: random internal nodes over F features
    N = 2 * 63 + 1
    feature = np.full(N, -1, np.int64)
    left = np.full(N, -1, np.int64)
    right = np.full(N, -1, np.int64)
    for i in range(62):
        feature[i] = rng.integers(0, F)
        left[i], right[i] = 2 * i + 1, 2 * i + 2
    thr = torch.as_tensor(rng.integers(0, 255, N).astype(np.float32), device=DEV)
    tr = Tree(torch.as_tensor(feature, device=DEV), thr, torch.as_tensor(left, device=DEV),
            torch.as_tensor(right, device=DEV), torch.as_tensor(rng.normal(size=N).astype(np.float32), device=DEV), 0)
    leaf = torch.as_tensor(rng.integers(62, 125, n), device=DEV)

    @dataclass
    class P:
        learning_rate: float = 0.1
        leaf_net_features: int = 8
        leaf_net_min_samples: int = 50
        leaf_net_l2: float = 1.0
        leaf_net_hidden: int = 0
    dev_out = NL.fit_leaf_networks_binned(tr, fm, gd, hd, leaf, P(), n=n)
    keep = NL.RANK_MAX_FEATURES
    try:
        NL.RANK_MAX_FEATURES = 0                            # host ranking
        host_out = NL.fit_leaf_networks_binned(tr, fm, gd, hd, leaf, P(), n=n)
    finally:
        NL.RANK_MAX_FEATURES = keep
    assert dev_out.leaf_net_feats is not None
    assert torch.equal(dev_out.leaf_net_feats.cpu(), host_out.leaf_net_feats.cpu())
    for a in ("value", "leaf_net_linear", "leaf_net_lo", "leaf_net_hi"):
        assert torch.equal(getattr(dev_out, a), getattr(host_out, a)), a
