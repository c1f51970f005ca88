"""Write golden vectors of the reference's boosting fits.

The trajectory of a boosting fit -- interaction steering, linear leaves,
target standardisation, many trees composed -- is fixed only by running the
reference.  This script imports the reference package from its sources
(read-only: no bytecode is written, and the C grower it would compile on
first use is the same grow.c built by ``make -C oracle ref`` into
oracle/_ref/) and fits on seeded synthetic data on the CPU.

``Booster.fit`` itself cannot run here: its CPU branch imports the Numba
grower module (yabt/boosting.py:432-433), and numba is not installed.  The
loop below therefore calls the reference's own functions in the order and
with the arguments of ``Booster.fit`` for the parameters used (no sampling,
no eval set, no refinement; yabt/boosting.py:271-515): ``Binner``,
``loss.base_score``/``grad_hess``, ``FeatureInteractionDetector``,
``grow_tree_c``, ``Tree.apply``, ``fit_leaf_networks``,
``Tree.net_contribution``; predictions come from the reference's
``Booster.predict_margin`` and estimator ``predict``/``predict_proba``.

It stores the per-tree node arrays, leaf models and predictions as .npz
files; it runs only where the reference sources are mounted, and the
fixtures are what tests/test_gpu_grow_ref.py and tests/test_boost_oracle.py
read.

    python tests/golden/make_booster_golden.py
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import sys

sys.dont_write_bytecode = True

import numpy as np  # noqa: E402
import torch  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libgrow_ref.so")


def cfg1(n, seed):
    """X ~ N(0,1) (n, 20); y = sin x0 + 0.5 x1 x2 + x3^2 + 0.3 sum x4..x9 + N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, 20)).astype(np.float32)
    y = (np.sin(X[:, 0]) + 0.5 * X[:, 1] * X[:, 2] + X[:, 3] ** 2 + 0.3 * X[:, 4:10].sum(axis=1)
         + rng.normal(scale=0.1, size=n)).astype(np.float32)
    return X, y


def logistic(n, F, seed):
    """X ~ N(0,1) (n, F); y ~ Bernoulli(sigmoid(X w)), w ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, F)).astype(np.float32)
    w = rng.normal(size=F)
    y = (rng.random(n) < 1 / (1 + np.exp(-(X @ w)))).astype(np.float32)
    return X, y


def sparse_regression(n, F, seed):
    """X: 90% zeros, the rest N(0,1); y = x0 + 2 x5 - x7 x9 + N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    X = np.where(rng.random((n, F)) < 0.1, rng.normal(size=(n, F)), 0.0).astype(np.float32)
    y = (X[:, 0] + 2 * X[:, 5] - X[:, 7] * X[:, 9] + rng.normal(scale=0.1, size=n)).astype(np.float32)
    return X, y


# The reference's sparse-layout helpers live in yabt/grow_numba.py, whose
# import needs numba (absent here); these two compute the same layout and
# density from the binned matrix.
def build_sparse_layout(binned):
    """The CSR layout of yabt/grow_numba.py:341-367: default_bin[f] is column
    f's most frequent bin (the lowest of equally frequent ones), and row r's
    explicit cells are its columns whose bin differs, in column order, as
    (indptr, indices, data, default_bin), all int64."""
    b = np.ascontiguousarray(binned.detach().cpu().numpy())
    n, F = b.shape
    default_bin = np.array([np.bincount(b[:, f], minlength=256).argmax() for f in range(F)], dtype=np.int64)
    r, c = np.nonzero(b != default_bin.astype(b.dtype))     # row-major: grouped by row, columns ascending
    indptr = np.searchsorted(r, np.arange(n + 1)).astype(np.int64)
    return indptr, c.astype(np.int64), b[r, c].astype(np.int64), default_bin


def estimate_density(binned, sample_rows=4096):
    """yabt/grow_numba.py:375-395's estimate: the share of cells outside their
    column's most frequent bin, over an evenly spaced sample of at most
    sample_rows rows (np.linspace indices, truncated)."""
    b = binned.detach().cpu().numpy()
    if b.shape[0] > sample_rows:
        b = b[np.linspace(0, b.shape[0] - 1, sample_rows).astype(np.int64)]
    modal = sum(int(np.bincount(col, minlength=256).max()) for col in b.T)
    return float(1.0 - modal / max(1, b.size))


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tree_arrays(trees, K=8):
    """Concatenated node arrays of a list of reference Trees (offsets per tree)."""
    off = [0]
    cols = {k: [] for k in ("feature", "threshold", "left", "right", "value")}
    nets = {k: [] for k in ("linear", "lo", "hi")}
    feats = np.full((len(trees), K), -1, np.int64)
    for t, tr in enumerate(trees):
        N = tr.feature.shape[0]
        off.append(off[-1] + N)
        for k in cols:
            cols[k].append(getattr(tr, k).detach().cpu().numpy())
        if tr.leaf_net_feats is not None:
            f = tr.leaf_net_feats.cpu().numpy()
            feats[t, :f.size] = f
            pad = lambda a, v: np.concatenate([a, np.full((N, K - a.shape[1]), v, np.float32)], 1)
            nets["linear"].append(pad(tr.leaf_net_linear.cpu().numpy(), 0.0))
            nets["lo"].append(pad(tr.leaf_net_lo.cpu().numpy(), -np.inf))
            nets["hi"].append(pad(tr.leaf_net_hi.cpu().numpy(), np.inf))
        else:
            nets["linear"].append(np.zeros((N, K), np.float32))
            nets["lo"].append(np.full((N, K), -np.inf, np.float32))
            nets["hi"].append(np.full((N, K), np.inf, np.float32))
    out = {k: np.concatenate(v) for k, v in cols.items()}
    out.update({k: np.concatenate(v).astype(np.float32) for k, v in nets.items()})
    out["node_off"] = np.array(off, np.int64)
    out["net_feats"] = feats
    return out


def booster_fit(yabt, booster, X, y):
    """The reference Booster's fit loop for p.subsample == p.colsample == 1,
    no eval set, refine_steps == refit_every == 0, no adaptive / GOSS /
    product / kernel features (yabt/boosting.py:271-515), run on the CPU with
    the C grower (the branch of boosting.py:443-465 taken when c_grower is on)."""
    from yabt.adaptive_features import FeatureInteractionDetector
    from yabt.binning import Binner
    from yabt.boosting import _INTERACTION_MIN_ROWS
    from yabt.grow_c import grow_tree_c
    from yabt.neural_leaves import fit_leaf_networks

    p, loss = booster.p, booster.loss
    booster.device_ = dev = "cpu"
    gen = torch.Generator(device="cpu").manual_seed(p.seed)
    booster.binner = Binner(max_bins=p.max_bins).fit(X)
    binned = booster.binner.transform(X, device=dev)
    Xraw = torch.from_numpy(booster.binner.impute(X)).to(dev)
    yt = torch.as_tensor(np.asarray(y, dtype=np.float32), device=dev)
    n, F = Xraw.shape
    use_interaction_aware = p.interaction_aware and n >= _INTERACTION_MIN_ROWS
    if p.detect_interactions or use_interaction_aware:
        booster.interaction_detector = FeatureInteractionDetector(F, device=dev)
    booster.base_score = loss.base_score(yt)
    margin = torch.full((n,), booster.base_score, device=dev)
    tp = booster._tree_params()
    bfm = np.ascontiguousarray(binned.detach().cpu().numpy().T, dtype=np.uint8)
    sl = None                      # Booster._get_sparse_layout (boosting.py:240-258, 438-439)
    if p.sparse_hist is True or (p.sparse_hist == "auto"
                                 and estimate_density(binned) <= p.sparse_hist_max_density):
        sl = build_sparse_layout(binned)
    booster.sparse_used_ = sl is not None
    for _ in range(p.n_estimators):
        grad, hess = loss.grad_hess(margin, yt)
        imat = None
        if use_interaction_aware and booster.interaction_detector is not None:
            imat = booster.interaction_detector.normalized_matrix()
        tree = grow_tree_c(binned, grad, hess, booster.binner, tp, None, interaction_matrix=imat,
                           interaction_boost=p.interaction_boost, sparse_layout=sl,
                           n_threads=p.c_grower_threads, binned_fmajor=bfm)
        leaf_idx = tree.apply(Xraw)
        if p.neural_leaves:
            tree = fit_leaf_networks(tree, Xraw, yt, margin, loss, p, gen, leaf_idx=leaf_idx)
        if booster.interaction_detector is not None:
            booster.interaction_detector.update_from_path_pairs(tree.path_feature_pairs())
        contrib = tree.value[leaf_idx]
        if tree.leaf_net_feats is not None:
            contrib = contrib + tree.net_contribution(Xraw, leaf_idx)
        margin = margin + contrib
        booster.trees.append(tree)
    return booster


def main() -> None:
    if not os.path.exists(REF_SO):
        raise SystemExit(f"{REF_SO} missing: run make -C oracle ref first")
    sys.path.insert(0, REF)
    import yabt
    from yabt import grow_c
    from yabt.boosting import Booster, LogLoss, MSELoss
    lib = ctypes.CDLL(REF_SO)
    grow_c._configure(lib)
    grow_c._LIB = lib  # the reference's loader returns this handle instead of compiling

    common = dict(device="cpu", sparse_hist=False, c_grower=True, refine_steps=0)

    # regression: the 20 000 x 20 estimator workload, 25 trees, 31 leaves, 255 bins
    X, y = cfg1(20_000, 0)
    Xt, _ = cfg1(4_000, 11)
    est = yabt.YABTRegressor(n_estimators=25, max_leaves=31, learning_rate=0.1, max_bins=255,
                             neural_leaves=True, **common)
    est._cat_idx = []
    yt = est._transform_y(np.asarray(y, dtype=np.float32), fit=True)      # sklearn_api.py:290-291
    est.booster_ = booster_fit(yabt, Booster(est._boost_params(), MSELoss()), est._encode(X, yt, True), yt)
    arr = tree_arrays(est.booster_.trees)
    np.savez_compressed(os.path.join(HERE, "booster_regression_20kx20.npz"),
                        x_digest=np.array(digest(X, y, Xt)), base=np.float64(est.booster_.base_score),
                        y_mean=np.float64(est._y_mean), y_std=np.float64(est._y_std),
                        pred=est.predict(Xt).astype(np.float32), torch_threads=np.int64(torch.get_num_threads()),
                        **arr)

    # binary classification: 50 000 x 28, 28 bins, depth 8, 10 trees, no leaf models
    X, y = logistic(50_000, 28, 1)
    Xt, _ = logistic(4_000, 28, 2)
    clf = yabt.YABTClassifier(n_estimators=10, max_leaves=256, max_depth=8, max_bins=28,
                              neural_leaves=False, **common)
    clf._cat_idx = []
    clf.classes_ = np.unique(y)                                          # sklearn_api.py:321-338
    clf.n_classes_ = len(clf.classes_)
    clf._is_binary = True
    yb = (y == clf.classes_[1]).astype(np.float32)
    clf.booster_ = booster_fit(yabt, Booster(clf._boost_params(), LogLoss()), clf._encode(X, yb, True), yb)
    arr = tree_arrays(clf.booster_.trees)
    np.savez_compressed(os.path.join(HERE, "booster_logistic_50kx28.npz"),
                        x_digest=np.array(digest(X, y, Xt)), base=np.float64(clf.booster_.base_score),
                        proba=clf.predict_proba(Xt)[:, 1].astype(np.float32),
                        torch_threads=np.int64(torch.get_num_threads()), **arr)

    # sparse regression: 30 000 x 60, 90% zeros, depth 6, 10 trees; sparse_hist
    # "auto" picks cgrow's sparse histogram builder
    X, y = sparse_regression(30_000, 60, 3)
    Xt, _ = sparse_regression(4_000, 60, 4)
    est = yabt.YABTRegressor(n_estimators=10, max_leaves=64, max_depth=6, max_bins=255, neural_leaves=False,
                             **dict(common, sparse_hist="auto"))
    est._cat_idx = []
    yt = est._transform_y(np.asarray(y, dtype=np.float32), fit=True)
    est.booster_ = booster_fit(yabt, Booster(est._boost_params(), MSELoss()), est._encode(X, yt, True), yt)
    assert est.booster_.sparse_used_, "the sparse builder was expected"
    arr = tree_arrays(est.booster_.trees)
    np.savez_compressed(os.path.join(HERE, "booster_sparse_30kx60.npz"),
                        x_digest=np.array(digest(X, y, Xt)), base=np.float64(est.booster_.base_score),
                        y_mean=np.float64(est._y_mean), y_std=np.float64(est._y_std),
                        pred=est.predict(Xt).astype(np.float32), torch_threads=np.int64(torch.get_num_threads()),
                        **arr)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.startswith("booster_")))


if __name__ == "__main__":
    main()
