"""CPU oracle of the boosting loop around the grower (TEST INFRASTRUCTURE ONLY).

Restates in numpy, with the C oracle grower (grow_oracle.c) for the trees and
neural_oracle.py for the linear leaves, the reference's training loop and
prediction:

* Binner fit / transform / impute, numpy path (yabt/binning.py:29-129);
* the losses' base scores and g, h in float32 (yabt/boosting.py:27-58);
* the loop of Booster.fit without sampling (yabt/boosting.py:271-534):
  g, h -> interaction matrix -> grow -> leaf ids -> linear leaves -> path
  pairs -> margin update, with the sparse-histogram choice and layout
  (yabt/boosting.py:240-258, yabt/grow_numba.py:341-395);
* the interaction detector (yabt/adaptive_features.py:121-160);
* leaf-model feature selection (yabt/neural_leaves.py:21-39): the order of
  equal split-use counts is the one torch's CPU argsort gives, as in the
  reference (the same library call);
* Booster._margin (yabt/boosting.py:536-545) with Tree.predict
  (yabt/tree.py:82-135): routing by ``x <= threshold``, value plus the
  clamped linear term summed over inputs in order.

Only tests/ use it, as the reference the GPU booster is compared against.
Pinned by tests/test_boost_oracle.py: loss closed forms and base scores, the
detector against hand-counted pairs, the margin update and prediction against
direct per-row evaluation, the leaf ids against raw-space routing of the
training rows, monotone training loss, and whole fits against the
reference's own boosting fits (tests/golden/booster_*.npz, written by
tests/golden/make_booster_golden.py): in the fp32 mode every tree of the
regression (linear leaves, interaction steering, 25 trees) and logistic (10
depth-8 trees) fits is the reference's, predictions within 1e-6.
"""

from __future__ import annotations

import numpy as np

from . import neural_oracle as N
from . import oracle as O

LEAF = -1


# --------------------------------------------------------------------------
# binner (binning.py:29-129, numpy path)
# --------------------------------------------------------------------------

class Binner:
    def __init__(self, max_bins: int = 256):
        self.max_bins = max_bins

    def fit(self, X: np.ndarray) -> "Binner":
        X = np.asarray(X, dtype=np.float32)
        n, F = X.shape
        med = np.nanmedian(X, axis=0) if n else np.zeros(F, np.float32)
        self.medians_ = np.where(np.isnan(med), 0.0, med)
        Xq = X[np.random.default_rng(0).choice(n, 200_000, replace=False)] if n > 200_000 else X
        qpts = np.linspace(0, 1, self.max_bins + 1)[1:-1]
        self.edges_ = []
        self.scales_ = np.empty(F, np.float32)
        for f in range(F):
            col = Xq[:, f]
            col = col[~np.isnan(col)]
            if col.size == 0:
                col = np.zeros(1, np.float32)
            self.edges_.append(np.unique(np.quantile(col, qpts).astype(np.float32)))
            q25, q75 = np.quantile(col, [0.25, 0.75])
            s = float(q75 - q25)
            if s == 0.0:
                s = float(col.std()) or 1.0
            self.scales_[f] = s
        return self

    def impute(self, X: np.ndarray) -> np.ndarray:
        X = np.asarray(X, dtype=np.float32)
        return np.where(np.isnan(X), self.medians_, X).astype(np.float32)

    def transform(self, X: np.ndarray, imputed: bool = False) -> np.ndarray:
        """(n, F) uint8, bin = #{edges < x} (searchsorted, left); features in
        a thread pool (searchsorted releases the GIL).  ``imputed``: X is
        already impute(X)."""
        from concurrent.futures import ThreadPoolExecutor
        Xi = np.asarray(X, np.float32) if imputed else self.impute(X)
        out = np.empty(Xi.shape, np.uint8)

        def one(f):
            out[:, f] = np.searchsorted(self.edges_[f], Xi[:, f], side="left").astype(np.uint8)

        with ThreadPoolExecutor(max_workers=8) as ex:
            list(ex.map(one, range(len(self.edges_))))
        return out

    def nbins(self) -> np.ndarray:
        return np.array([min(len(e) + 1, 256) for e in self.edges_], np.int32)

    def edge_value(self, f: int, b: int) -> np.float32:
        e = self.edges_[f]
        return e[min(b, len(e) - 1)]


# --------------------------------------------------------------------------
# losses (boosting.py:27-58), float32
# --------------------------------------------------------------------------

def base_score(loss: str, y: np.ndarray) -> float:
    """The mean, or the logit of the clamped mean (boosting.py:31-33, 49-50);
    the float32 mean is torch's CPU reduction, the call the reference makes."""
    import torch
    mu = torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32)).mean()
    if loss == "mse":
        return float(mu)
    p = float(mu.clamp(1e-6, 1 - 1e-6))
    return float(np.log(p / (1 - p)))


def grad_hess(loss: str, m: np.ndarray, y: np.ndarray):
    """g, h in float32; the logistic p is torch's CPU sigmoid, the call the
    reference makes (boosting.py:36)."""
    m = m.astype(np.float32)
    y = y.astype(np.float32)
    if loss == "mse":
        return (m - y).astype(np.float32), np.ones_like(y)
    import torch
    p = torch.sigmoid(torch.from_numpy(np.ascontiguousarray(m))).numpy()
    return (p - y).astype(np.float32), np.maximum(p * (np.float32(1) - p), np.float32(1e-6)).astype(np.float32)


def loss_value(loss: str, m: np.ndarray, y: np.ndarray) -> float:
    m = m.astype(np.float64)
    y = y.astype(np.float64)
    if loss == "mse":
        return float(0.5 * np.mean((m - y) ** 2))
    return float(np.mean(np.maximum(m, 0) - m * y + np.log1p(np.exp(-np.abs(m)))))


# --------------------------------------------------------------------------
# interaction detector (adaptive_features.py:121-160)
# --------------------------------------------------------------------------

def path_pairs(feature, left, right) -> list[tuple[int, int]]:
    """(ancestor feature, split feature) for every split node and each of its
    ancestors (tree.py:186-203), by walking down from the root."""
    pairs = []
    stack = [(0, [])]
    while stack:
        nid, anc = stack.pop()
        f = int(feature[nid])
        if f < 0:
            continue
        pairs.extend((a, f) for a in anc)
        stack.append((int(left[nid]), anc + [f]))
        stack.append((int(right[nid]), anc + [f]))
    return pairs


class Interactions:
    def __init__(self, F: int):
        self.m = np.zeros((F, F), np.float32)

    def update(self, pairs) -> None:
        for a, b in pairs:
            if a != b:
                self.m[a, b] += 1
                self.m[b, a] += 1

    def normalized(self) -> np.ndarray:
        m = self.m
        mx = m.max()
        if mx <= 0:
            return m.copy()
        bg = np.float32(m[m > 0].sum(dtype=np.float64)) / np.float32(np.count_nonzero(m))
        return np.maximum((m - bg) / (mx - bg + np.float32(1e-8)), np.float32(0)).astype(np.float32)


# --------------------------------------------------------------------------
# trees
# --------------------------------------------------------------------------

def sparse_layout(bins: np.ndarray):
    """The sparse histogram layout (yabt/grow_numba.py:341-367): each
    feature's most frequent bin over all rows (lowest on ties) is its
    default; (indptr, indices, data) is the row-major CSR of the other
    cells.  bins: (n, F) uint8."""
    n, F = bins.shape
    default = np.array([np.bincount(bins[:, f], minlength=256).argmax() for f in range(F)], np.int64)
    nondef = bins != default[None, :].astype(bins.dtype)
    indptr = np.zeros(n + 1, np.int64)
    np.cumsum(nondef.sum(axis=1), out=indptr[1:])
    r, c = np.nonzero(nondef)
    return indptr, c.astype(np.int64), bins[r, c].astype(np.int64), default


def estimate_density(bins: np.ndarray, sample_rows: int = 4096) -> float:
    """Share of non-modal cells over np.linspace(0, n - 1, sample_rows) rows
    (yabt/grow_numba.py:375-395), which gates the sparse layout."""
    n, F = bins.shape
    if n > sample_rows:
        bins = bins[np.linspace(0, n - 1, sample_rows).astype(np.int64)]
    m = bins.shape[0]
    modal = sum(int(np.bincount(bins[:, f], minlength=256).max()) for f in range(F))
    return float(1.0 - modal / max(1, m * F))


def thresholds(binner: Binner, feature, thr_bin) -> np.ndarray:
    return np.array([binner.edge_value(int(f), int(b)) if f >= 0 else np.float32(0)
                     for f, b in zip(feature, thr_bin)], np.float32)


def route(X: np.ndarray, feature, threshold, left, right) -> np.ndarray:
    """Leaf per row: x[f] <= threshold goes left (tree.py:82-116)."""
    n = X.shape[0]
    node = np.zeros(n, np.int64)
    active = np.ones(n, bool)
    while active.any():
        f = feature[node]
        active = f >= 0
        if not active.any():
            break
        idx = np.nonzero(active)[0]
        go_left = X[idx, f[idx]] <= threshold[node[idx]]
        node[idx] = np.where(go_left, left[node[idx]], right[node[idx]])
    return node


def select_features(feature: np.ndarray, X: np.ndarray, g: np.ndarray, k: int) -> np.ndarray:
    """Split features by use count, most used first, padded by
    |x^T g - mean(x) sum(g)| / std(x) (neural_leaves.py:21-39)."""
    import torch
    k = min(k, X.shape[1])
    f = feature[feature >= 0]
    if f.size:
        vals, counts = np.unique(f, return_counts=True)
        order = torch.from_numpy(counts).argsort(descending=True).numpy()
        used = vals[order][:k]
    else:
        used = np.empty(0, np.int64)
    if used.size >= k:
        return used.astype(np.int64)
    Xd = X.astype(np.float64)
    gd = g.astype(np.float64)
    score = np.abs(Xd.T @ gd - Xd.mean(axis=0) * gd.sum())
    score = score / np.maximum(Xd.std(axis=0, ddof=1), 1e-6)
    score[used] = -np.inf
    extra = np.argsort(-score, kind="stable")[: k - used.size]
    return np.concatenate([used, extra]).astype(np.int64)


def linear_leaves(tree: dict, X: np.ndarray, g: np.ndarray, h: np.ndarray, leaf: np.ndarray,
                  k: int, min_samples: int, lam: float, lr: float) -> dict:
    """fit_leaf_networks with linear leaves (neural_leaves.py:131-184)."""
    feats = select_features(tree["feature"], X, g, k)
    if feats.size == 0:
        return tree
    Xs = X[:, feats].astype(np.float32)
    mu, sd = N.moments(Xs)
    Xn = N.standardise(Xs, mu, sd)
    n_nodes = tree["value"].shape[0]
    cnt = N.counts(leaf, n_nodes)
    elig = N.eligible_nodes(tree["feature"], cnt, min_samples)
    if not elig.any():
        return tree
    lo, hi = N.envelopes(Xs, leaf, n_nodes)
    W, db = N.fit_linear(Xn, g, h, leaf, elig, n_nodes, lam)
    value, lin = N.fold(tree["value"], W, db, mu, sd, lr)
    out = dict(tree)
    out.update(value=value, feats=feats, linear=lin, lo=lo, hi=hi)
    return out


def tree_output(tree: dict, X: np.ndarray, node: np.ndarray) -> np.ndarray:
    """value[node] + sum_j linear[node, j] * clamp(x_j, lo, hi), in float32,
    inputs added in order (tree.py:118-135)."""
    out = tree["value"][node].astype(np.float32)
    if tree.get("feats") is None:
        return out
    net = np.zeros(X.shape[0], np.float32)
    for j, f in enumerate(tree["feats"]):
        x = np.minimum(np.maximum(X[:, f], tree["lo"][node, j]), tree["hi"][node, j])
        net = (net + (tree["linear"][node, j] * x).astype(np.float32)).astype(np.float32)
    return (out + net).astype(np.float32)


# --------------------------------------------------------------------------
# the loop
# --------------------------------------------------------------------------

def prepare(X: np.ndarray, max_bins: int = 256) -> tuple:
    """(binner, bins (n, F) uint8, imputed X) of Booster.fit's set-up
    (boosting.py:305-307): what depends only on X and max_bins."""
    binner = Binner(max_bins).fit(X)
    Xr = binner.impute(X)
    return binner, binner.transform(Xr, imputed=True), Xr


def fit(X: np.ndarray, y: np.ndarray, *, loss: str = "mse", n_estimators: int = 10, learning_rate: float = 0.1,
        max_leaves: int = 31, max_depth: int = 64, reg_lambda: float = 1.0, gamma: float = 0.0,
        min_child_weight: float = 1e-3, min_samples_leaf: int = 20, max_bins: int = 256,
        subsample: float = 1.0, colsample: float = 1.0, seed: int = 0,
        interaction_aware: bool = True, interaction_boost: float = 0.5, neural_leaves: bool = True,
        leaf_net_features: int = 8, leaf_net_l2: float = 1.0, leaf_net_min_samples: int = 50,
        sparse_hist="auto", sparse_hist_max_density: float = 0.5, mode: int = O.MODE_FIXED,
        prepared: tuple | None = None, on_tree=None) -> dict:
    """Booster.fit (boosting.py:271-534).  Row and column samples are drawn
    from a CPU torch generator seeded with ``seed``, rows first, by the same
    calls as the reference (boosting.py:369-383).  Trees grown on all rows
    use the sparse histogram builder when ``sparse_hist`` is True, or "auto"
    and the estimated density is at most ``sparse_hist_max_density``
    (boosting.py:240-258, 438-439); it changes only the fp32 mode's sums.
    ``prepared``: prepare(X, max_bins) for this X, shared by one-vs-rest
    classes (multiclass.py:25-33 fits every class's binner on the same X).
    ``on_tree``: called after each tree as on_tree(t, inputs, grown) with the
    tree's grower inputs (dict: g, h, imat, fmask, rows, margin before the
    tree) and the grower's trace (O.grow's dict) -- for tests that grow the
    same tree another way."""
    import torch
    gen = torch.Generator(device="cpu").manual_seed(seed)
    binner, bins, Xr = prepared if prepared is not None else prepare(X, max_bins)
    yt = np.asarray(y, np.float32)
    n, F = Xr.shape
    bins_fm = np.ascontiguousarray(bins.T)
    nb = binner.nbins()
    use_ia = interaction_aware and n >= 2000
    det = Interactions(F) if use_ia else None
    base = base_score(loss, yt)
    margin = np.full(n, base, np.float32)
    sl = None
    if sparse_hist is True or (sparse_hist == "auto" and estimate_density(bins) <= sparse_hist_max_density):
        sl = sparse_layout(bins)
    trees, train_loss = [], []
    for _ in range(n_estimators):
        g, h = grad_hess(loss, margin, yt)
        rows = None
        if subsample < 1.0:
            rows = torch.randperm(n, generator=gen)[:int(n * subsample)].numpy()
        fmask = None
        if colsample < 1.0:
            fmask = np.zeros(F, bool)
            fmask[torch.randperm(F, generator=gen)[:max(1, int(F * colsample))].numpy()] = True
        imat = det.normalized() if det is not None else None
        bfm, gg, hh = ((bins_fm, g, h) if rows is None
                       else (np.ascontiguousarray(bins_fm[:, rows]), g[rows], h[rows]))
        t = O.grow(bfm, gg, hh, mode=mode, fmask=fmask, imat=imat, ib=interaction_boost, nbins=nb,
                   sparse=sl if rows is None else None,
                   lam=reg_lambda, gamma=gamma, mcw=min_child_weight, msl=min_samples_leaf,
                   lr=learning_rate, max_leaves=max_leaves, max_depth=max_depth)
        if on_tree is not None:
            on_tree(len(trees), dict(g=g, h=h, imat=imat, fmask=fmask, rows=rows, margin=margin.copy()), t)
        tree = {k: t[k] for k in ("feature", "thr_bin", "left", "right", "value")}
        tree["threshold"] = thresholds(binner, tree["feature"], tree["thr_bin"])
        if rows is None:
            leaf = O.leaf_of_rows(t, n)
        else:
            leaf = route(Xr, tree["feature"], tree["threshold"], tree["left"], tree["right"])
        if neural_leaves:
            g2, h2 = grad_hess(loss, (margin + tree["value"][leaf]).astype(np.float32), yt)
            tree = linear_leaves(tree, Xr, g2, h2, leaf, leaf_net_features, leaf_net_min_samples,
                                 leaf_net_l2, learning_rate)
        if det is not None:
            det.update(path_pairs(tree["feature"], tree["left"], tree["right"]))
        margin = (margin + tree_output(tree, Xr, leaf)).astype(np.float32)
        trees.append(tree)
        train_loss.append(loss_value(loss, margin, yt))
    return {"trees": trees, "base": base, "binner": binner, "margin": margin, "train_loss": train_loss}


def predict_margin(model: dict, X: np.ndarray, n_trees: int | None = None) -> np.ndarray:
    """Booster._margin: base + tree outputs in order (boosting.py:536-545)."""
    Xr = model["binner"].impute(X)
    out = np.full(Xr.shape[0], model["base"], np.float32)
    for tree in model["trees"][:n_trees]:
        node = route(Xr, tree["feature"], tree["threshold"], tree["left"], tree["right"])
        out = (out + tree_output(tree, Xr, node)).astype(np.float32)
    return out
