"""Newton boosting on the GPU (mirror of yabt/boosting.py:60-561 and
yabt/multiclass.py:9-48).

``BoostParams`` carries every field of the reference with the same defaults,
so parameter sets written for the reference construct unchanged.  ``Booster``
runs the reference's training loop (boosting.py:271-534) with the data kept
on the HIP device from binning to the last margin update:

* g, h by ``yabt_grad_hess``; trees by the HIP grower (``yabt_grow``, or
  ``yabt_grow_ref`` with ``grower_arithmetic="reference"``), whose
  final partition gives every training row's leaf, so the routing pass
  ``tree.apply(Xraw)`` of boosting.py:492 is not needed (rows are the same:
  ``bin <= b  <=>  x <= edge_value(f, b)``); with row subsampling the grower
  sees a subset and the full set is routed by ``yabt_apply``;
* linear leaf models by ``fit_leaf_networks`` (``yabt_leaf_moments``,
  ``yabt_leaf_fit``);
* the margin update by ``yabt_margin_update``; evaluation-set and
  ``predict_margin`` outputs by ``yabt_predict`` over packed forests.

Interaction steering (``FeatureInteractionDetector``, adaptive_features.py:
113-180) keeps its (F, F) count matrix on the host: the counts are integers,
so its normalisation is the reference's own fp32 expression.

The reference's grower switches (``levelwise`` "auto"/False, ``numba_grower``,
``c_grower``, ``c_grower_threads``) all select the leaf-wise grower here;
``sparse_hist`` / ``sparse_hist_max_density`` pick cgrow's sparse or dense
histogram builder as the reference does, which matters only to
``grower_arithmetic="reference"`` (exact sums are the same either way).  Features outside the tree-growing path raise
``NotImplementedError`` when switched on: differentiable refinement and
refits, adaptive features, GOSS, product features, kernel splits, auto-tuning,
stochastic routing, MLP leaves and the level-wise grower (``levelwise=True``).
There is no CPU execution: ``device="cpu"`` is rejected.
"""

from __future__ import annotations

import threading
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, fields, replace

import numpy as np
import torch

from . import boost_ops
from .binning import Binner
from .grow_hip import grow_device, grow_tree_hip, leaf_ids, nbins_of, tree_from_result
from .losses import LogLoss, MSELoss
from .neural_leaves import feature_major, fit_leaf_networks
from .tree import Tree, TreeParams

# interaction steering is switched off below this row count (boosting.py:21-24)
_INTERACTION_MIN_ROWS = 2000


@dataclass
class BoostParams:
    """The reference's parameter set (boosting.py:60-200), same names and defaults."""
    n_estimators: int = 500
    learning_rate: float = 0.1
    max_leaves: int = 31
    max_depth: int = 64
    reg_lambda: float = 1.0
    gamma: float = 0.0
    min_split_gain_rel: float = 0.0
    min_child_weight: float = 1e-3
    min_samples_leaf: int = 20
    subsample: float = 1.0
    colsample: float = 1.0
    max_bins: int = 256
    refine_steps: int = 0
    refine_lr: float = 0.02
    refine_min_gain: float = 1e-4
    refit_every: int = 0
    refit_steps: int = 30
    refit_lr: float = 0.05
    adaptive_features: bool = False
    feature_importance_alpha: float = 0.1
    goss_enabled: bool = False
    goss_ratio: float = 0.9
    detect_interactions: bool = False
    interaction_aware: bool = True
    interaction_boost: float = 0.5
    product_features: bool = False
    product_max_features: int = 5
    product_max_order: int = 3
    product_min_corr: float = 0.03
    product_corr_gain: float = 1.3
    kernel_splits: bool = False
    kernel_candidates: int = 8
    kernel_gamma: float = 0.0
    kernel_min_samples: int = 64
    kernel_importance_weighting: bool | str = False
    neural_leaves: bool = True
    leaf_net_hidden: int = 0
    leaf_net_features: int = 8
    leaf_net_l2: float = 1.0
    leaf_net_steps: int = 40
    leaf_net_lr: float = 0.05
    leaf_net_min_samples: int = 50
    auto_tune: bool = False
    stochastic_routing: bool = False
    routing_tau: float = 0.05
    levelwise: bool | str = "auto"
    numba_grower: bool | str = "auto"
    c_grower: bool | str = "auto"
    c_grower_threads: int = 0
    sparse_hist: bool | str = "auto"
    sparse_hist_max_density: float = 0.5
    early_stopping_rounds: int = 0
    seed: int = 0
    device: str = "auto"
    verbose: bool = False
    # This backend's own switch (not a reference field): "exact" grows with
    # exact fixed-point histograms on the device; "reference" reproduces the
    # reference C grower's fp32 arithmetic and row order, giving its trees
    # bit for bit at a higher cost per split.
    grower_arithmetic: str = "exact"

    def resolve_device(self) -> str:
        """"auto" -> "cuda" (boosting.py:196-199); this backend runs on a HIP device only."""
        if self.device == "auto":
            return "cuda"
        return self.device


PARAM_NAMES = [f.name for f in fields(BoostParams)]

# (field, value that keeps it off, what it is) for the features outside the grower path
_OFF = [
    ("refine_steps", 0, "differentiable refinement"),
    ("refit_every", 0, "global leaf refits"),
    ("adaptive_features", False, "adaptive feature selection"),
    ("goss_enabled", False, "GOSS sampling"),
    ("product_features", False, "product features"),
    ("kernel_splits", False, "kernel splits"),
    ("auto_tune", False, "auto-tuning"),
    ("stochastic_routing", False, "stochastic routing"),
    ("leaf_net_hidden", 0, "MLP leaves"),
]


def check_supported(p: BoostParams) -> None:
    for name, off, what in _OFF:
        if getattr(p, name) != off:
            raise NotImplementedError(f"{what} ({name}={getattr(p, name)!r}) is not provided by this backend")
    if p.grower_arithmetic not in ("exact", "reference"):
        raise ValueError("grower_arithmetic must be 'exact' or 'reference'")
    if p.levelwise is True:
        raise NotImplementedError("the level-wise grower (levelwise=True) is not provided by this backend")
    if p.resolve_device() not in ("cuda",) and not str(p.resolve_device()).startswith("cuda:"):
        raise NotImplementedError(f"device={p.device!r}: this backend runs on a HIP device only")
    if not torch.cuda.is_available():
        raise RuntimeError("yabt_amd: no HIP device available")


class FeatureInteractionDetector:
    """Ancestor/descendant split-pair counts (adaptive_features.py:113-180),
    held on the host in fp32."""

    def __init__(self, n_features: int, device: str = "cpu"):
        self.n_features = n_features
        self.device = device
        self.interaction_scores = torch.zeros((n_features, n_features), device=device)
        self.update_count = 0

    def update_from_path_pairs(self, pairs: list[tuple[int, int]]) -> None:
        """Symmetric +1 per (a, b) pair with a != b (adaptive_features.py:129-145)."""
        if not pairs:
            return
        idx = torch.tensor(pairs, dtype=torch.long, device=self.device)
        a, b = idx[:, 0], idx[:, 1]
        keep = a != b
        a, b = a[keep], b[keep]
        ones = torch.ones(a.shape[0], device=self.device)
        self.interaction_scores.index_put_((a, b), ones, accumulate=True)
        self.interaction_scores.index_put_((b, a), ones, accumulate=True)
        self.update_count += 1

    def normalized_matrix(self) -> torch.Tensor:
        """((m - bg) / (max - bg + 1e-8)).clamp_min(0), bg = mean of the nonzero
        counts; m itself while it is all zero (adaptive_features.py:147-160)."""
        m = self.interaction_scores
        mx = m.max()
        if mx <= 0:
            return m
        bg = m[m > 0].mean()
        return ((m - bg) / (mx - bg + 1e-8)).clamp_min(0)

    def get_top_interactions(self, k: int = 5) -> list[tuple[int, int, float]]:
        """Top-k pairs of the upper triangle by count per update (adaptive_features.py:162-180)."""
        if self.update_count == 0:
            return []
        scores = self.interaction_scores / (self.update_count + 1e-8)
        s = scores.tolist()
        pairs = [(i, j, s[i][j]) for i in range(self.n_features) for j in range(i + 1, self.n_features)]
        pairs.sort(key=lambda x: x[2], reverse=True)
        return pairs[:k]


class Booster:
    """Newton boosting with the HIP grower (boosting.py:202-561)."""

    def __init__(self, params: BoostParams, loss):
        self.p = params
        self.loss = loss
        self.trees: list[Tree] = []
        self.binner: Binner | None = None
        self.base_score: float = 0.0
        self.best_iter: int | None = None
        self.interaction_detector: FeatureInteractionDetector | None = None
        self.tuning_report_: dict | None = None
        self.product_spec_: list[tuple[int, ...]] = []
        self._forest: boost_ops.Forest | None = None

    def _tree_params(self) -> TreeParams:
        p = self.p
        return TreeParams(max_leaves=p.max_leaves, max_depth=p.max_depth, reg_lambda=p.reg_lambda,
                          gamma=p.gamma, min_child_weight=p.min_child_weight,
                          min_samples_leaf=p.min_samples_leaf, learning_rate=p.learning_rate)

    def _device(self) -> torch.device:
        d = self.p.resolve_device()
        return torch.device("cuda", torch.cuda.current_device()) if d == "cuda" else torch.device(d)

    # rows the reference's density estimate samples (grow_numba.py:375)
    _DENSITY_SAMPLE_ROWS = 4096

    def _sparse_default_bins(self, lay, n: int, F: int) -> torch.Tensor | None:
        """The reference's sparse-histogram choice for unsubsampled trees
        (boosting.py:240-258, 438-439): ``sparse_hist`` True always, "auto" when
        the estimated share of non-modal cells is at most
        ``sparse_hist_max_density``.  The estimate takes the modal count per
        feature over np.linspace(0, n - 1, 4096) rows (grow_numba.py:375-395);
        the layout's default bin is each feature's most frequent bin over all
        rows, lowest bin on ties (grow_numba.py:356-359).  Only the default
        bins are needed: the explicit entries are the bins outside them.
        Returns the (F,) device default bins, or None for the dense builder."""
        p = self.p
        if p.sparse_hist is False or n == 0:
            return None
        fm = lay.fm[:, :n]
        if p.sparse_hist is not True:
            idx = np.arange(n) if n <= self._DENSITY_SAMPLE_ROWS else \
                np.linspace(0, n - 1, self._DENSITY_SAMPLE_ROWS).astype(np.int64)
            cols = fm[:, torch.from_numpy(idx).to(fm.device)].long()
            counts = torch.zeros((F, 256), dtype=torch.int64, device=fm.device)
            counts.scatter_add_(1, cols, torch.ones_like(cols))
            modal = int(counts.max(dim=1).values.sum())
            dens = 1.0 - modal / max(1, idx.size * F)
            if not dens <= p.sparse_hist_max_density:
                return None
        full = torch.stack([torch.bincount(fm[f], minlength=256) for f in range(F)])
        return full.argmax(dim=1).to(torch.int32).contiguous()

    def prepare(self, X: np.ndarray) -> tuple:
        """Binning on the device: fit, then both bin layouts and the imputed
        matrix from one pass over the raw X (binning.py:29-118).  The result
        depends only on X and ``max_bins``, so boosters fitted on the same X
        (one-vs-rest classes) can share it through ``fit(..., prepared=)``."""
        dev = self._device()
        Xd = torch.from_numpy(np.ascontiguousarray(np.asarray(X, dtype=np.float32))).to(dev)
        binner = Binner(max_bins=self.p.max_bins).fit(Xd)
        lay, Xraw = binner.layouts(Xd)
        return binner, lay, Xraw

    def fit(self, X: np.ndarray, y: np.ndarray,
            eval_set: tuple[np.ndarray, np.ndarray] | None = None, prepared: tuple | None = None,
            on_tree=None) -> "Booster":
        """The reference's training loop (boosting.py:271-534) on the device.
        ``prepared``: the result of ``prepare(X)`` for this X, if already made
        (optionally followed by ``feature_major`` of its imputed X, for the
        leaf models).
        ``on_tree``: called after each tree grown on all rows as
        on_tree(t, inputs, result) with the grower's inputs (dict: layouts,
        grad, hess, nbins, imat, fmask, and the grower keywords) and its
        GrowResult -- e.g. to grow the same tree in the other arithmetic
        (yabt_amd.divergence)."""
        p = self.p
        check_supported(p)
        dev = self._device()
        self.device_ = dev
        gen = torch.Generator(device="cpu").manual_seed(p.seed)
        self.trees = []
        self.best_iter = None
        self._forest = None

        self.binner, lay, Xraw = (prepared if prepared is not None else self.prepare(X))[:3]
        n, F = Xraw.shape
        binned = lay.rm[:n, :F]          # (n, F) view, used for row subsamples
        yt = torch.as_tensor(np.asarray(y, dtype=np.float32), device=dev)

        use_interaction_aware = p.interaction_aware and n >= _INTERACTION_MIN_ROWS
        self.interaction_detector = (FeatureInteractionDetector(F)
                                     if p.detect_interactions or use_interaction_aware else None)

        # one scalar of set-up, taken from the host copy of y with the loss's
        # own torch expression, as the reference's CPU fit computes it
        self.base_score = self.loss.base_score(torch.as_tensor(np.asarray(y, dtype=np.float32)))
        margin = torch.full((n,), self.base_score, device=dev)

        if eval_set is not None:
            Xv = self.binner.impute_device(eval_set[0])
            yv = torch.as_tensor(np.asarray(eval_set[1], dtype=np.float32), device=dev)
            margin_v = torch.full((Xv.shape[0],), self.base_score, device=dev)
            best_val, rounds_since_best = float("inf"), 0

        tp = self._tree_params()
        nbins = nbins_of(self.binner, F)
        # cgrow's histogram builder for unsubsampled trees: only the reference
        # arithmetic depends on it (exact sums are the same either way)
        sparse_db = (self._sparse_default_bins(lay, n, F) if p.grower_arithmetic == "reference" else None)

        # feature-major copy of Xraw for the leaf models, made at the first tree
        X_fm = prepared[3] if prepared is not None and len(prepared) > 3 else None
        for t in range(p.n_estimators):
            grad, hess = boost_ops.grad_hess(self.loss, margin, yt)

            tp_t = tp
            if p.min_split_gain_rel > 0.0:
                tp_t = replace(tp, gamma=p.gamma + p.min_split_gain_rel * float(grad.var()))

            rows = None
            if p.subsample < 1.0:
                m = int(n * p.subsample)
                rows = torch.randperm(n, generator=gen)[:m].to(dev)

            fmask = None
            if p.colsample < 1.0:
                k = max(1, int(F * p.colsample))
                fmask = torch.zeros(F, dtype=torch.bool, device=dev)
                fmask[torch.randperm(F, generator=gen)[:k].to(dev)] = True

            imat = None
            if use_interaction_aware and self.interaction_detector is not None:
                imat = self.interaction_detector.normalized_matrix()

            if rows is None:
                gkw = dict(fmask=fmask, imat=imat, ib=p.interaction_boost, lam=tp_t.reg_lambda, gamma=tp_t.gamma,
                           mcw=tp_t.min_child_weight, msl=tp_t.min_samples_leaf, lr=tp_t.learning_rate,
                           max_leaves=tp_t.max_leaves, max_depth=tp_t.max_depth)
                res = grow_device(lay, grad, hess, nbins, **gkw,
                                  default_bin=sparse_db if sparse_db is not None else "auto",
                                  arithmetic=p.grower_arithmetic)
                if on_tree is not None:
                    on_tree(t, dict(layouts=lay, grad=grad, hess=hess, nbins=nbins, **gkw), res)
                tree = tree_from_result(res, self.binner, F, dev)
                leaf_idx = leaf_ids(res, n, F, tp_t.max_leaves)
            else:
                tree = grow_tree_hip(binned[rows], grad[rows], hess[rows], self.binner, tp_t, fmask,
                                     interaction_matrix=imat, interaction_boost=p.interaction_boost,
                                     arithmetic=p.grower_arithmetic)
                leaf_idx = tree.apply(Xraw)

            if p.neural_leaves:
                if X_fm is None:
                    X_fm = feature_major(Xraw)
                tree = fit_leaf_networks(tree, Xraw, yt, margin, self.loss, p, gen, leaf_idx=leaf_idx,
                                         X_fmajor=X_fm)

            if self.interaction_detector is not None:
                self.interaction_detector.update_from_path_pairs(tree.path_feature_pairs())

            if X_fm is not None:
                boost_ops.margin_update(margin, leaf_idx, tree, X_fm, x_kind=2)
            else:
                boost_ops.margin_update(margin, leaf_idx, tree, Xraw)
            self.trees.append(tree)

            if eval_set is not None:
                boost_ops.predict(boost_ops.Forest([tree], dev), Xv, out=margin_v, accumulate=True)
                vl = float(self.loss.loss(margin_v, yv))
                if vl < best_val - 1e-7:
                    best_val, self.best_iter, rounds_since_best = vl, t, 0
                else:
                    rounds_since_best += 1
                if p.verbose and t % 50 == 0:
                    print(f"[{t}] train={float(self.loss.loss(margin, yt)):.5f} val={vl:.5f}")
                if p.early_stopping_rounds and rounds_since_best >= p.early_stopping_rounds:
                    break
        self.margin_ = margin
        return self

    def top_interactions(self, k: int = 5) -> list[tuple[int, int, float]]:
        if self.interaction_detector is None:
            return []
        return self.interaction_detector.get_top_interactions(k)

    def forest(self, n_trees: int | None = None) -> boost_ops.Forest:
        """The first n_trees trees packed for yabt_predict (cached for all trees)."""
        dev = getattr(self, "device_", None) or self._device()
        if n_trees is None or n_trees >= len(self.trees):
            if self._forest is None or self._forest.T != len(self.trees):
                self._forest = boost_ops.Forest(self.trees, dev)
            return self._forest
        return boost_ops.Forest(self.trees[:n_trees], dev)

    def _margin(self, Xt: torch.Tensor, n_trees: int | None = None, soft: bool | None = None) -> torch.Tensor:
        """base_score + the first n_trees trees' outputs (boosting.py:536-545)."""
        if soft:
            raise NotImplementedError("stochastic routing is not provided by this backend")
        return boost_ops.predict(self.forest(n_trees), Xt, self.base_score)

    def predict_margin(self, X: np.ndarray, use_best_iter: bool = True) -> np.ndarray:
        """Raw margins of X (boosting.py:547-561)."""
        dev = getattr(self, "device_", None) or self._device()
        Xt = self.binner.impute_device(np.asarray(X, dtype=np.float32))
        n_trees = None
        if use_best_iter and self.best_iter is not None and self.p.refit_every == 0:
            n_trees = self.best_iter + 1
        return self._margin(Xt, n_trees).cpu().numpy()


class MulticlassBooster:
    """One-vs-rest: one LogLoss booster per class, softmax over the per-class
    margins (multiclass.py:9-48).

    The class boosters do not depend on each other, so they are fitted
    concurrently: ``concurrency`` host threads (default 4, the device's
    hardware queues per process), each fitting one class at a time on a
    default-priority stream of its own.  A single tree's growth leaves most
    of the device idle (its rounds are latency-bound), so the classes' trees
    overlap.  Each class's booster is the one a sequential fit would make:
    its inputs are its own, its sums exact and its random generator seeded
    per booster."""

    def __init__(self, params: BoostParams, concurrency: int = 4):
        self.params = params
        self.concurrency = concurrency
        self.boosters_: list[Booster] = []
        self.classes_: np.ndarray | None = None

    def fit(self, X: np.ndarray, y: np.ndarray,
            eval_set: tuple[np.ndarray, np.ndarray] | None = None) -> "MulticlassBooster":
        self.classes_ = np.unique(y)
        self.boosters_ = []
        # every class's booster bins the same X the same way (multiclass.py:25-33):
        # bin once and share the binner, the bin layouts and the imputed X
        prepared = Booster(self.params, LogLoss()).prepare(X) if len(self.classes_) else None
        if prepared is not None and self.params.neural_leaves:
            prepared = prepared + (feature_major(prepared[2]),)
        if prepared is not None:
            # the shared inputs are complete before any other stream reads them
            torch.cuda.current_stream(prepared[2].device).synchronize()

        def one(label):
            yb = (y == label).astype(np.float32)
            evb = None
            if eval_set is not None:
                evb = (eval_set[0], (eval_set[1] == label).astype(np.float32))
            return Booster(self.params, LogLoss()).fit(X, yb, eval_set=evb, prepared=prepared)

        workers = max(1, min(int(self.concurrency), len(self.classes_)))
        if workers == 1:
            self.boosters_ = [one(label) for label in self.classes_]
            return self
        dev = prepared[2].device
        streams = [torch.cuda.Stream(dev) for _ in range(workers)]
        free = list(streams)
        lock = threading.Lock()

        def on_stream(label):
            with lock:
                s = free.pop()
            try:
                with torch.cuda.stream(s):
                    b = one(label)
                    s.synchronize()
                return b
            finally:
                with lock:
                    free.append(s)

        with ThreadPoolExecutor(max_workers=workers) as ex:
            self.boosters_ = list(ex.map(on_stream, list(self.classes_)))
        return self

    def predict_margin(self, X: np.ndarray) -> np.ndarray:
        return np.stack([b.predict_margin(X) for b in self.boosters_], axis=1)

    def predict_proba(self, X: np.ndarray) -> np.ndarray:
        m = self.predict_margin(X)
        e = np.exp(m - m.max(axis=1, keepdims=True))
        return e / e.sum(axis=1, keepdims=True)

    def predict(self, X: np.ndarray) -> np.ndarray:
        return self.classes_[np.argmax(self.predict_proba(X), axis=1)]


__all__ = ["BoostParams", "Booster", "MulticlassBooster", "FeatureInteractionDetector", "LogLoss", "MSELoss",
           "PARAM_NAMES", "check_supported"]
