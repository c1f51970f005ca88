"""Quantile binner (mirror of yabt/binning.py:9-129, numpy path).

Bin semantics: with interior edges e_0 < ... < e_{k-1} of feature f,
bin(x) = #{j : e_j < x}, so ``bin(x) <= b  <=>  x <= e_b`` and a split on
binned data is exactly the raw-space split ``x <= edge_value(f, b)``.

Edges are the numpy linear-method quantiles at linspace(0, 1, max_bins+1)[1:-1]
over at most 200 000 rows (a seeded subsample above that), rounded to float32
and de-duplicated; scales are the inter-quartile range (std, or 1, if zero).
The reference switches to a batched torch.quantile on CUDA machines
(binning.py:48-51); this binner always takes the numpy path so edges do not
depend on the machine.
"""

from __future__ import annotations

import numpy as np
import torch

MAX_BINS = 256


class Binner:
    def __init__(self, max_bins: int = MAX_BINS):
        if not 2 <= max_bins <= 256:
            raise ValueError("max_bins must be in [2, 256]")
        self.max_bins = max_bins
        self.edges_: list[torch.Tensor] | None = None
        self.medians_: np.ndarray | None = None
        self.scales_: torch.Tensor | None = None

    def fit(self, X: np.ndarray) -> "Binner":
        X = np.asarray(X, dtype=np.float32)
        n, F = X.shape
        med = np.nanmedian(X, axis=0) if n else np.zeros(F, np.float32)
        self.medians_ = np.where(np.isnan(med), 0.0, med)
        if n > 200_000:
            Xq = X[np.random.default_rng(0).choice(n, 200_000, replace=False)]
        else:
            Xq = X
        qpts = np.linspace(0, 1, self.max_bins + 1)[1:-1]
        edges, scales = [], np.empty(F, dtype=np.float32)
        for f in range(F):
            col = Xq[:, f]
            col = col[~np.isnan(col)]
            if col.size == 0:
                col = np.zeros(1, dtype=np.float32)
            edges.append(torch.from_numpy(np.unique(np.quantile(col, qpts).astype(np.float32))))
            q25, q75 = np.quantile(col, [0.25, 0.75])
            s = float(q75 - q25)
            if s == 0.0:
                s = float(col.std()) or 1.0
            scales[f] = s
        self.edges_ = edges
        self.scales_ = torch.from_numpy(scales)
        return self

    def impute(self, X: np.ndarray) -> np.ndarray:
        """Median-impute NaNs (the raw matrix used for routing and leaf models)."""
        X = np.asarray(X, dtype=np.float32)
        return np.where(np.isnan(X), self.medians_, X).astype(np.float32)

    def transform(self, X: np.ndarray, device: str | torch.device = "cpu") -> torch.Tensor:
        """(n, F) uint8 codes, bin = #{edges < x}."""
        assert self.edges_ is not None, "Binner not fitted"
        Xt = torch.from_numpy(np.ascontiguousarray(self.impute(X))).to(device)
        n, F = Xt.shape
        out = torch.empty((n, F), dtype=torch.uint8, device=Xt.device)
        for f in range(F):
            e = self.edges_[f].to(Xt.device)
            out[:, f] = torch.searchsorted(e, Xt[:, f].contiguous()).to(torch.uint8)
        return out

    def edge_value(self, feature: int, bin_idx: int) -> float:
        """Raw-space threshold equivalent to ``bin <= bin_idx``."""
        e = self.edges_[feature]
        return float(e[min(bin_idx, len(e) - 1)])


class IdentityBinner:
    """Binner for data that is already binned: bins 0..nbins-1 with
    edge_value(f, b) = b, so raw X := float(bin) routes exactly like the bins."""

    def __init__(self, F: int, nbins: int = MAX_BINS):
        self.max_bins = nbins
        e = torch.arange(nbins - 1, dtype=torch.float32)
        self.edges_ = [e for _ in range(F)]
        self.scales_ = torch.ones(F, dtype=torch.float32)
        self.medians_ = np.zeros(F, dtype=np.float32)

    def edge_value(self, feature: int, bin_idx: int) -> float:
        e = self.edges_[feature]
        return float(e[min(bin_idx, len(e) - 1)])
