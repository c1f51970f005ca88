"""Quantile binner on the GPU (mirror of yabt/binning.py:9-129, numpy path).

Bin semantics: with interior edges e_0 < ... < e_{k-1} of feature f,
bin(x) = #{j : e_j < x}, so ``bin(x) <= b  <=>  x <= e_b`` and a split on
binned data is exactly the raw-space split ``x <= edge_value(f, b)``.

``fit`` runs ``yabt_bin_fit`` (csrc/binner.hip): per feature, numpy's linear
quantiles at linspace(0, 1, max_bins+1)[1:-1] of at most 200 000 rows (the
reference's seeded subsample above that, drawn on the host with the same
numpy call), rounded to float32 and de-duplicated; the inter-quartile scale
(numpy's float32 std when zero, 1 if that is zero too); the NaN-ignoring
median of all rows.  The results equal the reference's numpy path bit for bit
(the reference switches to torch.quantile on CUDA machines, binning.py:48-51,
whose fp32 interpolation can move an edge by an ulp; this binner keeps the
numpy definition, so edges do not depend on the machine).

``transform`` / ``layouts`` run ``yabt_bin_transform``: median imputation and
the bin search in one pass, written straight into the grower's feature-major
and row-major layouts (and the imputed fp32 matrix the leaf models and the
routing read).  Fitted edges, scales and medians are also kept on the host
with the reference's attribute names and types.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

MAX_BINS = 256
SAMPLE_ROWS = 200_000


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _round16(x: int) -> int:
    return (x + 15) // 16 * 16


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("yabt_amd: no HIP device available")
    return torch.device("cuda", torch.cuda.current_device())


def _on_device(X) -> torch.Tensor:
    """X as a float32 (n, F) device tensor with unit column stride."""
    if isinstance(X, torch.Tensor):
        dev = X.device if X.device.type == "cuda" else _device()
        Xd = X.detach().to(dev, torch.float32)
    else:
        Xd = torch.from_numpy(np.ascontiguousarray(np.asarray(X, dtype=np.float32))).to(_device())
    if Xd.dim() != 2:
        raise ValueError("X must be 2-D (n, F)")
    return Xd if Xd.stride(1) == 1 else Xd.contiguous()


class Binner:
    def __init__(self, max_bins: int = MAX_BINS):
        if not 2 <= max_bins <= 256:
            raise ValueError("max_bins must be in [2, 256]")
        self.max_bins = max_bins
        self.edges_: list[torch.Tensor] | None = None
        self.medians_: np.ndarray | None = None
        self.scales_: torch.Tensor | None = None
        self._dev = None        # (device, edges (F, 255), nedges (F), medians (F))

    def fit(self, X) -> "Binner":
        """X: numpy array or torch tensor (n, F); NaN marks a missing value."""
        lib = _lib.load()
        Xd = _on_device(X)
        dev = Xd.device
        n, F = Xd.shape
        rows = None
        m = n
        if n > SAMPLE_ROWS:   # the reference's subsample (binning.py:36-38), same generator and call
            idx = np.random.default_rng(0).choice(n, SAMPLE_ROWS, replace=False)
            rows = torch.from_numpy(idx.astype(np.int64)).to(dev)
            m = SAMPLE_ROWS
        edges = torch.empty((F, 255), dtype=torch.float32, device=dev)
        nedges = torch.empty(F, dtype=torch.int32, device=dev)
        scales = torch.empty(F, dtype=torch.float32, device=dev)
        medians = torch.empty(F, dtype=torch.float32, device=dev)
        nbytes = int(lib.yabt_bin_fit_workspace_bytes(m, F))
        if nbytes == 0:
            raise ValueError("yabt_bin_fit: invalid sizes")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.yabt_bin_fit(_ptr(Xd), Xd.stride(0), n, F, _ptr(rows), m, self.max_bins, _ptr(ws), nbytes,
                                    _ptr(edges), 255, _ptr(nedges), _ptr(scales), _ptr(medians), _stream(dev)),
                   "yabt_bin_fit")
        ne_h = nedges.cpu().numpy()
        e_h = edges.cpu().numpy()
        self.edges_ = [torch.from_numpy(e_h[f, :ne_h[f]].copy()) for f in range(F)]
        self.scales_ = scales.cpu()
        self.medians_ = medians.cpu().numpy()
        self._dev = (dev, edges, nedges, medians)
        return self

    def _device_tables(self, dev: torch.device):
        assert self.edges_ is not None, "Binner not fitted"
        if self._dev is None or self._dev[0] != dev:
            F = len(self.edges_)
            edges = torch.zeros((F, 255), dtype=torch.float32)
            for f, e in enumerate(self.edges_):
                edges[f, :e.numel()] = e
            nedges = torch.tensor([e.numel() for e in self.edges_], dtype=torch.int32)
            medians = torch.as_tensor(np.asarray(self.medians_, np.float32))
            self._dev = (dev, edges.to(dev), nedges.to(dev), medians.to(dev))
        return self._dev[1:]

    def _run(self, Xd: torch.Tensor, fm=None, rm=None, imp=None) -> None:
        lib = _lib.load()
        dev = Xd.device
        n, F = Xd.shape
        if F != len(self.edges_):
            raise ValueError(f"X has {F} features, the binner was fitted on {len(self.edges_)}")
        edges, nedges, medians = self._device_tables(dev)
        _lib.check(lib.yabt_bin_transform(
            _ptr(Xd), Xd.stride(0), n, F, _ptr(edges), 255, _ptr(nedges), _ptr(medians),
            _ptr(fm), fm.stride(0) if fm is not None else 0, _ptr(rm), rm.stride(0) if rm is not None else 0,
            _ptr(imp), imp.stride(0) if imp is not None else 0, _stream(dev)), "yabt_bin_transform")

    def transform(self, X, device: str | torch.device = "cuda") -> torch.Tensor:
        """(n, F) uint8 codes, bin = #{edges < x} after median imputation,
        computed on the GPU and returned on ``device``."""
        Xd = _on_device(X)
        n, F = Xd.shape
        out = torch.empty((n, F), dtype=torch.uint8, device=Xd.device)
        if n:
            self._run(Xd, rm=out)
        return out.to(device)

    def layouts(self, X):
        """Bins in both grower layouts plus the imputed fp32 matrix, from one
        pass over X: (BinLayouts, Xraw (n, F) fp32 on the device)."""
        from .grow_hip import BinLayouts
        Xd = _on_device(X)
        dev = Xd.device
        n, F = Xd.shape
        fm = torch.zeros((F, max(16, _round16(n))), dtype=torch.uint8, device=dev)
        rm = torch.zeros((max(n, 1), _lib.row_stride(F)), dtype=torch.uint8, device=dev)
        imp = torch.empty((n, F), dtype=torch.float32, device=dev)
        if n:
            self._run(Xd, fm=fm, rm=rm, imp=imp)
        return BinLayouts(fm, rm, n, F), imp

    def impute_device(self, X) -> torch.Tensor:
        """Median-imputed fp32 (n, F) on the device."""
        Xd = _on_device(X)
        n, F = Xd.shape
        imp = torch.empty((n, F), dtype=torch.float32, device=Xd.device)
        if n:
            self._run(Xd, imp=imp)
        return imp

    def impute(self, X: np.ndarray) -> np.ndarray:
        """Median-impute NaNs on the host (binning.py:114-118, the reference's
        numpy expression on its fitted medians)."""
        X = np.asarray(X, dtype=np.float32)
        return np.where(np.isnan(X), self.medians_, X).astype(np.float32)

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
