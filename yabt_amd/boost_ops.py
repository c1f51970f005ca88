"""Device operations of the boosting step (csrc/boost.hip) on torch tensors.

* ``grad_hess``: the loss's g, h at the margin, or at margin + value[leaf]
  (yabt/boosting.py:35-38,52-54, yabt/neural_leaves.py:147), by
  ``yabt_grad_hess`` for the library's own losses; a user loss without a
  ``loss_id`` keeps its own ``grad_hess`` (its code, evaluated on the device).
* ``margin_update``: margin += value[leaf] + clamped linear-leaf term
  (yabt/boosting.py:508-511) by ``yabt_margin_update``.
* ``Forest`` / ``predict``: a list of trees packed once into concatenated
  node arrays and evaluated by ``yabt_predict`` in one launch
  (yabt/boosting.py:536-545).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .tree import Tree

KMAX = 8


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError("yabt_amd boosting ops need tensors on a HIP device")
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise ValueError("all tensors must be on one device")
    return dev


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.float().contiguous()


def grad_hess(loss, margin: torch.Tensor, y: torch.Tensor, leaf: torch.Tensor | None = None,
              value: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(g, h) of ``loss`` at margin (+ value[leaf] when both are given)."""
    loss_id = getattr(loss, "loss_id", None)
    if loss_id is None:
        m = margin if leaf is None else margin + value[leaf]
        return loss.grad_hess(m, y)
    dev = _need_device(margin, y)
    n = int(margin.shape[0])
    m = _f32(margin)
    yy = _f32(y)
    li = None if leaf is None else leaf.to(dev, torch.int64).contiguous()
    va = None if value is None else _f32(value.to(dev))
    g = torch.empty(n, dtype=torch.float32, device=dev)
    h = torch.empty(n, dtype=torch.float32, device=dev)
    nv = 0 if va is None else int(va.numel())
    _lib.check(_lib.load().yabt_grad_hess(int(loss_id), _ptr(m), _ptr(li), _ptr(va), nv, _ptr(yy), n,
                                          _ptr(g), _ptr(h), _stream(dev)), "yabt_grad_hess")
    return g, h


def margin_update(margin: torch.Tensor, leaf: torch.Tensor, tree: Tree, X: torch.Tensor,
                  x_kind: int = 0) -> torch.Tensor:
    """In place: margin += tree.value[leaf] (+ tree.net_contribution(X, leaf)).
    X is fp32 (n, F) row-major (x_kind 0), uint8 feature-major (F, ld >= n)
    (x_kind 1, inputs float(bin)) or fp32 feature-major (F, ld >= n) (x_kind 2)."""
    dev = _need_device(margin, leaf)
    if margin.dtype != torch.float32 or not margin.is_contiguous():
        raise ValueError("margin must be a contiguous float32 tensor (updated in place)")
    n = int(margin.shape[0])
    li = leaf.to(torch.int64).contiguous()
    value = _f32(tree.value.to(dev))
    K = 0
    feats = lin = lo = hi = None
    Xp, ldx = None, 0
    if tree.leaf_net_feats is not None:
        if tree.leaf_net_linear is None:
            raise NotImplementedError("MLP leaves are not provided by this backend")
        feats = tree.leaf_net_feats.to(dev, torch.int32).contiguous()
        K = int(feats.numel())
        lin = _f32(tree.leaf_net_linear.to(dev))
        if tree.leaf_net_lo is not None:
            lo, hi = _f32(tree.leaf_net_lo.to(dev)), _f32(tree.leaf_net_hi.to(dev))
        else:
            lo = torch.full_like(lin, float("-inf"))
            hi = torch.full_like(lin, float("inf"))
        if x_kind == 0:
            if X.dtype != torch.float32 or X.dim() != 2 or X.shape[0] != n or X.stride(1) != 1:
                raise ValueError("X must be fp32 (n, F) with unit column stride")
            if int(feats.max()) >= X.shape[1] or int(feats.min()) < 0:
                raise ValueError("leaf-model inputs out of range of X")
        else:
            dt = torch.uint8 if x_kind == 1 else torch.float32
            if X.dtype != dt or X.dim() != 2 or X.shape[1] < n or X.stride(1) != 1:
                raise ValueError(f"X must be {'uint8' if x_kind == 1 else 'fp32'} (F, ld >= n)")
            if int(feats.max()) >= X.shape[0] or int(feats.min()) < 0:
                raise ValueError("leaf-model inputs out of range of X")
        Xp, ldx = X, X.stride(0)
    _lib.check(_lib.load().yabt_margin_update(_ptr(margin), n, _ptr(li), _ptr(value), int(value.numel()), K,
                                              _ptr(feats), _ptr(lin),
                                              _ptr(lo), _ptr(hi), int(x_kind), _ptr(Xp), ldx, _stream(dev)),
               "yabt_margin_update")
    return margin


class Forest:
    """Trees packed for ``yabt_predict``: tree t owns nodes
    [node_off[t], node_off[t+1]) of the concatenated arrays; linear leaves are
    padded to K inputs (net_k[t] = 0 for trees without them)."""

    def __init__(self, trees: list[Tree], dev: torch.device):
        self.T = len(trees)
        self.dev = dev
        sizes = [int(t.feature.shape[0]) for t in trees]
        off = [0]
        for s in sizes:
            off.append(off[-1] + s)
        self.n_total = off[-1]
        self.node_off = torch.tensor(off, dtype=torch.int64, device=dev)
        cat = (lambda xs, dt: torch.cat([x.to(dev, dt) for x in xs]) if xs
               else torch.zeros(1, dtype=dt, device=dev))
        self.feature = cat([t.feature for t in trees], torch.int64).contiguous()
        self.threshold = cat([t.threshold for t in trees], torch.float32).contiguous()
        self.left = cat([t.left for t in trees], torch.int64).contiguous()
        self.right = cat([t.right for t in trees], torch.int64).contiguous()
        self.value = cat([t.value for t in trees], torch.float32).contiguous()
        ks = [0 if t.leaf_net_feats is None else int(t.leaf_net_feats.numel()) for t in trees]
        self.K = max(ks, default=0)
        if self.K > KMAX:
            raise ValueError(f"linear leaves over more than {KMAX} inputs are not supported")
        if self.K > 0:
            if any(t.leaf_net_feats is not None and t.leaf_net_linear is None for t in trees):
                raise NotImplementedError("MLP leaves are not provided by this backend")
            K = self.K
            self.net_k = torch.tensor(ks, dtype=torch.int32, device=dev)
            feats = torch.full((self.T, K), -1, dtype=torch.int32)
            lin = torch.zeros((self.n_total, K), dtype=torch.float32, device=dev)
            lo = torch.full((self.n_total, K), float("-inf"), dtype=torch.float32, device=dev)
            hi = torch.full((self.n_total, K), float("inf"), dtype=torch.float32, device=dev)
            for t, (tr, k) in enumerate(zip(trees, ks)):
                if k == 0:
                    continue
                a, b = off[t], off[t + 1]
                feats[t, :k] = tr.leaf_net_feats.cpu().to(torch.int32)
                lin[a:b, :k] = tr.leaf_net_linear.to(dev, torch.float32)
                if tr.leaf_net_lo is not None:
                    lo[a:b, :k] = tr.leaf_net_lo.to(dev, torch.float32)
                    hi[a:b, :k] = tr.leaf_net_hi.to(dev, torch.float32)
            self.max_feat = int(feats.max())
            self.net_feats = feats.to(dev).contiguous()
            self.linear, self.lo, self.hi = lin, lo, hi
        else:
            self.max_feat = -1
            self.net_k = self.net_feats = self.linear = self.lo = self.hi = None
        self.max_split_feat = int(self.feature.max()) if self.n_total else -1


def predict(forest: Forest, X: torch.Tensor, base: float = 0.0, out: torch.Tensor | None = None,
            accumulate: bool = False) -> torch.Tensor:
    """out = (out if accumulate else base) + sum of the forest's tree outputs
    for each row of raw X (n, F) fp32."""
    dev = _need_device(X)
    if X.dtype != torch.float32 or X.dim() != 2 or X.stride(1) != 1:
        X = X.float().contiguous()
    n, F = X.shape
    if max(forest.max_feat, forest.max_split_feat) >= F:
        raise ValueError("the forest uses features beyond X's columns")
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an output tensor")
        out = torch.empty(n, dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or not out.is_contiguous() or out.shape[0] != n:
        raise ValueError("out must be a contiguous float32 (n,) tensor")
    if n == 0:
        return out
    ldx = X.stride(0)
    _lib.check(_lib.load().yabt_predict(
        _ptr(X), ldx, n, F, forest.T, _ptr(forest.node_off), forest.n_total, _ptr(forest.feature),
        _ptr(forest.threshold), _ptr(forest.left), _ptr(forest.right), _ptr(forest.value), forest.K,
        _ptr(forest.net_k), _ptr(forest.net_feats), _ptr(forest.linear), _ptr(forest.lo), _ptr(forest.hi),
        ctypes.c_float(float(base)), int(bool(accumulate)), _ptr(out), _stream(dev)), "yabt_predict")
    return out
