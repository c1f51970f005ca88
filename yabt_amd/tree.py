"""Tree output type and grower parameters (mirror of yabt/tree.py:22-135,183-203).

``Tree`` keeps the reference's field names and meaning so code written against
the reference's ``Tree`` reads ours unchanged: flat node arrays, ``feature ==
-1`` for leaves, raw-space ``threshold`` with ``x[f] <= threshold`` going left,
lr-folded ``value``, and the optional linear-leaf fields.  Kernel-split and MLP
leaf fields are kept (always None here) for type compatibility.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

LEAF = -1
KERNEL_SPLIT = -2


@dataclass
class TreeParams:
    """Per-tree growth parameters (yabt/tree.py:22-36)."""
    max_leaves: int = 31
    max_depth: int = 64
    reg_lambda: float = 1.0
    gamma: float = 0.0
    min_child_weight: float = 1e-3
    min_samples_leaf: int = 20
    learning_rate: float = 0.1
    kernel_splits: bool = False
    kernel_candidates: int = 8
    kernel_gamma: float = 0.0
    kernel_min_samples: int = 64
    kernel_importance_weighting: bool = False


@dataclass
class Tree:
    """Flat tensor tree (yabt/tree.py:39-76)."""
    feature: torch.Tensor
    threshold: torch.Tensor
    left: torch.Tensor
    right: torch.Tensor
    value: torch.Tensor
    depth: int
    kernel_id: torch.Tensor | None = None
    kernel_centers: torch.Tensor | None = None
    kernel_prec: torch.Tensor | None = None
    leaf_net_feats: torch.Tensor | None = None
    leaf_net_linear: torch.Tensor | None = None
    leaf_net_W1: torch.Tensor | None = None
    leaf_net_b1: torch.Tensor | None = None
    leaf_net_W2: torch.Tensor | None = None
    leaf_net_lo: torch.Tensor | None = None
    leaf_net_hi: torch.Tensor | None = None
    gate_scale: torch.Tensor | None = None

    @property
    def is_leaf(self) -> torch.Tensor:
        return self.feature == LEAF

    def apply(self, X: torch.Tensor) -> torch.Tensor:
        """Leaf (node) index per row of raw X (n, F) (yabt/tree.py:82-116), by
        the routing kernel (yabt_apply); CPU inputs are routed on the current
        HIP device and the result is returned on X's device."""
        if self.kernel_id is not None:
            raise NotImplementedError("kernel splits are not supported by this backend")
        from .grow_hip import apply_hip
        return apply_hip(X, self.feature, self.threshold, self.left, self.right)

    def net_contribution(self, X: torch.Tensor, node: torch.Tensor) -> torch.Tensor:
        """Per-row linear-leaf output, inputs clamped to the leaf's envelope
        (yabt/tree.py:118-128)."""
        if self.leaf_net_feats is None:
            return torch.zeros(X.shape[0], device=X.device)
        if self.leaf_net_linear is None:
            raise NotImplementedError("MLP leaves are not supported by this backend")
        Xs = X[:, self.leaf_net_feats]
        if self.leaf_net_lo is not None:
            Xs = Xs.clamp(self.leaf_net_lo[node], self.leaf_net_hi[node])
        return (self.leaf_net_linear[node] * Xs).sum(dim=1)

    def predict(self, X: torch.Tensor) -> torch.Tensor:
        """value[leaf] + linear-leaf term per row (yabt/tree.py:130-135): one
        ``yabt_predict`` launch; CPU inputs are evaluated on the current HIP
        device and the result is returned on X's device."""
        from .boost_ops import Forest, predict
        from .grow_hip import _device
        dev = X.device if X.device.type == "cuda" else _device()
        return predict(Forest([self], dev), X.to(dev)).to(X.device)

    def num_leaves(self) -> int:
        return int((self.feature == LEAF).sum())

    def path_feature_pairs(self) -> list[tuple[int, int]]:
        """(ancestor feature, descendant feature) pairs along root-to-leaf
        paths, one per (split node, ancestor split) (yabt/tree.py:186-203; the
        same multiset, listed in node-id order)."""
        feature = self.feature.tolist()
        left, right = self.left.tolist(), self.right.tolist()
        # children always get larger ids than their parent (grow.c:338-339), so
        # one pass in id order sees every parent before its children
        ancestors: list[list[int]] = [[] for _ in feature]
        pairs: list[tuple[int, int]] = []
        for nid, f in enumerate(feature):
            if f < 0:
                continue
            pairs.extend((a, f) for a in ancestors[nid])
            for child in (left[nid], right[nid]):
                ancestors[child] = ancestors[nid] + [f]
        return pairs
