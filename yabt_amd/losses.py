"""Losses producing the grower's g and h (mirror of yabt/boosting.py:27-58).

Same classes, static methods and formulas as the reference, evaluated with
torch on the margin's device.  ``loss_id`` names the loss to the device
kernel of the boosting step (``yabt_grad_hess``: 0 squared error, 1 logistic),
which computes the same formulas in fp32.
"""

from __future__ import annotations

import numpy as np
import torch


class LogLoss:
    """Binary log loss on logits (boosting.py:27-42)."""
    is_classification = True
    loss_id = 1

    @staticmethod
    def base_score(y: torch.Tensor) -> float:
        p = float(y.mean().clamp(1e-6, 1 - 1e-6))
        return float(np.log(p / (1 - p)))

    @staticmethod
    def grad_hess(margin: torch.Tensor, y: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        p = torch.sigmoid(margin)
        return p - y, (p * (1 - p)).clamp_min(1e-6)

    @staticmethod
    def loss(margin: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        return torch.nn.functional.binary_cross_entropy_with_logits(margin, y)


class MSELoss:
    """Squared error (boosting.py:45-58); h = 1."""
    is_classification = False
    loss_id = 0

    @staticmethod
    def base_score(y: torch.Tensor) -> float:
        return float(y.mean())

    @staticmethod
    def grad_hess(margin: torch.Tensor, y: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return margin - y, torch.ones_like(y)

    @staticmethod
    def loss(margin: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        return 0.5 * (margin - y).square().mean()
