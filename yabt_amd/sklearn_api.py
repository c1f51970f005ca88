"""Scikit-learn style estimators on the GPU booster (mirror of
yabt/sklearn_api.py:238-363).

``YABTRegressor`` standardises y (mean, population std, 1 if zero) and
predicts ``margin * std + mean``; ``YABTClassifier`` is binary log loss on
``classes_`` (the second class positive) with ``predict_proba`` =
[1 - p, p], p = expit(margin), and one-vs-rest ``MulticlassBooster`` for more
than two classes.  Hyperparameters are the ``BoostParams`` fields, passed as
keyword arguments.  Categorical target encoding (``categorical_features``)
is not provided by this backend.
"""

from __future__ import annotations

import numpy as np
from scipy.special import expit
from sklearn.base import BaseEstimator, ClassifierMixin, RegressorMixin

from .boosting import PARAM_NAMES, Booster, BoostParams, LogLoss, MSELoss, MulticlassBooster


def _require_single_target(y: np.ndarray) -> np.ndarray:
    """(n,) or (n, 1) targets only (sklearn_api.py:224-236)."""
    if y.ndim == 2 and y.shape[1] == 1:
        return y.ravel()
    if y.ndim > 1:
        raise ValueError(f"y has shape {y.shape}; this estimator predicts a single target")
    return y


class _YABTBase(BaseEstimator):
    def __init__(self, **kwargs):
        defaults = BoostParams()
        for name in PARAM_NAMES:
            setattr(self, name, kwargs.pop(name, getattr(defaults, name)))
        self.cat_smoothing = kwargs.pop("cat_smoothing", 10.0)
        if kwargs:
            raise TypeError(f"Unknown parameters: {sorted(kwargs)}")

    @classmethod
    def _get_param_names(cls):
        return sorted(PARAM_NAMES + ["cat_smoothing"])

    def _boost_params(self) -> BoostParams:
        return BoostParams(**{n: getattr(self, n) for n in PARAM_NAMES})

    @staticmethod
    def _no_categoricals(categorical_features) -> None:
        if categorical_features:
            raise NotImplementedError("categorical target encoding is not provided by this backend")

    @staticmethod
    def _X(X) -> np.ndarray:
        return np.asarray(X, dtype=np.float32)

    def _margin(self, X) -> np.ndarray:
        return self.booster_.predict_margin(self._X(X))


class YABTRegressor(_YABTBase, RegressorMixin):
    """Squared-error regressor; standardises the target internally."""

    def _transform_y(self, y: np.ndarray, fit: bool) -> np.ndarray:
        if fit:
            self._y_mean = float(y.mean())
            self._y_std = float(y.std()) or 1.0
        return (y - self._y_mean) / self._y_std

    def fit(self, X, y, eval_set=None, categorical_features: list[int] | None = None):
        self._no_categoricals(categorical_features)
        y = _require_single_target(np.asarray(y, dtype=np.float32))
        yt = self._transform_y(y, fit=True)
        ev = None
        if eval_set is not None:
            ev = (self._X(eval_set[0]), self._transform_y(np.asarray(eval_set[1], dtype=np.float32), fit=False))
        self.booster_ = Booster(self._boost_params(), MSELoss())
        self.booster_.fit(self._X(X), yt, eval_set=ev)
        return self

    def predict(self, X) -> np.ndarray:
        return self._margin(X) * self._y_std + self._y_mean


class YABTClassifier(_YABTBase, ClassifierMixin):
    """Binary log-loss classifier; one-vs-rest for more than two classes."""

    def fit(self, X, y, eval_set=None, categorical_features: list[int] | None = None):
        self._no_categoricals(categorical_features)
        y = np.asarray(y, dtype=np.float32)
        self.classes_ = np.unique(y)
        self.n_classes_ = len(self.classes_)
        self._is_binary = self.n_classes_ == 2
        Xe = self._X(X)
        if self._is_binary:
            yt = (y == self.classes_[1]).astype(np.float32)
            ev = None
            if eval_set is not None:
                yv = (np.asarray(eval_set[1], dtype=np.float32) == self.classes_[1]).astype(np.float32)
                ev = (self._X(eval_set[0]), yv)
            self.booster_ = Booster(self._boost_params(), LogLoss())
            self.booster_.fit(Xe, yt, eval_set=ev)
        else:
            ev = None if eval_set is None else (self._X(eval_set[0]), eval_set[1])
            self.booster_ = MulticlassBooster(self._boost_params())
            self.booster_.fit(Xe, y, eval_set=ev)
        return self

    def predict_proba(self, X) -> np.ndarray:
        """Class probabilities, (n_samples, n_classes)."""
        Xe = self._X(X)
        if self._is_binary:
            p = expit(self.booster_.predict_margin(Xe))
            return np.stack([1 - p, p], axis=1)
        return self.booster_.predict_proba(Xe)

    def predict(self, X) -> np.ndarray:
        Xe = self._X(X)
        if self._is_binary:
            return self.classes_[(self.booster_.predict_margin(Xe) > 0).astype(int)]
        return self.booster_.predict(Xe)


__all__ = ["YABTRegressor", "YABTClassifier"]
