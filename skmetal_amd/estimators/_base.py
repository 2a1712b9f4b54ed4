"""Base class of the GPU wrappers: the API of skmetal/estimators/_base.py.

A wrapper holds the scikit-learn estimator it accelerates and answers, per
input, whether that input goes to the GPU.  The routing rules are skmetal's
(skmetal/estimators/_base.py:20-52), checked in this order; the first that
applies keeps the call on scikit-learn:
  1. the calling thread's device is "cpu";
  2. X is sparse;
  3. X is not float32;
  4. n * d is below the global threshold;
  5. n or d is below the estimator's (min_rows, min_cols) entry.
Everything the wrapper does not implement is read from the wrapped
estimator (fitted attributes included).
"""

from __future__ import annotations

import numpy as np
from sklearn.base import BaseEstimator
from sklearn.utils.validation import check_array

from .._config import _get_device, get_config


def _cpu_reason(name: str, X) -> str | None:
    """Why X stays on scikit-learn for the estimator class `name`, or None."""
    cfg = get_config()
    if _get_device() == "cpu":
        return "forced by set_device"
    if hasattr(X, "nnz"):
        return "sparse matrix"
    if X.dtype != np.float32:
        return f"dtype={X.dtype}, need float32"
    n, d = X.shape
    if n * d < cfg.threshold:
        return f"{n}x{d} = {n * d:,} < {cfg.threshold:,} threshold"
    limits = cfg.thresholds.get(name)
    if limits is not None and (n < limits[0] or d < limits[1]):
        return f"{n}x{d} < per-estimator min {limits[0]}x{limits[1]}"
    return None


class BaseGPUEstimator(BaseEstimator):
    """Wraps one scikit-learn estimator (``_estimator``)."""

    _estimator: BaseEstimator | None

    def __init__(self, _estimator=None):
        self._estimator = _estimator
        self._fitted = False

    def _validate_data(self, X, y=None):
        """X as float32 C-order with at least two rows; y as a float32 vector."""
        X = check_array(X, dtype=np.float32, order="C", ensure_min_samples=2)
        if y is not None:
            y = check_array(y, dtype=np.float32, order="C", ensure_2d=False)
        return X, y

    def _should_use_gpu(self, X) -> bool:
        name = type(self._estimator).__name__ if self._estimator is not None else type(self).__name__
        reason = _cpu_reason(name, X)
        if get_config().verbose:
            where = "gpu ({}x{})".format(*X.shape) if reason is None else f"cpu ({reason})"
            print(f"[skmetal_amd] {type(self).__name__}: device={where}")
        return reason is None

    def _fallback_fit(self, X, y, **kwargs):
        self._estimator.fit(X, y, **kwargs)
        self._fitted = True
        return self

    def _fallback_predict(self, X):
        return self._estimator.predict(X)

    def _fallback_transform(self, X):
        return self._estimator.transform(X)

    def score(self, X, y=None, **kwargs):
        return self._estimator.score(X, y, **kwargs)

    def predict(self, X):
        return self._fallback_predict(X)

    def transform(self, X):
        return self._fallback_transform(X)

    def __sklearn_is_fitted__(self) -> bool:
        return self._fitted

    def __getattr__(self, name):
        # only called for names not found on the wrapper itself
        if name in ("_estimator", "_fitted"):
            raise AttributeError(name)
        inner = self.__dict__.get("_estimator")
        if inner is not None and hasattr(inner, name):
            return getattr(inner, name)
        raise AttributeError(f"{type(self).__name__!r} object has no attribute {name!r}")
