"""Type-keyed dispatch from scikit-learn estimators to their GPU wrappers: the
API of skmetal/_dispatch.py (``_is_supported``, ``_get_gpu_impl``,
``_wrap_estimator``, ``_wrap_pipeline``).

The wrapper class for an estimator is looked up by the estimator's exact type
in ``estimators._registry.GPU_REGISTRY`` and imported on first use.  A
Pipeline is rebuilt step by step (names, memory and verbosity kept), each
step wrapped on its own type; unsupported steps are kept as they are.
"""

from __future__ import annotations

import importlib
import warnings

from sklearn.pipeline import Pipeline

from ._config import get_config
from .estimators._registry import GPU_REGISTRY


def _is_supported(estimator) -> bool:
    """True when a GPU wrapper is registered for the estimator's exact type."""
    return type(estimator) in GPU_REGISTRY


def _get_gpu_impl(estimator) -> type:
    """The GPU wrapper class registered for the estimator's type."""
    module_name, class_name = GPU_REGISTRY[type(estimator)]
    try:
        return getattr(importlib.import_module(module_name), class_name)
    except (ImportError, AttributeError) as exc:
        raise ImportError(f"the GPU wrapper {module_name}.{class_name} registered for "
                          f"{type(estimator).__name__} cannot be loaded: {exc}") from exc


def _wrap_estimator(estimator):
    """The estimator inside its GPU wrapper, or the estimator itself when none
    is registered (with a warning when verbose)."""
    if _is_supported(estimator):
        return _get_gpu_impl(estimator)(estimator)
    if get_config().verbose:
        warnings.warn(f"{type(estimator).__name__} has no MI355X implementation; it runs on scikit-learn.",
                      stacklevel=3)
    return estimator


def _wrap_pipeline(pipeline: Pipeline) -> Pipeline:
    """A new Pipeline whose steps are wrapped by type (step names are not read)."""
    return Pipeline([(name, _wrap_estimator(step)) for name, step in pipeline.steps], memory=pipeline.memory,
                    verbose=pipeline.verbose)
