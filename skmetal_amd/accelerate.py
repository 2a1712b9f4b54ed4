"""``accelerate`` and ``accelerate_context``: the API of skmetal/accelerate.py.

``accelerate`` takes, in order of precedence:
  - a Pipeline      -> a new Pipeline with every registered step wrapped;
  - a class         -> the class, changed so that calling it with an
                       estimator or Pipeline as first argument returns that
                       object accelerated (any other call constructs as before);
  - an estimator    -> its GPU wrapper (the estimator itself when none is
                       registered);
  - a callable      -> a function that calls it and accelerates what it returns;
  - nothing         -> itself, for use as ``@accelerate()``.
Anything else is returned unchanged with a warning.

``accelerate_context(enabled)`` routes the calling thread to "gpu" (or
"cpu") for the duration of a ``with`` block; blocks nest.
"""

from __future__ import annotations

import warnings
from functools import wraps
from typing import Any

from sklearn.pipeline import Pipeline

from ._config import _pop_thread_device, _push_thread_device
from ._dispatch import _wrap_estimator, _wrap_pipeline


def _is_model(obj: Any) -> bool:
    return isinstance(obj, Pipeline) or hasattr(obj, "fit")


def _accelerated(obj: Any) -> Any:
    """The accelerated form of an estimator or Pipeline."""
    return _wrap_pipeline(obj) if isinstance(obj, Pipeline) else _wrap_estimator(obj)


def _accelerate_class(cls: type) -> type:
    base_new = cls.__new__
    base_init = cls.__init__

    @wraps(base_new)
    def __new__(klass, *args, **kwargs):
        if args and _is_model(args[0]):
            return _accelerated(args[0])
        if base_new is object.__new__:
            return object.__new__(klass)
        return base_new(klass)

    @wraps(base_init)
    def __init__(self, *args, **kwargs):
        # reached only when __new__ returned an instance of cls
        if args and _is_model(args[0]):
            return
        base_init(self, *args, **kwargs)

    cls.__new__ = __new__
    cls.__init__ = __init__
    return cls


def _accelerate_factory(factory):
    @wraps(factory)
    def build(*args, **kwargs):
        made = factory(*args, **kwargs)
        return _accelerated(made) if _is_model(made) else made

    return build


def accelerate(obj: Any | None = None) -> Any:
    """Accelerate a scikit-learn estimator, Pipeline, class or factory
    (skmetal/accelerate.py:17-37)."""
    if obj is None:
        return accelerate
    if isinstance(obj, Pipeline):
        return _wrap_pipeline(obj)
    if isinstance(obj, type):
        return _accelerate_class(obj)
    if hasattr(obj, "fit"):
        return _wrap_estimator(obj)
    if callable(obj):
        return _accelerate_factory(obj)
    warnings.warn(f"accelerate() was given a {type(obj).__name__}, which is not an estimator, Pipeline, class or "
                  "callable; it is returned unchanged.", stacklevel=2)
    return obj


class accelerate_context:
    """``with accelerate_context(enabled):`` routes the calling thread to the GPU
    (enabled) or to scikit-learn (not enabled) until the block ends; other
    threads are not affected (skmetal/accelerate.py:95-113)."""

    def __init__(self, enabled: bool = True):
        self.enabled = enabled

    def __enter__(self):
        _push_thread_device("gpu" if self.enabled else "cpu")
        return self

    def __exit__(self, *exc):
        _pop_thread_device()
        return False
