"""Dispatch configuration: the API of skmetal/_config.py.

Functions kept by name, signature and meaning (skmetal/_config.py:119-199):
``get_config``, ``set_device``, ``set_threshold``, ``set_dtype``,
``set_verbose``, ``set_thresholds``, ``update_threshold``,
``reset_thresholds``, and the ``PER_ESTIMATOR_THRESHOLDS`` table
(skmetal/_config.py:6-32).

State is one process-wide ``Config`` plus, per thread, an optional device
override.  ``accelerate_context`` keeps a stack per thread of the devices
the thread routed to when each block began, and re-pins the thread to that
device when the block ends (skmetal's semantics); ``set_device`` sets the
process-wide value and the calling thread's override together, so the
caller reads back what it set even inside a context.  Writers hold one lock; readers do not need it (every field is a
single reference replaced atomically).
"""

from __future__ import annotations

import threading

# (min_rows, min_cols) below which an estimator stays on scikit-learn.  The
# values are skmetal's (skmetal/_config.py:6-32); this package consults the
# KMeans entry only and keeps the rest so that configuration code written for
# skmetal runs unchanged.
PER_ESTIMATOR_THRESHOLDS: dict[str, tuple[int, int]] = {
    "KMeans": (1_000, 10),
    "StandardScaler": (1_000, 10),
    "LinearRegression": (50_000, 50),
    "TruncatedSVD": (5_000, 20),
    "PCA": (5_000, 10),
    "ElasticNet": (50_000, 50),
    "Lasso": (50_000, 50),
    "LogisticRegression": (500_000, 500),
    "Ridge": (10_000_000, 10_000),
    "MinMaxScaler": (500_000, 10),
    "KNeighborsClassifier": (5_000_000, 10_000),
    "KNeighborsRegressor": (5_000_000, 10_000),
    "RobustScaler": (100_000, 10),
    "DBSCAN": (1_000, 2),
    "HistGradientBoostingClassifier": (10_000, 10),
    "HistGradientBoostingRegressor": (10_000, 10),
    "GaussianNB": (10_000, 10),
    "SVC": (5_000, 10),
    "SVR": (5_000, 10),
    "NearestNeighbors": (5_000, 10),
}

DEVICES = ("gpu", "cpu", "auto")
DTYPES = ("float32",)


class _ThreadState(threading.local):
    """Per-thread routing state: the device override (None: the process-wide
    value applies) and the stack accelerate_context saves overrides on."""

    def __init__(self):
        self.device: str | None = None
        self.saved: list[str | None] = []


_thread = _ThreadState()
_write_lock = threading.Lock()


class Config:
    """Routing configuration.

    device      "gpu" (default), "cpu" (always scikit-learn) or "auto"; reading
                it gives the calling thread's value
    threshold   smallest n_samples * n_features sent to the GPU
    dtype       compute dtype; "float32" only
    verbose     print every routing decision
    thresholds  class name -> (min_rows, min_cols)
    """

    def __init__(self, device: str = "gpu", threshold: int = 1, dtype: str = "float32", verbose: bool = False,
                 thresholds: dict | None = None):
        self.global_device = device
        self.threshold = threshold
        self.dtype = dtype
        self.verbose = verbose
        self.thresholds = dict(PER_ESTIMATOR_THRESHOLDS) if thresholds is None else thresholds

    @property
    def device(self) -> str:
        return self.global_device if _thread.device is None else _thread.device

    @device.setter
    def device(self, value: str) -> None:
        self.global_device = value

    def __repr__(self) -> str:
        on_gpu = [name for name, (rows, _) in self.thresholds.items() if rows < 10**8]
        return (f"Config(device={self.device!r}, threshold={self.threshold}, dtype={self.dtype!r}, "
                f"verbose={self.verbose}, {len(on_gpu)} of {len(self.thresholds)} estimators GPU-eligible)")


_config = Config()


def get_config() -> Config:
    """The configuration object (its ``device`` reads the calling thread's value)."""
    return _config


def _get_device() -> str:
    """The device routing uses on the calling thread."""
    return _config.device


def _set_thread_device(device: str | None) -> None:
    """Set the calling thread's device override, or drop it (None)."""
    _thread.device = device


def _push_thread_device(device: str) -> None:
    """accelerate_context's entry: save the device the thread routes to now
    (its override, or the process-wide value), then override it."""
    _thread.saved.append(_get_device())
    _thread.device = device


def _pop_thread_device() -> None:
    """accelerate_context's exit: pin the thread to the device saved by the
    matching push, as skmetal does (skmetal/accelerate.py:104-113): after
    the block the thread keeps that device even if ``set_device`` later
    changes the process-wide value from another thread."""
    if _thread.saved:
        _thread.device = _thread.saved.pop()


def set_device(device: str) -> None:
    """Route to "gpu", "cpu" (scikit-learn everywhere) or "auto".  Sets the
    process-wide value and the calling thread's override."""
    if device not in DEVICES:
        raise ValueError(f"device must be one of {', '.join(repr(d) for d in DEVICES)}, not {device!r}")
    with _write_lock:
        _config.global_device = device
        _thread.device = device


def set_threshold(threshold: int) -> None:
    """Inputs with fewer than ``threshold`` elements (n * d) stay on the CPU."""
    with _write_lock:
        _config.threshold = int(threshold)


def set_dtype(dtype: str) -> None:
    """Compute dtype of the GPU path; only "float32" is accepted."""
    if dtype not in DTYPES:
        raise ValueError(f"dtype {dtype!r} is not supported on the GPU path (float32 only)")
    with _write_lock:
        _config.dtype = dtype


def set_verbose(verbose: bool) -> None:
    """Print every routing decision (True) or none (False)."""
    with _write_lock:
        _config.verbose = bool(verbose)


def set_thresholds(thresholds: dict) -> None:
    """Replace the whole per-estimator table (class name -> (min_rows, min_cols))."""
    with _write_lock:
        _config.thresholds = dict(thresholds)


def update_threshold(name: str, min_rows: int, min_cols: int) -> None:
    """Set one estimator's (min_rows, min_cols): smaller inputs stay on the CPU."""
    with _write_lock:
        table = dict(_config.thresholds)
        table[name] = (min_rows, min_cols)
        _config.thresholds = table


def reset_thresholds() -> None:
    """Restore PER_ESTIMATOR_THRESHOLDS."""
    with _write_lock:
        _config.thresholds = dict(PER_ESTIMATOR_THRESHOLDS)
