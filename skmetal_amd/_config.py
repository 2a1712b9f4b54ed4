"""Configuration API (mirrors skmetal/_config.py of the reference).

Thread-safe global configuration with a per-thread device override used by
``accelerate_context``.  Only the KMeans entry of the per-estimator
threshold table is consulted by this package; the other names are kept so
that code written against skmetal's configuration functions keeps working.
"""

import threading

PER_ESTIMATOR_THRESHOLDS: dict[str, tuple[int, int]] = {
    # (min_rows, min_cols) below which an estimator stays on the CPU
    # (skmetal/_config.py:6-32; KMeans :20)
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


class Config:
    """Global configuration for GPU dispatch.

    Attributes
    ----------
    device : str
        ``"gpu"``, ``"cpu"`` (scikit-learn) or ``"auto"``.
    threshold : int
        Minimum ``n_samples * n_features`` for GPU dispatch.
    dtype : str
        Compute dtype; only ``"float32"``.
    verbose : bool
        Print every routing decision.
    thresholds : dict
        Per-estimator ``(min_rows, min_cols)``.
    """

    def __init__(self, device="gpu", threshold=1, dtype="float32", verbose=False, thresholds=None):
        self._device = device
        self.threshold = threshold
        self.dtype = dtype
        self.verbose = verbose
        self.thresholds = thresholds if thresholds is not None else dict(PER_ESTIMATOR_THRESHOLDS)

    @property
    def device(self) -> str:
        val = getattr(_thread_local, "device", _UNSET)
        return self._device if val is _UNSET else val

    @device.setter
    def device(self, val: str):
        self._device = val

    def __repr__(self):
        n_gpu = sum(1 for v in self.thresholds.values() if v[0] < 1e8)
        n_cpu = len(self.thresholds) - n_gpu
        return (
            f"device={self.device}, threshold={self.threshold}, verbose={self.verbose}\n"
            f"  estimators routed to GPU: {n_gpu}  |  estimators routed to CPU: {n_cpu}"
        )


_config = Config()
_lock = threading.Lock()
_thread_local = threading.local()
_UNSET = object()


def get_config() -> Config:
    return _config


def _get_device() -> str:
    val = getattr(_thread_local, "device", _UNSET)
    return _config._device if val is _UNSET else val


def _set_thread_device(device) -> None:
    if device is None:
        if hasattr(_thread_local, "device"):
            del _thread_local.device
    else:
        _thread_local.device = device


def set_device(device: str) -> None:
    """``"gpu"`` (default), ``"cpu"`` (force scikit-learn) or ``"auto"``."""
    with _lock:
        if device not in ("gpu", "cpu", "auto"):
            raise ValueError("device must be 'gpu', 'cpu', or 'auto'")
        _config._device = device
        _thread_local.device = device


def set_threshold(threshold: int) -> None:
    with _lock:
        _config.threshold = int(threshold)


def set_dtype(dtype: str) -> None:
    with _lock:
        if dtype != "float32":
            raise ValueError("Only float32 is supported for GPU operations.")
        _config.dtype = dtype


def set_verbose(verbose: bool) -> None:
    with _lock:
        _config.verbose = bool(verbose)


def set_thresholds(thresholds: dict) -> None:
    with _lock:
        _config.thresholds = dict(thresholds)


def update_threshold(name: str, min_rows: int, min_cols: int) -> None:
    with _lock:
        _config.thresholds[name] = (min_rows, min_cols)


def reset_thresholds() -> None:
    with _lock:
        _config.thresholds = dict(PER_ESTIMATOR_THRESHOLDS)
