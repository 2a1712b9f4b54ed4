"""Synthetic test problems shared by the CPU and GPU tests."""

from __future__ import annotations

import numpy as np


def mixed_scale_problem(n, d, k, seed, kind):
    """Columns of very different magnitudes in one X.

    kind "quantised": d - 1 clustered columns at ~1e3 next to one column of
    multiples of 1e-5 (integers 0..40 per cluster plus a per-row jitter);
    kind "1e6": half the columns at ~1e3, half at ~1e-3 (10^6 : 1);
    kind "cluster": in every column, half the clusters sit at ~1e3 and half at
    ~1e-3, so one column holds centres 10^6 apart."""
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, k, n)
    if kind == "quantised":
        cen = rng.uniform(-1e3, 1e3, (k, d))
        X = cen[ids] + rng.standard_normal((n, d)) * 30.0
        q = rng.integers(0, 40, k)[ids] + rng.integers(0, 3, n)
        X[:, d - 1] = q * 1e-5
    elif kind == "1e6":
        cen = rng.uniform(-1e3, 1e3, (k, d))
        X = cen[ids] + rng.standard_normal((n, d)) * 30.0
        X[:, d // 2:] *= 1e-6
    else:
        cen = rng.uniform(-1.0, 1.0, (k, d)) * np.where(np.arange(k) % 2 == 0, 1e3, 1e-3)[:, None]
        X = cen[ids] + rng.standard_normal((n, d)) * np.where(ids % 2 == 0, 30.0, 3e-5)[:, None]
    X = X.astype(np.float32)
    C0 = np.stack([X[np.flatnonzero(ids == j)[0]] for j in range(k)])
    return X, C0
