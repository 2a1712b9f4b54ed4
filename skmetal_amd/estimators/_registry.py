"""Estimator registry: sklearn class -> (module, GPU wrapper class).

Mirrors skmetal/estimators/_registry.py; this package accelerates KMeans
only, and registers it only when the MI355X path initialised.
"""

from sklearn.cluster import KMeans

from .. import _bridge

GPU_REGISTRY: dict[type, tuple[str, str]] = {}

if _bridge.HIP_AVAILABLE:
    GPU_REGISTRY[KMeans] = ("skmetal_amd.estimators.cluster", "HipKMeans")
