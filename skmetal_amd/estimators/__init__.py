"""GPU-accelerated estimators."""

from ._base import BaseGPUEstimator  # noqa: F401
from ._registry import GPU_REGISTRY  # noqa: F401
from .cluster import HipKMeans, MetalKMeans  # noqa: F401

__all__ = ["BaseGPUEstimator", "GPU_REGISTRY", "HipKMeans", "MetalKMeans"]
