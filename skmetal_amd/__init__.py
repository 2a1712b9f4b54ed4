"""skmetal_amd: MI355X (gfx950) acceleration of scikit-learn's KMeans Lloyd path.

The public API mirrors skmetal's (skmetal/__init__.py:46-86)::

    import skmetal_amd as skmetal
    from sklearn.cluster import KMeans

    model = skmetal.accelerate(KMeans(n_clusters=50, n_init=1))
    model.fit(X)          # Lloyd iterations run on the GPU, X resident in HBM

``HIP_AVAILABLE`` (alias ``METAL_AVAILABLE``) reports whether the GPU path
initialised; without it ``accelerate`` leaves estimators on scikit-learn.
"""

from ._about import __version__, __version_info__
from ._config import (
    get_config,
    reset_thresholds,
    set_device,
    set_dtype,
    set_threshold,
    set_thresholds,
    set_verbose,
    update_threshold,
)
from .accelerate import accelerate, accelerate_context
from ._bridge import HIP_AVAILABLE, METAL_AVAILABLE

if HIP_AVAILABLE:
    from ._bridge import device_info
else:

    def device_info() -> dict:  # type: ignore[misc]
        raise RuntimeError("skmetal_amd: device_info() requires an MI355X (gfx950) GPU and libskmetal_hip.so.")


__all__ = [
    "__version__",
    "__version_info__",
    "HIP_AVAILABLE",
    "METAL_AVAILABLE",
    "accelerate",
    "accelerate_context",
    "device_info",
    "get_config",
    "set_device",
    "set_threshold",
    "set_dtype",
    "set_verbose",
    "set_thresholds",
    "update_threshold",
    "reset_thresholds",
]
