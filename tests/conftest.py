import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for _p in (ROOT, ROOT / "tests"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(autouse=True)
def reset_config():
    """Reset skmetal_amd's global config before every test (tests/conftest.py:7-17 of skmetal)."""
    try:
        from skmetal_amd._config import PER_ESTIMATOR_THRESHOLDS, _set_thread_device, get_config
    except ImportError:
        yield
        return
    cfg = get_config()
    cfg.device = "gpu"
    _set_thread_device(None)
    cfg.threshold = 1
    cfg.dtype = "float32"
    cfg.verbose = False
    cfg.thresholds = dict(PER_ESTIMATOR_THRESHOLDS)
    yield
