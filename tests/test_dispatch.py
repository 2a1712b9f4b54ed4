"""CPU tests of the dispatch layer: which objects ``accelerate`` wraps and
how, the order of the routing rules, and the per-thread device override of
``accelerate_context`` -- the behaviour of skmetal's accelerate.py,
_dispatch.py and estimators/_base.py, exercised with a toy estimator
registered for the test."""

from __future__ import annotations

import threading
import warnings

import numpy as np
import pytest
from scipy import sparse
from sklearn.pipeline import Pipeline
from sklearn.preprocessing import StandardScaler

import skmetal_amd
from skmetal_amd.estimators._base import BaseGPUEstimator


class Toy:
    """A minimal estimator type with a registered GPU wrapper."""

    def __init__(self, k=1):
        self.k = k

    def fit(self, X, y=None):
        self.fitted_ = True
        return self


class ToyGPU(BaseGPUEstimator):
    pass


@pytest.fixture
def registry(monkeypatch):
    from skmetal_amd.estimators import _registry

    monkeypatch.setitem(_registry.GPU_REGISTRY, Toy, (__name__, "ToyGPU"))
    skmetal_amd.update_threshold("Toy", 100, 4)
    yield
    skmetal_amd.reset_thresholds()


def test_estimator_and_pipeline_forms(registry):
    t = Toy()
    w = skmetal_amd.accelerate(t)
    assert isinstance(w, ToyGPU) and w._estimator is t
    scaler = StandardScaler()
    p = skmetal_amd.accelerate(Pipeline([("toy", Toy(2)), ("s", scaler)], verbose=False))
    assert isinstance(p, Pipeline)
    assert [name for name, _ in p.steps] == ["toy", "s"]
    assert isinstance(p.steps[0][1], ToyGPU) and p.steps[0][1].k == 2  # attribute read through the wrapper
    assert p.steps[1][1] is scaler


def test_factory_and_decorator_forms(registry):
    @skmetal_amd.accelerate
    def make(k):
        return Toy(k)

    @skmetal_amd.accelerate()
    def make_pipe():
        return Pipeline([("toy", Toy())])

    @skmetal_amd.accelerate
    def make_other():
        return 42

    assert isinstance(make(3), ToyGPU) and make(3).k == 3
    assert isinstance(make_pipe().steps[0][1], ToyGPU)
    assert make_other() == 42
    assert make.__name__ == "make"


def test_class_form(registry):
    @skmetal_amd.accelerate
    class Holder:
        def __init__(self, v=0):
            self.v = v

    assert isinstance(Holder(Toy()), ToyGPU)
    assert isinstance(Holder(Pipeline([("toy", Toy())])), Pipeline)
    h = Holder(5)
    assert isinstance(h, Holder) and h.v == 5


def test_unrecognised_object_is_returned_with_a_warning():
    with pytest.warns(UserWarning):
        assert skmetal_amd.accelerate(7) == 7


def test_routing_rule_order(registry):
    w = skmetal_amd.accelerate(Toy())
    X = np.zeros((200, 8), np.float32)
    assert w._should_use_gpu(X)
    assert not w._should_use_gpu(X[:99])                   # rows below the Toy entry
    assert not w._should_use_gpu(np.zeros((200, 3), np.float32))
    assert not w._should_use_gpu(X.astype(np.float64))     # dtype
    assert not w._should_use_gpu(sparse.csr_matrix(X))     # sparse, before the dtype rule reads X.dtype
    skmetal_amd.set_threshold(200 * 8 + 1)                 # global n * d threshold
    assert not w._should_use_gpu(X)
    skmetal_amd.set_threshold(1)
    skmetal_amd.set_device("cpu")
    assert not w._should_use_gpu(X)
    skmetal_amd.set_device("auto")                         # "auto" routes by the thresholds
    assert w._should_use_gpu(X)


def test_verbose_prints_each_decision(registry, capsys):
    w = skmetal_amd.accelerate(Toy())
    skmetal_amd.set_verbose(True)
    try:
        w._should_use_gpu(np.zeros((200, 8), np.float32))
        w._should_use_gpu(np.zeros((50, 8), np.float32))
    finally:
        skmetal_amd.set_verbose(False)
    out = capsys.readouterr().out.splitlines()
    assert out[0].endswith("device=gpu (200x8)")
    assert "device=cpu" in out[1] and "per-estimator min 100x4" in out[1]


def test_context_nests_and_stays_on_its_thread():
    cfg = skmetal_amd.get_config()
    seen = {}
    inside = threading.Event()
    done = threading.Event()

    def other():
        inside.wait(5)
        seen["other"] = cfg.device
        done.set()

    th = threading.Thread(target=other)
    th.start()
    with skmetal_amd.accelerate_context(enabled=False):
        assert cfg.device == "cpu"
        with skmetal_amd.accelerate_context(enabled=True):
            assert cfg.device == "gpu"
        assert cfg.device == "cpu"
        inside.set()
        done.wait(5)
    th.join()
    assert seen["other"] == "gpu"
    assert cfg.device == "gpu"


def test_context_exit_pins_the_thread_to_its_entry_device():
    """skmetal/accelerate.py:95-113: the block saves the device the thread
    routed to at entry and sets it as the thread's own on exit, so a later
    set_device from another thread no longer reaches that thread."""
    cfg = skmetal_amd.get_config()
    skmetal_amd.set_device("gpu")
    seen = {}
    exited = threading.Event()
    changed = threading.Event()

    def worker():
        with skmetal_amd.accelerate_context(enabled=False):
            seen["inside"] = cfg.device
        seen["after_exit"] = cfg.device
        exited.set()
        changed.wait(5)
        seen["after_set_device"] = cfg.device

    th = threading.Thread(target=worker)
    th.start()
    exited.wait(5)
    skmetal_amd.set_device("cpu")  # process-wide value and this thread's own
    changed.set()
    th.join()
    try:
        assert seen == {"inside": "cpu", "after_exit": "gpu", "after_set_device": "gpu"}
        # a thread that never entered a block follows the process-wide value
        fresh = {}
        t2 = threading.Thread(target=lambda: fresh.setdefault("d", cfg.device))
        t2.start()
        t2.join()
        assert fresh["d"] == "cpu"
    finally:
        skmetal_amd.set_device("gpu")


def test_set_device_is_seen_by_its_caller_inside_a_context():
    with skmetal_amd.accelerate_context(enabled=True):
        skmetal_amd.set_device("cpu")
        assert skmetal_amd.get_config().device == "cpu"
    skmetal_amd.set_device("gpu")


def test_wrapper_reads_through_and_fails_on_unknown_names(registry):
    w = skmetal_amd.accelerate(Toy(9))
    assert w.k == 9
    with pytest.raises(AttributeError):
        w.no_such_attribute
    assert not w.__sklearn_is_fitted__()


def test_unregistered_estimator_warns_only_when_verbose():
    s = StandardScaler()
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert skmetal_amd.accelerate(s) is s
    skmetal_amd.set_verbose(True)
    try:
        with pytest.warns(UserWarning):
            assert skmetal_amd.accelerate(s) is s
    finally:
        skmetal_amd.set_verbose(False)
