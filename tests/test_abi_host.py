"""CPU checks of the drop-in boundary and the host-side mirror of skmetal's API.

No GPU is needed: the library is loaded but no compute entry point is called.

* libskmetal_hip.so exports exactly the functions include/skmetal_hip.h
  declares, and the ctypes registry binds every one of them;
* the reference's KMeans entry points (skmetal/_bridge.py:111-142, 352-363,
  627-639) are among them with the reference's names;
* without a usable GPU the package imports, reports HIP_AVAILABLE False,
  leaves estimators on scikit-learn (skmetal/estimators/_registry.py
  registers nothing it cannot run) and the GPU entry points raise instead of
  computing on the CPU;
* the estimator wrapper's host logic (tolerance scaling, n_init rules, routing
  thresholds, configuration API) behaves like skmetal's / scikit-learn's.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "skmetal_hip.h"
LIB = ROOT / "skmetal_amd" / "libskmetal_hip.so"

# the KMeans subset of skmetal's C ABI (skmetal_bridge/.../include/bridge.h:11-12,
# 37-45, 60 and the lazily bound skmetal_kmeans_inertia, _bridge.py:627-639)
REFERENCE_KMEANS_ABI = {
    "skmetal_init",
    "skmetal_warmup",
    "skmetal_device_info",
    "skmetal_kmeans_assign",
    "skmetal_kmeans_batch_fused",
    "skmetal_kmeans_inertia",
    "skmetal_compute_mindists",
}

# every name of skmetal's ctypes registry (skmetal/_bridge.py:107-345), which
# its loader binds eagerly when the library loads (:345-349)
REFERENCE_REGISTRY = [
    "skmetal_pairwise_distance", "skmetal_scaler_fit", "skmetal_column_minmax", "skmetal_kmeans_assign",
    "skmetal_kmeans_batch_fused", "skmetal_compute_mindists", "skmetal_gemm", "skmetal_fista_fit",
    "skmetal_column_transform", "skmetal_sv_init", "skmetal_sv_hook", "skmetal_sv_shortcut",
    "skmetal_knn_vote_classify", "skmetal_knn_vote_regress", "skmetal_knn_vote_classify_weighted",
    "skmetal_knn_vote_regress_weighted", "skmetal_knn_tiled_kneighbors", "skmetal_rbf_kernel_square",
    "skmetal_rbf_kernel_cross", "skmetal_tree_predict_all", "skmetal_svc_predict_binary", "skmetal_logreg_irls_fit",
    "skmetal_logreg_lbfgs_fit", "skmetal_ridge_fit_solve", "skmetal_multinomial_lbfgs_fit",
    "skmetal_minmax_transform", "skmetal_convert_f32_to_f16", "skmetal_convert_f16_to_f32", "skmetal_gemm_f16",
]
# the registry names this library implements; the others return SKMETAL_ENOSYS
PROVIDED = REFERENCE_KMEANS_ABI | {"skmetal_gemm"}
NOT_PROVIDED = set(REFERENCE_REGISTRY) - PROVIDED


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"SKMETAL_API\s+[\w\s\*]+?\b(skmetal_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib_path() -> Path:
    if not LIB.exists():  # built by __graft_entry__.build(); build here if nothing is
        from skmetal_amd import _build

        _build.build()
    return LIB


def test_header_declares_reference_kmeans_abi():
    names = _declared()
    assert REFERENCE_KMEANS_ABI <= names
    assert set(REFERENCE_REGISTRY) <= names
    extra = names - REFERENCE_KMEANS_ABI - set(REFERENCE_REGISTRY)
    assert all(n.startswith("skmetal_hip_") for n in extra), extra


def test_reference_loader_binds_every_registry_name(lib_path):
    # what skmetal/_bridge.py:345-349 does when the library loads: getattr of
    # every registry name (a missing one raises AttributeError at import)
    lib = ctypes.CDLL(str(lib_path))
    for name in REFERENCE_REGISTRY:
        f = getattr(lib, name)
        f.restype = ctypes.c_int
    assert len(NOT_PROVIDED) == 25


def test_registry_names_outside_kmeans_return_enosys(lib_path):
    # the stubs touch no device: callable without a GPU
    lib = ctypes.CDLL(str(lib_path))
    lib.skmetal_hip_last_error.restype = ctypes.c_char_p
    for name in sorted(NOT_PROVIDED):
        f = getattr(lib, name)
        f.restype = ctypes.c_int
        assert f() == 7, name  # SKMETAL_ENOSYS
        assert name in lib.skmetal_hip_last_error().decode()
    lib.skmetal_init()  # the library's last error is shared: leave it at the init result


def test_library_exports_every_declared_symbol(lib_path):
    lib = ctypes.CDLL(str(lib_path))
    for name in sorted(_declared()):
        assert hasattr(lib, name), f"{name} declared in skmetal_hip.h but not exported"


@pytest.mark.skipif(shutil.which("nm") is None, reason="binutils nm not available")
def test_library_exports_nothing_undeclared(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    ours = {s for s in exported if s.startswith("skmetal")}
    assert ours == _declared()


def test_ctypes_registry_binds_the_header():
    from skmetal_amd import _bridge

    bound = {entry[0] for entry in _bridge._REGISTRY}
    assert bound == _declared() - NOT_PROVIDED


def test_without_gpu_the_package_imports_and_refuses_to_compute():
    import skmetal_amd
    from skmetal_amd import _bridge
    from skmetal_amd.estimators import GPU_REGISTRY

    if _bridge.HIP_AVAILABLE:
        pytest.skip("a GPU is present")
    assert skmetal_amd.HIP_AVAILABLE is False and skmetal_amd.METAL_AVAILABLE is False
    assert GPU_REGISTRY == {}
    assert "no HIP device" in _bridge.last_error() or "not available" in _bridge.last_error().lower()
    X = np.zeros((8, 2), np.float32)
    with pytest.raises(RuntimeError):
        _bridge.kmeans_assign(X, X[:2].copy(), np.empty(8, np.int32), 8, 2, 2)
    with pytest.raises(RuntimeError):
        _bridge.kmeans_fit(X, X[:2].copy(), np.empty(8, np.int32), 10, 0.0)
    with pytest.raises(RuntimeError):
        skmetal_amd.device_info()


def test_accelerate_without_gpu_returns_sklearn_estimator():
    from sklearn.cluster import KMeans
    from sklearn.pipeline import Pipeline
    from sklearn.preprocessing import StandardScaler

    import skmetal_amd
    from skmetal_amd import _bridge

    if _bridge.HIP_AVAILABLE:
        pytest.skip("a GPU is present")
    km = KMeans(n_clusters=3, n_init=1)
    assert skmetal_amd.accelerate(km) is km
    pipe = skmetal_amd.accelerate(Pipeline([("s", StandardScaler()), ("k", KMeans(n_clusters=2))]))
    assert isinstance(pipe.steps[1][1], KMeans)


def _wrapper(**kw):
    from sklearn.cluster import KMeans

    from skmetal_amd.estimators.cluster import HipKMeans

    return HipKMeans(KMeans(**kw))


def test_small_inputs_route_to_sklearn_and_match_it():
    """Below KMeans' (1_000, 10) threshold (skmetal/_config.py:20) fit is sklearn's own."""
    from sklearn.cluster import KMeans

    rng = np.random.default_rng(0)
    X = rng.standard_normal((300, 4)).astype(np.float32)
    init = X[:3].copy()
    w = _wrapper(n_clusters=3, init=init, n_init=1, max_iter=50)
    w.fit(X)
    ref = KMeans(n_clusters=3, init=init, n_init=1, max_iter=50).fit(X)
    np.testing.assert_array_equal(w.labels_, ref.labels_)
    np.testing.assert_allclose(w.cluster_centers_, ref.cluster_centers_)


def test_large_inputs_without_gpu_fail_loudly():
    from skmetal_amd import _bridge

    if _bridge.HIP_AVAILABLE:
        pytest.skip("a GPU is present")
    rng = np.random.default_rng(1)
    X = rng.standard_normal((2000, 12)).astype(np.float32)
    w = _wrapper(n_clusters=4, init=X[:4].copy(), n_init=1)
    with pytest.raises(RuntimeError):
        w.fit(X)


def test_routing_rules():
    from skmetal_amd import set_device, set_threshold, update_threshold

    X = np.zeros((5000, 16), np.float32)
    w = _wrapper(n_clusters=2)
    assert w._should_use_gpu(X)
    assert not w._should_use_gpu(X[:999])          # rows below 1_000
    assert not w._should_use_gpu(X[:, :9].copy())  # columns below 10
    assert not w._should_use_gpu(X.astype(np.float64))
    set_threshold(10**9)
    assert not w._should_use_gpu(X)
    set_threshold(1)
    update_threshold("KMeans", 10, 2)
    assert w._should_use_gpu(X[:20, :2].copy())
    set_device("cpu")
    assert not w._should_use_gpu(X)


def test_config_api_validation_and_context():
    from skmetal_amd import (accelerate_context, get_config, reset_thresholds, set_device, set_dtype,
                             update_threshold)
    from skmetal_amd._config import PER_ESTIMATOR_THRESHOLDS

    with pytest.raises(ValueError):
        set_device("tpu")
    with pytest.raises(ValueError):
        set_dtype("float64")
    update_threshold("KMeans", 1, 1)
    assert get_config().thresholds["KMeans"] == (1, 1)
    reset_thresholds()
    assert get_config().thresholds == PER_ESTIMATOR_THRESHOLDS
    set_device("gpu")
    with accelerate_context(enabled=False):
        assert get_config().device == "cpu"
    assert get_config().device == "gpu"


@pytest.mark.parametrize("n,d", [(1, 1), (2, 3), (17, 5), (1000, 100), (4099, 130), (20000, 9), (65, 768)])
def test_column_variance_is_numpys(n, d):
    """The library's host column variances are numpy's float32 np.var(X, axis=0)
    bit for bit (row-order fp32 chains, fp64 divisions)."""
    from skmetal_amd import _bridge

    rng = np.random.default_rng(n + d)
    X = (rng.standard_normal((n, d)) * rng.uniform(0.01, 100, d) + rng.uniform(-1e3, 1e3, d)).astype(np.float32)
    np.testing.assert_array_equal(_bridge.column_variance(X), np.var(X, axis=0))


def test_tolerance_matches_sklearn():
    from sklearn.cluster._kmeans import _tolerance as sk_tolerance

    from skmetal_amd.estimators.cluster import _tolerance

    rng = np.random.default_rng(2)
    X = (rng.standard_normal((500, 7)) * rng.uniform(0.1, 5, 7)).astype(np.float32)
    for tol in (0.0, 1e-4, 0.3):
        assert _tolerance(X, tol) == sk_tolerance(X, tol)  # the same bits


def test_same_clustering_is_permutation_invariant():
    from skmetal_amd.estimators.cluster import _same_clustering

    rng = np.random.default_rng(3)
    a = rng.integers(0, 5, 200)
    perm = rng.permutation(5)
    assert _same_clustering(a, perm[a], 5)
    b = perm[a].copy()
    b[0] = (b[0] + 1) % 5
    assert not _same_clustering(a, b, 5)


def test_n_init_rules_follow_sklearn():
    w = _wrapper(n_clusters=3, n_init="auto")
    assert w._resolve_n_init("k-means++") == 1
    assert w._resolve_n_init("random") == 10
    w = _wrapper(n_clusters=3, n_init=5)
    assert w._resolve_n_init("random") == 5
    with pytest.warns(RuntimeWarning):
        assert w._resolve_n_init(np.zeros((3, 2), np.float32)) == 1


def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr


def test_synthetic_workloads_are_deterministic():
    from skmetal_amd import _synth

    X1, C1 = _synth.generate("c1", seed=5, scale=0.02)
    X2, C2 = _synth.generate("c1", seed=5, scale=0.02)
    assert X1.dtype == np.float32 and X1.flags.c_contiguous and X1.shape == (2000, 32)
    assert C1.shape == (8, 32)
    np.testing.assert_array_equal(X1, X2)
    np.testing.assert_array_equal(C1, C2)
    # init rows are rows of X
    assert all((X1 == c).all(axis=1).any() for c in C1)
