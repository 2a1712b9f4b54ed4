"""GPU: skmetal_gemm, the reference's fp32 GEMM entry point (bridge.h:14-19).

C = alpha op(A) op(B) + beta C against an fp64 product, to the fp32 bound of a
K-term dot product: |C - C_ref| <= 4 K 2^-24 (|alpha| |op(A)| |op(B)| +
|beta| |C|) elementwise.  Then the reference's own MetalKMeans.transform
formula (skmetal/estimators/cluster.py:135-146: sqrt(max(||x||^2 + ||c||^2
- 2 gemm(X, C^T), 0))) run on this gemm against scikit-learn's transform.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bridge():
    from skmetal_amd import _bridge

    if not _bridge.HIP_AVAILABLE:
        pytest.fail(f"GPU path unavailable on a GPU run: {_bridge.last_error()}")
    return _bridge


def _check(got, A, B, C0, alpha, beta, ta, tb):
    a = (A.T if ta else A).astype(np.float64)
    b = (B.T if tb else B).astype(np.float64)
    ref = alpha * (a @ b) + (beta * C0.astype(np.float64) if beta != 0.0 else 0.0)
    bound = abs(alpha) * (np.abs(a) @ np.abs(b))
    if beta != 0.0:
        bound = bound + abs(beta) * np.abs(C0)
    K = a.shape[1]
    tol = 4.0 * K * 2.0**-24 * bound + 1e-30
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= tol), f"max err/tol {np.max(err / tol):.3g}"


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 5, 3), (500, 50, 100), (333, 257, 129), (64, 4096, 768)])
def test_gemm_matches_fp64(bridge, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    got = bridge.gemm(A, B, trans_A=ta, trans_B=tb)
    assert got.shape == (M, N) and got.dtype == np.float32
    _check(got, A, B, None, 1.0, 0.0, ta, tb)


@pytest.mark.parametrize("alpha,beta", [(2.5, 0.0), (-1.0, 1.0), (0.5, -3.0)])
def test_gemm_alpha_beta(bridge, alpha, beta):
    rng = np.random.default_rng(11)
    A = rng.standard_normal((130, 70)).astype(np.float32)
    B = rng.standard_normal((70, 90)).astype(np.float32)
    C0 = rng.standard_normal((130, 90)).astype(np.float32)
    C = C0.copy()
    got = bridge.gemm(A, B, alpha=alpha, beta=beta, C=C)
    _check(got, A, B, C0, alpha, beta, False, False)


def test_gemm_beta_zero_ignores_c(bridge):
    # beta == 0: C is write-only (a NaN-filled C must not leak into the result)
    from skmetal_amd._bridge import _lib

    rng = np.random.default_rng(12)
    A = rng.standard_normal((40, 30)).astype(np.float32)
    B = rng.standard_normal((30, 20)).astype(np.float32)
    C = np.full((40, 20), np.nan, np.float32)
    rc = _lib.skmetal_gemm(A.ctypes.data, B.ctypes.data, C.ctypes.data, 40, 20, 30, ctypes.c_float(1.0),
                           ctypes.c_float(0.0), 0, 0)
    assert rc == 0
    _check(C, A, B, None, 1.0, 0.0, False, False)


def test_gemm_rejects_bad_arguments(bridge):
    from skmetal_amd._bridge import _lib

    A = np.ones((2, 2), np.float32)
    assert _lib.skmetal_gemm(None, A.ctypes.data, A.ctypes.data, 2, 2, 2, ctypes.c_float(1.0), ctypes.c_float(0.0),
                             0, 0) == 1
    assert _lib.skmetal_gemm(A.ctypes.data, A.ctypes.data, A.ctypes.data, 0, 2, 2, ctypes.c_float(1.0),
                             ctypes.c_float(0.0), 0, 0) == 1
    with pytest.raises(ValueError):
        bridge.gemm(np.ones((3, 4), np.float32), np.ones((5, 2), np.float32))


def test_reference_transform_formula_on_gemm(bridge):
    # skmetal's MetalKMeans.transform computed with this library's gemm, against
    # scikit-learn's transform: the expanded form in fp32 loses ~1e-7 ||x||^2
    from sklearn.cluster import KMeans

    rng = np.random.default_rng(13)
    X = (rng.standard_normal((3000, 40)) + rng.integers(0, 5, (3000, 1)) * 4.0).astype(np.float32)
    km = KMeans(n_clusters=6, n_init=1, random_state=0).fit(X)
    centers = km.cluster_centers_.astype(np.float32)
    X_norms = np.einsum("ij,ij->i", X, X)[:, np.newaxis]
    C_norms = np.einsum("ij,ij->i", centers, centers)[np.newaxis, :]
    cross = bridge.gemm(X, np.ascontiguousarray(centers.T))
    got = np.sqrt(np.maximum(X_norms + C_norms - 2.0 * cross, 0.0))
    ref = km.transform(X)
    scale = np.sqrt(X_norms + C_norms)
    assert np.all(np.abs(got**2 - ref**2) <= 1e-5 * scale**2)
