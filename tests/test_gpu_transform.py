"""GPU parity of KMeans.transform (skmetal_hip_kmeans_transform): the distances
must be scikit-learn's, i.e. equal to the oracle's restatement of
euclidean_distances for fp32 data.

Both evaluate d^2 = -2 x.c + ||x||^2 + ||c||^2 in fp64 from the same fp32
inputs, but sum the dot products in different orders (BLAS blocks, the kernel
a sequential fma chain), so their fp64 values may differ by the forward error
of that expression, |e| <= 2 d 2^-53 (||x||^2 + ||c||^2).  Where d^2 is far
from 0 that moves a distance by at most 1 ulp; where x ~ c it can decide
between 0 and sqrt(|e|) (the kernel's chain gives exactly 0 for x = c).  The
check allows 1 ulp plus that error carried through the square root, and
requires 99% of the distances to be bit-exact.
"""

from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def bridge():
    from skmetal_amd import _bridge

    if not _bridge.HIP_AVAILABLE:
        pytest.fail(f"GPU path unavailable on a GPU run: {_bridge.last_error()}")
    return _bridge


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(D, ref, X, C, what):
    assert D.shape == ref.shape and D.dtype == np.float32
    X64, C64 = X.astype(np.float64), C.astype(np.float64)
    eps = 2.0 * X.shape[1] * 2.0**-53 * ((X64 * X64).sum(1)[:, None] + (C64 * C64).sum(1)[None, :])
    r = ref.astype(np.float64)
    tol = np.spacing(ref).astype(np.float64) + np.minimum(np.sqrt(eps), eps / (2.0 * np.maximum(r, 1e-300)))
    bad = np.abs(D.astype(np.float64) - r) > tol
    assert not bad.any(), f"{what}: {int(bad.sum())} distances off, e.g. {D[bad][:4]} vs {ref[bad][:4]}"
    exact = float(np.mean(D == ref))
    assert exact >= 0.99, f"{what}: only {exact:.5f} of the distances are bit-exact"


def _cases():
    meta = json.loads((GOLDEN / "transform.json").read_text())
    with np.load(GOLDEN / "transform.npz") as z:
        a = {key: z[key] for key in z.files}
    return [(c["name"], a[c["name"] + "__X"], a[c["name"] + "__C"], a[c["name"] + "__D"]) for c in meta["cases"]]


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_transform_golden(bridge, case):
    name, X, C, D = case
    _say(f"transform golden {name} {X.shape} k={C.shape[0]}")
    _check(bridge.kmeans_transform(X, C), D, X, C, name)


@pytest.mark.parametrize("n,d,k", [(1, 1, 1), (63, 5, 65), (1000, 1, 3), (777, 300, 10), (4097, 33, 130),
                                   (5000, 100, 50), (100003, 120, 21), (70001, 64, 37)])
def test_transform_vs_oracle(bridge, n, d, k):
    _say(f"transform vs oracle n={n} d={d} k={k}")
    rng = np.random.default_rng(n * 7 + d + k)
    X = (rng.standard_normal((n, d)) * rng.uniform(0.5, 3.0, d) + rng.uniform(-5, 5, d)).astype(np.float32)
    C = X[rng.choice(n, size=min(k, n), replace=False)]
    if C.shape[0] < k:
        C = np.concatenate([C, (rng.standard_normal((k - C.shape[0], d))).astype(np.float32)])
    _check(bridge.kmeans_transform(X, C), oracle.transform(X, C), X, C, f"{n}x{d} k={k}")


def test_transform_full_size_headline_workload(bridge):
    """500,000 x 100 against 50 centres: a 100 MB distance matrix."""
    from skmetal_amd import _synth

    X, C0 = _synth.generate("c2", seed=0)
    bridge.kmeans_transform(X[:1000], C0)
    t = time.perf_counter()
    D = bridge.kmeans_transform(X, C0)
    _say(f"transform 500000x100 k=50: {(time.perf_counter() - t) * 1e3:.1f} ms (host buffers, PCIe included)")
    _check(D, oracle.transform(X, C0), X, C0, "c2 transform")


def test_accelerate_transform_and_fit_transform(bridge):
    from sklearn.cluster import KMeans

    import skmetal_amd

    rng = np.random.default_rng(5)
    cen = rng.uniform(-10, 10, (6, 12))
    X = (cen[rng.integers(0, 6, 8000)] + rng.standard_normal((8000, 12))).astype(np.float32)
    Y = (cen[rng.integers(0, 6, 3000)] + rng.standard_normal((3000, 12))).astype(np.float32)
    kw = dict(n_clusters=6, init="k-means++", n_init=1, random_state=2)
    model = skmetal_amd.accelerate(KMeans(**kw))
    FT = model.fit_transform(X)
    C = model.cluster_centers_
    _check(FT, oracle.transform(X, C), X, C, "fit_transform")
    _check(model.transform(Y), oracle.transform(Y, C), Y, C, "transform")
    ref = KMeans(**kw).fit(X)
    np.testing.assert_allclose(model.transform(Y), ref.transform(Y), rtol=1e-4, atol=1e-4)
