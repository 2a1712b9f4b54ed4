"""GPU parity of skmetal's k-means|| seeding with its distance rounds on the
device (skmetal_hip_lloyd_mindists; MetalKMeans._kmeans_parallel_init,
skmetal/estimators/cluster.py:70-116) against the oracle, and of the
MetalKMeans mirror's fit."""

from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from oracle import parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bridge():
    from skmetal_amd import _bridge

    if not _bridge.HIP_AVAILABLE:
        pytest.fail(f"GPU path unavailable on a GPU run: {_bridge.last_error()}")
    return _bridge


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _blobs(n, d, k, seed):
    rng = np.random.default_rng(seed)
    C = rng.normal(0, 10, (k, d))
    return (C[rng.integers(0, k, n)] + rng.normal(0, 1, (n, d))).astype(np.float32)


def _check(got, ref, X, rows, what):
    """Both are the fp32 cast of the fp64 expanded distance; the fp64 sums
    differ in order, so values agree to 1 ulp plus that rounding."""
    X64 = X.astype(np.float64)
    xx = np.einsum("ij,ij->i", X64, X64)
    cc = xx[np.asarray(rows)].max()
    eps = 2.0 * X.shape[1] * 2.0**-53 * (xx + cc)
    r = ref.astype(np.float64)
    tol = np.spacing(ref).astype(np.float64) + np.minimum(np.sqrt(eps), eps / (2.0 * np.maximum(r, 1e-300)))
    bad = np.abs(got.astype(np.float64) - r) > tol
    assert not bad.any(), f"{what}: {int(bad.sum())} distances off, e.g. {got[bad][:4]} vs {ref[bad][:4]}"
    # at a candidate's own row (x = c) the device's sums cancel exactly, where the
    # oracle's BLAS product leaves fp64 noise; elsewhere the casts agree
    own = np.zeros(X.shape[0], dtype=bool)
    own[np.asarray(rows)] = True
    assert np.all(got[own] == 0.0), f"{what}: x = c not exactly 0"
    exact = float(np.mean(got[~own] == ref[~own]))
    assert exact >= 0.99, f"{what}: only {exact:.5f} bit-exact"


@pytest.mark.parametrize("n,d,m", [(1000, 5, 1), (4097, 33, 20), (3001, 100, 70), (777, 1, 9),
                                   (150001, 120, 37)])  # more 64-row spans than resident blocks; rows of 120
def test_mindists_match_oracle(bridge, n, d, m):
    _say(f"k-means|| mindists n={n} d={d} m={m}")
    X = _blobs(n, d, 6, n + m)
    rng = np.random.default_rng(m)
    a = rng.choice(n, m, replace=False)
    b = rng.choice(n, 5, replace=False)
    f = oracle.parallel_mindists(X)
    with bridge.LloydHandle(n, d, 2) as h:
        h.load(X, center=False)
        _check(h.mindists(a, reset=True), f(a, True), X, a, "first round")
        _check(h.mindists(b), f(b, False), X, np.concatenate([a, b]), "second round")
        _check(h.mindists([]), f([], False), X, np.concatenate([a, b]), "no new rows")
        _check(h.mindists(b[:2], reset=True), f(b[:2], True), X, b[:2], "reset")


def test_mindists_errors(bridge):
    X = _blobs(500, 4, 3, 0)
    with bridge.LloydHandle(500, 4, 2) as h:
        h.load(X, center=False)
        with pytest.raises(RuntimeError):
            h.mindists([1, 2])            # the first round must reset
        with pytest.raises(RuntimeError):
            h.mindists([1, 500], reset=True)
        with pytest.raises(RuntimeError):
            h.mindists([-1], reset=True)
        assert np.isfinite(h.mindists([7], reset=True)).all()


@pytest.mark.parametrize("n,d,k,seed", [(20000, 20, 8, 0), (5000, 100, 50, 1), (3000, 7, 3, 2)])
def test_parallel_init_matches_oracle(bridge, n, d, k, seed):
    from skmetal_amd.estimators.cluster import kmeans_parallel_init

    _say(f"k-means|| init n={n} d={d} k={k} seed={seed}")
    X = _blobs(n, d, k, seed + 10)
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=False)
        got, got_rows = kmeans_parallel_init(X, k, np.random.RandomState(seed), h, trace=True)
    ref, ref_rows = oracle.kmeans_parallel_init(X, k, np.random.RandomState(seed), trace=True)
    assert got.shape == (k, d) and got.dtype == np.float32
    _check_init(got, got_rows, ref, ref_rows, k, f"n={n} d={d} k={k}")


def _check_init(got, got_rows, ref, ref_rows, k, what):
    """Candidate rows are integer picks: identical, in order.  Up to k
    candidates are the centroids themselves (bit for bit); more are pruned by
    one Lloyd iteration, the device's against scikit-learn's (the reference's
    prune): the same labels of the candidates give centres equal within the
    fp32 parity tolerance."""
    np.testing.assert_array_equal(np.asarray(got_rows), np.asarray(ref_rows), err_msg=f"{what}: candidate rows")
    if len(ref_rows) <= k:
        np.testing.assert_array_equal(got, ref, err_msg=what)
    else:
        parity.check_centers(got, ref, what=f"{what}: pruned centroids")


def test_parallel_init_matches_reference_method(bridge):
    """The device path against the reference method's own draws and prune
    (tests/golden/kpar.npz, written by make_kpar_fixtures.py): every
    candidate row, then the centroids."""
    from skmetal_amd.estimators.cluster import kmeans_parallel_init
    from test_kpar_oracle import KPAR

    for c, a in KPAR:
        X = a["X"]
        n, d = X.shape
        _say(f"k-means|| vs reference vectors {c['name']}")
        with bridge.LloydHandle(n, d, c["k"]) as h:
            h.load(X, center=False)
            got, rows = kmeans_parallel_init(X, c["k"], np.random.RandomState(c["seed"]), h, trace=True)
        _check_init(got, rows, a["centroids"], a["final_rows"], c["k"], c["name"])


def test_metal_kmeans_fit(bridge):
    from sklearn.cluster import KMeans

    from skmetal_amd.estimators.cluster import MetalKMeans

    X = _blobs(30000, 24, 10, 4)
    # three steps per attempt: the reference's k-means|| prune often seeds two
    # centres in one blob, so longer runs cross near-ties at every step and any
    # two fp32 implementations drift apart; over three steps a near-tie row
    # moves a centre by far less than the tolerance
    m = MetalKMeans(KMeans(n_clusters=10, n_init=2, random_state=0, max_iter=3))
    assert m._should_use_gpu(X)
    m.fit(X)
    est = m._estimator
    assert est.labels_.shape == (30000,) and est.labels_.min() >= 0 and est.labels_.max() < 10
    assert est.cluster_centers_.shape == (10, 24) and est.n_iter_ >= 1
    # the reference's fit sequence (cluster.py:20-67), all on the oracle: its
    # k-means||, then per attempt skmetal's batch_fused loop contract with tol
    # as given (reference_loop) and the inertia of its labels and centres; the
    # attempt of lowest inertia is kept (a k-means|| prune can end above
    # scikit-learn's fit)
    rng = np.random.RandomState(0)
    best = None
    for _ in range(2):
        out = oracle.reference_loop(X, oracle.kmeans_parallel_init(X, 10, rng), 3, 1e-4)
        inertia = oracle.inertia(X, out["centers"], out["labels"])
        if best is None or inertia < best[0]:
            best = (inertia, out)
    inertia, out = best
    parity.check_inertia(est.inertia_, inertia, rtol=1e-5, what="MetalKMeans inertia")
    parity.check_centers(est.cluster_centers_, out["centers"], what="MetalKMeans centres")
    _, b1, b2 = oracle.assign(X, out["estep_centers"], return_gap=True)
    parity.check_labels(est.labels_, out["labels"], b1, b2, X, what="MetalKMeans labels")
    # labels_ are the last step's E-step (the reference's contract); predict is
    # the E-step on the final centres
    ref_p, p1, p2 = oracle.assign(X, est.cluster_centers_, return_gap=True)
    parity.check_labels(m.predict(X), ref_p, p1, p2, X, what="MetalKMeans predict")
    m2 = MetalKMeans(KMeans(n_clusters=10, n_init=2, random_state=0, max_iter=3))
    np.testing.assert_array_equal(m2.fit_predict(X), est.labels_)   # the device fit, not sklearn's
    D = m.transform(X[:1000])
    assert D.shape == (1000, 10) and np.mean(np.argmin(D, axis=1) == ref_p[:1000]) >= 0.99


def test_mindists_candidate_buffer_growth(bridge):
    # rounds with more new rows than any before regrow the device candidate list
    X = _blobs(5000, 12, 4, 9)
    f = oracle.parallel_mindists(X)
    rng = np.random.default_rng(3)
    seen = []
    with bridge.LloydHandle(5000, 12, 4) as h:
        h.load(X, center=False)
        for i, m in enumerate((3, 40, 150, 2)):
            rows = rng.choice(5000, m, replace=False)
            seen.extend(rows.tolist())
            _check(h.mindists(rows, reset=(i == 0)), f(rows, i == 0), X, seen, f"round {i} (m={m})")


def test_parallel_init_large_k_matches_oracle(bridge):
    """k = 512: int(2 + ln 512) = 8 rounds of 512 draws each (the draw blocks,
    repeated passes, the candidate buffers growing), then ~4,000 candidates
    pruned by one Lloyd iteration of k = 512 on the device's generic path."""
    from skmetal_amd.estimators.cluster import kmeans_parallel_init

    n, d, k = 60_000, 24, 512
    X = _blobs(n, d, 40, 21)
    _say(f"k-means|| init n={n} d={d} k={k}")
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=False)
        got, got_rows = kmeans_parallel_init(X, k, np.random.RandomState(5), h, trace=True)
    ref, ref_rows = oracle.kmeans_parallel_init(X, k, np.random.RandomState(5), trace=True)
    assert len(ref_rows) > 8 * k // 2
    _check_init(got, got_rows, ref, ref_rows, k, f"n={n} d={d} k={k}")
