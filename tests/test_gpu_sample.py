"""GPU: numpy's RandomState.choice(n, size, replace=False, p=w / w.sum()) on the
device (skmetal_hip_lloyd_sample_prepare / _draw through LloydHandle.choice),
against numpy's own choice on the same weights and seeds.

The draws of MetalKMeans._kmeans_parallel_init (skmetal/estimators/cluster.py:
94-98: w = maximum(dists, 1e-30) with dists the k-means|| distances) and of
scikit-learn's init="random" (sklearn/cluster/_kmeans.py:1010-1013: unit
weights).  Picks are integer work: the rows must be identical, in order, and
the RandomState must be left where numpy leaves it.  numpy is the oracle here;
its weights are the device's own distances, downloaded.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

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


def _numpy_choice(dists, size, seed):
    rs = np.random.RandomState(seed)
    d = np.maximum(dists, 1e-30)
    rows = rs.choice(d.shape[0], size=size, p=d / d.sum(), replace=False)
    return rows, rs.rand()


def _device_choice(h, size, seed, exact=False, weights="mindists"):
    rs = np.random.RandomState(seed)
    rows = h.choice(rs, size, weights=weights, exact=exact)
    return rows, rs.rand(), h.sample_exact


def _blobs(n, d, k, seed, spread=10.0):
    rng = np.random.default_rng(seed)
    C = rng.normal(0, spread, (k, d))
    return (C[rng.integers(0, k, n)] + rng.normal(0, 1, (n, d))).astype(np.float32)


@pytest.mark.parametrize("n,d,size,cand", [(1, 17, 1, 1), (2, 4, 2, 1), (9, 3, 5, 2), (1000, 20, 50, 3),
                                           (8193, 33, 40, 5), (50_000, 100, 64, 7), (500_000, 100, 50, 10)])
def test_choice_matches_numpy(bridge, n, d, size, cand):
    _say(f"choice n={n} d={d} size={size}")
    X = _blobs(n, d, 6, n + d)
    rows0 = np.random.default_rng(n).choice(n, size=min(cand, n), replace=False)
    with bridge.LloydHandle(n, d, 1) as h:
        h.load(X, center=False)
        dists = h.mindists(rows0, reset=True)
        mixed = 0
        for seed in range(4):
            ref, ref_next = _numpy_choice(dists, size, seed)
            got, got_next, _ = _device_choice(h, size, seed)
            assert np.array_equal(got, ref), f"seed {seed}: {got[:8]} vs {ref[:8]}"
            assert got_next == ref_next, "the RandomState was not left where numpy leaves it"
            got_x, _, n_exact = _device_choice(h, size, seed, exact=True)
            assert np.array_equal(got_x, ref)
            assert n_exact >= size
            # a margin of 1/(4n): about half the draws take the exact search,
            # the rest stay with the certified one, in the same pass
            got_w, _, n_w = _device_choice(h, size, seed, exact=2)
            assert np.array_equal(got_w, ref)
            mixed += 0 < n_w < size
        if size >= 8:
            assert mixed > 0, "no pass split its draws between the two searches"


def test_choice_repeats_take_more_passes(bridge):
    # a few rows carry nearly all the weight: numpy draws the same rows again
    # and runs further passes with the found rows zeroed
    n, d = 3000, 17
    rng = np.random.default_rng(4)
    X = rng.normal(0, 1e-3, (n, d)).astype(np.float32)
    X[rng.choice(n, 12, replace=False)] += 40.0
    with bridge.LloydHandle(n, d, 2) as h:
        h.load(X, center=False)
        dists = h.mindists([0], reset=True)
        for seed in range(6):
            ref, ref_next = _numpy_choice(dists, 20, seed)
            got, got_next, _ = _device_choice(h, 20, seed)
            assert np.array_equal(got, ref) and got_next == ref_next
            got_x, _, _ = _device_choice(h, 20, seed, exact=True)
            assert np.array_equal(got_x, ref)


def test_choice_subnormal_and_zero_probabilities(bridge):
    # one far row: every other row's floored weight 1e-30 over a total of
    # ~1e9 (fp32 subnormal p) or ~1e18 (p rounds to 0: size 3 is then more
    # than the rows with p > 0, numpy's error)
    n, d = 2000, 20
    for far, what in [(3e4, "subnormal"), (1e9, "zero")]:
        X = np.zeros((n, d), np.float32)
        X[7, 0] = far
        X[11, 1] = 1.0
        with bridge.LloydHandle(n, d, 2) as h:
            h.load(X, center=False)
            dists = h.mindists([0], reset=True)
            for size in (1, 2, 3):
                try:
                    ref, ref_next = _numpy_choice(dists, size, 0)
                except ValueError as e:
                    with pytest.raises(ValueError, match=str(e)):
                        _device_choice(h, size, 0)
                    continue
                got, got_next, _ = _device_choice(h, size, 0)
                assert np.array_equal(got, ref) and got_next == ref_next, what


def test_choice_nan_probabilities_raise_numpy_error(bridge):
    # squared distances that overflow fp32: p = inf / inf = NaN
    n, d = 100, 17
    X = np.zeros((n, d), np.float32)
    X[3, :] = 3e19
    with bridge.LloydHandle(n, d, 2) as h:
        h.load(X, center=False)
        dists = h.mindists([0], reset=True)
        with pytest.raises(ValueError, match="probabilities contain NaN"):
            _numpy_choice(dists, 2, 0)
        with pytest.raises(ValueError, match="probabilities contain NaN"):
            _device_choice(h, 2, 0)


@pytest.mark.parametrize("n,size", [(5, 5), (1000, 10), (8192 * 3 + 5, 100), (500_000, 50)])
def test_unit_weights_match_numpy(bridge, n, size):
    # scikit-learn's init="random": p = ones(n, float32) / n
    with bridge.LloydHandle(n, 17, 1) as h:
        h.load(np.zeros((n, 17), np.float32), center=False)
        for seed in range(3):
            rs = np.random.RandomState(seed)
            w = np.ones(n, dtype=np.float32)
            ref = rs.choice(n, size=size, replace=False, p=w / w.sum())
            got, got_next, _ = _device_choice(h, size, seed, weights="unit")
            assert np.array_equal(got, ref) and got_next == rs.rand()


def test_choice_rejects_bad_calls(bridge):
    import ctypes

    from skmetal_amd._bridge import _lib

    with bridge.LloydHandle(100, 17, 2) as h:
        h.load(np.zeros((100, 17), np.float32), center=False)
        with pytest.raises(RuntimeError):
            h.choice(np.random.RandomState(0), 3)  # no k-means|| distances yet
        with pytest.raises(ValueError):
            h.choice(np.random.RandomState(0), 3, weights="other")
        with pytest.raises(ValueError, match="larger sample"):
            h.choice(np.random.RandomState(0), 101, weights="unit")
        u = np.array([0.5, 1.0])
        out = np.zeros(2, np.int64)
        ne = ctypes.c_int(0)
        assert _lib.skmetal_hip_lloyd_sample_draw(h._h, None, 0, u.ctypes.data, 2, out.ctypes.data, 0,
                                                  ctypes.byref(ne)) != 0  # u = 1 is outside [0, 1)
        bad = np.array([100], np.int64)
        assert _lib.skmetal_hip_lloyd_sample_draw(h._h, bad.ctypes.data, 1, u.ctypes.data, 1, out.ctypes.data, 0,
                                                  ctypes.byref(ne)) != 0  # zeroed row out of range


def test_random_init_seeds_match_sklearn(bridge):
    # KMeans(init="random"): each init's seed rows come from the device sampler
    # and equal scikit-learn's _init_centroids draws from the same RandomState,
    # init after init; a whole n_init=3 fit then lands on scikit-learn's inertia
    from sklearn.cluster import KMeans

    import skmetal_amd
    from skmetal_amd.estimators.cluster import HipKMeans

    X = _blobs(20_000, 24, 8, 3, spread=30.0)
    k = 8
    est = KMeans(n_clusters=k, init="random", n_init=3, random_state=11)
    rs_ref = np.random.RandomState(11)
    rs_got = np.random.RandomState(11)
    xx = np.einsum("ij,ij->i", X, X)
    w = np.ones(X.shape[0], dtype=X.dtype)
    with bridge.LloydHandle(X.shape[0], X.shape[1], k) as h:
        h.load(X, center=True)
        for _ in range(3):
            ref = est._init_centroids(X, x_squared_norms=xx, init="random", random_state=rs_ref, sample_weight=w)
            got = HipKMeans(est)._initial_centers(X, "random", k, rs_got, h)
            assert np.array_equal(got, ref)
    assert rs_got.rand() == rs_ref.rand()

    kw = dict(n_clusters=k, init="random", n_init=3, max_iter=100, random_state=11)
    ref = KMeans(**kw).fit(X)
    got = skmetal_amd.accelerate(KMeans(**kw)).fit(X)
    assert got.inertia_ == pytest.approx(ref.inertia_, rel=1e-4)
