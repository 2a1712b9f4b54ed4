"""CPU checks of the estimator layer's host logic: scikit-learn's
same-clustering rule for n_init > 1, the feature-count check of predict /
transform / score, and the size checks the bridge applies before it hands
raw pointers to the library."""

from __future__ import annotations

import numpy as np
import pytest


def _same_clustering_loop(a, b, k):
    # sklearn/cluster/_k_means_common.pyx _is_same_clustering, as a plain loop
    mapping = [-1] * k
    for x, y in zip(a.tolist(), b.tolist()):
        if mapping[x] == -1:
            mapping[x] = y
        elif mapping[x] != y:
            return False
    return True


def test_same_clustering_matches_the_loop():
    from skmetal_amd.estimators.cluster import _same_clustering

    rng = np.random.default_rng(0)
    for _ in range(500):
        k = int(rng.integers(1, 10))
        n = int(rng.integers(1, 60))
        a = rng.integers(0, k, n).astype(np.int32)
        b = rng.permutation(k)[a].astype(np.int32)
        kind = rng.integers(0, 3)
        if kind == 1:
            b[rng.integers(0, n)] = rng.integers(0, k)       # one row moved
        elif kind == 2:
            b = (b // 2).astype(np.int32)                    # two labels merged: still a function of a
        assert _same_clustering(a, b, k) == _same_clustering_loop(a, b, k)


def test_same_clustering_large_is_fast():
    import time

    from skmetal_amd.estimators.cluster import _same_clustering

    rng = np.random.default_rng(1)
    a = rng.integers(0, 50, 500_000).astype(np.int32)
    b = rng.permutation(50)[a].astype(np.int32)
    t = time.perf_counter()
    assert _same_clustering(a, b, 50)
    b[123_456] = (b[123_456] + 1) % 50
    assert not _same_clustering(a, b, 50)
    assert time.perf_counter() - t < 0.5


def test_feature_count_is_checked_like_sklearn():
    from sklearn.cluster import KMeans

    from skmetal_amd.estimators.cluster import _check_n_features

    km = KMeans(n_clusters=2)
    km.n_features_in_ = 5
    _check_n_features(km, np.zeros((3, 5), np.float32))
    with pytest.raises(ValueError, match="X has 4 features, but KMeans is expecting 5 features"):
        _check_n_features(km, np.zeros((3, 4), np.float32))


@pytest.mark.parametrize("bad", ["X", "centroids", "assignments", "dists"])
def test_bridge_rejects_arrays_of_the_wrong_size(bad):
    from skmetal_amd import _bridge

    n, d, k = 10, 4, 3
    X = np.zeros((n, d), np.float32)
    C = np.zeros((k, d), np.float32)
    lab = np.zeros(n, np.int32)
    dist = np.zeros(n, np.float32)
    if bad == "X":
        X = np.zeros((n, d - 1), np.float32)
    elif bad == "centroids":
        C = np.zeros((k, d + 1), np.float32)
    elif bad == "assignments":
        lab = np.zeros(n - 1, np.int32)
    else:
        dist = np.zeros(n + 1, np.float32)
    with pytest.raises(ValueError):
        if bad == "dists":
            _bridge.compute_mindists(X, C, lab, dist, n, d, k)
        else:
            _bridge.kmeans_assign(X, C, lab, n, d, k)
