"""GPU parity of the device k-means++ seeding (skmetal_hip_kmeans_plusplus /
skmetal_hip_lloyd_plusplus) against scikit-learn's picks and the oracle.

With the same random draws the device must pick exactly the rows the oracle
(a restatement of sklearn/cluster/_kmeans.py:174-263 with fp64 reductions)
picks, and on the golden inputs exactly the rows scikit-learn 1.7.2 picked.
"""

from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle import parity

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


def _cases():
    meta = json.loads((GOLDEN / "plusplus.json").read_text())
    with np.load(GOLDEN / "plusplus.npz") as z:
        arrays = {key: z[key] for key in z.files}
    return [(c, arrays[c["name"] + "__X"], arrays[c["name"] + "__idx"]) for c in meta["cases"]]


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0]["name"] for c in CASES])
def test_plusplus_golden_picks(bridge, case):
    c, X, idx = case
    n, d = X.shape
    _say(f"plusplus golden {c['name']} n={n} d={d} k={c['k']}")
    rs = np.random.RandomState(c["seed"])
    if c.get("centred"):
        with bridge.LloydHandle(n, d, c["k"]) as h:
            h.load(X, center=True)
            got = h.plusplus(rs, c["n_local_trials"])
            cen = h.centers()
        np.testing.assert_array_equal(got, idx)
        # the seeded centres are the chosen rows of X (centred, then shifted back)
        parity.check_centers(cen, X[idx], what="seeded centres")
    else:
        centers, got = bridge.kmeans_plusplus(X, c["k"], rs, c["n_local_trials"])
        np.testing.assert_array_equal(got, idx)
        np.testing.assert_array_equal(centers, X[idx])


def _blobs(n, d, k, seed, spread=10.0):
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-spread, spread, (k, d))
    ids = rng.integers(0, k, n)
    return (cen[ids] + rng.standard_normal((n, d))).astype(np.float32)


SHAPES = [
    # n, d, k, n_local_trials (None: 2 + int(ln k))
    (1, 3, 1, None),
    (255, 2, 9, None),
    (1000, 1, 10, None),
    (2049, 7, 30, 20),       # two candidate passes of 16
    (3000, 300, 8, None),    # two LDS feature segments
    (300, 3, 300, None),     # k = n: every row once
    (70000, 16, 16, 3),      # 274 row blocks in the running sum
    (20000, 100, 50, None),
    (5000, 50, 20, None),    # rows of 52 floats (the 64-float instance), 4 candidates
    (4000, 120, 12, 8),      # rows of 120 floats (the 128-float instance), 8 candidates
]


@pytest.mark.parametrize("n,d,k,trials", SHAPES)
def test_plusplus_vs_oracle(bridge, n, d, k, trials):
    _say(f"plusplus vs oracle n={n} d={d} k={k} trials={trials}")
    X = _blobs(n, d, max(1, k // 2), seed=n + d + k)
    T, first, u = bridge.plusplus_draws(np.random.RandomState(k), n, k, trials)
    ref = oracle.kmeans_plusplus(X, k, first, u, T)
    _, got = bridge.kmeans_plusplus(X, k, np.random.RandomState(k), trials)
    np.testing.assert_array_equal(got, ref)
    if k == n:
        assert sorted(got.tolist()) == list(range(n))


def test_plusplus_duplicate_rows_zero_potential(bridge):
    """Once every distinct row is taken the potential is 0 and every draw is 0:
    searchsorted then returns row 0 (the first running sum >= 0), as numpy does."""
    rng = np.random.default_rng(4)
    X = np.repeat(rng.uniform(-3, 3, (3, 5)), [300, 200, 100], axis=0).astype(np.float32)
    T, first, u = bridge.plusplus_draws(np.random.RandomState(8), X.shape[0], 6)
    ref = oracle.kmeans_plusplus(X, 6, first, u, T)
    _, got = bridge.kmeans_plusplus(X, 6, np.random.RandomState(8))
    np.testing.assert_array_equal(got, ref)


def test_plusplus_is_deterministic(bridge):
    X = _blobs(50000, 24, 20, seed=2)
    a = bridge.kmeans_plusplus(X, 40, np.random.RandomState(5))[1]
    b = bridge.kmeans_plusplus(X, 40, np.random.RandomState(5))[1]
    np.testing.assert_array_equal(a, b)


def test_plusplus_rejects_bad_trials(bridge):
    X = _blobs(100, 4, 3, seed=1)
    with bridge.LloydHandle(100, 4, 3) as h:
        h.load(X)
        with pytest.raises(RuntimeError, match="n_local_trials"):
            h.plusplus_with(65, 0, np.zeros(2 * 65))
        with pytest.raises(RuntimeError, match="first index"):
            h.plusplus_with(2, 100, np.zeros(4))


def test_plusplus_full_size_headline_workload(bridge):
    """500,000 x 100, k = 50 (centred, as KMeans.fit seeds): device vs oracle, and the time."""
    from skmetal_amd import _synth

    X, _ = _synth.generate("c2", seed=0)
    n, d = X.shape
    k = 50
    mean = oracle.mean_f32(X)
    Xc = X - mean
    T, first, u = bridge.plusplus_draws(np.random.RandomState(0), n, k)
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=True)
        h.plusplus_with(T, first, u)  # warm
        t = time.perf_counter()
        got = h.plusplus_with(T, first, u)
        dt = time.perf_counter() - t
    _say(f"device k-means++ 500000x100 k=50: {dt * 1e3:.2f} ms")
    ref = oracle.kmeans_plusplus(Xc, k, first, u, T)
    np.testing.assert_array_equal(got, ref)


def test_accelerate_fit_plusplus_n_init(bridge):
    """KMeans(init='k-means++', n_init=3): three device seedings from one random
    state and one upload of X, the best kept, as scikit-learn does."""
    from sklearn.cluster import KMeans

    import skmetal_amd

    X = _blobs(20000, 16, 10, seed=21)
    kw = dict(n_clusters=10, init="k-means++", n_init=3, max_iter=100, random_state=7)
    model = skmetal_amd.accelerate(KMeans(**kw)).fit(X)
    ref = KMeans(**kw).fit(X)
    parity.check_centers(model.cluster_centers_, ref.cluster_centers_, what="n_init=3 centres")
    parity.check_inertia(model.inertia_, ref.inertia_, rtol=1e-5, atol=parity.centring_floor(X),
                         what="n_init=3 inertia")
