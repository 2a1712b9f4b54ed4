"""Pins the oracle's k-means++ seeding (oracle.kmeans_plusplus, a restatement of
sklearn/cluster/_kmeans.py:174-263) and the host-side draw order
(skmetal_amd._bridge.plusplus_draws) before the GPU seeding is checked against them.

  * scikit-learn's docstring vector (kmeans_plusplus on 6 points, seed 0 -> rows [3, 2]);
  * golden picks of scikit-learn 1.7.2's kmeans_plusplus on 9 small inputs
    (tests/golden/plusplus.npz, written by make_plusplus_fixtures.py): blobs,
    a 1-feature line, exact duplicate rows (zero potentials), 1 and 20 trials,
    k = 1, and KMeans.fit's seeding on centred X;
  * invariants: distinct rows picked while any row is at a positive distance,
    the first pick is the seed's choice(n, p=w / w.sum());
  * planted mistakes (the worst candidate kept instead of the best, closest
    distances not min-updated, an exclusive running sum) that the golden picks
    must reject.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from skmetal_amd._bridge import plusplus_draws

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cases():
    meta = json.loads((GOLDEN / "plusplus.json").read_text())
    with np.load(GOLDEN / "plusplus.npz") as z:
        arrays = {key: z[key] for key in z.files}
    for c in meta["cases"]:
        yield c, arrays[c["name"] + "__X"], arrays[c["name"] + "__idx"]


CASES = list(_cases())


def _inputs(c, X):
    if c.get("centred"):
        X = X - X.mean(axis=0)
    T, first, u = plusplus_draws(np.random.RandomState(c["seed"]), X.shape[0], c["k"], c["n_local_trials"])
    return X, T, first, u


def test_docstring_vector():
    X = np.array([[1, 2], [1, 4], [1, 0], [10, 2], [10, 4], [10, 0]], np.float32)
    T, first, u = plusplus_draws(np.random.RandomState(0), 6, 2)
    assert T == 2
    np.testing.assert_array_equal(oracle.kmeans_plusplus(X, 2, first, u, T), [3, 2])


@pytest.mark.parametrize("case", CASES, ids=[c[0]["name"] for c in CASES])
def test_oracle_matches_sklearn_picks(case):
    c, X, idx = case
    Xi, T, first, u = _inputs(c, X)
    np.testing.assert_array_equal(oracle.kmeans_plusplus(Xi, c["k"], first, u, T), idx)


def test_draws_follow_sklearn_order():
    """The first draw is choice(n, p=w / w.sum()) on float32 unit weights, then the
    uniforms; drawing them at once leaves the generator where k - 1 calls would."""
    n, k, T = 1000, 7, 3
    a = np.random.RandomState(4)
    T2, first, u = plusplus_draws(a, n, k, T)
    b = np.random.RandomState(4)
    w = np.ones(n, np.float32)
    assert first == b.choice(n, p=w / w.sum())
    for c in range(k - 1):
        np.testing.assert_array_equal(u[c], b.uniform(size=T))
    assert a.randint(1 << 30) == b.randint(1 << 30)


def test_distinct_rows_while_potential_positive():
    rng = np.random.default_rng(3)
    X = rng.standard_normal((800, 5)).astype(np.float32)
    T, first, u = plusplus_draws(np.random.RandomState(1), 800, 40)
    idx = oracle.kmeans_plusplus(X, 40, first, u, T)
    assert len(set(idx.tolist())) == 40


def _planted(X, k, first, U, T, mistake):
    """oracle.kmeans_plusplus with one plausible mistake."""
    X = np.ascontiguousarray(X, np.float32)
    n = X.shape[0]
    idx = [first]
    closest = oracle._upcast_sqdist(X, np.array([first]))[0]
    pot = float(closest.astype(np.float64).sum())
    for c in range(1, k):
        r = U[c - 1] * float(np.float32(pot))
        cum = np.cumsum(closest, dtype=np.float64)
        if mistake == "exclusive":
            cum = np.concatenate([[0.0], cum[:-1]])
        cid = np.searchsorted(cum, r)
        cid = np.clip(cid, None, n - 1)
        dist = oracle._upcast_sqdist(X, cid)
        np.minimum(closest[None, :], dist, out=dist)
        cpot = dist.astype(np.float64).sum(axis=1)
        b = int(np.argmax(cpot)) if mistake == "worst" else int(np.argmin(cpot))
        if mistake == "no_min":
            dist = oracle._upcast_sqdist(X, cid)
        pot = float(cpot[b])
        closest = dist[b]
        idx.append(int(cid[b]))
    return np.array(idx)


@pytest.mark.parametrize("mistake", ["worst", "no_min", "exclusive"])
def test_planted_mistakes_are_caught(mistake):
    wrong = 0
    for c, X, idx in CASES:
        Xi, T, first, u = _inputs(c, X)
        wrong += not np.array_equal(_planted(Xi, c["k"], first, u, T, mistake), idx)
    assert wrong >= 3
