"""The oracle's restatement of skmetal's k-means|| seeding
(MetalKMeans._kmeans_parallel_init, skmetal/estimators/cluster.py:70-116),
checked on the CPU: its distances against scikit-learn and brute force, the
loop's rules (first draw, round count, the {0} taken set, the cyclic fill) by
properties, and the whole seeding against golden vectors of the reference's
own method (tests/golden/kpar.npz, written by make_kpar_fixtures.py, which runs
MetalKMeans._kmeans_parallel_init with numpy distances in place of its two
bridge calls): the candidate rows of every round, the final candidate list and
the k centroids, bit for bit."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
from sklearn.metrics.pairwise import euclidean_distances

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def kpar_cases():
    """(case metadata, arrays) of the reference's k-means|| fixtures."""
    meta = json.loads((GOLDEN / "kpar.json").read_text())
    with np.load(GOLDEN / "kpar.npz") as z:
        arrays = {key: z[key] for key in z.files}
    return [(c, {key[len(c["name"]) + 2:]: v for key, v in arrays.items() if key.startswith(c["name"] + "__")})
            for c in meta["cases"]]


KPAR = kpar_cases()


@pytest.mark.parametrize("case", KPAR, ids=[c[0]["name"] for c in KPAR])
def test_oracle_matches_reference_method(case):
    c, a = case
    X = a["X"]
    C, rows = oracle.kmeans_parallel_init(X, c["k"], np.random.RandomState(c["seed"]), trace=True)
    rows = np.asarray(rows, dtype=np.int64)
    for r in range(c["rounds"]):
        ref = a[f"round{r}_rows"]
        np.testing.assert_array_equal(rows[: len(ref)], ref, err_msg=f"candidates at round {r}")
    np.testing.assert_array_equal(rows, a["final_rows"])
    np.testing.assert_array_equal(C, a["centroids"])


def test_reference_vectors_show_the_taken_set_quirk():
    # the reference's taken set starts as {0} (cluster.py:86): in the case that
    # draws every row, row 0 never joins and the first row joins twice
    c, a = next(x for x in KPAR if x[0]["name"] == "all_rows_10x3_k10")
    rows = list(a["final_rows"])
    first = np.random.RandomState(c["seed"]).randint(c["n"])
    assert first != 0 and 0 not in rows and rows.count(first) == 2


def _blobs(n, d, k, seed):
    rng = np.random.default_rng(seed)
    C = rng.normal(0, 10, (k, d))
    return (C[rng.integers(0, k, n)] + rng.normal(0, 1, (n, d))).astype(np.float32)


@pytest.mark.parametrize("n,d", [(500, 3), (777, 33), (300, 100)])
def test_mindists_match_sklearn_and_brute_force(n, d):
    X = _blobs(n, d, 5, n + d)
    f = oracle.parallel_mindists(X)
    rows_a, rows_b = [3, 17, 250], [9, 120]
    got_a = f(rows_a, True)
    got_b = f(rows_b, False)
    for got, rows in ((got_a, rows_a), (got_b, rows_a + rows_b)):
        sk = euclidean_distances(X[rows], X, squared=True).min(axis=0)
        brute = ((X.astype(np.float64)[None, :, :] - X.astype(np.float64)[rows][:, None, :]) ** 2).sum(-1).min(0)
        assert got.dtype == np.float32
        # the expanded form's fp64 rounding is far below fp32's: a few ulps of the
        # norms at most, against brute force
        scale = np.einsum("ij,ij->i", X.astype(np.float64), X.astype(np.float64)) + 1.0
        assert np.all(np.abs(got - brute) <= 1e-6 * scale)
        assert np.mean(got == sk) >= 0.99
        assert np.all(got[rows] <= 1e-6 * scale[rows])  # x = c: zero up to the expanded form's fp64 rounding
    assert np.all(got_b <= got_a)


def test_first_draw_rounds_and_taken_set():
    X = _blobs(2000, 8, 6, 1)
    for k in (1, 2, 7, 50):
        calls = []
        base = oracle.parallel_mindists(X)

        def counted(rows, reset):
            calls.append((list(rows), reset))
            return base(rows, reset)

        C, rows = oracle.kmeans_parallel_init(X, k, np.random.RandomState(5), mindists=counted, trace=True)
        assert rows[0] == np.random.RandomState(5).randint(X.shape[0])     # :77
        assert len(calls) == max(1, int(2 + np.log(k)))                   # :83
        assert calls[0] == ([rows[0]], True) and all(not r for _, r in calls[1:])
        assert 0 not in rows[1:]                                          # taken set starts as {0} (:85)
        assert len(set(rows[1:])) == len(rows) - 1
        assert len(rows) <= 1 + len(calls) * min(k, X.shape[0])
        assert C.shape == (k, X.shape[1]) and C.dtype == np.float32


def test_fewer_candidates_than_k_repeat_cyclically():
    # k > n: the first round draws every row; row 0 is never taken, and the
    # first row is taken again, since the taken set starts as {0}, not {first}
    X = _blobs(6, 2, 2, 3)
    C, rows = oracle.kmeans_parallel_init(X, 8, np.random.RandomState(0), trace=True)
    first = np.random.RandomState(0).randint(6)
    assert first != 0
    assert sorted(rows) == sorted([first] + [1, 2, 3, 4, 5])
    for i in range(8):
        assert np.array_equal(C[i], X[rows[i % len(rows)]])


def test_planted_mistake_in_distances_is_caught():
    # the same loop over distances that keep only the last round's candidates
    # (the reference recomputes against all of them) draws differently
    X = _blobs(3000, 4, 8, 7)
    base = oracle.parallel_mindists(X)

    def last_round_only(rows, reset):
        return base(rows, True)

    a = oracle.kmeans_parallel_init(X, 8, np.random.RandomState(2), trace=True)[1]
    b = oracle.kmeans_parallel_init(X, 8, np.random.RandomState(2), mindists=last_round_only, trace=True)[1]
    assert a != b
