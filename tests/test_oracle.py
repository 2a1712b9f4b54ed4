"""Pins the oracle (CPU restatement of sklearn's Lloyd) before anything is checked against it.

Checks, in the order a plausible mistake would be caught:
  * skmetal's only known-answer vector for the path (tests/test_kernels.py:93-99);
  * sklearn's own hand-computed vectors (sklearn/cluster/tests/test_k_means.py:
    :85-111 relocation toy, :115-153 _relocate_empty_clusters_dense);
  * closed forms: k=1 (mean, total sum of squares), init = distinct rows of X
    (labels = arange, inertia 0), the unit-weight toy;
  * brute force: argmin over explicit direct-form distances; lowest index on ties;
    row permutation <-> label permutation;
  * numpy's float32 column mean, bit for bit;
  * sklearn golden trajectories (tests/golden/*.npz written by make_fixtures.py);
  * two planted mistakes (dropping ||c||^2, '<=' ties) that these checks must reject.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from golden_io import load_golden
from oracle import parity

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_known_answer_assign():
    # tests/test_kernels.py:93-99 of skmetal
    X = np.array([[0.0, 0.0], [1.0, 1.0], [10.0, 10.0], [9.0, 9.0]], np.float32)
    C = np.array([[0.0, 0.0], [10.0, 10.0]], np.float32)
    np.testing.assert_array_equal(oracle.assign(X, C), [0, 0, 1, 1])


def test_mean_f32_bit_exact():
    rng = np.random.default_rng(3)
    for n, d in [(1, 3), (257, 7), (20000, 33)]:
        X = (rng.standard_normal((n, d)) * 7 + 3).astype(np.float32)
        assert np.array_equal(oracle.mean_f32(X), X.mean(axis=0))


def test_assign_brute_force_and_ties():
    rng = np.random.default_rng(4)
    X = rng.standard_normal((3000, 13)).astype(np.float32)
    C = rng.standard_normal((37, 13)).astype(np.float32)
    lab, best, second = oracle.assign(X, C, return_gap=True)
    D = ((X.astype(np.float64)[:, None, :] - C.astype(np.float64)[None]) ** 2).sum(-1)
    ref = D.argmin(1)
    np.testing.assert_array_equal(lab, ref)
    np.testing.assert_allclose(best, D.min(1), rtol=1e-10, atol=1e-9)
    Ds = np.sort(D, axis=1)
    np.testing.assert_allclose(second, Ds[:, 1], rtol=1e-10, atol=1e-9)
    # duplicate centres: the lower index always wins
    C2 = np.concatenate([C[:5], C[:5]])
    lab2 = oracle.assign(X, C2)
    assert lab2.max() < 5


def test_assign_row_permutation():
    rng = np.random.default_rng(5)
    X = rng.standard_normal((1000, 9)).astype(np.float32)
    C = rng.standard_normal((11, 9)).astype(np.float32)
    p = rng.permutation(1000)
    np.testing.assert_array_equal(oracle.assign(X[p], C), oracle.assign(X, C)[p])


def test_k1_closed_form():
    rng = np.random.default_rng(6)
    X = (rng.standard_normal((5000, 6)) * 3 + 1).astype(np.float32)
    out = oracle.lloyd(X, X[:1], max_iter=5)
    Xd = X.astype(np.float64)
    np.testing.assert_allclose(out["centers"][0], Xd.mean(0), rtol=0, atol=2e-6)
    # sklearn (and the oracle) evaluate inertia on fp32-centred X with the
    # centred fp32 centre; on those exact values:
    #   sum ||x-c||^2 = sum ||x-mu||^2 + n ||mu-c||^2
    m32 = X.mean(axis=0)
    Xc = (X - m32).astype(np.float64)
    c = (out["centers"][0] - m32).astype(np.float64)
    mu = Xc.mean(0)
    np.testing.assert_allclose(out["inertia"], ((Xc - mu) ** 2).sum() + len(X) * ((mu - c) ** 2).sum(), rtol=1e-11)
    assert out["n_iter"] == 2  # labels all 0 twice -> strict convergence at iteration 1


def test_init_equal_rows_closed_form():
    rng = np.random.default_rng(7)
    X = rng.standard_normal((40, 5)).astype(np.float32) * 10
    out = oracle.lloyd(X, X, max_iter=3)
    np.testing.assert_array_equal(out["labels"], np.arange(40))
    assert out["inertia"] == pytest.approx(0.0, abs=1e-8)


def test_unit_toy_closed_form():
    X = np.array([[0, 0], [0.5, 0], [0.5, 1], [1, 1]], np.float32)
    out = oracle.lloyd(X, np.array([[0, 0], [1, 1]], np.float32), max_iter=300)
    np.testing.assert_array_equal(out["labels"], [0, 0, 1, 1])
    np.testing.assert_allclose(out["centers"], [[0.25, 0], [0.75, 1]], atol=1e-7)
    assert out["inertia"] == pytest.approx(0.25)
    assert out["n_iter"] == 2


def test_sklearn_relocated_clusters_vector():
    # sklearn/cluster/tests/test_k_means.py:85-111 (unit weights)
    X = np.array([[0, 0], [0.5, 0], [0.5, 1], [1, 1]], np.float32)
    out = oracle.lloyd(X, np.array([[0.5, 0.5], [3, 3]], np.float32), max_iter=300)
    assert out["n_iter"] == 3
    assert out["inertia"] == pytest.approx(0.25)
    ok_a = np.array_equal(out["labels"], [0, 0, 1, 1]) and np.allclose(out["centers"], [[0.25, 0], [0.75, 1]])
    ok_b = np.array_equal(out["labels"], [1, 1, 0, 0]) and np.allclose(out["centers"], [[0.75, 1], [0.25, 0]])
    assert ok_a or ok_b


def test_sklearn_relocate_empty_vector():
    # sklearn/cluster/tests/test_k_means.py:115-153: weights [8,1,1], sums [[-36],[10],[9.5]]
    X = np.array([-10.0, -9.5, -9, -8.5, -8, -1, 1, 9, 9.5, 10], np.float32).reshape(-1, 1)
    C_old = np.full((3, 1), -10.0, np.float32)
    C_new, shift, n_empty = oracle.mstep(X, np.zeros(10, np.int32), C_old)
    assert n_empty == 2
    np.testing.assert_allclose(C_new, [[-36 / 8], [10], [9.5]], rtol=1e-7)
    np.testing.assert_allclose(shift, np.abs(C_new[:, 0] + 10.0), rtol=1e-7)


def test_average_centers_copies_heaviest_row_in_loop_order():
    # more clusters than distinct points: relocation is skipped (max distance 0)
    # and empty clusters copy row argmax(weight) as it stands in the loop
    # (_k_means_common.pyx:274-295): raw sum if it comes later, average if earlier.
    X = np.array([[1.0], [1.0], [1.0], [2.0]], np.float32)
    C_old = np.array([[5.0], [1.0], [2.0]], np.float32)
    labels = np.array([1, 1, 1, 2], np.int32)  # cluster 0 empty, heaviest is 1
    dist0 = oracle.mindists(X, C_old, labels)
    assert dist0.max() == 0.0
    C_new, _, n_empty = oracle.mstep(X, labels, C_old)
    assert n_empty == 1
    np.testing.assert_allclose(C_new, [[3.0], [1.0], [2.0]])  # raw sum 1+1+1 copied
    C_old2 = np.array([[1.0], [2.0], [5.0]], np.float32)
    labels2 = np.array([0, 0, 0, 1], np.int32)  # cluster 2 empty, heaviest 0 already averaged
    C_new2, _, _ = oracle.mstep(X, labels2, C_old2)
    np.testing.assert_allclose(C_new2, [[1.0], [2.0], [1.0]])


def test_c_and_numpy_restatements_agree():
    rng = np.random.default_rng(8)
    for n, d, k in [(600, 5, 4), (1200, 17, 25), (400, 3, 40)]:
        cen = rng.uniform(-8, 8, (6, d))
        X = (cen[rng.integers(0, 6, n)] + rng.standard_normal((n, d))).astype(np.float32)
        C0 = X[rng.choice(n, k, replace=False)]
        a = oracle.lloyd(X, C0, 40)
        b = oracle.numpy_lloyd(X, C0, 40)
        assert a["n_iter"] == b["n_iter"]
        np.testing.assert_array_equal(a["labels"], b["labels"])
        np.testing.assert_allclose(a["centers"], b["centers"], rtol=0, atol=1e-6)
        assert a["inertia"] == pytest.approx(b["inertia"], rel=1e-12)


def _golden_cases():
    manifest = json.loads((GOLDEN / "manifest.json").read_text())
    return [c["name"] for c in manifest["cases"]]


@pytest.mark.parametrize("name", _golden_cases())
def test_oracle_matches_sklearn_golden(name):
    """Oracle vs sklearn's recorded outputs.

    sklearn's labels are only reproducible up to near-tie rows (its BLAS
    rounding varies from run to run), so its recorded trajectory (one run,
    stepped with its own lloyd_iter_chunked_dense) is checked in lockstep:
    from sklearn's centres after m-1 steps, the oracle's E-step must give
    sklearn's labels up to near-ties and the oracle's M-step on sklearn's
    labels must give sklearn's centres.  The oracle's own full run must match
    sklearn's fit end to end whenever the trajectory met no label mismatch.
    """
    g = load_golden(name)
    X, C0 = g["X"], g["C0"]
    mean = X.mean(axis=0)
    Xc = X - mean
    prev = C0
    n_mism = 0
    for m in range(len(g["trace"])):
        n_mism += parity.check_lockstep(Xc, prev - mean, g["trace"][m] - mean,
                                        g["trace_labels"][m].astype(np.int32),
                                        what=f"{name} iteration {m + 1}")
        prev = g["trace"][m]
    # sklearn's final labels are the E-step of its final centres
    _, best, second = oracle.assign(Xc, g["centers"] - mean, return_gap=True)
    parity.check_labels(g["labels"], oracle.assign(Xc, g["centers"] - mean), best, second, Xc,
                        what=f"{name} final labels")
    # sklearn's fp32 inertia_ vs an fp64 recomputation from its labels/centres
    ref_inertia = oracle.inertia(Xc, g["centers"] - mean, g["labels"])
    scale = float((Xc.astype(np.float64) ** 2).sum())
    assert abs(float(g["inertia"]) - ref_inertia) <= 1e-4 * ref_inertia + 1e-7 * scale

    tol_abs = oracle.sklearn_tolerance(X, float(g["tol"])) if "tol" in g else 0.0
    out = oracle.lloyd(X, C0, int(g["max_iter"]), tol_abs)
    if n_mism == 0:
        assert out["n_iter"] == int(g["n_iter"])
        parity.check_centers(out["centers"], g["centers"], what=f"{name} centers")
        _, best, second = oracle.assign(Xc, out["centers"] - mean, return_gap=True)
        parity.check_labels(g["labels"], out["labels"], best, second, Xc, what=f"{name} labels")
        assert abs(out["inertia"] - ref_inertia) <= parity.INERTIA_RTOL * ref_inertia + 1e-9 * scale


def _assign_without_cnorm(X, C):
    X = X.astype(np.float64)
    C = C.astype(np.float64)
    return np.argmin(-2.0 * X @ C.T, axis=1)


def _assign_last_tie(X, C):
    X = X.astype(np.float64)
    C = C.astype(np.float64)
    D = (C * C).sum(1)[None] - 2.0 * X @ C.T
    return D.shape[1] - 1 - np.argmin(D[:, ::-1], axis=1)


def test_planted_mistakes_are_caught():
    X = np.array([[0.0, 0.0], [1.0, 1.0], [10.0, 10.0], [9.0, 9.0]], np.float32)
    C = np.array([[0.0, 0.0], [10.0, 10.0]], np.float32)
    assert not np.array_equal(_assign_without_cnorm(X, C), [0, 0, 1, 1])
    rng = np.random.default_rng(9)
    Xr = rng.standard_normal((500, 4)).astype(np.float32)
    Cr = rng.standard_normal((6, 4)).astype(np.float32)
    Cdup = np.concatenate([Cr, Cr])
    assert _assign_last_tie(Xr, Cdup).min() >= 6  # would fail the duplicate-centre check
    assert oracle.assign(Xr, Cdup).max() < 6


@pytest.mark.parametrize("tol,n_iter", [(0.3, 1), (0.25001, 1), (0.25, 2), (0.1, 2), (0.0, 5), (-1.0, 5)])
def test_reference_loop_stopping_rule(tol, n_iter):
    """skmetal's batch_fused stop (KMeansBridge.swift:306-310) on the unit toy:
    step 1 moves both centres by exactly 0.25, step 2 by 0, so the loop stops
    after step 1 when 0.25 < tol, after step 2 when 0 < tol <= 0.25, and never
    early for tol <= 0."""
    X = np.array([[0, 0], [0.5, 0], [0.5, 1], [1, 1]], np.float32)
    C0 = np.array([[0, 0], [1, 1]], np.float32)
    out = oracle.reference_loop(X, C0, 5, tol)
    assert out["n_iter"] == n_iter
    np.testing.assert_array_equal(out["labels"], [0, 0, 1, 1])
    np.testing.assert_allclose(out["centers"], [[0.25, 0], [0.75, 1]], atol=1e-7)


def test_reference_loop_zero_iterations_and_last_estep_labels():
    X = np.array([[0, 0], [0.5, 0], [0.5, 1], [1, 1]], np.float32)
    out = oracle.reference_loop(X, np.array([[0, 0], [1, 1]], np.float32), 0, 1.0)
    assert out["n_iter"] == 0 and out["labels"] is None
    # labels are the last step's E-step, against the centres that step started from:
    # one step from centres where row 1 sits on centre 0's side, which the update then moves
    X2 = np.array([[0.0], [1.0], [2.0], [10.0]], np.float32)
    C2 = np.array([[1.4], [10.0]], np.float32)
    one = oracle.reference_loop(X2, C2, 1, 0.0)
    np.testing.assert_array_equal(one["labels"], [0, 0, 0, 1])
    np.testing.assert_allclose(one["centers"], [[1.0], [10.0]], atol=1e-6)
