"""Pins the oracle's KMeans.transform (oracle.transform, a restatement of
euclidean_distances for fp32 data, sklearn/metrics/pairwise.py:582-652):

  * scikit-learn 1.7.2's KMeans.transform on 4 small inputs, bit for bit
    (tests/golden/transform.npz, written by make_transform_fixtures.py):
    blobs, 130 features, a 1e4 offset with 1e-3..1e3 column scales
    (cancellation in the expanded form), rows equal to centres;
  * closed forms: 1-feature |x - c|, a 3-4-5 triangle, 0 for x = c;
  * planted mistakes (fp32 arithmetic, the root taken in fp64 before the cast
    to fp32) that the golden distances reject.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cases():
    meta = json.loads((GOLDEN / "transform.json").read_text())
    with np.load(GOLDEN / "transform.npz") as z:
        a = {key: z[key] for key in z.files}
    return [(c["name"], a[c["name"] + "__X"], a[c["name"] + "__C"], a[c["name"] + "__D"]) for c in meta["cases"]]


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_sklearn_transform(case):
    _, X, C, D = case
    np.testing.assert_array_equal(oracle.transform(X, C), D)


def test_closed_forms():
    X = np.array([[0.0, 0.0], [3.0, 4.0], [-1.5, 2.0]], np.float32)
    C = np.array([[0.0, 0.0], [3.0, 4.0]], np.float32)
    D = oracle.transform(X, C)
    np.testing.assert_array_equal(D[:, 0], [0.0, 5.0, 2.5])
    np.testing.assert_array_equal(D[:2, 1], [5.0, 0.0])
    x = np.array([[1.25], [-7.0], [2.0]], np.float32)
    c = np.array([[0.5], [2.0]], np.float32)
    np.testing.assert_array_equal(oracle.transform(x, c), np.abs(x - c.T))


def _fp32_expanded(X, C):
    d = -2.0 * (X @ C.T) + (X * X).sum(1)[:, None] + (C * C).sum(1)[None, :]
    return np.sqrt(np.maximum(d, 0)).astype(np.float32)


def _root_before_cast(X, C):
    X64, C64 = X.astype(np.float64), C.astype(np.float64)
    d = -2.0 * (X64 @ C64.T) + (X64 * X64).sum(1)[:, None] + (C64 * C64).sum(1)[None, :]
    return np.sqrt(np.maximum(d, 0)).astype(np.float32)


@pytest.mark.parametrize("mistake", [_fp32_expanded, _root_before_cast])
def test_planted_mistakes_are_caught(mistake):
    assert any(not np.array_equal(mistake(X, C), D, equal_nan=False) for _, X, C, D in CASES)
