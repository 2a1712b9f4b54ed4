"""GPU parity: libskmetal_hip.so (through its C ABI) against the oracle.

Every test here runs the HIP kernels on an MI355X and checks them with the
rules of oracle/parity.py:
  labels  -- equal except near-ties (gap < 1e-5 ||x||^2),
  centres -- row-relative error <= 1e-4,
  inertia -- relative error <= 1e-5 against an fp64 recomputation.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle import parity
from problems import mixed_scale_problem

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


def test_native_library_is_the_in_tree_build(bridge):
    path = Path(bridge.library_path())
    assert path.name == "libskmetal_hip.so"
    assert path.parent == Path(bridge.__file__).resolve().parent
    info = bridge.device_info()
    assert info["has_unified_memory"] is False
    assert info["recommended_working_set_size_bytes"] > 100 * 2**30


def test_known_answer_assign(bridge):
    # skmetal tests/test_kernels.py:93-99
    X = np.array([[0.0, 0.0], [1.0, 1.0], [10.0, 10.0], [9.0, 9.0]], dtype=np.float32)
    centroids = np.array([[0.0, 0.0], [10.0, 10.0]], dtype=np.float32)
    assignments = np.empty(4, dtype=np.int32)
    bridge.kmeans_assign(X, centroids, assignments, 4, 2, 2)
    np.testing.assert_array_equal(assignments, [0, 0, 1, 1])


ASSIGN_SHAPES = [
    (1, 1, 1), (2, 3, 2), (63, 7, 5), (64, 4, 4), (65, 33, 9), (257, 2, 64), (1000, 32, 8),
    (3001, 100, 50), (2048, 16, 65), (999, 20, 200), (4096, 129, 17), (1500, 300, 70),
    (700, 5, 1024), (513, 768, 96), (3000, 257, 530), (1000, 1000, 300),
]


@pytest.mark.parametrize("n,d,k", ASSIGN_SHAPES)
def test_assign_vs_oracle(bridge, n, d, k):
    _say(f"assign n={n} d={d} k={k}")
    rng = np.random.default_rng(n * 131 + d * 7 + k)
    X = (rng.standard_normal((n, d)) * 3).astype(np.float32)
    C = (rng.standard_normal((k, d)) * 3).astype(np.float32)
    out = np.full(n, -7, dtype=np.int32)
    bridge.kmeans_assign(X, C, out, n, d, k)
    ref, best, second = oracle.assign(X, C, return_gap=True)
    assert out.min() >= 0 and out.max() < k
    parity.check_labels(out, ref, best, second, X, what=f"assign {n}x{d} k={k}")


def test_assign_one_hot_layout(bridge):
    """Each row equals one centre exactly: checks the MFMA lane/register layout."""
    k, d = 64, 64
    C = np.eye(k, d, dtype=np.float32) * 10
    rng = np.random.default_rng(0)
    truth = rng.integers(0, k, 4096).astype(np.int32)
    X = C[truth].copy()
    out = np.empty(4096, np.int32)
    bridge.kmeans_assign(X, C, out, 4096, d, k)
    np.testing.assert_array_equal(out, truth)


def test_assign_duplicate_centres_lowest_index(bridge):
    rng = np.random.default_rng(1)
    X = rng.standard_normal((3000, 12)).astype(np.float32)
    base = rng.standard_normal((7, 12)).astype(np.float32)
    C = np.concatenate([base, base, base])
    out = np.empty(3000, np.int32)
    bridge.kmeans_assign(X, C, out, 3000, 12, 21)
    ref = oracle.assign(X, C)
    np.testing.assert_array_equal(out, ref)
    assert out.max() < 7


@pytest.mark.parametrize("d", [3, 37, 100, 128, 161])
def test_mindists_and_inertia_vs_oracle(bridge, d):
    """Per-row distances and their total; d covers each row-distance path
    (contiguous chunks for row strides of at most 32, 64, 104 and 128 floats,
    column slabs above)."""
    rng = np.random.default_rng(2 + d)
    n, k = 5000, 13
    X = (rng.standard_normal((n, d)) * 2).astype(np.float32)
    C = rng.standard_normal((k, d)).astype(np.float32)
    lab = rng.integers(0, k, n).astype(np.int32)
    dists = np.empty(n, np.float32)
    bridge.compute_mindists(X, C, lab, dists, n, d, k)
    ref = oracle.mindists(X, C, lab)
    np.testing.assert_allclose(dists, ref, rtol=2e-6, atol=1e-5)
    v = bridge.kmeans_inertia(X, C, lab, n, d, k)
    parity.check_inertia(v, oracle.inertia(X, C, lab), what="kmeans_inertia")


@pytest.mark.parametrize("n,d,k", [(20000, 100, 50), (9000, 33, 7), (12000, 128, 200), (6000, 200, 33)])
def test_fit_inertia_from_final_estep(bridge, n, d, k):
    """The fit's inertia comes from its final E-step (k_assign3 adds each
    row's direct-form distance to its new centre); it equals the separate
    row-distance pass over the same labels and centres up to the fp64
    summation order, and the oracle's inertia of those labels and centres."""
    rng = np.random.default_rng(11 + d)
    X = (rng.standard_normal((n, d)) * 2 + rng.integers(-3, 4, (n, 1))).astype(np.float32)
    C0 = X[rng.choice(n, k, replace=False)].copy()
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=False)
        h.set_centers(C0)
        n_iter, inertia = h.run(4, 0.0, strict=True)
        ref = h.inertia()
        C, lab = h.centers(), h.labels()
    _say(f"fit inertia n={n} d={d} k={k}: {inertia!r} row-distance pass {ref!r}")
    assert inertia == pytest.approx(ref, rel=1e-12)
    parity.check_inertia(inertia, oracle.inertia(X, C, lab), what="fit inertia")


def test_fit_inertia_full_size_headline_workload(bridge):
    """The 500,000 x 100, k = 50 workload: a 10-step sklearn-rule fit from the
    seeded init ends on a step that changed labels, so its inertia comes from
    the final E-step; it matches the row-distance pass over the same labels
    and centres (the profile of the fit's end runs this test)."""
    from skmetal_amd import _synth

    X, C0 = _synth.generate("c2", seed=0)
    with bridge.LloydHandle(*X.shape, C0.shape[0]) as h:
        h.load(X, center=True)
        for rep in range(2):
            h.set_centers(C0)
            n_iter, inertia = h.run(10, 0.0, strict=True)
            ref = h.inertia()
            _say(f"c2 fit {rep}: n_iter={n_iter} inertia={inertia!r} row-distance pass {ref!r}")
            assert n_iter == 10
            assert inertia == pytest.approx(ref, rel=1e-12)


def _lockstep_gpu(bridge, X, C0, steps, what, center=True, elem_rtol=None):
    """Run `steps` single GPU steps from C0, checking each against the oracle
    (in the coordinates the device runs in: X centred on its fp32 column mean,
    as scikit-learn's fit does, or X as given)."""
    n, d = X.shape
    k = C0.shape[0]
    mean = X.mean(axis=0) if center else np.zeros(d, np.float32)
    Xc = X - mean
    prev = C0
    n_mism = 0
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=center)
        for m in range(steps):
            h.set_centers(prev)
            h.iterate(1)
            lab = h.labels()
            Cn = h.centers()
            n_mism += parity.check_lockstep(Xc, prev - mean, Cn - mean, lab, what=f"{what} step {m + 1}",
                                            elem_rtol=elem_rtol)
            prev = Cn
    return n_mism


# (n, d, k) covering every row stride of the split kernel (with and without a
# 16-wide K tail, pad columns; d = 100 has an LDS row shorter than its MFMA
# span) and 1..4 blocks of 16 centres
SPLIT_SHAPES = [(3000, 17, 5), (4100, 33, 16), (5000, 64, 17), (6000, 80, 48), (20000, 97, 50), (7000, 100, 64)]


def _blob_problem(n, d, k, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-6, 6, (k, d))
    X = ((cen[rng.integers(0, k, n)] + rng.standard_normal((n, d))) * scale).astype(np.float32)
    C0 = X[np.sort(rng.choice(n, k, replace=False))].copy()
    return X, C0


def _split_engaged(bridge, X, C0):
    n, d = X.shape
    with bridge.LloydHandle(n, d, C0.shape[0]) as h:
        h.load(X, center=True)
        h.set_centers(C0)
        return h.info()


@pytest.mark.parametrize("n,d,k", SPLIT_SHAPES)
def test_split_estep_lockstep(bridge, n, d, k):
    """Fused steps with the E-step and sums on bf16 MFMAs over the exact
    three-part split, against the oracle step by step."""
    _say(f"split lockstep n={n} d={d} k={k}")
    X, C0 = _blob_problem(n, d, k, seed=n + d + k)
    info = _split_engaged(bridge, X, C0)
    assert info["fused"] and info["split"], info
    _lockstep_gpu(bridge, X, C0, 3, what=f"split {n}x{d} k={k}")


@pytest.mark.parametrize("n,k", [(1, 1), (5, 3), (31, 4), (33, 7), (100, 20), (257, 64)])
def test_split_tiny_problems(bridge, n, k):
    """Partial 32-row tiles and waves with no tile at all (most of the grid)."""
    _say(f"split tiny n={n} k={k}")
    rng = np.random.default_rng(n * 7 + k)
    X = (rng.standard_normal((n, 40)) * 3).astype(np.float32)
    C0 = X[np.sort(rng.choice(n, k, replace=False))].copy()
    info = _split_engaged(bridge, X, C0)
    assert info["fused"] and info["split"], info
    _lockstep_gpu(bridge, X, C0, 2, what=f"split tiny {n} k={k}")
    C = C0.copy()
    lab = np.empty(n, np.int32)
    n_iter, _ = bridge.kmeans_fit(X, C, lab, 50, 0.0, strict=True)
    out = oracle.lloyd(X, C0, 50)
    assert n_iter == out["n_iter"]
    parity.check_centers(C, out["centers"], what=f"tiny fit n={n} k={k}")


def test_split_assign_duplicate_centres_lowest_index(bridge):
    """Identical centres give identical split distances: the lowest index wins."""
    rng = np.random.default_rng(11)
    X = rng.standard_normal((3000, 40)).astype(np.float32)
    base = rng.standard_normal((7, 40)).astype(np.float32)
    C = np.concatenate([base, base, base])
    out = np.empty(3000, np.int32)
    bridge.kmeans_assign(X, C, out, 3000, 40, 21)
    ref, best, second = oracle.assign(X, C, return_gap=True)
    assert out.max() < 7
    parity.check_labels(out, ref, best, second, X, what="split duplicate centres")


@pytest.mark.parametrize("d,reps,extra", [(100, 3, 0), (40, 2, 0), (64, 4, 0), (100, 1, 2), (64, 2, 3), (40, 3, 4)])
def test_split_fused_duplicate_centres_lowest_index(bridge, d, reps, extra):
    """Every row is an exact tie between copies of its centre: the lowest
    index must win, exactly as scikit-learn's strict '<' scan picks it.  With
    extra > 0 the last 16-centre block holds at most four centres (the stacked
    block, whose distances take all nine part products) and they are copies
    of earlier ones."""
    rng = np.random.default_rng(d + reps + 10 * extra)
    n = 9000
    base = rng.uniform(-5, 5, (16, d)).astype(np.float32)
    X = (base[rng.integers(0, 16, n)] + rng.standard_normal((n, d))).astype(np.float32)
    C = np.concatenate([base] * reps + [base[:extra]])[:64]
    k = C.shape[0]
    mean = X.mean(axis=0)
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=True)
        h.set_centers(C)
        assert h.info()["split"]
        h.iterate(1)
        lab = h.labels()
    ref = oracle.assign(X - mean, C - mean)
    np.testing.assert_array_equal(lab, ref)
    assert lab.max() < 16


@pytest.mark.parametrize("n,d,k", [(3000, 101, 10), (40, 20, 40), (2000, 17, 64)])
def test_split_edge_shapes_lockstep(bridge, n, d, k):
    """d just past the fused limit (generic path with k <= 64), k = n, the
    smallest split row stride with 64 centres."""
    _say(f"split edge n={n} d={d} k={k}")
    X, C0 = _blob_problem(n, d, k, seed=3 * n + d)
    info = _split_engaged(bridge, X, C0)
    assert info["split"] or info["asplit"], info
    _lockstep_gpu(bridge, X, C0, 2, what=f"split edge {n}x{d} k={k}")


@pytest.mark.parametrize("scale", [1e-15, 1e-3, 1e4, 1e15])
def test_split_estep_scaled_data(bridge, scale):
    """The bf16 parts share fp32's exponent range: no scaling for any data
    magnitude within the split's range."""
    _say(f"split scale {scale}")
    X, C0 = _blob_problem(6000, 40, 30, seed=5, scale=scale)
    assert _split_engaged(bridge, X, C0)["split"]
    _lockstep_gpu(bridge, X, C0, 2, what=f"split scale {scale}")


@pytest.mark.parametrize("kind", ["quantised", "1e6", "cluster"])
@pytest.mark.parametrize("n,d,k", [(20000, 100, 50), (6000, 40, 13), (8000, 48, 150)])
def test_split_mixed_scale_columns(bridge, n, d, k, kind):
    """Per-element fp32 accuracy of the split path: columns (or clusters) whose
    values are 10^5..10^8 times smaller than the rest keep their own relative
    accuracy -- every lockstep step checks centres per row, per column and per
    element at the scale of the cluster's own values, the last at the fp32
    level (FP32_ELEM_RTOL)."""
    _say(f"split mixed scale {kind} n={n} d={d} k={k}")
    X, C0 = mixed_scale_problem(n, d, k, seed=n + d + k, kind=kind)
    info = _split_engaged(bridge, X, C0)
    assert info["split"] or info["asplit"], info
    # "cluster" runs on X as given: centring would move the small clusters'
    # values to the scale of the column mean
    _lockstep_gpu(bridge, X, C0, 3, what=f"mixed scale {kind} {n}x{d} k={k}", center=kind != "cluster",
                  elem_rtol=parity.FP32_ELEM_RTOL)


@pytest.mark.parametrize("kind", ["quantised", "cluster"])
def test_split_mixed_scale_assign(bridge, kind):
    """The separate E-step (assign entry point) on mixed-scale columns."""
    X, C0 = mixed_scale_problem(5000, 100, 200, seed=21, kind=kind)
    out = np.empty(len(X), np.int32)
    bridge.kmeans_assign(X, C0, out, X.shape[0], X.shape[1], C0.shape[0])
    ref, best, second = oracle.assign(X, C0, return_gap=True)
    parity.check_labels(out, ref, best, second, X, what=f"mixed scale assign {kind}")


def test_split_switched_off_by_env(bridge, monkeypatch):
    """SKMETAL_HIP_SPLIT=0 keeps the fp32 MFMA E-step; both agree with the oracle."""
    monkeypatch.setenv("SKMETAL_HIP_SPLIT", "0")
    X, C0 = _blob_problem(8000, 100, 50, seed=9)
    info = _split_engaged(bridge, X, C0)
    assert info["fused"] and not info["split"], info
    _lockstep_gpu(bridge, X, C0, 2, what="fp32 E-step")


@pytest.mark.parametrize("n,d,k", [(5000, 40, 100), (3000, 130, 300)])
def test_asplit_generic_path_lockstep(bridge, n, d, k):
    """k > 64: the separate E-step over the split (several centre passes and
    feature segments) with the sorted update, step by step against the oracle."""
    _say(f"asplit lockstep n={n} d={d} k={k}")
    X, C0 = _blob_problem(n, d, k, seed=n + k)
    info = _split_engaged(bridge, X, C0)
    assert not info["fused"] and info["asplit"], info
    _lockstep_gpu(bridge, X, C0, 2, what=f"asplit {n}x{d} k={k}")


def test_split_off_for_non_finite_data(bridge):
    X, C0 = _blob_problem(3000, 40, 8, seed=3)
    X[17, 5] = np.inf
    with bridge.LloydHandle(3000, 40, 8) as h:
        h.load(X, center=False)
        h.set_centers(C0)
        assert not h.info()["split"] and not h.info()["asplit"]


def test_split_off_below_its_range(bridge):
    """Data whose largest magnitude is below 2^-50 keeps the fp32 E-step."""
    X, C0 = _blob_problem(3000, 40, 8, seed=4, scale=1e-17)
    with bridge.LloydHandle(3000, 40, 8) as h:
        h.load(X, center=False)
        h.set_centers(C0)
        assert h.info()["fused"] and not h.info()["split"]
    _lockstep_gpu(bridge, X, C0, 2, what="fp32 E-step for 1e-17 data")


def _golden_names():
    return [c["name"] for c in json.loads((GOLDEN / "manifest.json").read_text())["cases"]]


def _load_golden(name):
    from golden_io import load_golden

    return load_golden(name)


@pytest.mark.parametrize("name", _golden_names())
def test_lockstep_golden(bridge, name):
    g = _load_golden(name)
    _say(f"lockstep golden {name} {g['X'].shape}")
    _lockstep_gpu(bridge, g["X"], g["C0"], min(len(g["trace"]), 6), name)


@pytest.mark.parametrize("name", _golden_names())
def test_fit_vs_sklearn_golden(bridge, name):
    """Full GPU fit vs sklearn's recorded fit and the oracle."""
    g = _load_golden(name)
    X, C0 = g["X"], g["C0"]
    _say(f"fit golden {name} {X.shape} k={C0.shape[0]}")
    n, d = X.shape
    k = C0.shape[0]
    tol_abs = oracle.sklearn_tolerance(X, float(g["tol"])) if "tol" in g else 0.0
    C = C0.copy()
    lab = np.empty(n, np.int32)
    n_iter, inertia = bridge.kmeans_fit(X, C, lab, int(g["max_iter"]), tol_abs, strict=True)
    mean = X.mean(axis=0)
    Xc = X - mean
    # final labels are the E-step of the final centres
    ref_lab, best, second = oracle.assign(Xc, C - mean, return_gap=True)
    parity.check_labels(lab, ref_lab, best, second, Xc, what=f"{name} final E-step")
    parity.check_inertia(inertia, oracle.inertia(Xc, C - mean, lab), atol=parity.centring_floor(X),
                         what=f"{name} inertia")
    # end to end against sklearn whenever the oracle's own trajectory matches sklearn's
    out = oracle.lloyd(X, C0, int(g["max_iter"]), tol_abs)
    if out["n_iter"] == int(g["n_iter"]) and parity.center_rel_err(out["centers"], g["centers"]) <= 1e-5:
        assert n_iter == int(g["n_iter"]), f"{name}: n_iter {n_iter} vs sklearn {int(g['n_iter'])}"
        parity.check_centers(C, g["centers"], what=f"{name} centres vs sklearn")
        _, best, second = oracle.assign(Xc, g["centers"] - mean, return_gap=True)
        parity.check_labels(lab, g["labels"], best, second, Xc, what=f"{name} labels vs sklearn")


def test_fit_is_deterministic(bridge):
    from skmetal_amd import _synth

    X, C0 = _synth.generate("c2", seed=3, scale=0.05)
    outs = []
    for _ in range(2):
        C = C0.copy()
        lab = np.empty(X.shape[0], np.int32)
        n_iter, inertia = bridge.kmeans_fit(X, C, lab, 15, 0.0, strict=False)
        outs.append((C, lab, n_iter, inertia))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
    assert outs[0][2:] == outs[1][2:]


def test_fit_is_deterministic_generic_path(bridge):
    """k > 64: assign + sorted update + record finalize, bitwise equal across runs."""
    rng = np.random.default_rng(21)
    cen = rng.uniform(-5, 5, (150, 40))
    X = (cen[rng.integers(0, 150, 60000)] + rng.standard_normal((60000, 40))).astype(np.float32)
    C0 = X[np.sort(rng.choice(60000, 120, replace=False))]
    outs = []
    for _ in range(2):
        C = C0.copy()
        lab = np.empty(X.shape[0], np.int32)
        n_iter, inertia = bridge.kmeans_fit(X, C, lab, 12, 0.0, strict=False)
        outs.append((C, lab, n_iter, inertia))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
    assert outs[0][2:] == outs[1][2:]


def test_empty_cluster_relocation_matches_oracle(bridge):
    g = _load_golden("empty_1000x10_k20")
    X, C0 = g["X"], g["C0"]
    C = C0.copy()
    lab = np.empty(X.shape[0], np.int32)
    n_iter, inertia = bridge.kmeans_fit(X, C, lab, 300, 0.0, strict=True)
    assert np.all(np.isfinite(C))
    assert len(np.unique(lab)) == 20
    out = oracle.lloyd(X, C0, 300)
    assert n_iter == out["n_iter"]
    parity.check_centers(C, out["centers"], what="relocation fit")


# the relocation paths: k_reloc after every step (default), the loop's halt
# with the device kernels started by the host, and the host relocation
_RELOC_PATHS = {
    "in-stream": {},
    "halt+device": {"SKMETAL_HIP_INLINE_RELOCATE": "0"},
    "host": {"SKMETAL_HIP_HOST_RELOCATE": "1"},
}


def _fit_each_relocation_path(bridge, monkeypatch, X, C0, max_iter):
    res = {}
    for where, env in _RELOC_PATHS.items():
        for var in ("SKMETAL_HIP_INLINE_RELOCATE", "SKMETAL_HIP_HOST_RELOCATE"):
            monkeypatch.delenv(var, raising=False)
        for var, val in env.items():
            monkeypatch.setenv(var, val)
        C = C0.copy()
        lab = np.empty(X.shape[0], np.int32)
        res[where] = bridge.kmeans_fit(X, C, lab, max_iter, 0.0, strict=True) + (C,)
    for var in ("SKMETAL_HIP_INLINE_RELOCATE", "SKMETAL_HIP_HOST_RELOCATE"):
        monkeypatch.delenv(var, raising=False)
    return res


@pytest.mark.parametrize("n_dup", [1, 4, 9])
@pytest.mark.parametrize("k_base", [12, 72])
def test_relocation_of_several_empty_clusters(bridge, n_dup, k_base, monkeypatch):
    """Duplicated initial centres leave n_dup clusters empty after the first
    E-step (lowest index wins ties); every relocation path must follow the
    oracle's (sklearn's) rule and agree with the others.  k_base = 12 runs
    the fused step to convergence; 72 runs the assign + update step for the
    first 3 steps (the relocation is in the first; with up to 81 centres on 6
    blobs later steps meet near ties that fp32 rounding may settle either
    way)."""
    rng = np.random.default_rng(40 + n_dup + k_base)
    cen = rng.uniform(-8, 8, (6, 8))
    X = (cen[rng.integers(0, 6, 6000)] + rng.standard_normal((6000, 8))).astype(np.float32)
    base = X[np.sort(rng.choice(6000, k_base, replace=False))]
    C0 = np.concatenate([base, base[:n_dup]])  # the copies come later: they get no rows
    max_iter = 60 if k_base == 12 else 3
    out = oracle.lloyd(X, C0, max_iter)
    res = _fit_each_relocation_path(bridge, monkeypatch, X, C0, max_iter)
    for where, (n_iter, inertia, C) in res.items():
        assert n_iter == out["n_iter"], f"{where}: n_iter {n_iter} vs oracle {out['n_iter']}"
        parity.check_centers(C, out["centers"], what=f"{where} relocation n_dup={n_dup} k={len(C0)}")
    for where in ("halt+device", "host"):
        parity.check_centers(res["in-stream"][2], res[where][2], rtol=1e-5,
                             what=f"in-stream vs {where} relocation")


@pytest.mark.parametrize("d", [100, 200])
def test_relocation_wide_rows(bridge, d, monkeypatch):
    """Four empty clusters relocated on rows of 100 and 200 features (the
    contiguous and the column-slab row-distance paths of the relocation):
    the step that relocates against the oracle, then three steps across the
    relocation paths (16 centres on 6 blobs meet near ties in later steps
    that the oracle's fp64 distances may settle otherwise)."""
    rng = np.random.default_rng(70 + d)
    cen = rng.uniform(-8, 8, (6, d))
    X = (cen[rng.integers(0, 6, 6000)] + rng.standard_normal((6000, d))).astype(np.float32)
    base = X[np.sort(rng.choice(6000, 12, replace=False))]
    C0 = np.concatenate([base, base[:4]])
    out = oracle.lloyd(X, C0, 1)
    res = _fit_each_relocation_path(bridge, monkeypatch, X, C0, 1)
    for where, (n_iter, inertia, C) in res.items():
        assert n_iter == out["n_iter"], f"{where}: n_iter {n_iter} vs oracle {out['n_iter']}"
        parity.check_centers(C, out["centers"], what=f"{where} relocation d={d}")
    res = _fit_each_relocation_path(bridge, monkeypatch, X, C0, 3)
    for where in ("halt+device", "host"):
        assert res["in-stream"][0] == res[where][0]
        parity.check_centers(res["in-stream"][2], res[where][2], rtol=1e-5,
                             what=f"in-stream vs {where} relocation d={d}, 3 steps")


@pytest.mark.parametrize("n,tied,step,kb", [(20000, 5, 1e-2, 16), (150000, 600, 4e-3, 16), (20000, 5, 1e-2, 80),
                                          (300000, 600, 4e-3, 80)])
def test_relocation_candidates_near_the_top(bridge, n, tied, step, kb):
    """On the split paths (kb = 16: the fused step; kb = 80: the separate
    E-step and the sorted update) the relocated rows are searched among the
    E-step's approximate distances (||x||^2 + the row's minimum of ||c||^2 -
    2 x.c), with direct-form distances only for the rows within a margin of
    each block's top.  A group of far rows whose distances differ by far less
    than that margin (one coordinate stepped by `step`) must still move in the
    oracle's order.  With 600 of them in consecutive rows, a block holds more
    candidates than its list and falls back to every row's direct form."""
    rng = np.random.default_rng(n + kb)
    d, E = 64, 3
    cen = rng.uniform(-6, 6, (8, d))
    X = (cen[rng.integers(0, 8, n)] + rng.standard_normal((n, d))).astype(np.float32)
    rows = np.arange(1000, 1000 + tied) if tied > 256 else np.sort(rng.choice(n, tied, replace=False))
    far = np.repeat((cen[0] + 40.0)[None, :], tied, axis=0)
    far[:, 0] += step * rng.permutation(tied)  # distinct distances, in no row order
    X[rows] = far.astype(np.float32)
    others = np.setdiff1d(np.arange(n), rows)
    base = X[np.sort(rng.choice(others, kb, replace=False))]
    C0 = np.concatenate([base, base[:E]])  # the copies come later: E empty clusters
    info = _split_engaged(bridge, X, C0)
    assert info["split"] if kb <= 64 else (info["asplit"] and not info["fused"]), info
    _say(f"relocation near the top n={n} far rows={tied} k={kb + E}")
    # one step against the oracle: labels up to near-ties (80 centres on 8
    # blobs meet some), the oracle's M-step and relocation on the device's
    # labels against the device's centres
    mean = X.mean(axis=0)
    with bridge.LloydHandle(n, d, kb + E) as h:
        h.load(X, center=True)
        h.set_centers(C0)
        h.iterate(1)
        lab, Cn = h.labels(), h.centers()
    parity.check_lockstep(X - mean, C0 - mean, Cn - mean, lab, what=f"relocation near the top n={n} k={kb + E}")
    # the relocated centres are the rows the oracle moves: the stepped
    # coordinate tells them apart
    ref, _, n_empty = oracle.mstep(X - mean, lab, C0 - mean)
    assert n_empty == E
    np.testing.assert_allclose((Cn - mean)[kb:kb + E, 0], ref[kb:kb + E, 0], rtol=0, atol=step / 8)


@pytest.mark.parametrize("wl,steps", [("c1", 4), ("c2", 3)])
def test_workload_lockstep_full_size(bridge, wl, steps):
    from skmetal_amd import _synth

    X, C0 = _synth.generate(wl, seed=0)
    _say(f"lockstep {wl} {X.shape} k={C0.shape[0]}")
    _lockstep_gpu(bridge, X, C0, steps, wl)


def test_c2_fixed_iterations_inertia_monotone(bridge):
    from skmetal_amd import _synth

    X, C0 = _synth.generate("c2", seed=0)
    n, d = X.shape
    prev = np.inf
    with bridge.LloydHandle(n, d, C0.shape[0]) as h:
        h.load(X, center=True)
        h.set_centers(C0)
        for _ in range(6):
            h.iterate(1)
            v = h.inertia()  # labels of this E-step against the centres of its M-step
            assert v <= prev * (1 + 1e-6)
            prev = v


@pytest.mark.parametrize("n,d,k,blobs", [(3000, 1, 5, 4), (5000, 2000, 30, 12), (20000, 64, 300, 90),
                                         (8000, 129, 130, 60), (50000, 32, 8, 8)])
def test_lockstep_update_geometries(bridge, n, d, k, blobs):
    """Column tiles (d > 1024), several cluster groups, d = 1, many row ranges."""
    _say(f"lockstep geometry n={n} d={d} k={k}")
    rng = np.random.default_rng(n + d + k)
    cen = rng.uniform(-5, 5, (blobs, d))
    X = (cen[rng.integers(0, blobs, n)] + rng.standard_normal((n, d))).astype(np.float32)
    C0 = X[np.sort(rng.choice(n, k, replace=False))]
    _lockstep_gpu(bridge, X, C0, 3, f"geometry {n}x{d} k={k}")


def test_step_mode_selection(bridge):
    """k <= 64 and padded d <= 128 take the fused E-step + sums kernel; others the generic path."""
    with bridge.LloydHandle(500_000, 100, 50) as h:
        assert h.info()["fused"] is True
    with bridge.LloydHandle(10_000, 16, 100) as h:
        assert h.info()["fused"] is False
    with bridge.LloydHandle(10_000, 200, 8) as h:
        assert h.info()["fused"] is False


def _sampled_steps(bridge, X, C0, steps, sample, seed, what):
    """Full-size GPU steps from C0.  Labels are checked against the oracle's
    E-step on a row sample (the full n x k oracle E-step would take minutes);
    centres are checked in full: the oracle's M-step (sums, relocation,
    averaging) applied to the GPU's labels must reproduce the GPU's centres."""
    import time

    t0 = time.perf_counter()
    n, d = X.shape
    k = C0.shape[0]
    mean = X.mean(axis=0)
    Xc = X - mean
    idx = np.sort(np.random.default_rng(seed).choice(n, size=min(sample, n), replace=False))
    prev = C0
    with bridge.LloydHandle(n, d, k) as h:
        h.load(X, center=True)
        for m in range(steps):
            _say(f"{what} step {m + 1} ({time.perf_counter() - t0:.1f} s)")
            h.set_centers(prev)
            h.iterate(1)
            lab = h.labels()
            Cn = h.centers()
            assert lab.min() >= 0 and lab.max() < k
            ref, best, second = oracle.assign(Xc[idx], prev - mean, return_gap=True)
            parity.check_labels(lab[idx], ref, best, second, Xc[idx], what=f"{what} step {m + 1} sampled labels")
            C_ref, _, n_empty = oracle.mstep(Xc, lab, prev - mean)
            C_got = (Cn - mean).astype(np.float64)
            err = parity.center_rel_err(C_ref, C_got)
            if err > parity.CENTER_RTOL and n_empty >= 3:
                counts = np.bincount(lab, minlength=k)
                C_got = parity._match_relocated(C_got, C_ref, np.flatnonzero(counts == 0))
                err = parity.center_rel_err(C_ref, C_got)
            assert err <= parity.CENTER_RTOL, f"{what} step {m + 1}: centres error {err:.3e}"
            col = parity.center_col_err(C_got, C_ref)
            assert col <= parity.CENTER_RTOL, f"{what} step {m + 1}: per-column centres error {col:.3e}"
            mem = parity.center_member_err(C_got, C_ref, Xc, lab)
            assert mem <= parity.CENTER_RTOL, f"{what} step {m + 1}: per-element centres error {mem:.3e}"
            prev = Cn


@pytest.mark.timeout(600)
@pytest.mark.parametrize("wl,scale,steps", [("c3", 1.0, 3), ("c4", 1.0, 3), ("c5", 1.0, 2)])
def test_workload_sampled_full_size(bridge, wl, scale, steps):
    """The large-k workloads (generic assign/update path) at their real shapes:
    1M x 128 k=256, 4M x 64 k=1024 (Zipf-skewed clusters), and the
    768-feature k=4096 embedding workload, 2M x 768 with X at 6.1 GB resident
    (buffers past 2^31 bytes).  Labels are checked on 20,000 sampled rows,
    centres in full (per row, per column and per element)."""
    import time

    from skmetal_amd import _synth

    t = time.perf_counter()
    X, C0 = _synth.generate(wl, seed=0, scale=scale)
    _say(f"{wl}: generated {X.shape} in {time.perf_counter() - t:.1f} s")
    _say(f"sampled lockstep {wl} {X.shape} k={C0.shape[0]}")
    _sampled_steps(bridge, X, C0, steps, 20000, 7, wl)


def _separated_blobs(n, d, k, seed):
    """k well-separated blobs (centres ~U[-10,10]^d, sigma 1) and one initial
    centre per blob: scikit-learn's trajectory has no near-ties to diverge on."""
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-10, 10, (k, d))
    ids = rng.integers(0, k, n)
    X = (cen[ids] + rng.standard_normal((n, d))).astype(np.float32)
    C0 = np.stack([X[np.flatnonzero(ids == j)[0]] for j in range(k)])
    return X, C0


@pytest.mark.parametrize("tol,max_iter", [(0.0, 6), (1e-4, 50), (1e3, 50), (0.5, 50)])
@pytest.mark.parametrize("n,d,k", [(20000, 100, 50), (5000, 130, 150), (3000, 12, 7)])
def test_batch_fused_reference_contract(bridge, n, d, k, tol, max_iter):
    """skmetal_kmeans_batch_fused through the C ABI against the oracle running
    skmetal's loop contract (KMeansBridge.swift:187-320): the stop on the root
    of the largest centre shift (strict '<' tol), no label stop, the labels of
    the last step's E-step, n_iter = steps run.  Separated blobs with one
    initial centre per blob: step 1 moves every centre by ~sqrt(d), step 2 by
    exactly 0."""
    _say(f"batch_fused n={n} d={d} k={k} tol={tol} max_iter={max_iter}")
    X, C0 = _separated_blobs(n, d, k, seed=n + k)
    C = C0.copy()
    lab = np.full(n, -7, np.int32)
    n_iter = bridge.kmeans_batch_fused(X, C, lab, n, d, k, (n + 255) // 256, max_iter, tol)
    ref = oracle.reference_loop(X, C0, max_iter, tol)
    assert n_iter == ref["n_iter"]
    np.testing.assert_array_equal(lab, ref["labels"])
    parity.check_centers(C, ref["centers"], what="batch_fused centres")


def test_batch_fused_zero_iterations_writes_nothing(bridge):
    X, C0 = _separated_blobs(2000, 20, 5, seed=3)
    C = C0.copy()
    lab = np.full(2000, -7, np.int32)
    assert bridge.kmeans_batch_fused(X, C, lab, 2000, 20, 5, 8, 0, 1e-4) == 0
    np.testing.assert_array_equal(C, C0)
    assert (lab == -7).all()


def test_accelerate_kmeans_matches_sklearn(bridge):
    """skmetal's user-facing path: accelerate(KMeans(...)).fit/predict/score on the
    GPU against scikit-learn's own KMeans from the same initial centres."""
    from sklearn.cluster import KMeans

    import skmetal_amd
    from skmetal_amd.estimators.cluster import HipKMeans

    X, C0 = _separated_blobs(20000, 32, 8, 11)
    kw = dict(n_clusters=8, init=C0, n_init=1, max_iter=100, tol=1e-4)
    model = skmetal_amd.accelerate(KMeans(**kw))
    assert isinstance(model, HipKMeans)
    model.fit(X)
    ref = KMeans(**kw).fit(X)
    parity.check_centers(model.cluster_centers_, ref.cluster_centers_, what="accelerate centres")
    mean = X.mean(axis=0)
    _, best, second = oracle.assign(X - mean, ref.cluster_centers_ - mean, return_gap=True)
    parity.check_labels(model.labels_, ref.labels_, best, second, X - mean, what="accelerate labels")
    assert model.n_iter_ == ref.n_iter_
    parity.check_inertia(model.inertia_, ref.inertia_, rtol=1e-5, atol=parity.centring_floor(X),
                         what="accelerate inertia")
    Y, _ = _separated_blobs(5000, 32, 8, 12)
    pred = model.predict(Y)
    ref_pred = ref.predict(Y)
    _, best, second = oracle.assign(Y, ref.cluster_centers_, return_gap=True)
    parity.check_labels(pred, ref_pred, best, second, Y, what="accelerate predict")
    assert model.score(Y) == pytest.approx(ref.score(Y), rel=1e-5)


def test_accelerate_kmeans_plusplus_same_draws_as_sklearn(bridge):
    """k-means++ init is drawn from the estimator's random_state exactly as
    scikit-learn draws it, so a seeded fit reproduces scikit-learn's."""
    from sklearn.cluster import KMeans

    import skmetal_amd

    X, _ = _separated_blobs(10000, 32, 8, 13)
    kw = dict(n_clusters=8, init="k-means++", n_init=1, max_iter=50, random_state=3)
    model = skmetal_amd.accelerate(KMeans(**kw)).fit(X)
    ref = KMeans(**kw).fit(X)
    parity.check_centers(model.cluster_centers_, ref.cluster_centers_, what="k-means++ centres")
    assert model.n_iter_ == ref.n_iter_


@pytest.mark.parametrize("bad,msg", [(np.nan, "NaN"), (np.inf, "infinity"), (-np.inf, "infinity")])
def test_fit_rejects_non_finite_like_sklearn(bridge, bad, msg):
    """fit checks finiteness on the device (max |x| of the resident X) and then
    raises scikit-learn's own error."""
    from sklearn.cluster import KMeans

    import skmetal_amd
    from skmetal_amd.estimators.cluster import HipKMeans

    X, _ = _separated_blobs(3000, 12, 4, 5)
    X[17, 3] = bad
    model = skmetal_amd.accelerate(KMeans(n_clusters=4, n_init=1, random_state=0))
    assert isinstance(model, HipKMeans) and model._should_use_gpu(X)  # the GPU path, not the CPU fallback
    with pytest.raises(ValueError, match=msg):
        model.fit(X)
    with pytest.raises(ValueError, match=msg):
        KMeans(n_clusters=4, n_init=1, random_state=0).fit(X)


def test_fit_extreme_finite_values(bridge):
    """Finite values whose centring overflows fp32 pass the check (scikit-learn
    accepts them) and the fit still returns finite labels."""
    from sklearn.cluster import KMeans

    import skmetal_amd

    X = np.zeros((2000, 12), np.float32)
    X[:1000, 0] = 3.0e38
    X[1000:, 0] = -3.0e38
    X[:, 1:] = np.random.default_rng(1).standard_normal((2000, 11)).astype(np.float32)
    model = skmetal_amd.accelerate(KMeans(n_clusters=2, n_init=1, random_state=0))
    assert model._should_use_gpu(X)
    with np.errstate(over="ignore", invalid="ignore"):
        model.fit(X)
    assert model.labels_.shape == (2000,)
    assert model.labels_.min() >= 0 and model.labels_.max() < 2
