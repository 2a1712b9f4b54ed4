"""Write the golden fixtures for the KMeans Lloyd path.

Runs scikit-learn's ``KMeans(algorithm="lloyd")`` -- the CPU implementation
skmetal routes ``KMeans`` to -- on small and C1-sized inputs and stores its
outputs as compressed ``.npz`` files (numeric arrays only; load with
``np.load(path)``, no pickle).  Inputs that are cheap to regenerate
(the c1 workload) are stored as generator name + seed + SHA-256 instead of
the array itself.

Run from the repository root:  python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import sklearn  # noqa: E402
from sklearn.cluster import KMeans  # noqa: E402
from sklearn.cluster._k_means_lloyd import lloyd_iter_chunked_dense  # noqa: E402
from sklearn.datasets import make_blobs  # noqa: E402
from sklearn.utils._openmp_helpers import _openmp_effective_n_threads  # noqa: E402

from skmetal_amd import _synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def _fit(X, C0, max_iter, tol):
    km = KMeans(n_clusters=C0.shape[0], init=C0, n_init=1, max_iter=max_iter, tol=tol,
                algorithm="lloyd")
    km.fit(X)
    return km


def _trajectory(X, C0, steps):
    """Centres and labels after each Lloyd step of ONE sklearn run.

    Steps sklearn's own lloyd_iter_chunked_dense (the loop body of
    _kmeans_single_lloyd) on the centred data, as KMeans.fit does, so every
    recorded step follows from the previous recorded one.
    Returns (centres [steps,k,d] in caller coordinates, labels [steps,n]).
    """
    Xc = X.copy()
    mean = Xc.mean(axis=0)
    Xc -= mean
    centers = C0 - mean
    k, d = centers.shape
    w = np.ones(X.shape[0], dtype=X.dtype)
    centers_new = np.zeros_like(centers)
    weight = np.zeros(k, dtype=X.dtype)
    labels = np.full(X.shape[0], -1, dtype=np.int32)
    shift = np.zeros(k, dtype=X.dtype)
    nt = _openmp_effective_n_threads()
    cs, ls = [], []
    for _ in range(steps):
        lloyd_iter_chunked_dense(Xc, w, centers, centers_new, weight, labels, shift, nt)
        centers, centers_new = centers_new, centers
        cs.append(centers + mean)
        ls.append(labels.copy())
    return np.stack(cs).astype(np.float32), np.stack(ls).astype(np.int32)


def small_case(name, X, C0, max_iter=300, tol=0.0):
    X = np.ascontiguousarray(X, dtype=np.float32)
    C0 = np.ascontiguousarray(C0, dtype=np.float32)
    km = _fit(X, C0, max_iter, tol)
    trace, trace_labels = _trajectory(X, C0, min(km.n_iter_, 8))
    np.savez_compressed(
        OUT / f"{name}.npz",
        X=X, C0=C0, max_iter=np.int64(max_iter), tol=np.float64(tol),
        centers=km.cluster_centers_.astype(np.float32), labels=km.labels_.astype(np.int32),
        inertia=np.float64(km.inertia_), n_iter=np.int64(km.n_iter_),
        trace=trace, trace_labels=trace_labels,
    )
    return dict(name=name, n=X.shape[0], d=X.shape[1], k=C0.shape[0], n_iter=int(km.n_iter_),
                inertia=float(km.inertia_))


def workload_case(name, wl, seed, max_iter, scale=1.0):
    X, C0 = _synth.generate(wl, seed=seed, scale=scale)
    km = _fit(X, C0, max_iter, 0.0)
    k = C0.shape[0]
    trace, trace_labels = _trajectory(X, C0, km.n_iter_)
    lab_t = np.uint8 if k <= 256 else np.int32
    np.savez_compressed(
        OUT / f"{name}.npz",
        workload=np.array(wl), seed=np.int64(seed), scale=np.float64(scale),
        sha256=np.array(_synth.sha256(X)), C0=C0, max_iter=np.int64(max_iter),
        centers=km.cluster_centers_.astype(np.float32),
        labels=km.labels_.astype(lab_t),
        inertia=np.float64(km.inertia_), n_iter=np.int64(km.n_iter_),
        trace=trace, trace_labels=trace_labels.astype(lab_t),
    )
    return dict(name=name, workload=wl, n=X.shape[0], d=X.shape[1], k=k,
                n_iter=int(km.n_iter_), inertia=float(km.inertia_))


def main():
    rng = np.random.default_rng(20261201)
    manifest = dict(sklearn=sklearn.__version__, numpy=np.__version__, cases=[])
    cases = manifest["cases"]

    # unit-weight toy (closed form: centres [[.25,0],[.75,1]], inertia .25)
    X = np.array([[0, 0], [0.5, 0], [0.5, 1], [1, 1]], np.float32)
    cases.append(small_case("toy_unit", X, np.array([[0, 0], [1, 1]], np.float32)))

    # test_correctness.py:106 shape: make_blobs(2000, centers=10, n_features=50)
    X, _ = make_blobs(n_samples=2000, centers=10, n_features=50, random_state=42)
    X = X.astype(np.float32)
    C0 = X[np.sort(rng.choice(2000, 10, replace=False))]
    cases.append(small_case("blobs_2000x50_k10", X, C0))
    cases.append(small_case("blobs_2000x50_k10_tol", X, C0, tol=1e-4))

    # test_comprehensive.py:328-336 shape: 1000x10, 5 blobs, k=20; duplicated
    # initial rows force empty clusters and the relocation path
    X, _ = make_blobs(n_samples=1000, n_features=10, centers=5, random_state=42)
    X = X.astype(np.float32)
    idx = np.sort(rng.choice(1000, 17, replace=False))
    C0 = np.concatenate([X[idx], X[idx[:3]]])
    cases.append(small_case("empty_1000x10_k20", X, C0))

    # more clusters than distinct points (relocation impossible, max distance 0)
    base = rng.standard_normal((3, 6)).astype(np.float32) * 4
    X = base[rng.integers(0, 3, 200)]
    C0 = np.concatenate([base, base[:2]])
    cases.append(small_case("dup_points_k5", X, C0))

    # ragged feature counts and k above one 64-wide cluster chunk
    for name, n, d, k, b in [("odd_3000x7_k6", 3000, 7, 6, 6), ("odd_2500x33_k9", 2500, 33, 9, 9),
                             ("k100_5000x16", 5000, 16, 100, 40), ("k200_4000x20", 4000, 20, 200, 30)]:
        X, _ = make_blobs(n_samples=n, n_features=d, centers=b, random_state=n + d)
        X = X.astype(np.float32)
        C0 = X[np.sort(rng.choice(n, k, replace=False))]
        cases.append(small_case(name, X, C0))

    # the c1 workload at full size (100,000 x 32, k=8, 20 iterations)
    cases.append(workload_case("c1_full", "c1", seed=0, max_iter=20))
    # c2's law at 2% of its rows (10,000 x 100, k=50)
    cases.append(workload_case("c2_small", "c2", seed=0, max_iter=50, scale=0.02))

    (OUT / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
