"""Write the golden fixture for skmetal's k-means|| seeding.

Runs skmetal's own ``MetalKMeans._kmeans_parallel_init``
(skmetal/estimators/cluster.py:70-116) from the reference checkout, in the
build container only.  Its two bridge calls are replaced by numpy distances:
``kmeans_assign`` (cluster.py:92) gives each row its nearest candidate and
``compute_mindists`` (:93) the squared distance to it, both from the direct
form sum((x - c)^2) in float64, cast to float32 (the Metal kernels compute
fp32 distances).  Everything else -- the first draw (:79), the number of rounds
(:84), the taken set (:86, :99-102), ``rng.choice`` (:98), the cyclic fill
(:106-110) and the prune by one scikit-learn KMeans iteration (:112-116) -- is
the reference's code, run as it is.

Recorded per case: X, the seed, the candidate rows each round starts from (the
candidate array the method hands to ``kmeans_assign``), the final candidate
rows (the array the prune fits, or the cyclic fill's source) and the k
centroids the method returns.  One compressed ``.npz`` of numeric arrays (load
with ``np.load``, no pickle) and a JSON index.

Run from the repository root, where the reference is checked out:
    python tests/golden/make_kpar_fixtures.py [reference root, default /root/reference]
"""

from __future__ import annotations

import json
import sys
import warnings
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def _sqdist(X, C):
    """fp32 cast of the float64 direct-form squared distances, [n x m]."""
    X64 = X.astype(np.float64)
    out = np.empty((X.shape[0], C.shape[0]), dtype=np.float32)
    for j in range(C.shape[0]):
        out[:, j] = ((X64 - C[j].astype(np.float64)) ** 2).sum(axis=1).astype(np.float32)
    return out


def _row_ids(X, rows):
    """Row index in X of every row of `rows` (the rows of X are distinct)."""
    ids = []
    for r in rows:
        hit = np.flatnonzero(np.all(X == r, axis=1))
        assert hit.size >= 1, "a candidate is not a row of X"
        ids.append(int(hit[0]))
    return np.asarray(ids, dtype=np.int64)


def cases():
    rng = np.random.default_rng(11)

    def blobs(n, d, m, scale):
        cen = rng.normal(0, scale, (m, d))
        return (cen[rng.integers(0, m, n)] + rng.normal(0, 1, (n, d))).astype(np.float32)

    yield "blobs_2000x5_k8", blobs(2000, 5, 8, 10), 8, 0
    yield "blobs_3000x20_k16", blobs(3000, 20, 12, 6), 16, 1
    yield "blobs_1500x3_k40", blobs(1500, 3, 30, 8), 40, 2
    yield "line_600x1_k3", (rng.standard_normal((600, 1)) * 5).astype(np.float32), 3, 3
    yield "blobs_2000x64_k32", blobs(2000, 64, 32, 10), 32, 4
    # every row drawn each round: fewer candidates than k, the cyclic fill
    yield "all_rows_10x3_k10", rng.uniform(-1, 1, (10, 3)).astype(np.float32), 10, 5


def main():
    ref = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    sys.path.insert(0, str(ref))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # the reference warns that Metal is absent
        from skmetal.estimators import cluster as refcluster
    import sklearn
    import sklearn.cluster

    rec = {}

    def kmeans_assign(X, c_arr, assignments, n, d, ck):
        rec["rounds"].append(np.array(c_arr, copy=True))
        assignments[:] = np.argmin(_sqdist(X, c_arr), axis=1).astype(assignments.dtype)

    def compute_mindists(X, c_arr, assignments, dists, n, d, ck):
        D = _sqdist(X, c_arr)
        dists[:] = D[np.arange(n), assignments.astype(np.int64)]

    base_kmeans = sklearn.cluster.KMeans

    class RecordingKMeans(base_kmeans):
        def fit(self, X, y=None, sample_weight=None):
            rec["final"] = np.array(X, copy=True)
            return super().fit(X, y, sample_weight)

    class NumpyRecordingArrays:
        """numpy, with np.array of a Python list recorded (the candidate
        arrays the method builds, cluster.py:89 and :105)."""

        def __getattr__(self, name):
            return getattr(np, name)

        def array(self, obj, *args, **kwargs):
            out = np.array(obj, *args, **kwargs)
            if isinstance(obj, list):
                rec["arrays"].append(out.copy())
            return out

    refcluster.kmeans_assign = kmeans_assign
    refcluster.compute_mindists = compute_mindists
    refcluster.np = NumpyRecordingArrays()
    sklearn.cluster.KMeans = RecordingKMeans
    init = refcluster.MetalKMeans._kmeans_parallel_init

    arrays, meta = {}, []
    try:
        for name, X, k, seed in cases():
            rec.clear()
            rec["rounds"], rec["arrays"] = [], []
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                C = init(None, X, k, np.random.RandomState(seed))
            if "final" in rec:
                final = rec["final"]
            else:
                # the cyclic fill (cluster.py:105-110): the candidate array is
                # the last one the method builds from its list
                final = rec["arrays"][-1]
            arrays[f"{name}__X"] = X
            arrays[f"{name}__centroids"] = np.asarray(C, dtype=np.float32)
            arrays[f"{name}__final_rows"] = _row_ids(X, final)
            for r, c_arr in enumerate(rec["rounds"]):
                arrays[f"{name}__round{r}_rows"] = _row_ids(X, c_arr)
            meta.append(dict(name=name, n=int(X.shape[0]), d=int(X.shape[1]), k=int(k), seed=int(seed),
                             rounds=len(rec["rounds"]), pruned="final" in rec))
    finally:
        sklearn.cluster.KMeans = base_kmeans
        refcluster.np = np
    np.savez_compressed(OUT / "kpar.npz", **arrays)
    (OUT / "kpar.json").write_text(json.dumps(dict(sklearn=sklearn.__version__, numpy=np.__version__,
                                                   source="skmetal/estimators/cluster.py:70-116",
                                                   cases=meta), indent=1) + "\n")
    print(f"wrote {len(meta)} k-means|| cases")


if __name__ == "__main__":
    main()
