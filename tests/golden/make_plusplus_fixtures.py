"""Write the golden fixture for k-means++ seeding.

Runs scikit-learn's ``kmeans_plusplus`` (sklearn/cluster/_kmeans.py:68-263, the
seeding ``KMeans(init="k-means++")`` uses) on small float32 inputs and stores,
per case, X, the seed, n_local_trials and the row indices scikit-learn chose,
in one compressed ``.npz`` of numeric arrays (load with ``np.load``, no pickle).
Also records the picks of ``KMeans.fit``'s own seeding, which runs on the
column-centred X (``_kmeans.py:1477-1484``), for one case.

Run from the repository root:  python tests/golden/make_plusplus_fixtures.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import sklearn  # noqa: E402
from sklearn.cluster import kmeans_plusplus  # noqa: E402
from sklearn.datasets import make_blobs  # noqa: E402

OUT = Path(__file__).resolve().parent


def cases():
    # scikit-learn's docstring example (sklearn/cluster/_kmeans.py:132-141): indices [3, 2]
    yield "docstring", np.array([[1, 2], [1, 4], [1, 0], [10, 2], [10, 4], [10, 0]], np.float32), 2, 0, None
    X, _ = make_blobs(400, 12, centers=6, random_state=3)
    yield "blobs_400x12_k6", X.astype(np.float32), 6, 7, None
    X, _ = make_blobs(600, 33, centers=10, cluster_std=2.0, random_state=5)
    yield "blobs_600x33_k20", X.astype(np.float32), 20, 11, None
    rng = np.random.RandomState(2)
    X = rng.standard_normal((300, 1)).astype(np.float32) * 4
    yield "line_300x1_k8", X, 8, 2, None
    X = np.repeat(rng.uniform(-3, 3, (5, 4)), [40, 30, 20, 20, 10], axis=0).astype(np.float32)
    yield "dup_120x4_k7", X, 7, 4, None          # 5 distinct rows: zero potentials once they are taken
    X = rng.uniform(-1, 1, (300, 24)).astype(np.float32)
    yield "uniform_300x24_k12_t1", X, 12, 9, 1   # one trial per centre
    yield "uniform_300x24_k12_t20", X, 12, 9, 20  # more trials than one pass of the kernel holds
    X = (rng.standard_normal((257, 3)) * [1.0, 100.0, 0.01]).astype(np.float32)
    yield "aniso_257x3_k1", X, 1, 5, None


def main():
    arrays, meta = {}, []
    for name, X, k, seed, trials in cases():
        _, idx = kmeans_plusplus(X, k, random_state=seed, n_local_trials=trials)
        T = trials if trials is not None else 2 + int(np.log(k))
        arrays[f"{name}__X"] = X
        arrays[f"{name}__idx"] = idx.astype(np.int64)
        meta.append(dict(name=name, k=int(k), seed=int(seed), n_local_trials=int(T)))
    # KMeans.fit seeds on the centred X
    X, _ = make_blobs(500, 20, centers=8, random_state=8)
    X = X.astype(np.float32) + 50.0
    Xc = X - X.mean(axis=0)
    _, idx = kmeans_plusplus(Xc, 8, random_state=13)
    arrays["fit_centred_500x20_k8__X"] = X
    arrays["fit_centred_500x20_k8__idx"] = idx.astype(np.int64)
    meta.append(dict(name="fit_centred_500x20_k8", k=8, seed=13, n_local_trials=2 + int(np.log(8)), centred=True))
    np.savez_compressed(OUT / "plusplus.npz", **arrays)
    (OUT / "plusplus.json").write_text(json.dumps(dict(sklearn=sklearn.__version__, numpy=np.__version__,
                                                       cases=meta), indent=1) + "\n")
    print(f"wrote {len(meta)} k-means++ cases")


if __name__ == "__main__":
    main()
