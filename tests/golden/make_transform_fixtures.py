"""Write the golden fixture for KMeans.transform.

Runs scikit-learn's ``KMeans.transform`` (sklearn/cluster/_kmeans.py:1124-1148:
euclidean_distances to the fitted centres) on small float32 inputs and stores
X, the centres and the distance matrix per case in one compressed ``.npz`` of
numeric arrays (load with ``np.load``, no pickle).

Run from the repository root:  python tests/golden/make_transform_fixtures.py
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import sklearn
from sklearn.cluster import KMeans
from sklearn.datasets import make_blobs

OUT = Path(__file__).resolve().parent


def cases():
    X, _ = make_blobs(300, 7, centers=5, random_state=1)
    yield "blobs_300x7_k5", X.astype(np.float32), 5
    X, _ = make_blobs(200, 130, centers=9, cluster_std=3.0, random_state=2)
    yield "blobs_200x130_k9", X.astype(np.float32), 9
    rng = np.random.RandomState(3)
    X = (rng.standard_normal((150, 3)) * [1e-3, 1.0, 1e3] + 1e4).astype(np.float32)  # large offset: cancellation
    yield "offset_150x3_k4", X, 4
    X = np.repeat(rng.uniform(-2, 2, (6, 2)), 10, axis=0).astype(np.float32)  # rows equal to centres
    yield "dup_60x2_k6", X, 6


def main():
    arrays, meta = {}, []
    for name, X, k in cases():
        km = KMeans(n_clusters=k, n_init=1, random_state=0).fit(X)
        arrays[f"{name}__X"] = X
        arrays[f"{name}__C"] = km.cluster_centers_.astype(np.float32)
        arrays[f"{name}__D"] = km.transform(X).astype(np.float32)
        meta.append(dict(name=name, k=int(k)))
    np.savez_compressed(OUT / "transform.npz", **arrays)
    (OUT / "transform.json").write_text(json.dumps(dict(sklearn=sklearn.__version__, cases=meta), indent=1) + "\n")
    print(f"wrote {len(meta)} transform cases")


if __name__ == "__main__":
    main()
