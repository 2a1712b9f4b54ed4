"""Deterministic synthetic KMeans workloads (fp32, C-order).

The five Lloyd workloads the library is measured and parity-tested on:

=====  ======================  ======  =======================================================
name   n x d                   k       data
=====  ======================  ======  =======================================================
c1     100,000 x 32            8       8 equal isotropic blobs, centres ~U[-10,10]^32, sigma 1
c2     500,000 x 100           50      50 equal blobs, centres ~U[-10,10]^100, sigma 1
c3     1,000,000 x 128         256     256 equal blobs, centres ~N(0, 4 I), sigma 1
c4     4,000,000 x 64          1024    1024 blobs with Zipf(s=1.2) sizes, centres ~N(0, 9 I)
c5     2,000,000 x 768         4096    normalise(u + 0.2 z), u one of 4096 random unit
                                       directions, z ~ N(0, I_768)
=====  ======================  ======  =======================================================

Rows are shuffled.  Init is ``X[rng.choice(n, k, replace=False)]`` drawn from
an independent stream (seed + 1).  ``scale`` shrinks n for quick runs while
keeping d, k and the data law.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    n: int
    d: int
    k: int
    iters: int
    description: str


WORKLOADS = {
    "c1": Workload("c1", 100_000, 32, 8, 20, "8 equal blobs U[-10,10]^32 sigma=1"),
    "c2": Workload("c2", 500_000, 100, 50, 50, "50 equal blobs U[-10,10]^100 sigma=1"),
    "c3": Workload("c3", 1_000_000, 128, 256, 30, "256 blobs N(0,4I) sigma=1"),
    "c4": Workload("c4", 4_000_000, 64, 1024, 20, "1024 Zipf(1.2)-sized blobs N(0,9I) sigma=1"),
    "c5": Workload("c5", 2_000_000, 768, 4096, 10, "L2-normalised u+0.2z, 4096 unit directions"),
}


def _blob_sizes_equal(n: int, b: int) -> np.ndarray:
    sizes = np.full(b, n // b, dtype=np.int64)
    sizes[: n - sizes.sum()] += 1
    return sizes


def _blob_sizes_zipf(n: int, b: int, s: float) -> np.ndarray:
    w = np.arange(1, b + 1, dtype=np.float64) ** (-s)
    w /= w.sum()
    sizes = np.floor(w * n).astype(np.int64)
    sizes = np.maximum(sizes, 1)
    # hand the rounding remainder to the largest blobs, deterministically
    rem = n - int(sizes.sum())
    i = 0
    while rem != 0:
        step = 1 if rem > 0 else -1
        if sizes[i % b] + step >= 1:
            sizes[i % b] += step
            rem -= step
        i += 1
    return sizes


def _fill_blobs(rng, centres: np.ndarray, sizes: np.ndarray, sigma: float) -> np.ndarray:
    n = int(sizes.sum())
    d = centres.shape[1]
    X = rng.standard_normal((n, d), dtype=np.float32)
    if sigma != 1.0:
        X *= np.float32(sigma)
    lab = np.repeat(np.arange(len(sizes)), sizes)
    perm = rng.permutation(n)
    lab = lab[perm]
    # add centres in row blocks to bound peak memory
    step = 1 << 18
    c32 = centres.astype(np.float32)
    for s in range(0, n, step):
        X[s : s + step] += c32[lab[s : s + step]]
    return X


def _fill_directions_parallel(rng, u: np.ndarray, sizes: np.ndarray, sigma: float) -> np.ndarray:
    """c5's rows, normalise(u_label + sigma z), filled in blocks of 65,536 rows
    on host threads.  Each block draws from its own generator spawned from
    `rng` (after the label permutation), so the result does not depend on the
    thread count."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    n = int(sizes.sum())
    d = u.shape[1]
    lab = np.repeat(np.arange(len(sizes)), sizes)[rng.permutation(n)]
    block = 1 << 16
    nblk = (n + block - 1) // block
    gens = rng.spawn(nblk)
    u32 = u.astype(np.float32)
    X = np.empty((n, d), dtype=np.float32)

    def fill(b):
        r0, r1 = b * block, min(n, (b + 1) * block)
        blk = X[r0:r1]
        gens[b].standard_normal(out=blk, dtype=np.float32)
        blk *= np.float32(sigma)
        blk += u32[lab[r0:r1]]
        blk /= np.linalg.norm(blk, axis=1, keepdims=True).astype(np.float32)

    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(fill, range(nblk)))
    return X


def generate(name: str, seed: int = 0, scale: float = 1.0):
    """Return (X, C0) for workload ``name`` (fp32 C-order)."""
    w = WORKLOADS[name]
    n = max(w.k, int(round(w.n * scale)))
    rng = np.random.default_rng(seed)
    if name == "c1" or name == "c2":
        cen = rng.uniform(-10.0, 10.0, size=(w.k, w.d))
        X = _fill_blobs(rng, cen, _blob_sizes_equal(n, w.k), 1.0)
    elif name == "c3":
        cen = rng.standard_normal((w.k, w.d)) * 2.0
        X = _fill_blobs(rng, cen, _blob_sizes_equal(n, w.k), 1.0)
    elif name == "c4":
        cen = rng.standard_normal((w.k, w.d)) * 3.0
        X = _fill_blobs(rng, cen, _blob_sizes_zipf(n, w.k, 1.2), 1.0)
    elif name == "c5":
        u = rng.standard_normal((w.k, w.d))
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        X = _fill_directions_parallel(rng, u, _blob_sizes_equal(n, w.k), 0.2)
    else:
        raise KeyError(name)
    X = np.ascontiguousarray(X, dtype=np.float32)
    C0 = initial_centres(X, w.k, seed + 1)
    return X, C0


def initial_centres(X: np.ndarray, k: int, seed: int) -> np.ndarray:
    idx = np.random.default_rng(seed).choice(X.shape[0], size=k, replace=False)
    return np.ascontiguousarray(X[np.sort(idx)], dtype=np.float32)


def sha256(X: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(X).view(np.uint8)).hexdigest()
