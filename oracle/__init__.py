"""Oracle for the KMeans Lloyd path -- TEST INFRASTRUCTURE ONLY.

CPU restatement of scikit-learn 1.7.2's dense Lloyd k-means (the CPU path
skmetal dispatches ``KMeans`` to), used only to check results, by
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``.  Nothing in the product package imports this module.

Two independent restatements live here:

* ``lloyd_oracle.c`` (compiled to ``liboracle.so`` by ``make -C oracle``),
  fp64 arithmetic on fp32 data, OpenMP-parallel so it handles the 500k x 100
  workload in seconds; every function cites the sklearn file:line it follows.
* ``numpy_lloyd`` below, a vectorised numpy restatement of the same steps for
  small inputs, used to cross-check the C one.

Parity status per function (what pins it, see tests/test_oracle.py):

* ``assign``      -- skmetal's known-answer vector (tests/test_kernels.py:93-99),
                     brute force over all k on random inputs, permutation and
                     duplicate-centre invariants, sklearn golden labels.
* ``mstep``       -- closed forms (k=1 mean, init=X rows), sklearn's
                     _relocate_empty_clusters_dense vector
                     (sklearn/cluster/tests/test_k_means.py:115-153),
                     sklearn golden centres.
* ``lloyd``       -- sklearn golden trajectories (tests/golden/*.npz written by
                     tests/golden/make_fixtures.py), the unit-weight toy case,
                     strict-convergence n_iter, monotone inertia.
* ``reference_loop`` -- skmetal's batch_fused stopping contract over ``assign`` /
                     ``mstep``: the unit toy case's closed-form shift sequence
                     (0.25, then 0) at tol just above, at and below 0.25, tol 0,
                     max_iter 0 (tests/test_oracle.py).
* ``inertia``     -- closed form (sum of squares about the mean for k=1),
                     sklearn golden inertia.
* ``mean_f32``    -- bit-exact against numpy's float32 X.mean(axis=0).
* ``kmeans_plusplus`` -- scikit-learn's kmeans_plusplus picks on 9 golden inputs
                     (tests/golden/plusplus.npz, make_plusplus_fixtures.py) and its
                     docstring vector; planted mistakes (tests/test_plusplus_oracle.py).
* ``transform``   -- scikit-learn's KMeans.transform bit for bit on 4 golden inputs
                     (tests/golden/transform.npz), closed forms, planted mistakes
                     (tests/test_transform_oracle.py).
* ``kmeans_parallel_init`` (skmetal's k-means||) -- its distances against
                     scikit-learn's euclidean_distances(squared=True) and brute
                     force; the first draw, the round count, the {0} taken-set
                     rule and the cyclic fill by properties; the whole
                     seeding (every round's candidate rows, the final list,
                     the centroids) bit for bit against golden vectors of the
                     reference's own MetalKMeans._kmeans_parallel_init, run in
                     the build container with numpy distances in place of its
                     two Metal calls (tests/golden/kpar.npz, 6 cases;
                     tests/test_kpar_oracle.py).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64


def build(force: bool = False) -> Path:
    """Compile liboracle.so with gcc (make -C oracle)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.oracle_mean_f32.argtypes = [_f32p, _i64, _i64, _f32p]
        L.oracle_mean_f32.restype = None
        L.oracle_assign.argtypes = [_f32p, _i64, _i64, _f32p, _i64, _i32p, _f64p, _f64p]
        L.oracle_assign.restype = None
        L.oracle_sums.argtypes = [_f32p, _i64, _i64, _i32p, _i64, _f64p, _i64p]
        L.oracle_sums.restype = None
        L.oracle_mindists.argtypes = [_f32p, _i64, _i64, _f32p, _i32p, _f64p]
        L.oracle_mindists.restype = None
        L.oracle_inertia.argtypes = [_f32p, _i64, _i64, _f32p, _i32p]
        L.oracle_inertia.restype = ctypes.c_double
        L.oracle_mstep.argtypes = [_f32p, _i64, _i64, _i32p, _f32p, _i64, _f32p, _f64p]
        L.oracle_mstep.restype = ctypes.c_int
        L.oracle_lloyd.argtypes = [_f32p, _i64, _i64, _f32p, _i64, ctypes.c_int, ctypes.c_double,
                                   _f32p, _i32p, _f64p, _f32p]
        L.oracle_lloyd.restype = ctypes.c_int
        L.oracle_num_threads.argtypes = []
        L.oracle_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def mean_f32(X):
    X = _f32(X)
    n, d = X.shape
    out = np.empty(d, np.float32)
    lib().oracle_mean_f32(_p(X, _f32p), n, d, _p(out, _f32p))
    return out


def assign(X, C, return_gap: bool = False):
    """Labels (int32) by strict-'<' argmin of ||c||^2 - 2 x.c (fp64).

    With return_gap, also returns (best, second) true squared distances.
    """
    X = _f32(X)
    C = _f32(C)
    n, d = X.shape
    k = C.shape[0]
    labels = np.empty(n, np.int32)
    if return_gap:
        best = np.empty(n, np.float64)
        second = np.empty(n, np.float64)
        lib().oracle_assign(_p(X, _f32p), n, d, _p(C, _f32p), k, _p(labels, _i32p),
                            _p(best, _f64p), _p(second, _f64p))
        return labels, best, second
    lib().oracle_assign(_p(X, _f32p), n, d, _p(C, _f32p), k, _p(labels, _i32p), None, None)
    return labels


def sums(X, labels, k):
    X = _f32(X)
    labels = np.ascontiguousarray(labels, dtype=np.int32)
    n, d = X.shape
    s = np.empty((k, d), np.float64)
    c = np.empty(k, np.int64)
    lib().oracle_sums(_p(X, _f32p), n, d, _p(labels, _i32p), k, _p(s, _f64p), _p(c, _i64p))
    return s, c


def mindists(X, C, labels):
    X = _f32(X)
    C = _f32(C)
    labels = np.ascontiguousarray(labels, dtype=np.int32)
    n, d = X.shape
    out = np.empty(n, np.float64)
    lib().oracle_mindists(_p(X, _f32p), n, d, _p(C, _f32p), _p(labels, _i32p), _p(out, _f64p))
    return out


def inertia(X, C, labels) -> float:
    X = _f32(X)
    C = _f32(C)
    labels = np.ascontiguousarray(labels, dtype=np.int32)
    n, d = X.shape
    return float(lib().oracle_inertia(_p(X, _f32p), n, d, _p(C, _f32p), _p(labels, _i32p)))


def mstep(X, labels, C_old):
    """One M-step (sums, relocation, averaging, shift). Returns (C_new, shift, n_empty)."""
    X = _f32(X)
    C_old = _f32(C_old)
    labels = np.ascontiguousarray(labels, dtype=np.int32)
    n, d = X.shape
    k = C_old.shape[0]
    C_new = np.empty_like(C_old)
    shift = np.empty(k, np.float64)
    ne = lib().oracle_mstep(_p(X, _f32p), n, d, _p(labels, _i32p), _p(C_old, _f32p), k,
                            _p(C_new, _f32p), _p(shift, _f64p))
    return C_new, shift, int(ne)


def lloyd(X, C_init, max_iter: int, tol_abs: float = 0.0, trace: bool = False):
    """sklearn KMeans(init=C_init, n_init=1, algorithm='lloyd').fit(X), unit weights.

    Returns dict(centers, labels, inertia, n_iter[, trace]).
    """
    X = _f32(X)
    C_init = _f32(C_init)
    n, d = X.shape
    k = C_init.shape[0]
    C_out = np.empty((k, d), np.float32)
    labels = np.empty(n, np.int32)
    inert = ctypes.c_double(0.0)
    tr = np.empty((max_iter, k, d), np.float32) if trace else None
    n_iter = lib().oracle_lloyd(_p(X, _f32p), n, d, _p(C_init, _f32p), k, int(max_iter),
                                float(tol_abs), _p(C_out, _f32p), _p(labels, _i32p),
                                ctypes.byref(inert), _p(tr, _f32p) if trace else None)
    if n_iter < 0:
        raise MemoryError("oracle_lloyd allocation failed")
    out = dict(centers=C_out, labels=labels, inertia=inert.value, n_iter=int(n_iter))
    if trace:
        out["trace"] = tr[:n_iter]
    return out


def reference_loop(X, C_init, max_iter: int, tol: float):
    """skmetal's loop contract for skmetal_kmeans_batch_fused
    (skmetal_bridge/Sources/SkMetalBridge/KMeansBridge.swift:187-320) over this
    oracle's Lloyd step: up to max_iter steps of ``assign`` + ``mstep`` on X
    centred on its fp32 column mean (empty clusters relocated as scikit-learn
    does); after each step the loop stops when the fp32 root of the largest
    squared centre shift is below tol, strictly (:306-310); no label-based
    stop and no final E-step.  The squared shifts are fp64 sums of the fp32
    coordinates' differences, rounded to fp32, as the library computes them.
    Returns dict(centers (caller coordinates), labels (the last step's E-step;
    None when max_iter = 0), estep_centers (the centres that E-step used),
    n_iter)."""
    X = _f32(X)
    mean = X.mean(axis=0)
    Xc = X - mean
    C = _f32(C_init) - mean
    labels = None
    C_prev = C
    n_iter = 0
    for it in range(int(max_iter)):
        labels = assign(Xc, C)
        C_prev = C
        C_new, _, _ = mstep(Xc, labels, C)
        sq = ((C_new.astype(np.float64) - C.astype(np.float64)) ** 2).sum(axis=1).astype(np.float32)
        C = C_new
        n_iter = it + 1
        if np.sqrt(np.float32(sq.max(initial=0.0))) < np.float32(tol):
            break
    return dict(centers=(C + mean).astype(np.float32), labels=labels,
                estep_centers=(C_prev + mean).astype(np.float32), n_iter=n_iter)


def sklearn_tolerance(X, tol: float) -> float:
    """sklearn's _tolerance (sklearn/cluster/_kmeans.py:279-287) for dense X."""
    if tol == 0:
        return 0.0
    return float(np.mean(np.var(np.asarray(X, dtype=np.float32), axis=0)) * tol)


# ---------------------------------------------------------------------------
# Independent numpy restatement (small inputs only), used to cross-check C.
# ---------------------------------------------------------------------------

def numpy_lloyd(X, C_init, max_iter: int, tol_abs: float = 0.0):
    """Vectorised restatement of the same sklearn steps, fp64 arithmetic."""
    X = _f32(X)
    mean = X.mean(axis=0)  # numpy float32 mean, as sklearn
    Xc = X - mean
    C = _f32(C_init) - mean
    Xd = Xc.astype(np.float64)
    n, d = X.shape
    k = C.shape[0]
    old = np.full(n, -1, np.int32)
    strict = False
    it = 0
    for it in range(max_iter):
        Cd = C.astype(np.float64)
        D = (Cd * Cd).sum(1)[None, :] - 2.0 * Xd @ Cd.T
        labels = np.argmin(D, axis=1).astype(np.int32)  # first minimum, as strict '<'
        counts = np.bincount(labels, minlength=k).astype(np.int64)
        S = np.zeros((k, d), np.float64)
        np.add.at(S, labels, Xd)
        empty = np.flatnonzero(counts == 0)
        if empty.size:
            dist = ((Xd - Cd[labels]) ** 2).sum(1)
            if dist.max() > 0:
                order = np.lexsort((np.arange(n), -dist))
                for e, j in enumerate(empty):
                    far = order[e]
                    o = labels[far]
                    S[o] -= Xd[far]
                    S[j] = Xd[far]
                    counts[j] = 1
                    counts[o] -= 1
        amax = int(np.argmax(counts))
        cur = S.copy()
        for j in range(k):
            if counts[j] > 0:
                cur[j] = cur[j] / counts[j]
            else:
                cur[j] = cur[amax]
        C_new = cur.astype(np.float32)
        shift = np.sqrt(((C_new.astype(np.float64) - C.astype(np.float64)) ** 2).sum(1))
        C = C_new
        if np.array_equal(labels, old):
            strict = True
            break
        if (shift ** 2).sum() <= tol_abs:
            break
        old = labels
    n_iter = it + 1
    Cd = C.astype(np.float64)
    if not strict:
        D = (Cd * Cd).sum(1)[None, :] - 2.0 * Xd @ Cd.T
        labels = np.argmin(D, axis=1).astype(np.int32)
    inert = float(((Xd - Cd[labels]) ** 2).sum())
    return dict(centers=(C + mean).astype(np.float32), labels=labels, inertia=inert, n_iter=n_iter)


def _upcast_sqdist(Xc, rows, X64=None, xx=None):
    """sklearn/metrics/pairwise.py:391-446,582-640 (_euclidean_distances with
    fp32 data -> _euclidean_distances_upcast): fp64 -2 c.x + ||c||^2 + ||x||^2 of
    the candidate rows against every row, cast to fp32, negatives set to 0."""
    if X64 is None:
        X64 = Xc.astype(np.float64)
        xx = np.einsum("ij,ij->i", X64, X64)
    C64 = X64[rows]
    cc = xx[rows]
    d = -2.0 * (C64 @ X64.T)
    d += cc[:, None]
    d += xx[None, :]
    d = d.astype(np.float32)
    np.maximum(d, 0, out=d)
    return d


def kmeans_plusplus(X, k: int, first: int, uniforms, n_local_trials: int, trace: bool = False):
    """Greedy k-means++ with the random draws given: sklearn/cluster/_kmeans.py:174-263
    (_kmeans_plusplus), unit sample weights.

    first    -- the first centre's row (random_state.choice, :225)
    uniforms -- [(k-1) x n_local_trials] values of random_state.uniform (:243)

    Reductions are exact in fp64 (sequential cumsum as stable_cumsum, :244-246;
    potentials as fp64 sums of the fp32 minima, where scikit-learn uses an fp32
    BLAS dot product, :236,257), and the potential enters the draws rounded to
    fp32 as scikit-learn's fp32 current_pot does (:243).  Returns the k row
    indices (and, with trace, each centre's candidate rows and potentials)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    n = X.shape[0]
    T = int(n_local_trials)
    U = np.asarray(uniforms, dtype=np.float64).reshape(max(k - 1, 0), T)
    idx = np.empty(k, np.int64)
    idx[0] = first
    X64 = X.astype(np.float64)
    xx = np.einsum("ij,ij->i", X64, X64)
    closest = _upcast_sqdist(X, np.array([first]), X64, xx)[0]         # :234-236
    pot = float(np.sum(closest.astype(np.float64)))                    # :237
    cands, pots = [np.array([first])], [np.array([pot])]
    for c in range(1, k):
        r = U[c - 1] * float(np.float32(pot))                          # :243
        cum = np.cumsum(closest, dtype=np.float64)                     # :244-246 stable_cumsum
        cid = np.searchsorted(cum, r)                                  # side='left'
        np.clip(cid, None, n - 1, out=cid)                             # :248
        dist = _upcast_sqdist(X, cid, X64, xx)                         # :251-253
        np.minimum(closest[None, :], dist, out=dist)                   # :256
        cpot = dist.astype(np.float64).sum(axis=1)                     # :257
        b = int(np.argmin(cpot))                                       # :260 first minimum
        pot = float(cpot[b])
        closest = dist[b]
        idx[c] = cid[b]
        cands.append(cid)
        pots.append(cpot)
    if trace:
        return idx, cands, pots
    return idx


def parallel_mindists(X):
    """The k-means|| rounds' distances on the CPU: returns mindists(rows, reset),
    the fp32 squared distance of every row of X to its nearest candidate so far
    (_upcast_sqdist of each candidate row, min), lowered with `rows`; reset
    starts from +inf."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    X64 = X.astype(np.float64)
    xx = np.einsum("ij,ij->i", X64, X64)
    state = {}

    def mindists(rows, reset):
        if reset:
            state["c"] = np.full(X.shape[0], np.inf, dtype=np.float32)
        if len(rows):
            np.minimum(state["c"], _upcast_sqdist(X, np.asarray(rows, dtype=np.int64), X64, xx).min(axis=0),
                       out=state["c"])
        return state["c"].copy()

    return mindists


def kmeans_parallel_init(X, k: int, rng, mindists=None, trace: bool = False):
    """skmetal's k-means|| seeding, MetalKMeans._kmeans_parallel_init
    (skmetal/estimators/cluster.py:70-116), with `rng` a numpy RandomState:
    first row rng.randint(n) (:77); max(1, int(2 + ln k)) rounds (:83); each
    round the squared distance of every row to its assigned candidate, i.e. the
    nearest one (:91-93; here _upcast_sqdist, min over the candidates), floored
    at 1e-30 and normalised in fp32 (:94-95), then rng.choice(n, min(k, n),
    p, replace=False) (:97-98); new indices join in draw order, the taken set
    starting as {0} as the reference's does (:85,99-102); more than k
    candidates are pruned by one scikit-learn KMeans iteration from the first
    k (:112-116), fewer are repeated cyclically (:105-110).
    mindists(rows, reset) may replace the CPU distances (the device's, for a
    cross-check).  Returns the k centroids (and, with trace, the candidate rows)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    n, d = X.shape
    if mindists is None:
        mindists = parallel_mindists(X)
    first = int(rng.randint(n))
    rows, taken, new = [first], {0}, [first]
    for r in range(max(1, int(2 + np.log(k)))):
        dists = np.maximum(mindists(new, r == 0), 1e-30)
        probs = dists / dists.sum()
        new = []
        for i in rng.choice(n, size=min(k, n), p=probs, replace=False):
            if i not in taken:
                taken.add(i)
                rows.append(int(i))
                new.append(int(i))
    cand = X[np.asarray(rows, dtype=np.int64)]
    if cand.shape[0] <= k:
        out = np.empty((k, d), dtype=np.float32)
        for i in range(k):
            out[i] = cand[i % cand.shape[0]]
    else:
        from sklearn.cluster import KMeans

        out = KMeans(n_clusters=k, init=cand[:k], n_init=1, max_iter=1, random_state=rng).fit(cand)
        out = out.cluster_centers_.astype(np.float32)
    return (out, rows) if trace else out


def transform(X, C):
    """sklearn/cluster/_kmeans.py:1124-1148 (KMeans.transform = euclidean_distances(X,
    cluster_centers_)) for fp32 data: sklearn/metrics/pairwise.py:582-652 upcast
    chunks, d = (-2 x.c + ||x||^2) + ||c||^2 in fp64, cast to fp32, negatives to 0
    (:428-431), np.sqrt in fp32 (:441)."""
    X64 = np.asarray(X, dtype=np.float32).astype(np.float64)
    C64 = np.asarray(C, dtype=np.float32).astype(np.float64)
    d = -2.0 * (X64 @ C64.T)
    d += np.einsum("ij,ij->i", X64, X64)[:, None]
    d += np.einsum("ij,ij->i", C64, C64)[None, :]
    d = d.astype(np.float32)
    np.maximum(d, 0, out=d)
    return np.sqrt(d)
