"""KMeans on the MI355X: the Lloyd loop runs in libskmetal_hip.so.

``HipKMeans`` takes the place of skmetal's ``MetalKMeans``
(skmetal/estimators/cluster.py:18-146) and of ``MetalKMeansMLX``
(skmetal/estimators/_mlx_kmeans.py:35-156) as the registered ``KMeans``
implementation.  It follows scikit-learn's ``KMeans.fit``
(sklearn/cluster/_kmeans.py:1427-1554) with ``algorithm="lloyd"``:

* ``init`` may be an array (used as given, ``n_init`` forced to 1),
  ``"k-means++"``, ``"random"`` or a callable, drawn from the estimator's
  ``random_state`` in the same order scikit-learn draws them; k-means++
  (sklearn/cluster/_kmeans.py:174-260) runs on the GPU on the centred X that
  is already resident for the Lloyd loop, with scikit-learn's random draws;
* X is uploaded once for all ``n_init`` runs;
* ``tol`` is scaled by the mean feature variance (``_tolerance``,
  _kmeans.py:279-287) and the loop stops on strict label convergence;
* for ``n_init > 1`` the run with the lowest inertia that is not the same
  clustering as the best so far is kept (_kmeans.py:1516-1527).

Estimator attributes set after ``fit``: ``cluster_centers_``, ``labels_``
(int32), ``inertia_``, ``n_iter_``, ``n_features_in_``.
"""

from __future__ import annotations

import warnings
from concurrent.futures import ThreadPoolExecutor

import numpy as np
from sklearn.exceptions import ConvergenceWarning
from sklearn.utils.validation import _assert_all_finite, check_array, check_random_state

from .. import _bridge
from .._config import get_config
from ._base import BaseGPUEstimator


def _tolerance(X: np.ndarray, tol: float) -> float:
    """sklearn/cluster/_kmeans.py:279-287 for dense float32 X: np.mean of
    np.var(X, axis=0), times tol.  The column variances come from the library
    (numpy's float32 np.var bit for bit, in host threads: numpy's own np.var
    is most of a fit's time on large X)."""
    if tol == 0:
        return 0.0
    return float(np.mean(_bridge.column_variance(X)) * tol)


def _same_clustering(a: np.ndarray, b: np.ndarray, k: int) -> bool:
    """scikit-learn's _is_same_clustering (sklearn/cluster/_k_means_common.pyx:
    _is_same_clustering): True when every label of `a` is paired with one label
    of `b` only.  rep[j] takes the b of some row labelled j in a (whichever
    write lands); the pairing is a function exactly when every row's b equals
    its label's rep."""
    a = np.asarray(a, dtype=np.intp)
    rep = np.empty(k, dtype=np.asarray(b).dtype)
    rep[a] = b
    return bool(np.array_equal(rep[a], b))


def _check_n_features(est, X) -> None:
    """scikit-learn's feature-count check for a fitted estimator."""
    expected = getattr(est, "n_features_in_", None)
    if expected is not None and X.shape[1] != expected:
        raise ValueError(f"X has {X.shape[1]} features, but {type(est).__name__} is expecting {expected} "
                         "features as input.")


class HipKMeans(BaseGPUEstimator):
    """GPU KMeans (Lloyd) with X resident in MI355X HBM."""

    def _resolve_n_init(self, init) -> int:
        est = self._estimator
        n_init = est.n_init
        if n_init in ("auto", "warn"):
            if isinstance(init, str) and init == "k-means++":
                n_init = 1
            elif isinstance(init, str) and init == "random":
                n_init = 10
            elif callable(init):
                n_init = 10
            else:
                n_init = 1
        if not isinstance(init, str) and not callable(init) and n_init != 1:
            warnings.warn(
                "Explicit initial center position passed: performing only one init in "
                f"{type(est).__name__} instead of n_init={n_init}.",
                RuntimeWarning,
                stacklevel=3,
            )
            n_init = 1
        return int(n_init)

    def _initial_centers(self, X, init, k, random_state, h):
        """sklearn/cluster/_kmeans.py:958-1029 (_init_centroids), unit weights,
        for the inits other than k-means++ (seeded on the device).  "random"
        draws random_state.choice(n, k, replace=False, p=ones / n) on the device
        (the same rows and draws as numpy's)."""
        if isinstance(init, str) and init == "random":
            seeds = h.choice(random_state, k, weights="unit")
            centers = X[seeds]
        elif callable(init):
            centers = init(X, k, random_state=random_state)
        else:
            centers = init
        centers = check_array(centers, dtype=np.float32, order="C", copy=True)
        if centers.shape != (k, X.shape[1]):
            raise ValueError(
                f"The shape of the initial centers {centers.shape} does not match "
                f"the number of clusters {k} and features {X.shape[1]}."
            )
        return np.ascontiguousarray(centers, dtype=np.float32)

    def fit(self, X, y=None, sample_weight=None):
        # the finiteness check is done on the device once X is resident
        # (scikit-learn's own check is a sum over X on the host)
        X = check_array(X, dtype=np.float32, order="C", ensure_min_samples=2, ensure_all_finite=False)
        if sample_weight is not None:
            if get_config().verbose:
                print("[skmetal_amd] HipKMeans: device=cpu (sample_weight is not supported on the GPU path)")
            return self._fallback_fit(X, y, sample_weight=sample_weight)
        if not self._should_use_gpu(X):
            return self._fallback_fit(X, y)

        est = self._estimator
        n, d = X.shape
        k = int(est.n_clusters)
        if n < k:
            raise ValueError(f"n_samples={n} should be >= n_clusters={k}.")
        init = est.init
        n_init = self._resolve_n_init(init)
        random_state = check_random_state(est.random_state)

        best = None
        plusplus = isinstance(init, str) and init == "k-means++"
        # The first seeding's random draws run while X is uploaded and centred.  The
        # tolerance's column variances (host threads, no device) run once the
        # upload is done, while the device seeds with k-means++ (both the upload's
        # staging and the variances are bound by the host's memory bandwidth), and
        # beside the upload for the other inits.  Nothing else draws from
        # random_state in between, so the draws are those of the serial order.
        with ThreadPoolExecutor(max_workers=2) as pool, _bridge.LloydHandle(n, d, k) as h:
            draws_f = pool.submit(_bridge.plusplus_draws, random_state, n, k) if plusplus else None
            tol_f = None if plusplus else pool.submit(_tolerance, X, est.tol)
            h.load(X, center=True)
            if tol_f is None:
                tol_f = pool.submit(_tolerance, X, est.tol)
            if not np.isfinite(h.max_abs()):
                # NaN or infinity in X (or a centring that overflowed): scikit-learn's
                # check raises its own error for the first two and passes the last
                _assert_all_finite(X, input_name="X", estimator_name=type(est).__name__)
            tol_abs = None
            for i in range(n_init):
                if plusplus:
                    T, first, u = draws_f.result() if i == 0 else _bridge.plusplus_draws(random_state, n, k)
                    h.plusplus_with(T, first, u)
                else:
                    h.set_centers(self._initial_centers(X, init, k, random_state, h))
                if tol_abs is None:
                    tol_abs = tol_f.result()
                n_iter, inertia = h.run(est.max_iter, tol_abs, strict=True)
                labels = h.labels()
                if best is None or (inertia < best[2] and not _same_clustering(labels, best[1], k)):
                    best = (h.centers(), labels, inertia, n_iter)

        centers, labels, inertia, n_iter = best
        if len(np.unique(labels)) < k:
            warnings.warn(
                f"Number of distinct clusters ({len(np.unique(labels))}) found smaller than "
                f"n_clusters ({k}). Possibly due to duplicate points in X.",
                ConvergenceWarning,
                stacklevel=2,
            )
        est.cluster_centers_ = centers
        est.labels_ = labels
        est.inertia_ = float(inertia)
        est.n_iter_ = int(n_iter)
        est.n_features_in_ = d
        est._n_features_out = k
        est._n_threads = 1
        self._fitted = True
        return self

    def _gpu_ready(self, X) -> bool:
        return self._fitted and self._should_use_gpu(X) and hasattr(self._estimator, "cluster_centers_")

    def predict(self, X):
        X, _ = self._validate_data(X)
        if not self._gpu_ready(X):
            return self._fallback_predict(X)
        _check_n_features(self._estimator, X)
        n, d = X.shape
        C = np.ascontiguousarray(self._estimator.cluster_centers_, dtype=np.float32)
        out = np.empty(n, dtype=np.int32)
        _bridge.kmeans_assign(X, C, out, n, d, C.shape[0])
        return out

    def transform(self, X):
        """Distances to the centres (sklearn/cluster/_kmeans.py:1124-1148) on the GPU."""
        X, _ = self._validate_data(X)
        if not self._gpu_ready(X):
            return self._fallback_transform(X)
        _check_n_features(self._estimator, X)
        C = np.ascontiguousarray(self._estimator.cluster_centers_, dtype=np.float32)
        return _bridge.kmeans_transform(X, C)

    def fit_predict(self, X, y=None, sample_weight=None):
        return self.fit(X, y, sample_weight=sample_weight)._estimator.labels_

    def fit_transform(self, X, y=None, sample_weight=None):
        return self.fit(X, y, sample_weight=sample_weight).transform(X)

    def score(self, X, y=None, sample_weight=None):
        X, _ = self._validate_data(X)
        if sample_weight is not None or not self._gpu_ready(X):
            return self._estimator.score(X, y, sample_weight=sample_weight)
        _check_n_features(self._estimator, X)
        n, d = X.shape
        C = np.ascontiguousarray(self._estimator.cluster_centers_, dtype=np.float32)
        lab = np.empty(n, dtype=np.int32)
        _bridge.kmeans_assign(X, C, lab, n, d, C.shape[0])
        v = _bridge.kmeans_inertia(X, C, lab, n, d, C.shape[0])
        if v < 0:
            raise RuntimeError(f"skmetal_kmeans_inertia failed: {_bridge.last_error()}")
        return -float(v)


def _prune_candidates(cand: np.ndarray, k: int) -> np.ndarray:
    """The reference's prune of more than k k-means|| candidates
    (skmetal/estimators/cluster.py:112-116: scikit-learn
    KMeans(n_clusters=k, init=cand[:k], n_init=1, max_iter=1).fit(cand)) on the
    device: scikit-learn's fit rules for it (the candidates centred on their
    mean, tol = 1e-4 times the mean column variance, one Lloyd iteration with
    the strict-convergence rule, then the final E-step) on this library's Lloyd
    loop, and scikit-learn's warning when fewer than k clusters stay
    distinct.  scikit-learn's fit draws nothing from the random_state it is
    given here, so neither does this."""
    m, d = cand.shape
    with _bridge.LloydHandle(m, d, k) as h:
        h.load(cand, center=True)
        h.set_centers(np.ascontiguousarray(cand[:k]))
        h.run(1, _tolerance(cand, 1e-4), strict=True)
        centers = h.centers()
        distinct = len(np.unique(h.labels()))
    if distinct < k:
        warnings.warn(
            f"Number of distinct clusters ({distinct}) found smaller than n_clusters ({k}). "
            "Possibly due to duplicate points in X.",
            ConvergenceWarning,
            stacklevel=3,
        )
    return centers


def kmeans_parallel_init(X: np.ndarray, k: int, rng, handle, trace: bool = False):
    """skmetal's k-means|| seeding, MetalKMeans._kmeans_parallel_init
    (skmetal/estimators/cluster.py:70-116), on the device: `handle` holds X
    (uploaded once) and keeps every row's squared distance to its nearest
    candidate, lowered with each round's new rows (skmetal_hip_lloyd_mindists).
    The distance to the assigned candidate that the reference's kmeans_assign +
    compute_mindists pair gives is that minimum.  Each round's draw is numpy's
    rng.choice(n, min(k, n), replace=False, p=maximum(dists, 1e-30) / sum) over
    the resident distances (LloydHandle.choice: the same rows, the same
    uniforms taken from rng); rounds = max(1, int(2 + ln k)); the set of taken
    indices starts as {0}, as the reference's does; more than k candidates are
    pruned by one Lloyd iteration from the first k in scikit-learn's rules
    (_prune_candidates), fewer are repeated cyclically.  Returns the k
    centroids (and, with trace, the candidate rows)."""
    n, d = X.shape
    first = int(rng.randint(n))
    n_rounds = max(1, int(2 + np.log(k)))
    rows = [first]
    taken = {0}
    new = [first]
    for r in range(n_rounds):
        handle.mindists(new, reset=(r == 0), download=False)
        idx = handle.choice(rng, min(k, n), weights="mindists")
        new = []
        for i in idx:
            if i not in taken:
                taken.add(i)
                rows.append(int(i))
                new.append(int(i))
    cand = X[np.asarray(rows, dtype=np.int64)]
    if cand.shape[0] <= k:
        centroids = np.empty((k, d), dtype=np.float32)
        centroids[: cand.shape[0]] = cand
        for i in range(cand.shape[0], k):
            centroids[i] = cand[i % cand.shape[0]]
    else:
        centroids = _prune_candidates(np.ascontiguousarray(cand, dtype=np.float32), k)
    return (centroids, rows) if trace else centroids


class MetalKMeans(BaseGPUEstimator):
    """skmetal's MetalKMeans (skmetal/estimators/cluster.py:18-146) on the MI355X,
    for code that wants its behaviour rather than scikit-learn's: k-means||
    seeding per init attempt (distance rounds on the device, X uploaded once
    for all attempts), then the reference's call sequence per attempt,
    kmeans_batch_fused with the estimator's tol as given and kmeans_inertia,
    keeping the attempt of lowest inertia.  n_iter_ is the last attempt's, as in
    the reference.  HipKMeans is the registered KMeans (scikit-learn's fit)."""

    def fit(self, X, y=None, **kwargs):
        X, _ = self._validate_data(X, y)
        if not self._should_use_gpu(X):
            return self._fallback_fit(X, y, **kwargs)
        est = self._estimator
        n, d = X.shape
        k = int(est.n_clusters)
        if n < k:
            raise ValueError(f"n_samples={n} should be >= n_clusters={k}.")
        max_iter = est.max_iter
        tol = est.tol
        n_init = est.n_init
        if n_init == "auto":
            init = getattr(est, "init", "k-means++")
            n_init = 1 if isinstance(init, str) and init == "k-means++" else (10 if n > 10000 else 5)
        rng = check_random_state(est.random_state)
        num_groups = max(1, (n + 255) // 256)

        best_inertia, best_centroids, best_assignments = np.inf, None, None
        actual_iters = 0
        with _bridge.LloydHandle(n, d, k) as h:
            h.load(X, center=False)
            for _ in range(int(n_init)):
                centroids = np.ascontiguousarray(kmeans_parallel_init(X, k, rng, h), dtype=np.float32)
                assignments = np.empty(n, dtype=np.int32)
                actual_iters = _bridge.kmeans_batch_fused(X, centroids, assignments, n, d, k, num_groups,
                                                          max_iter, tol)
                inertia = _bridge.kmeans_inertia(X, centroids, assignments, n, d, k)
                if inertia < best_inertia:
                    best_inertia = inertia
                    best_centroids = centroids.copy()
                    best_assignments = assignments.copy()
        if best_centroids is None:
            raise RuntimeError("MetalKMeans: no init attempt gave a valid inertia")
        est.cluster_centers_ = best_centroids
        est.labels_ = best_assignments.astype(np.int32)
        est.inertia_ = float(best_inertia)
        est.n_iter_ = int(actual_iters)
        est.n_features_in_ = d
        est._n_features_out = k
        self._fitted = True
        return self

    def fit_predict(self, X, y=None, **kwargs):
        # defined here so that attribute delegation to the wrapped estimator
        # does not run scikit-learn's own fit on the CPU
        return self.fit(X, y, **kwargs)._estimator.labels_

    def fit_transform(self, X, y=None, **kwargs):
        return self.fit(X, y, **kwargs).transform(X)

    def predict(self, X):
        X, _ = self._validate_data(X)
        if not self._fitted or not self._should_use_gpu(X):
            return self._fallback_predict(X)
        _check_n_features(self._estimator, X)
        C = np.ascontiguousarray(self._estimator.cluster_centers_, dtype=np.float32)
        out = np.empty(X.shape[0], dtype=np.int32)
        _bridge.kmeans_assign(X, C, out, X.shape[0], X.shape[1], C.shape[0])
        return out

    def transform(self, X):
        X, _ = self._validate_data(X)
        if not self._fitted or not self._should_use_gpu(X):
            return self._fallback_transform(X)
        _check_n_features(self._estimator, X)
        C = np.ascontiguousarray(self._estimator.cluster_centers_, dtype=np.float32)
        return _bridge.kmeans_transform(X, C)
