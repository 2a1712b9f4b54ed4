"""ctypes bridge to libskmetal_hip.so (mirrors skmetal/_bridge.py on the KMeans path).

Binds the reference's KMeans entry points with the reference's argtypes
(skmetal/_bridge.py:111-142, 352-363, 627-639) plus this library's additions
(``skmetal_hip_*``).  ``HIP_AVAILABLE`` (alias ``METAL_AVAILABLE``) is True
only when the library loaded *and* a gfx950 device initialised.  Wrappers
raise ``RuntimeError`` when the library is unavailable or a call fails; they
never compute anything on the CPU.
"""

from __future__ import annotations

import ctypes
import os
import warnings
from pathlib import Path

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_NAME = "libskmetal_hip.so"


def _find_library() -> str:
    env = os.environ.get("SKMETAL_HIP_LIB")
    candidates = [Path(env)] if env else []
    candidates.append(_PKG / LIB_NAME)
    for p in candidates:
        if p.exists():
            return str(p.resolve())
    raise RuntimeError(f"{LIB_NAME} not found; build it with `python -m skmetal_amd._build`")


_c_size = ctypes.c_size_t
_vp = ctypes.c_void_p

# (c_name, restype, argtypes...) -- the KMeans subset of the reference's registry
_REGISTRY = [
    ("skmetal_init", ctypes.c_int),
    ("skmetal_warmup", ctypes.c_int),
    ("skmetal_device_info", ctypes.c_int, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t),
     ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_uint64)),
    ("skmetal_kmeans_assign", ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size),
    ("skmetal_kmeans_batch_fused", ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size, _c_size, _c_size,
     ctypes.c_float, ctypes.POINTER(ctypes.c_int32)),
    ("skmetal_compute_mindists", ctypes.c_int, _vp, _vp, _vp, _vp, _c_size, _c_size, _c_size),
    ("skmetal_gemm", ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size, ctypes.c_float, ctypes.c_float,
     ctypes.c_int, ctypes.c_int),
    ("skmetal_kmeans_inertia", ctypes.c_float, _vp, _vp, _vp, _c_size, _c_size, _c_size),
    ("skmetal_hip_last_error", ctypes.c_char_p),
    ("skmetal_hip_release_cache", ctypes.c_int),
    ("skmetal_hip_kmeans_fit", ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size, _c_size, ctypes.c_double,
     ctypes.c_int, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_double)),
    ("skmetal_hip_lloyd_create", ctypes.c_int, _c_size, _c_size, _c_size, ctypes.POINTER(_vp)),
    ("skmetal_hip_lloyd_destroy", ctypes.c_int, _vp),
    ("skmetal_hip_lloyd_load", ctypes.c_int, _vp, _vp, ctypes.c_int),
    ("skmetal_hip_lloyd_set_centers", ctypes.c_int, _vp, _vp),
    ("skmetal_hip_lloyd_iterate", ctypes.c_int, _vp, _c_size, ctypes.POINTER(ctypes.c_float),
     ctypes.POINTER(ctypes.c_float)),
    ("skmetal_hip_lloyd_run", ctypes.c_int, _vp, _c_size, ctypes.c_double, ctypes.c_int,
     ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_double)),
    ("skmetal_hip_lloyd_info", ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)),
    ("skmetal_hip_lloyd_get_centers", ctypes.c_int, _vp, _vp),
    ("skmetal_hip_lloyd_get_labels", ctypes.c_int, _vp, _vp),
    ("skmetal_hip_lloyd_inertia", ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_double)),
    ("skmetal_hip_lloyd_plusplus", ctypes.c_int, _vp, _c_size, ctypes.c_int64, _vp, _vp),
    ("skmetal_hip_kmeans_plusplus", ctypes.c_int, _vp, _c_size, _c_size, _c_size, _c_size, ctypes.c_int64, _vp, _vp),
    ("skmetal_hip_kmeans_transform", ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size),
    ("skmetal_hip_column_variance", ctypes.c_int, _vp, _c_size, _c_size, _vp),
    ("skmetal_hip_lloyd_max_abs", ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_float)),
    ("skmetal_hip_lloyd_mindists", ctypes.c_int, _vp, _vp, _c_size, ctypes.c_int, _vp),
    ("skmetal_hip_lloyd_sample_prepare", ctypes.c_int, _vp, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
     ctypes.POINTER(ctypes.c_int64)),
    ("skmetal_hip_lloyd_sample_draw", ctypes.c_int, _vp, _vp, _c_size, _vp, _c_size, _vp, ctypes.c_int,
     ctypes.POINTER(ctypes.c_int)),
    ("skmetal_hip_kmeans_batch_fused_noalloc", ctypes.c_int, _vp, _vp, _vp, _c_size, _c_size, _c_size, _c_size,
     ctypes.c_float, ctypes.POINTER(ctypes.c_int32)),
]

SKMETAL_FIT_STRICT = 1

_lib = None
_load_error = None
HIP_AVAILABLE = False
try:
    _lib = ctypes.CDLL(_find_library())
    for _name, _restype, *_argtypes in _REGISTRY:
        _f = getattr(_lib, _name)
        _f.argtypes = list(_argtypes)
        _f.restype = _restype
    _rc = _lib.skmetal_init()
    if _rc != 0:
        raise RuntimeError(f"skmetal_init failed with code {_rc}: {_lib.skmetal_hip_last_error().decode()}")
    HIP_AVAILABLE = True
except Exception as _err:  # noqa: BLE001 -- report and keep importing, like the reference
    _load_error = _err
    warnings.warn(
        f"skmetal_amd: MI355X GPU path not available ({_err}). accelerate() leaves estimators on scikit-learn.",
        stacklevel=2,
    )

METAL_AVAILABLE = HIP_AVAILABLE  # name kept for code written against skmetal

_WARMUP_DONE = False


def library_path() -> str | None:
    return getattr(_lib, "_name", None) if _lib is not None else None


def _require():
    if _lib is None or not HIP_AVAILABLE:
        raise RuntimeError(f"skmetal_amd GPU path unavailable: {_load_error}")


def last_error() -> str:
    return _lib.skmetal_hip_last_error().decode() if _lib is not None else str(_load_error)


def ensure_warmed_up():
    global _WARMUP_DONE
    _require()
    if not _WARMUP_DONE:
        _check(_lib.skmetal_warmup(), "skmetal_warmup")
        _WARMUP_DONE = True


def _check(err: int, name: str, context: str = ""):
    if err != 0:
        msg = f"{name} failed with code {err}"
        if context:
            msg += f" ({context})"
        detail = last_error()
        if detail:
            msg += f": {detail}"
        raise RuntimeError(msg)


def _bridge_call(c_func, *args, context=""):
    """Call a C entry point converting numpy arrays / ints / floats as the reference does
    (skmetal/_bridge.py:78-103); raise RuntimeError on a non-zero return."""
    ensure_warmed_up()
    c_args = []
    for a in args:
        if isinstance(a, np.ndarray):
            c_args.append(a.ctypes.data)
        elif isinstance(a, bool):
            c_args.append(ctypes.c_int(int(a)))
        elif isinstance(a, int):
            c_args.append(ctypes.c_size_t(a))
        elif isinstance(a, (float, np.floating)):
            c_args.append(ctypes.c_float(a))
        else:
            c_args.append(a)
    _check(c_func(*c_args), c_func.__name__, context)


def _f32c(a, name):
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous float32 ndarray")
    return a


def _i32c(a, name):
    if not (isinstance(a, np.ndarray) and a.dtype.itemsize == 4 and a.dtype.kind in "iu" and a.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous 32-bit integer ndarray")
    return a


def _check_sizes(n, d, k, X, centroids, assignments, dists=None):
    """The arrays hold exactly the n x d, k x d and n elements the library
    will read or write through their pointers."""
    n, d, k = int(n), int(d), int(k)
    if X.size != n * d:
        raise ValueError(f"X has {X.size} elements, expected n * d = {n} * {d}")
    if centroids.size != k * d:
        raise ValueError(f"centroids has {centroids.size} elements, expected k * d = {k} * {d}")
    if assignments.size != n:
        raise ValueError(f"assignments has {assignments.size} elements, expected n = {n}")
    if dists is not None and dists.size != n:
        raise ValueError(f"dists has {dists.size} elements, expected n = {n}")


# ---- the reference's KMeans wrappers (skmetal/_bridge.py:576-639) ----

def kmeans_assign(X, centroids, assignments, n, d, k) -> None:
    """E-step: assignments[i] = nearest centroid of X[i]."""
    _f32c(X, "X"), _f32c(centroids, "centroids"), _i32c(assignments, "assignments")
    _check_sizes(n, d, k, X, centroids, assignments)
    _bridge_call(_lib.skmetal_kmeans_assign, X, centroids, assignments, n, d, k)


def kmeans_batch_fused(X, centroids, assignments, n, d, k, num_groups, max_iter, tol) -> int:
    """Lloyd fit on the GPU (centroids in/out); returns n_iter."""
    _f32c(X, "X"), _f32c(centroids, "centroids"), _i32c(assignments, "assignments")
    _check_sizes(n, d, k, X, centroids, assignments)
    n_iter_out = ctypes.c_int32(0)
    _bridge_call(_lib.skmetal_kmeans_batch_fused, X, centroids, assignments, n, d, k, num_groups, max_iter,
                 ctypes.c_float(tol), ctypes.byref(n_iter_out))
    return n_iter_out.value


def compute_mindists(X, centroids, assignments, dists, n, d, k) -> None:
    """dists[i] = ||X[i] - centroids[assignments[i]]||^2."""
    _f32c(X, "X"), _f32c(centroids, "centroids"), _i32c(assignments, "assignments"), _f32c(dists, "dists")
    _check_sizes(n, d, k, X, centroids, assignments, dists)
    _bridge_call(_lib.skmetal_compute_mindists, X, centroids, assignments, dists, n, d, k)


def kmeans_inertia(X, centroids, assignments, n, d, k) -> float:
    """Sum of squared distances to the assigned centroids (GPU); -1.0 on failure, as the reference."""
    _f32c(X, "X"), _f32c(centroids, "centroids"), _i32c(assignments, "assignments")
    _check_sizes(n, d, k, X, centroids, assignments)
    ensure_warmed_up()
    return float(_lib.skmetal_kmeans_inertia(X.ctypes.data, centroids.ctypes.data, assignments.ctypes.data,
                                             n, d, k))


def gemm(A, B, alpha: float = 1.0, beta: float = 0.0, trans_A: bool = False, trans_B: bool = False, C=None):
    """C = alpha * op(A) @ op(B) + beta * C in fp32 on the device (skmetal_gemm).

    The reference's gemm (skmetal/_bridge.py:499-560) with its argument checks;
    its last route, the bridge's fp32 GEMM, is the only one here.  C is read
    only when beta != 0 (then it must be given, [M x N] float32)."""
    _require()
    if A.dtype != np.float32 or B.dtype != np.float32:
        raise TypeError("A and B must be float32")
    if not (A.flags["C_CONTIGUOUS"] and B.flags["C_CONTIGUOUS"]):
        raise ValueError("A and B must be C-contiguous")
    M, K = (A.shape[1], A.shape[0]) if trans_A else (A.shape[0], A.shape[1])
    K2, N = (B.shape[1], B.shape[0]) if trans_B else (B.shape[0], B.shape[1])
    if K != K2:
        raise ValueError(f"Incompatible dimensions: A {A.shape}, B {B.shape}")
    if beta != 0.0:
        if C is None:
            raise ValueError("beta != 0 needs C")
        _f32c(C, "C")
        if C.shape != (M, N):
            raise ValueError(f"C has shape {C.shape}, expected {(M, N)}")
        out = C
    else:
        out = np.empty((M, N), dtype=np.float32)
    _bridge_call(_lib.skmetal_gemm, A, B, out, M, N, K, ctypes.c_float(alpha), ctypes.c_float(beta),
                 ctypes.c_int(int(trans_A)), ctypes.c_int(int(trans_B)), context=f"M={M} N={N} K={K}")
    return out


def device_info() -> dict:
    _require()
    name_buf = ctypes.create_string_buffer(256)
    max_threads = ctypes.c_size_t()
    unified = ctypes.c_uint8()
    working_set = ctypes.c_uint64()
    _check(_lib.skmetal_device_info(name_buf, 256, ctypes.byref(max_threads), ctypes.byref(unified),
                                    ctypes.byref(working_set)), "skmetal_device_info")
    return {
        "name": name_buf.value.decode("utf-8") if name_buf.value else "unknown",
        "max_threads_per_threadgroup": max_threads.value,
        "has_unified_memory": bool(unified.value),
        "recommended_working_set_size_bytes": working_set.value,
    }


# ---- additions ----

def kmeans_fit(X, centroids, labels, max_iter, tol_abs, strict=True):
    """Full sklearn-semantics Lloyd fit. centroids in/out, labels out.

    Returns (n_iter, inertia)."""
    _f32c(X, "X"), _f32c(centroids, "centroids"), _i32c(labels, "labels")
    ensure_warmed_up()
    n, d = X.shape
    k = centroids.shape[0]
    n_iter = ctypes.c_int32(0)
    inertia = ctypes.c_double(0.0)
    _check(_lib.skmetal_hip_kmeans_fit(X.ctypes.data, centroids.ctypes.data, labels.ctypes.data, n, d, k,
                                       int(max_iter), float(tol_abs), SKMETAL_FIT_STRICT if strict else 0,
                                       ctypes.byref(n_iter), ctypes.byref(inertia)), "skmetal_hip_kmeans_fit")
    return int(n_iter.value), float(inertia.value)


def plusplus_draws(random_state, n: int, k: int, n_local_trials: int | None = None, dtype=np.float32):
    """The random numbers scikit-learn's k-means++ takes from `random_state`, in its
    order (sklearn/cluster/_kmeans.py:225-243, unit sample weights of X's dtype):
    the first centre's row, ``choice(n, p=w / w.sum())``, then
    ``uniform(size=n_local_trials)`` for each further centre.  Drawing the k - 1
    uniform vectors at once consumes the generator exactly as k - 1 separate
    calls do.  Returns (n_local_trials, first_index, uniforms [(k-1) x T] float64)."""
    if n_local_trials is None:
        n_local_trials = 2 + int(np.log(k))
    w = np.ones(n, dtype=dtype)
    first = int(random_state.choice(n, p=w / w.sum()))
    u = np.ascontiguousarray(random_state.uniform(size=(k - 1) * n_local_trials), dtype=np.float64)
    return int(n_local_trials), first, u.reshape(k - 1, n_local_trials)


def kmeans_plusplus(X, n_clusters: int, random_state, n_local_trials: int | None = None):
    """k-means++ seeding of X (as given) on the GPU with scikit-learn's draws:
    returns (centers, indices) like sklearn.cluster.kmeans_plusplus (unit weights)."""
    _f32c(X, "X")
    ensure_warmed_up()
    n, d = X.shape
    T, first, u = plusplus_draws(random_state, n, n_clusters, n_local_trials, X.dtype)
    idx = np.empty(n_clusters, np.int64)
    _check(_lib.skmetal_hip_kmeans_plusplus(X.ctypes.data, n, d, n_clusters, T, first, u.ctypes.data,
                                            idx.ctypes.data), "skmetal_hip_kmeans_plusplus")
    return X[idx], idx


def column_variance(X):
    """numpy's float32 np.var(X, axis=0) bit for bit, in host threads (the
    library's; no device needed)."""
    _f32c(X, "X")
    if _lib is None:
        raise RuntimeError(f"{LIB_NAME} not loaded: {_load_error}")
    n, d = X.shape
    out = np.empty(d, np.float32)
    _check(_lib.skmetal_hip_column_variance(X.ctypes.data, n, d, out.ctypes.data), "skmetal_hip_column_variance")
    return out


def kmeans_transform(X, centroids):
    """Distances of every row of X to every centroid, [n x k] float32, as
    scikit-learn's KMeans.transform computes them (GPU)."""
    _f32c(X, "X"), _f32c(centroids, "centroids")
    ensure_warmed_up()
    n, d = X.shape
    k = centroids.shape[0]
    if centroids.shape[1] != d:
        raise ValueError(f"X has {d} features, centroids have {centroids.shape[1]}")
    out = np.empty((n, k), np.float32)
    _check(_lib.skmetal_hip_kmeans_transform(X.ctypes.data, centroids.ctypes.data, out.ctypes.data, n, d, k),
           "skmetal_hip_kmeans_transform")
    return out


class LloydHandle:
    """Device-resident Lloyd problem (X uploaded once, kept in HBM)."""

    def __init__(self, n: int, d: int, k: int):
        ensure_warmed_up()
        self.n, self.d, self.k = int(n), int(d), int(k)
        h = ctypes.c_void_p()
        _check(_lib.skmetal_hip_lloyd_create(self.n, self.d, self.k, ctypes.byref(h)), "skmetal_hip_lloyd_create")
        self._h = h

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.skmetal_hip_lloyd_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def load(self, X, center=True):
        _f32c(X, "X")
        assert X.shape == (self.n, self.d)
        _check(_lib.skmetal_hip_lloyd_load(self._h, X.ctypes.data, int(bool(center))), "skmetal_hip_lloyd_load")

    def set_centers(self, C):
        _f32c(C, "C")
        assert C.shape == (self.k, self.d)
        _check(_lib.skmetal_hip_lloyd_set_centers(self._h, C.ctypes.data), "skmetal_hip_lloyd_set_centers")

    def iterate(self, iters: int, kernel_times: bool = False):
        """Run `iters` fixed Lloyd steps; returns their time (ms), or with
        kernel_times (ms, (main, update, finalize)) where the second item holds
        the average per-step kernel times measured inside the same run."""
        ms = ctypes.c_float(0.0)
        km = (ctypes.c_float * 3)()
        _check(_lib.skmetal_hip_lloyd_iterate(self._h, int(iters), ctypes.byref(ms), km if kernel_times else None),
               "skmetal_hip_lloyd_iterate")
        if kernel_times:
            return float(ms.value), tuple(float(v) for v in km)
        return float(ms.value)

    def run(self, max_iter: int, tol_abs: float = 0.0, strict: bool = True):
        n_iter = ctypes.c_int32(0)
        inertia = ctypes.c_double(0.0)
        _check(_lib.skmetal_hip_lloyd_run(self._h, int(max_iter), float(tol_abs),
                                          SKMETAL_FIT_STRICT if strict else 0, ctypes.byref(n_iter),
                                          ctypes.byref(inertia)), "skmetal_hip_lloyd_run")
        return int(n_iter.value), float(inertia.value)

    def plusplus(self, random_state, n_local_trials: int | None = None):
        """Seed the centres with k-means++ on the loaded X, drawing from
        `random_state` as scikit-learn does; returns the chosen row indices."""
        T, first, u = plusplus_draws(random_state, self.n, self.k, n_local_trials)
        return self.plusplus_with(T, first, u)

    def plusplus_with(self, n_local_trials: int, first: int, uniforms):
        """k-means++ with given draws (first row, (k-1) x n_local_trials uniforms)."""
        u = np.ascontiguousarray(uniforms, dtype=np.float64)
        assert u.size == (self.k - 1) * n_local_trials
        idx = np.empty(self.k, np.int64)
        _check(_lib.skmetal_hip_lloyd_plusplus(self._h, int(n_local_trials), int(first), u.ctypes.data,
                                               idx.ctypes.data), "skmetal_hip_lloyd_plusplus")
        return idx

    def max_abs(self) -> float:
        """Largest |x| of the loaded X (NaN as +inf), measured on the device."""
        v = ctypes.c_float(0.0)
        _check(_lib.skmetal_hip_lloyd_max_abs(self._h, ctypes.byref(v)), "skmetal_hip_lloyd_max_abs")
        return float(v.value)

    def mindists(self, rows, reset: bool = False, download: bool = True):
        """k-means|| round: squared distance of every loaded row to its nearest
        candidate so far, lowered with the candidate rows `rows` (indices into X);
        reset starts from +inf.  Returns float32 [n] (None with download=False:
        the distances stay on the device for choice(weights="mindists"))."""
        r = np.ascontiguousarray(rows, dtype=np.int64).reshape(-1)
        out = np.empty(self.n, np.float32) if download else None
        _check(_lib.skmetal_hip_lloyd_mindists(self._h, r.ctypes.data if r.size else None, r.size, int(bool(reset)),
                                               out.ctypes.data if download else None), "skmetal_hip_lloyd_mindists")
        return out

    def choice(self, random_state, size: int, weights: str = "mindists", exact=False):
        """numpy's legacy ``random_state.choice(n, size, replace=False, p=w / w.sum())``
        on the device, for fp32 weights w: "mindists" = the k-means|| distances
        floored at 1e-30 (``np.maximum(dists, 1e-30)``), "unit" = ones.  Same
        rows, same draws taken from random_state, same errors.  The pass loop is
        numpy's: rand(size - found) uniforms, their rows, repeats dropped (first
        occurrence kept, in draw order), found rows zeroed, again until size rows.
        exact=True searches numpy's own cumsum for every draw; the default keeps
        the rows of a cumsum of another order where they provably agree;
        exact=2 gives that proof a margin of at least 1/(4n) (about half the
        draws take each search).  The count of draws searched exactly is kept in
        ``self.sample_exact``."""
        if weights not in ("mindists", "unit"):
            raise ValueError(f"weights={weights!r} is not 'mindists' or 'unit'")
        n = self.n
        size = int(size)
        psum = ctypes.c_double(0.0)
        nnz = ctypes.c_int64(0)
        _check(_lib.skmetal_hip_lloyd_sample_prepare(self._h, 0 if weights == "mindists" else 1, ctypes.byref(psum),
                                                     ctypes.byref(nnz)), "skmetal_hip_lloyd_sample_prepare")
        # numpy's checks, in numpy's order (fp32 p: atol = sqrt of fp32 epsilon)
        atol = max(np.sqrt(np.finfo(np.float64).eps), np.sqrt(np.finfo(np.float32).eps))
        if np.isnan(psum.value):
            raise ValueError("probabilities contain NaN")
        if abs(psum.value - 1.0) > atol:
            raise ValueError("probabilities do not sum to 1")
        if size > n:
            raise ValueError("Cannot take a larger sample than population when 'replace=False'")
        if size < 0:
            raise ValueError("negative dimensions are not allowed")
        if nnz.value < size:
            raise ValueError("Fewer non-zero entries in p than size")
        found = np.zeros(size, dtype=np.int64)
        n_uniq = 0
        n_exact = ctypes.c_int(0)
        self.sample_exact = 0
        while n_uniq < size:
            u = np.ascontiguousarray(random_state.rand(size - n_uniq), dtype=np.float64)
            rows = np.empty(u.size, dtype=np.int64)
            zero = found[:n_uniq]
            _check(_lib.skmetal_hip_lloyd_sample_draw(self._h, zero.ctypes.data if n_uniq else None, n_uniq,
                                                      u.ctypes.data, u.size, rows.ctypes.data, int(exact),
                                                      ctypes.byref(n_exact)), "skmetal_hip_lloyd_sample_draw")
            self.sample_exact += int(n_exact.value)
            _, first = np.unique(rows, return_index=True)
            first.sort()
            new = rows.take(first)
            found[n_uniq:n_uniq + new.size] = new
            n_uniq += new.size
        return found

    def info(self):
        fused = ctypes.c_int(0)
        partials = ctypes.c_int(0)
        _check(_lib.skmetal_hip_lloyd_info(self._h, ctypes.byref(fused), ctypes.byref(partials)),
               "skmetal_hip_lloyd_info")
        mode = int(fused.value)
        return dict(fused=bool(mode & 3), split=(mode & 3) == 2, asplit=bool(mode & 4), partials=int(partials.value))

    def centers(self):
        out = np.empty((self.k, self.d), np.float32)
        _check(_lib.skmetal_hip_lloyd_get_centers(self._h, out.ctypes.data), "skmetal_hip_lloyd_get_centers")
        return out

    def labels(self):
        out = np.empty(self.n, np.int32)
        _check(_lib.skmetal_hip_lloyd_get_labels(self._h, out.ctypes.data), "skmetal_hip_lloyd_get_labels")
        return out

    def inertia(self) -> float:
        v = ctypes.c_double(0.0)
        _check(_lib.skmetal_hip_lloyd_inertia(self._h, ctypes.byref(v)), "skmetal_hip_lloyd_inertia")
        return float(v.value)
