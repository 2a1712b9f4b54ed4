"""skmetal_hip_kmeans_batch_fused_noalloc through the C ABI against
skmetal_kmeans_batch_fused, on device buffers the test allocates itself.

The no-allocation entry point runs skmetal's loop contract on X as given;
skmetal_kmeans_batch_fused runs it on X centred on its column mean.  On
well-separated blobs with one initial centre per blob there are no near-ties,
so both give the same labels exactly, the same n_iter and centres within the
parity tolerance.  Two calls in a row, the second smaller, share the scratch
array; a last check covers the size limits.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import parity

pytestmark = pytest.mark.gpu


def _hip():
    for name in ("libamdhip64.so.7", "libamdhip64.so.6", "libamdhip64.so"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    pytest.fail("libamdhip64 not found")


class _Dev:
    """A device buffer holding a copy of a numpy array."""

    def __init__(self, hip, a):
        self.hip, self.nbytes = hip, a.nbytes
        self.ptr = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(a.nbytes)) == 0
        assert hip.hipMemcpy(self.ptr, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) == 0

    def get(self, like):
        out = np.empty_like(like)
        assert self.hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, ctypes.c_size_t(self.nbytes), 2) == 0
        return out

    def free(self):
        self.hip.hipFree(self.ptr)


def _blobs(n, d, k, seed):
    rng = np.random.default_rng(seed)
    cen = rng.uniform(-10, 10, (k, d))
    ids = rng.integers(0, k, n)
    X = (cen[ids] + rng.standard_normal((n, d))).astype(np.float32)
    C0 = np.stack([X[np.flatnonzero(ids == j)[0]] for j in range(k)])
    return X, C0


def _noalloc(lib, hip, X, C0, max_iter, tol):
    n, d = X.shape
    k = C0.shape[0]
    dX, dC, dL = _Dev(hip, X), _Dev(hip, C0), _Dev(hip, np.full(n, -7, np.int32))
    it = ctypes.c_int32(-1)
    try:
        rc = lib.skmetal_hip_kmeans_batch_fused_noalloc(dX.ptr, dC.ptr, dL.ptr, n, d, k, max_iter,
                                                         ctypes.c_float(tol), ctypes.byref(it))
        assert rc == 0, lib.skmetal_hip_last_error().decode()
        return dC.get(C0), dL.get(np.empty(n, np.int32)), it.value
    finally:
        for b in (dX, dC, dL):
            b.free()


def test_noalloc_matches_batch_fused_twice():
    from skmetal_amd import _bridge

    if not _bridge.HIP_AVAILABLE:
        pytest.fail(f"GPU path unavailable on a GPU run: {_bridge.last_error()}")
    lib = _bridge._lib
    hip = _hip()
    for (n, d, k, max_iter, tol) in [(400000, 100, 50, 20, 1e-4), (30000, 48, 20, 3, 0.0)]:
        print(f"no-alloc vs batch_fused n={n} d={d} k={k}", flush=True)
        X, C0 = _blobs(n, d, k, seed=n + d)
        C_ref = C0.copy()
        lab_ref = np.empty(n, np.int32)
        it_ref = _bridge.kmeans_batch_fused(X, C_ref, lab_ref, n, d, k, (n + 255) // 256, max_iter, tol)
        C, lab, it = _noalloc(lib, hip, X, C0, max_iter, tol)
        assert it == it_ref
        np.testing.assert_array_equal(lab, lab_ref)
        parity.check_centers(C, C_ref, what=f"no-alloc centres n={n}")


def test_noalloc_limits():
    from skmetal_amd import _bridge

    lib = _bridge._lib
    dummy = ctypes.c_void_p(16)  # never dereferenced: every case below is rejected first
    it = ctypes.c_int32(0)
    for (n, d, k) in [(1000, 33, 8), (1000, 100, 65), ((1 << 22) + 1, 32, 8)]:
        rc = lib.skmetal_hip_kmeans_batch_fused_noalloc(dummy, dummy, dummy, n, d, k, 5, ctypes.c_float(0.0),
                                                         ctypes.byref(it))
        assert rc != 0
        assert "this entry point takes" in lib.skmetal_hip_last_error().decode()
