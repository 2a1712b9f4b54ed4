"""Parity rules for the KMeans Lloyd path -- TEST INFRASTRUCTURE ONLY.

The acceptance rule compared against the oracle (and against sklearn's own
outputs in the golden fixtures):

* labels  -- identical, except rows whose oracle best-vs-second squared
             distance gap is below ``LABEL_GAP_REL * ||x||^2`` (x in the
             coordinates the distances were evaluated in);
* centres -- three checks, each at CENTER_RTOL:
             per centre row j: max_c |a_jc - b_jc| / max_c |b_jc|;
             per column c: max_j |a_jc - b_jc| / max_j |b_jc| (a column whose
             values are far smaller than the others' is held to its own scale);
             per element, in a lockstep step: |a_jc - b_jc| / mean |x_ic| over
             the rows i of cluster j (the scale an fp32 sum of those rows works
             at, so a cluster whose values in a column are far smaller than
             other clusters' is held to its own scale too);
* inertia -- |a - b| <= INERTIA_RTOL * |b| against an fp64 recomputation.
"""

from __future__ import annotations

import numpy as np

LABEL_GAP_REL = 1e-5
CENTER_RTOL = 1e-4
INERTIA_RTOL = 1e-5
# per-element centre error, relative to the cluster's own mean |x|, that fp32
# sums over chains of up to a few hundred rows stay within (used where the
# arithmetic itself is under test: columns and clusters of mixed scales)
FP32_ELEM_RTOL = 1e-5


def label_mismatches(labels, ref_labels, best, second, X, gap_rel=LABEL_GAP_REL):
    """Return (n_mismatch, n_unexcused, idx_unexcused)."""
    labels = np.asarray(labels).astype(np.int64)
    ref_labels = np.asarray(ref_labels).astype(np.int64)
    mism = np.flatnonzero(labels != ref_labels)
    if mism.size == 0:
        return 0, 0, mism
    Xm = np.asarray(X, dtype=np.float64)[mism]
    xx = (Xm * Xm).sum(1)
    gap = np.asarray(second, dtype=np.float64)[mism] - np.asarray(best, dtype=np.float64)[mism]
    bad = mism[gap >= gap_rel * np.maximum(xx, 1e-300)]
    return int(mism.size), int(bad.size), bad


def check_labels(labels, ref_labels, best, second, X, gap_rel=LABEL_GAP_REL, what="labels"):
    n_m, n_bad, bad = label_mismatches(labels, ref_labels, best, second, X, gap_rel)
    assert n_bad == 0, (
        f"{what}: {n_bad} of {n_m} mismatching rows are not near-ties "
        f"(first rows {bad[:8].tolist()})"
    )
    return n_m


def center_rel_err(C, C_ref):
    C = np.asarray(C, dtype=np.float64)
    R = np.asarray(C_ref, dtype=np.float64)
    num = np.abs(C - R).max(axis=1)
    den = np.maximum(np.abs(R).max(axis=1), 1e-30)
    return float((num / den).max())


def center_col_err(C, C_ref):
    """max over columns c of max_j |C_jc - R_jc| / max_j |R_jc|."""
    C = np.asarray(C, dtype=np.float64)
    R = np.asarray(C_ref, dtype=np.float64)
    floor = max(float(np.abs(R).max(initial=0.0)) * 1e-30, 1e-300)
    num = np.abs(C - R).max(axis=0)
    den = np.maximum(np.abs(R).max(axis=0), floor)
    return float((num / den).max())


def center_member_err(C, C_ref, X, labels):
    """max over (j, c) of |C_jc - R_jc| / mean_{i in cluster j} |x_ic|, over the
    clusters that have rows in `labels`."""
    from scipy import sparse

    C = np.asarray(C, dtype=np.float64)
    R = np.asarray(C_ref, dtype=np.float64)
    X = np.asarray(X)
    lab = np.asarray(labels, dtype=np.int64)
    k = R.shape[0]
    cnt = np.bincount(lab, minlength=k).astype(np.float64)
    absum = np.zeros_like(R)
    xmax = 0.0
    step = 1 << 18
    for s0 in range(0, len(lab), step):
        lb = lab[s0:s0 + step]
        blk = np.abs(X[s0:s0 + step])
        xmax = max(xmax, float(blk.max(initial=0.0)))
        onehot = sparse.csr_matrix((np.ones(len(lb), np.float64), (lb, np.arange(len(lb)))), shape=(k, len(lb)))
        absum += onehot @ blk.astype(np.float64)
    has = cnt > 0
    if not has.any():
        return 0.0
    scale = absum[has] / cnt[has, None]
    floor = max(xmax * 1e-30, 1e-300)
    return float((np.abs(C[has] - R[has]) / np.maximum(scale, floor)).max())


def check_centers(C, C_ref, rtol=CENTER_RTOL, what="centers"):
    err = center_rel_err(C, C_ref)
    assert err <= rtol, f"{what}: max row-relative error {err:.3e} > {rtol:.1e}"
    col = center_col_err(C, C_ref)
    assert col <= rtol, f"{what}: max per-column error {col:.3e} > {rtol:.1e}"
    return max(err, col)


def centring_floor(X) -> float:
    """Absolute inertia floor from fp32 centring: each element of X - mean carries
    a rounding error up to eps*|x|, so two implementations that centre with
    means differing in the last bit may differ by about n*d*(eps*max|x|)^2 even
    when the true inertia is zero (all points on their centres)."""
    X = np.asarray(X)
    eps = float(np.finfo(np.float32).eps)
    return 4.0 * X.size * (eps * float(np.abs(X).max(initial=0.0))) ** 2


def check_inertia(v, ref, rtol=INERTIA_RTOL, atol=0.0, what="inertia"):
    diff = abs(float(v) - float(ref))
    err = diff / max(abs(float(ref)), 1e-300)
    assert diff <= rtol * abs(float(ref)) + atol, (
        f"{what}: relative error {err:.3e} > {rtol:.1e} ({v} vs {ref}, atol {atol:.1e})")
    return err


def near_ties(best, second, X, gap_rel=LABEL_GAP_REL):
    """Rows whose best-vs-second gap is below gap_rel * ||x||^2."""
    Xd = np.asarray(X, dtype=np.float64)
    xx = (Xd * Xd).sum(1)
    gap = np.asarray(second, dtype=np.float64) - np.asarray(best, dtype=np.float64)
    return np.flatnonzero(gap < gap_rel * np.maximum(xx, 1e-300))


def _match_relocated(C, C_ref, rows):
    """C with the given rows best-matched (greedily) to those of C_ref."""
    C = np.asarray(C, dtype=np.float64).copy()
    R = np.asarray(C_ref, dtype=np.float64)
    rows = list(rows)
    free = list(rows)
    for r in rows:
        errs = [np.abs(C[f] - R[r]).max() for f in free]
        f = free.pop(int(np.argmin(errs)))
        C[r], C[f] = C[f].copy(), C[r].copy()
    return C


def check_lockstep(X, C_prev, C_next_ref, labels_ref, rtol=CENTER_RTOL, what="step", elem_rtol=None):
    """One Lloyd step from C_prev checked against a reference step.

    X and C_prev are in the coordinates the step runs in; labels_ref and
    C_next_ref are the reference's E-step labels and M-step centres for that
    step.  Labels must agree with the oracle's E-step up to near-ties; the
    oracle's M-step applied to labels_ref must reproduce C_next_ref.  When
    three or more clusters were empty, the reference may hand the relocated
    points to the empty clusters in a different order, so those rows are
    compared as a set.  elem_rtol (default rtol) bounds the per-element error
    at the cluster's own scale.  Returns the number of label mismatches.
    """
    import oracle

    labels, best, second = oracle.assign(X, C_prev, return_gap=True)
    n_m = check_labels(labels_ref, labels, best, second, X, what=f"{what} labels")
    C_new, _, n_empty = oracle.mstep(X, labels_ref, C_prev)
    C_got = np.asarray(C_next_ref, dtype=np.float64)
    err = center_rel_err(C_new, C_got)
    if err > rtol and n_empty >= 3:
        counts = np.bincount(np.asarray(labels_ref, dtype=np.int64), minlength=len(C_prev))
        C_got = _match_relocated(C_got, C_new, np.flatnonzero(counts == 0))
        err = center_rel_err(C_new, C_got)
    assert err <= rtol, f"{what}: centres row-relative error {err:.3e} > {rtol:.1e}"
    col = center_col_err(C_got, C_new)
    assert col <= rtol, f"{what}: centres per-column error {col:.3e} > {rtol:.1e}"
    mem = center_member_err(C_got, C_new, X, labels_ref)
    er = rtol if elem_rtol is None else elem_rtol
    assert mem <= er, f"{what}: centres per-element error (cluster scale) {mem:.3e} > {er:.1e}"
    return n_m
