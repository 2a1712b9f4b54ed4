"""CPU checks of the arithmetic the split kernels rely on, and of the parity
rule that has to tell an fp32-accurate M-step from a narrower one.

The split kernels (k_fused3, k_assign3) write every fp32 value as three bf16
parts, each rounded to nearest (v_cvt_pk_bf16_f32):
    hi = bf16(x), mid = bf16(x - hi), lo = (x - hi) - mid.
Here the same rounding is restated in integer arithmetic on the fp32 bits and
the claims made for it are checked against what the mathematics fixes:
x = hi + mid + lo exactly, the parts' magnitude bounds, and the bound on the
three part products the E-step leaves out.  Then the per-column and
per-element centre checks of oracle/parity.py are shown to reject an M-step
built from two fp16 parts under one global 2^s scale (the arithmetic the split
replaced) on mixed-scale columns, and to accept the three-part bf16 sums.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import parity
from problems import mixed_scale_problem


def bf16_rn(x):
    """fp32 -> nearest bf16 (ties to even), returned as fp32 values."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def split3(x):
    x = np.asarray(x, dtype=np.float32)
    hi = bf16_rn(x)
    r = (x - hi).astype(np.float32)
    mid = bf16_rn(r)
    lo = (r - mid).astype(np.float32)
    return hi, mid, lo


def _is_bf16(v):
    return np.all((np.asarray(v, np.float32).view(np.uint32) & 0xFFFF) == 0)


def _wide_fp32(rng, n, emin=-100, emax=100):
    """Random fp32 values with random mantissas over a wide exponent range,
    plus the mantissa patterns where rounding to 8 bits ties or carries."""
    mant = rng.integers(0, 1 << 23, n, dtype=np.int64)
    expo = rng.integers(emin + 127, emax + 127, n, dtype=np.int64)
    sign = rng.integers(0, 2, n, dtype=np.int64)
    v = ((sign << 31) | (expo << 23) | mant).astype(np.uint32).view(np.float32)
    edge = np.array([1.0, -1.0, 1 + 2 ** -8, 1 + 2 ** -9, 1 + 3 * 2 ** -9, 2 - 2 ** -23, 1 + 2 ** -9 + 2 ** -23,
                     1 + 2 ** -17, 1 + 2 ** -8 + 2 ** -17, 1.9 * 2.0 ** 60, 2 ** -100, np.pi, -np.e], dtype=np.float32)
    return np.concatenate([v, edge])


def test_bf16_rounding_restated():
    """bf16_rn agrees with a rounding written from the definition: the nearest
    of the two neighbouring 8-bit-significand values, ties to the even one."""
    rng = np.random.default_rng(0)
    x = _wide_fp32(rng, 20000).astype(np.float64)
    e = np.floor(np.log2(np.abs(x)))
    ulp = 2.0 ** (e - 7)
    lo = np.floor(x / ulp) * ulp
    hi = lo + ulp
    dl, dh = x - lo, hi - x
    even_lo = (np.floor(x / ulp) % 2) == 0
    ref = np.where(dl < dh, lo, np.where(dh < dl, hi, np.where(even_lo, lo, hi)))
    np.testing.assert_array_equal(bf16_rn(x.astype(np.float32)).astype(np.float64), ref)


def test_three_part_split_is_exact():
    rng = np.random.default_rng(1)
    x = _wide_fp32(rng, 200000)
    hi, mid, lo = split3(x)
    assert _is_bf16(hi) and _is_bf16(mid) and _is_bf16(lo)
    total = hi.astype(np.float64) + mid.astype(np.float64) + lo.astype(np.float64)
    np.testing.assert_array_equal(total, x.astype(np.float64))
    ax = np.abs(x.astype(np.float64))
    assert np.all(np.abs(mid.astype(np.float64)) <= 2.0 ** -8 * ax)
    assert np.all(np.abs(lo.astype(np.float64)) <= 2.0 ** -16 * ax)


def test_two_bf16_parts_are_not_enough():
    """Planted mistake: a two-part split (hi + mid) leaves up to 2^-17 |x| out,
    so the exactness check above is not vacuous."""
    rng = np.random.default_rng(2)
    x = _wide_fp32(rng, 20000)
    hi, mid, _ = split3(x)
    assert np.any(hi.astype(np.float64) + mid.astype(np.float64) != x.astype(np.float64))


def test_left_out_products_bound():
    """The E-step keeps hh, hm, mh, hl, lh, mm: the other three part products
    total at most (2^-23 + 2^-32) |x_i c_i| for every feature."""
    rng = np.random.default_rng(3)
    x = _wide_fp32(rng, 100000, -40, 40)
    c = _wide_fp32(rng, 100000, -40, 40)
    xh, xm, xl = (p.astype(np.float64) for p in split3(x))
    ch, cm, cl = (p.astype(np.float64) for p in split3(c))
    left = xm * cl + xl * cm + xl * cl
    kept = xh * ch + xh * cm + xm * ch + xh * cl + xl * ch + xm * cm
    exact = x.astype(np.float64) * c.astype(np.float64)
    np.testing.assert_allclose(kept + left, exact, rtol=1e-15, atol=0)
    bound = (2.0 ** -23 + 2.0 ** -32) * np.abs(exact)
    assert np.all(np.abs(left) <= bound)
    # and the bound is attained to within a factor of 2 (not loose by orders)
    assert np.max(np.abs(left) / np.maximum(np.abs(exact), 1e-300)) > 2.0 ** -25


def _sums_three_part(Xc, lab, k):
    """Per-cluster sums of hi, mid and lo each in fp32 (in row order), added in
    fp64: the split M-step's arithmetic up to its fp32 summation order."""
    hi, mid, lo = split3(Xc)
    out = np.zeros((k, Xc.shape[1]))
    for part in (hi, mid, lo):
        s = np.zeros((k, Xc.shape[1]), np.float32)
        np.add.at(s, lab, part)
        out += s.astype(np.float64)
    return out


def _sums_fp16_global_scale(Xc, lab, k):
    """The arithmetic the split replaced: x scaled by one 2^s (so the largest
    |x| lands in [2^13, 2^14)), then hi = fp16(v), lo = fp16(v - hi) with fp16
    subnormals, the sums of hi + lo unscaled."""
    m = float(np.abs(Xc).max())
    e = np.frexp(m)[1]
    sh = 14 - e if (e > 14 or e < -2) else 0
    v = (Xc.astype(np.float64) * 2.0 ** sh).astype(np.float32)
    hi = v.astype(np.float16)
    lo = (v - hi.astype(np.float32)).astype(np.float16)
    out = np.zeros((k, Xc.shape[1]))
    np.add.at(out, lab, hi.astype(np.float64) + lo.astype(np.float64))
    return out * 2.0 ** -sh


@pytest.mark.parametrize("kind", ["quantised", "1e6", "cluster"])
def test_column_check_rejects_the_fp16_global_scale_split(kind):
    X, C0 = mixed_scale_problem(4000, 20, 9, seed=7, kind=kind)
    Xc = X - X.mean(axis=0) if kind != "cluster" else X
    lab = oracle.assign(Xc, C0 - (X.mean(axis=0) if kind != "cluster" else 0))
    k = C0.shape[0]
    cnt = np.bincount(lab, minlength=k)
    assert cnt.min() > 0
    ref = oracle.mstep(Xc, lab, C0)[0].astype(np.float64)
    good = (_sums_three_part(Xc, lab, k) / cnt[:, None]).astype(np.float32)
    bad = (_sums_fp16_global_scale(Xc, lab, k) / cnt[:, None]).astype(np.float32)
    assert parity.center_col_err(good, ref) <= 1e-6
    assert parity.center_member_err(good, ref, Xc, lab) <= 1e-6
    # the row-relative check alone cannot see the narrower arithmetic ...
    assert parity.center_rel_err(bad, ref) <= parity.CENTER_RTOL
    # ... the per-element check at the cluster's own scale does, at the fp32
    # level the mixed-scale GPU tests apply
    assert parity.center_member_err(bad, ref, Xc, lab) > parity.FP32_ELEM_RTOL
