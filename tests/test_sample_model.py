"""CPU: the arithmetic that the device sampler (skmetal_amd/csrc/sample_kernels.hip)
reproduces, checked against numpy itself.

numpy's legacy RandomState.choice(n, size, replace=False, p=w / w.sum()) is the
oracle of the k-means|| draws (skmetal/estimators/cluster.py:94-98) and of
scikit-learn's init="random" (sklearn/cluster/_kmeans.py:1010-1013).  The
kernels restate three facts about it, each pinned here on numpy's own outputs:

* w.sum() of a contiguous fp32 array is a running total over 8192-element
  blocks, each summed pairwise (leaves of <= 128 on eight accumulators, halves
  split at a multiple of 8) -- a wrong leaf size, split rule or block length
  changes the sum on some of these arrays;
* choice's passes: rand(size - found) uniforms, searchsorted(cumsum(p) /
  cumsum(p)[-1], u, "right"), first occurrences kept in draw order, found rows'
  p zeroed, until size rows;
* the certified search's error bound: any order of adding non-negative terms
  whose every term passes through at most h roundings is within gamma_h of the
  exact sum relative to the total, so a tree-order prefix and numpy's
  sequential cumsum differ by at most 2 gamma_n of the total;
* the exact search's cumsum: numpy's sequential fp64 cumsum rebuilt chunk by
  chunk from exact integer sums on the running sum's binade grid.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

F32 = np.float32


def _half(length):
    h = length // 2
    return h - h % 8


def _pairwise(a, leaf=128):
    n = len(a)
    if n < 8:
        r = F32(0.0)
        for v in a:
            r = F32(r + v)
        return r
    if n <= leaf:
        r = [a[j] for j in range(8)]
        i = 8
        while i < n - n % 8:
            for j in range(8):
                r[j] = F32(r[j] + a[i + j])
            i += 8
        res = F32(F32(F32(r[0] + r[1]) + F32(r[2] + r[3])) + F32(F32(r[4] + r[5]) + F32(r[6] + r[7])))
        for v in a[i:]:
            res = F32(res + v)
        return res
    h = _half(n)
    return F32(_pairwise(a[:h], leaf) + _pairwise(a[h:], leaf))


def _numpy_sum_model(a, block=8192, leaf=128):
    r = F32(0.0)
    for b in range(0, len(a), block):
        r = F32(r + _pairwise(a[b:b + block], leaf))
    return r


@pytest.mark.parametrize("n", [1, 7, 8, 9, 127, 128, 129, 1000, 8191, 8192, 8193, 16385, 24577, 70001])
def test_fp32_sum_order_is_numpys(n):
    rng = np.random.default_rng(n)
    for t in range(3):
        a = (rng.random(n) ** (1 + 5 * t) * 10.0 ** rng.integers(-8, 8)).astype(np.float32)
        assert _numpy_sum_model(a) == a.sum()


def test_sum_model_discriminates():
    # each planted variant differs from numpy on at least one of these arrays:
    # a plain running sum, pairwise without the 8192 blocks, 64-weight leaves,
    # 4096-element blocks
    rng = np.random.default_rng(7)
    arrays = [(rng.random(n) ** 4 * 1e3).astype(np.float32) for n in (20001, 70001, 100003)]

    def running(a):
        r = F32(0.0)
        for v in a:
            r = F32(r + v)
        return r

    for variant in (running, _pairwise, lambda a: _numpy_sum_model(a, leaf=64),
                    lambda a: _numpy_sum_model(a, block=4096)):
        assert any(variant(a) != a.sum() for a in arrays)


def _choice_model(rs, n, size, p):
    p = np.array(p, dtype=np.float64)
    found = np.zeros(size, dtype=np.int64)
    n_uniq = 0
    while n_uniq < size:
        u = rs.rand(size - n_uniq)
        if n_uniq > 0:
            p[found[:n_uniq]] = 0
        cdf = np.cumsum(p)
        cdf /= cdf[-1]
        new = cdf.searchsorted(u, side="right")
        _, first = np.unique(new, return_index=True)
        first.sort()
        new = new.take(first)
        found[n_uniq:n_uniq + new.size] = new
        n_uniq += new.size
    return found


def test_choice_passes_are_numpys():
    # peaked weights (up to the 30th power) repeat rows and force further passes
    for seed in range(200):
        g = np.random.default_rng(seed)
        n = int(g.integers(2, 3000))
        size = int(g.integers(1, min(n, 60) + 1))
        w = np.maximum((g.random(n) ** g.integers(1, 30)).astype(np.float32), 1e-30)
        p = w / w.sum()
        if np.count_nonzero(p > 0) < size:
            continue
        r1, r2 = np.random.RandomState(seed), np.random.RandomState(seed)
        assert np.array_equal(r1.choice(n, size=size, p=p, replace=False), _choice_model(r2, n, size, p))
        assert r1.rand() == r2.rand()


def test_tree_prefix_within_bound_of_numpy_cumsum():
    # numpy's sequential cumsum against a chunked tree-order prefix (2048-row
    # chunks, running chunk totals, per-chunk scans): the gap stays inside
    # 2 gamma_{n + nc + 64} of the total, the bound the certified search uses
    u = 2.0**-53
    for seed, n in [(0, 5000), (1, 100_000), (2, 300_000)]:
        g = np.random.default_rng(seed)
        w = np.maximum((g.random(n) ** g.integers(1, 8)).astype(np.float32), 1e-30)
        p = (w / w.sum()).astype(np.float64)
        seq = np.cumsum(p)
        nc = -(-n // 2048)
        chunks = p.reshape(-1) if n % 2048 == 0 else np.concatenate([p, np.zeros(nc * 2048 - n)])
        chunks = chunks.reshape(nc, 2048)
        tot = chunks.sum(axis=1)
        pfx = np.concatenate([[0.0], np.cumsum(tot)])
        tree = (pfx[:-1, None] + np.cumsum(chunks, axis=1)).reshape(-1)[:n]
        h = n + nc + 64
        gam = h * u / (1 - h * u)
        T = pfx[-1]
        bound = 2 * gam * T / (1 - gam)
        assert np.max(np.abs(tree - seq)) <= bound
        # the bound is not vacuous: it is far below the smallest cdf step a
        # draw would have to fall between
        assert bound < 1e-9


def _grid_q(v, e):
    w = math.ldexp(v, 52 - e)
    if w >= 2.0**52:
        return None
    fl = math.floor(w)
    fr = w - fl
    if fr == 0.5:
        return None
    return int(fl) + (1 if fr > 0.5 else 0)


def _chunked_cumsum(p, ch=2048):
    """The exact search's cumsum: per chunk, while the running sum s stays in
    one binade [2^e, 2^(e+1)), fl(s + p) = s + 2^(e-52) RN(p / 2^(e-52)), so
    the chunk's sums are s plus an exact integer prefix on that grid; a chunk
    that starts at 0, leaves the binade or holds a tie (p / grid ending in
    exactly .5) is added in row order instead."""
    out = np.empty(len(p))
    s, walked = 0.0, 0
    for c0 in range(0, len(p), ch):
        chunk = [float(v) for v in p[c0:c0 + ch]]
        qs = None
        if s > 0.0:
            e = math.frexp(s)[1] - 1
            qs = [_grid_q(v, e) for v in chunk]
            if any(q is None for q in qs) or sum(qs) >= 2**53 or s + math.ldexp(float(sum(qs)), e - 52) >= 2.0**(e + 1):
                qs = None
        if qs is None:
            walked += 1
            r = s
            for i, v in enumerate(chunk):
                r = r + v
                out[c0 + i] = r
        else:
            acc = 0
            for i, q in enumerate(qs):
                acc += q
                out[c0 + i] = s + math.ldexp(float(acc), e - 52)
        s = out[c0 + len(chunk) - 1]
    return out, walked


def test_chunked_cumsum_is_numpys():
    # uniform, widely spread, a few dominant and many zero probabilities: the
    # grid sums and the walked chunks both give numpy's cumsum bit for bit, and
    # both kinds of chunk occur
    rng = np.random.default_rng(3)
    walked = chunks = 0
    for kind in range(4):
        n = 20_000 + 977 * kind
        if kind == 0:
            w = np.ones(n, np.float32)
        elif kind == 1:
            w = np.maximum((rng.random(n) ** 9).astype(np.float32), np.float32(1e-30))
        elif kind == 2:
            w = np.maximum((rng.random(n) * 1e-3).astype(np.float32), np.float32(1e-30))
            w[rng.integers(0, n, 5)] = 1e3
        else:
            w = rng.exponential(1.0, n).astype(np.float32)
            w[rng.choice(n, n // 3)] = 0.0
        p = (w / w.sum()).astype(np.float64)
        got, wk = _chunked_cumsum(p)
        assert np.array_equal(got, np.cumsum(p))
        walked += wk
        chunks += -(-n // 2048)
    assert 0 < walked < chunks
