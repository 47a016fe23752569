"""CPU checks that pin the track-02 oracle (``oracle/hc_sinkhorn_ref.py``).

The reference ships no golden vectors for ``hc_split_sinkhorn``: its only check
is a live comparison with the frozen PyTorch function
(``track-02/test_correctness.py:22-34``, atol 1e-5, rtol 1e-4). The oracle is
pinned here by what the mathematics fixes, chosen so that a plausible slip
(rows and columns swapped, a round too many or too few, eps in the wrong
place, the wrong slice of ``mixes``) fails at least one check:

* the vectorised float64 form equals an independently written scalar-loop
  form on random tokens;
* closed forms: with ``hc_scale = 0`` and a constant comb base every round
  maps the uniform entry ``x`` to ``x / (4x + eps)``, and pre / post are plain
  sigmoids of the base;
* the last operation is a column division: every column of the output sums to
  ``S / (S + eps)``, just below 1, for the pre-division column sum ``S``; with
  one round the rows sum to values far from 1;
* after the default 20 rounds the matrix is doubly stochastic to within a few
  eps, positive, and pre, post stay in their ranges;
* float32 stays within 1e-6 of float64 on the contest's input distribution.
"""
import math

import numpy as np
import pytest

from oracle.hc_sinkhorn_ref import hc_split_sinkhorn_loops, hc_split_sinkhorn_np

EPS = 1e-6


def inputs(n, seed, scale_std=1.0):
    g = np.random.default_rng(seed)
    mixes = g.standard_normal((n, 24))
    sc = g.standard_normal(3) * scale_std
    base = g.standard_normal(24)
    return mixes, sc, base


@pytest.mark.parametrize("iters", [0, 1, 2, 20])
def test_vectorised_equals_loops(iters):
    mixes, sc, base = inputs(16, seed=iters)
    pre, post, comb = hc_split_sinkhorn_np(mixes, sc, base, sinkhorn_iters=iters,
                                           dtype=np.float64)
    for t in range(16):
        p, q, c = hc_split_sinkhorn_loops(mixes[t], sc, base, sinkhorn_iters=iters)
        np.testing.assert_allclose(pre[t], p, rtol=1e-13, atol=0)
        np.testing.assert_allclose(post[t], q, rtol=1e-13, atol=0)
        np.testing.assert_allclose(comb[t], np.array(c), rtol=1e-12, atol=0)


@pytest.mark.parametrize("iters", [1, 2, 5, 20])
def test_closed_form_uniform(iters):
    mixes, _, base = inputs(3, seed=7)
    base[8:] = 0.37                      # constant comb base
    sc = np.zeros(3)
    pre, post, comb = hc_split_sinkhorn_np(mixes, sc, base, sinkhorn_iters=iters,
                                           dtype=np.float64)
    sig = lambda v: 1.0 / (1.0 + math.exp(-v))
    np.testing.assert_allclose(pre, np.tile([sig(v) + EPS for v in base[:4]], (3, 1)), rtol=1e-15)
    np.testing.assert_allclose(post, np.tile([2 * sig(v) for v in base[4:8]], (3, 1)), rtol=1e-15)
    x = 0.25 + EPS                       # softmax of a constant row, plus eps
    x = x / (4 * x + EPS)                # the first column division
    for _ in range(iters - 1):
        x = x / (4 * x + EPS)            # row division
        x = x / (4 * x + EPS)            # column division
    np.testing.assert_allclose(comb, np.full((3, 4, 4), x), rtol=1e-14)


def test_last_division_is_by_columns():
    """After a column division by S + eps every column sums to S / (S + eps):
    just below 1 (entries are at least eps / (1 + 5 eps), so S > 4e-6 and the
    sum exceeds 1 - 0.2). With one round the rows are left unnormalised."""
    mixes, sc, base = inputs(64, seed=3, scale_std=2.0)
    for iters in (1, 3):
        _, _, c = hc_split_sinkhorn_np(mixes, sc, base, sinkhorn_iters=iters, dtype=np.float64)
        colsum = c.sum(axis=-2)
        assert np.all(colsum < 1.0) and np.all(colsum > 0.8)
        if iters == 1:
            assert np.max(np.abs(c.sum(axis=-1) - 1.0)) > 1e-2


def test_doubly_stochastic_after_default_rounds():
    mixes, sc, base = inputs(256, seed=11)
    pre, post, comb = hc_split_sinkhorn_np(mixes, sc, base, dtype=np.float64)
    assert np.all(comb > 0)
    assert np.max(np.abs(comb.sum(axis=-1) - 1.0)) < 1e-4
    assert np.max(np.abs(comb.sum(axis=-2) - 1.0)) < 1e-5
    assert np.all(pre > EPS) and np.all(pre <= 1.0 + EPS)
    assert np.all(post > 0) and np.all(post < 2.0)


def test_slices_of_mixes():
    """pre reads mixes[:, :4], post mixes[:, 4:8], comb mixes[:, 8:] row-major:
    perturbing one input moves only its own output."""
    mixes, sc, base = inputs(1, seed=5)
    p0, q0, c0 = hc_split_sinkhorn_np(mixes, sc, base, dtype=np.float64)
    for k, (dp, dq, dc) in {2: (True, False, False), 6: (False, True, False),
                            8 + 4 * 2 + 1: (False, False, True)}.items():
        m = mixes.copy()
        m[0, k] += 0.5
        p, q, c = hc_split_sinkhorn_np(m, sc, base, dtype=np.float64)
        assert (not np.array_equal(p, p0)) == dp
        assert (not np.array_equal(q, q0)) == dq
        assert (not np.array_equal(c, c0)) == dc
        if dp:
            assert np.flatnonzero(p[0] != p0[0]).tolist() == [2]
        if dq:
            assert np.flatnonzero(q[0] != q0[0]).tolist() == [2]


def test_float32_close_to_float64():
    mixes, sc, base = inputs(4096, seed=13)
    r32 = hc_split_sinkhorn_np(mixes.astype(np.float32), sc.astype(np.float32),
                               base.astype(np.float32))
    r64 = hc_split_sinkhorn_np(mixes.astype(np.float32).astype(np.float64),
                               sc.astype(np.float32).astype(np.float64),
                               base.astype(np.float32).astype(np.float64), dtype=np.float64)
    for a, b in zip(r32, r64):
        assert a.dtype == np.float32
        assert np.max(np.abs(a - b)) < 1e-6
