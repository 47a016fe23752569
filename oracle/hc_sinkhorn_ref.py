"""CPU restatement of the reference ``hc_split_sinkhorn`` oracle (track 02).

TEST INFRASTRUCTURE ONLY. This module is the checker for the HIP path and the
reported CPU baseline; nothing in the product imports it.

Reference being restated (read as text, never imported or run):

* ``track-02/reference/reference.py:38-51`` -- the formula and its order:
  ``mixes`` is split into ``pre_raw = [..., :hc]``, ``post_raw = [...,
  hc:2hc]`` and ``comb_raw = [..., 2hc:]`` read row-major as ``[hc, hc]``
  (``:38-40``); ``pre = sigmoid(pre_raw * hc_scale[0] + hc_base[:hc]) + eps``
  (``:42``); ``post = 2 * sigmoid(post_raw * hc_scale[1] + hc_base[hc:2hc])``
  (``:43``); ``comb = comb_raw * hc_scale[2] + hc_base[2hc:]`` (``:44``), a
  softmax over the last axis (each row) plus ``eps`` (``:46``), one division
  of every column by its sum plus ``eps`` (``:47``), then ``sinkhorn_iters -
  1`` rounds of a row division followed by a column division, each by the
  sum plus ``eps`` (``:49-51``). A count below 1 runs no round (Python's
  ``range`` of a negative number is empty).
* ``track-02/requirements.md`` ("计算逻辑") -- the same, in words; inputs and
  outputs are fp32; ``hc_mult = 4``, ``sinkhorn_iters = 20``, ``eps = 1e-6``
  in the model.
* ``track-02/submission.py:340-346`` -- the drop-in accepts 3-D ``mixes`` with
  ``hc_mult = 4`` only (last dim 24).

Functions
---------
``hc_split_sinkhorn_np``     NumPy in the given float type (float32 follows
                             the reference's fp32 arithmetic op for op;
                             float64 is the accuracy reference).
``hc_split_sinkhorn_loops``  pure-Python scalar loops on one token, float64
                             (``math.exp``), for brute-force checks.
"""
from __future__ import annotations

import math

import numpy as np


def _sigmoid(x):
    with np.errstate(over="ignore"):  # exp(-x) = inf for very negative x: sigmoid 0
        return 1.0 / (1.0 + np.exp(-x))


def hc_split_sinkhorn_np(mixes, hc_scale, hc_base, hc_mult=4, sinkhorn_iters=20, eps=1e-6,
                         dtype=np.float32):
    """``reference.py:38-51`` on NumPy arrays of ``dtype``.

    mixes ``[..., (2 + hc) * hc]``, hc_scale ``[3]``, hc_base ``[(2 + hc) * hc]``.
    Returns ``(pre [..., hc], post [..., hc], comb [..., hc, hc])``.
    """
    hc = int(hc_mult)
    x = np.asarray(mixes, dtype=dtype)
    sc = np.asarray(hc_scale, dtype=dtype)
    base = np.asarray(hc_base, dtype=dtype)
    e = dtype(eps)
    lead = x.shape[:-1]
    pre = _sigmoid(x[..., :hc] * sc[0] + base[:hc]) + e                     # :42
    post = dtype(2) * _sigmoid(x[..., hc:2 * hc] * sc[1] + base[hc:2 * hc])  # :43
    comb = (x[..., 2 * hc:].reshape(*lead, hc, hc) * sc[2]
            + base[2 * hc:].reshape(hc, hc))                                 # :44
    comb = np.exp(comb - comb.max(axis=-1, keepdims=True))                  # :46 softmax(dim=-1)
    comb = comb / comb.sum(axis=-1, keepdims=True) + e
    comb = comb / (comb.sum(axis=-2, keepdims=True) + e)                    # :47
    for _ in range(sinkhorn_iters - 1):                                      # :49-51
        comb = comb / (comb.sum(axis=-1, keepdims=True) + e)
        comb = comb / (comb.sum(axis=-2, keepdims=True) + e)
    return pre.astype(dtype), post.astype(dtype), comb.astype(dtype)


def hc_split_sinkhorn_loops(mix, hc_scale, hc_base, hc_mult=4, sinkhorn_iters=20, eps=1e-6):
    """One token (``mix`` of length ``(2 + hc) * hc``) with explicit indices:
    ``comb[i][j] = mix[2hc + hc*i + j]``; a row is fixed ``i`` (the softmax
    and row-normalisation axis, ``dim=-1``), a column fixed ``j``."""
    hc = int(hc_mult)
    mix = [float(v) for v in mix]
    s = [float(v) for v in hc_scale]
    b = [float(v) for v in hc_base]
    sig = lambda v: 1.0 / (1.0 + math.exp(-v))
    pre = [sig(mix[k] * s[0] + b[k]) + eps for k in range(hc)]
    post = [2.0 * sig(mix[hc + k] * s[1] + b[hc + k]) for k in range(hc)]
    c = [[mix[2 * hc + hc * i + j] * s[2] + b[2 * hc + hc * i + j] for j in range(hc)]
         for i in range(hc)]
    for i in range(hc):
        mx = max(c[i])
        ex = [math.exp(c[i][j] - mx) for j in range(hc)]
        tot = sum(ex)
        c[i] = [ex[j] / tot + eps for j in range(hc)]

    def cols():
        for j in range(hc):
            tot = sum(c[i][j] for i in range(hc)) + eps
            for i in range(hc):
                c[i][j] = c[i][j] / tot

    def rows():
        for i in range(hc):
            tot = sum(c[i]) + eps
            c[i] = [v / tot for v in c[i]]

    cols()
    for _ in range(sinkhorn_iters - 1):
        rows()
        cols()
    return pre, post, c
