"""CPU restatement of the reference ``sparse_attn`` oracle.

TEST INFRASTRUCTURE ONLY. This module is the checker for the HIP path and the
reported CPU baseline; nothing in the product imports it.

Reference being restated (read as text, never imported or run):

* ``track-01/reference/reference.py:24-40`` -- the formula and its order:
  gather rows ``kv[b, idx]`` (``:27-30``), fp32 ``einsum`` of q and the
  gathered rows times ``scale`` (``:32``), the per-head sink appended as an
  extra logit (``:34-35``), softmax over ``topk + 1`` (``:36``), the sink column
  dropped (``:38``), fp32 ``einsum`` with the gathered rows (``:39``) and a
  round-to-nearest-even cast to q's dtype (``:40``).
* ``track-01/requirements.md:92-114`` -- argument meaning (q/kv bf16, sink fp32
  per head, idx int32, ``o`` in q's dtype).
* ``track-01/submission.py:313-322`` -- the ``-1`` sentinel: such a slot gets
  score -inf and a zero row, i.e. it is removed from the row.  The frozen
  oracle itself raises on ``-1`` (``torch.gather`` rejects it), so this
  extension is pinned separately: a ``-1`` slot must equal the same row with
  the slot deleted, and an all-``-1`` row gives ``o = 0`` (the sink takes all
  the mass, the limit of ``reference.py:35-36``).
* Any other out-of-range index (``< -1`` or ``>= kv_len``) raises
  ``RuntimeError``, as ``torch.gather`` does at ``reference.py:28``.

Functions
---------
``sparse_attn_ref``        torch-CPU fp32, the reference's operation order,
                           chunked over m so that large configs fit in memory.
``sparse_attn_fp64``       NumPy float64, per-query compaction of valid slots.
``sparse_attn_bruteforce`` pure-Python scalar loops (tiny shapes only).
``masked_fold_fp64``       float64 split-topk partials (running max, sum,
                           unnormalised output) merged with the sink folded in
                           last, the algebra of ``track-01/notes.md:32-41``.
``sparse_attn_lse_fp64``   float64 ``(o, lse)``: ``lse = ln(sum_t exp(s_t) +
                           exp(sink))``, the ``m_total + ln(l_total)`` of
                           ``track-01/submission.py:195-199``.
``merge_fp64``             float64 merge of partial ``(o_i, lse_i)`` over
                           disjoint slot subsets with the sink folded once.
``sparse_attn_bruteforce_lse``  scalar-loop ``lse`` (tiny shapes only).

No-mass convention (outside the reference, whose softmax is 0/0 there): a
query with no valid slot and ``sink = -inf`` gives ``o = 0`` and
``lse = -inf``.

Parity status: every function here is pinned by ``tests/test_oracle.py``
(cross-checks between the three independent restatements, closed forms,
a textbook softmax-attention special case, invariances and planted mistakes).
"""
from __future__ import annotations

import math

import numpy as np
import torch

__all__ = [
    "sparse_attn_ref",
    "sparse_attn_fp64",
    "sparse_attn_bruteforce",
    "masked_fold_fp64",
    "sparse_attn_lse_fp64",
    "merge_fp64",
    "sparse_attn_bruteforce_lse",
    "check_indices",
]


def check_indices(topk_idxs: torch.Tensor, kv_len: int) -> None:
    """Raise like ``torch.gather`` would at ``reference.py:28`` for bad indices.

    ``-1`` is the padding sentinel of ``submission.py:313-322`` and is allowed.
    """
    idx = topk_idxs.long()
    bad = (idx < -1) | (idx >= kv_len)
    if bool(bad.any()):
        v = int(idx[bad].flatten()[0])
        raise RuntimeError(
            f"sparse_attn: index {v} is out of bounds for kv_len {kv_len}")


def sparse_attn_ref(q, kv, attn_sink, topk_idxs, scale, chunk: int | None = None):
    """torch-CPU restatement of ``reference.py:24-40`` with ``-1`` masking.

    Same arithmetic as the reference (fp32 einsum, softmax over topk+1, cast
    to q's dtype); the only addition is the ``-1`` mask, applied as -inf on
    the score and a (finite) clamped gather index whose weight is then 0.
    ``chunk`` bounds the m-slice processed at once; queries are independent so
    chunking does not change any value.
    """
    b, m, h, d = q.shape
    kv_len = kv.shape[1]
    topk = topk_idxs.shape[-1]
    check_indices(topk_idxs, kv_len)
    if kv_len == 0:  # every slot is -1 here; give gather one harmless row
        kv = torch.zeros(b, 1, d, dtype=kv.dtype)
    idx = topk_idxs.long()
    valid = idx != -1
    safe = idx.clamp(min=0)
    out = torch.empty(b, m, h, d, dtype=q.dtype)
    if b == 0 or m == 0:
        return out
    if chunk is None:
        # keep the gathered fp32 block near 512 MiB
        per_q = max(1, topk * d * 4 * 3)
        chunk = max(1, min(m, (512 << 20) // max(1, b * per_q)))
    sink = attn_sink.float()
    for m0 in range(0, m, chunk):
        m1 = min(m, m0 + chunk)
        mc = m1 - m0
        flat_idx = safe[:, m0:m1].reshape(b, mc * topk)
        gathered = torch.gather(
            kv, 1, flat_idx.unsqueeze(-1).expand(-1, -1, d)).reshape(b, mc, topk, d)
        gf = gathered.float()
        scores = torch.einsum("bmhd,bmtd->bmht", q[:, m0:m1].float(), gf) * scale
        scores = scores.masked_fill(~valid[:, m0:m1, None, :], float("-inf"))
        s = sink[None, None, :, None].expand(b, mc, h, 1)
        attn = torch.softmax(torch.cat([scores, s], dim=-1), dim=-1)
        o = torch.einsum("bmht,bmtd->bmhd", attn[..., :-1], gf)
        out[:, m0:m1] = o.to(q.dtype)
    return out


def _as_f64(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


def sparse_attn_fp64(q, kv, attn_sink, topk_idxs, scale) -> np.ndarray:
    """float64 NumPy restatement, computed per query on the compacted slots.

    Independent of ``sparse_attn_ref``'s route: it deletes ``-1`` slots
    instead of masking them, takes the max over scores and the sink
    explicitly, and never casts to bf16. Returns float64 ``[b, m, h, d]``.
    """
    qn = _as_f64(q)
    kvn = _as_f64(kv)
    sk = _as_f64(attn_sink)
    idx = np.asarray(topk_idxs.numpy() if isinstance(topk_idxs, torch.Tensor)
                     else topk_idxs, dtype=np.int64)
    b, m, h, d = qn.shape
    kv_len = kvn.shape[1]
    if ((idx < -1) | (idx >= kv_len)).any():
        raise RuntimeError("sparse_attn: index out of bounds")
    out = np.zeros((b, m, h, d), dtype=np.float64)
    for bi in range(b):
        for mi in range(m):
            rows = idx[bi, mi]
            rows = rows[rows != -1]
            K = kvn[bi, rows]                        # [n, d]
            s = (qn[bi, mi] @ K.T) * float(scale)    # [h, n]
            z = np.concatenate([s, sk[:, None]], axis=1)
            zmax = z.max(axis=1, keepdims=True)
            e = np.exp(z - zmax)
            w = e / e.sum(axis=1, keepdims=True)
            out[bi, mi] = w[:, :-1] @ K
    return out


def sparse_attn_bruteforce(q, kv, attn_sink, topk_idxs, scale) -> np.ndarray:
    """Scalar pure-Python loops over (b, m, h, slot, d). Tiny shapes only.

    Each valid slot contributes ``exp(s_t - M) * kv[row_t]`` to the numerator
    and ``exp(s_t - M)`` to the denominator; the sink adds ``exp(sink - M)`` to
    the denominator only (``reference.py:34-39``); ``M`` is the max over the
    valid scores and the sink.
    """
    qn = _as_f64(q).tolist()
    kvn = _as_f64(kv).tolist()
    sk = _as_f64(attn_sink).tolist()
    idx = (topk_idxs.tolist() if isinstance(topk_idxs, torch.Tensor)
           else np.asarray(topk_idxs).tolist())
    b = len(qn)
    m = len(qn[0]) if b else 0
    h = len(qn[0][0]) if m else 0
    d = len(qn[0][0][0]) if h else 0
    kv_len = len(kvn[0]) if b else 0
    out = np.zeros((b, m, h, d), dtype=np.float64)
    for bi in range(b):
        for mi in range(m):
            rows = []
            for r in idx[bi][mi]:
                if r == -1:
                    continue
                if r < -1 or r >= kv_len:
                    raise RuntimeError("sparse_attn: index out of bounds")
                rows.append(r)
            for hi in range(h):
                qv = qn[bi][mi][hi]
                scores = []
                for r in rows:
                    acc = 0.0
                    kr = kvn[bi][r]
                    for di in range(d):
                        acc += qv[di] * kr[di]
                    scores.append(acc * float(scale))
                mx = max(scores + [sk[hi]])
                ws = [math.exp(s - mx) for s in scores]
                den = sum(ws) + math.exp(sk[hi] - mx)
                for di in range(d):
                    num = 0.0
                    for w, r in zip(ws, rows):
                        num += w * kvn[bi][r][di]
                    out[bi, mi, hi, di] = num / den
    return out


def masked_fold_fp64(q, kv, attn_sink, topk_idxs, scale, nsplit: int) -> np.ndarray:
    """Split the topk axis into ``nsplit`` contiguous parts, keep per part the
    running max ``m_s``, sum ``l_s`` and unnormalised output ``O_s``, merge them
    with ``exp(m_s - M)`` weights and fold the sink in last
    (``track-01/notes.md:32-41``: ``m_tot = max(m, sink)``,
    ``l_tot = exp(m - m_tot) * l + exp(sink - m_tot)``,
    ``o = exp(m - m_tot) * O / l_tot``). A part with no valid slot carries
    ``m = -inf, l = 0, O = 0`` and weight 0. Returns float64 ``[b, m, h, d]``.
    """
    qn = _as_f64(q)
    kvn = _as_f64(kv)
    sk = _as_f64(attn_sink)
    idx = np.asarray(topk_idxs.numpy() if isinstance(topk_idxs, torch.Tensor)
                     else topk_idxs, dtype=np.int64)
    b, m, h, d = qn.shape
    topk = idx.shape[-1]
    per = -(-topk // nsplit) if topk else 0
    out = np.zeros((b, m, h, d), dtype=np.float64)
    for bi in range(b):
        for mi in range(m):
            ms, ls, Os = [], [], []
            for s in range(nsplit):
                rows = idx[bi, mi, s * per:(s + 1) * per]
                rows = rows[rows != -1]
                if rows.size == 0:
                    ms.append(np.full(h, -np.inf))
                    ls.append(np.zeros(h))
                    Os.append(np.zeros((h, d)))
                    continue
                K = kvn[bi, rows]
                sc = (qn[bi, mi] @ K.T) * float(scale)
                mx = sc.max(axis=1)
                e = np.exp(sc - mx[:, None])
                ms.append(mx)
                ls.append(e.sum(axis=1))
                Os.append(e @ K)
            M = np.max(np.stack(ms), axis=0)
            L = np.zeros(h)
            O = np.zeros((h, d))
            for mx, l, Ob in zip(ms, ls, Os):
                empty = np.isneginf(mx)
                w = np.where(empty, 0.0, np.exp(np.where(empty, 0.0, mx - np.where(empty, 0.0, M))))
                L += w * l
                O += w[:, None] * Ob
            m_tot = np.maximum(M, sk)
            a = np.where(np.isneginf(M), 0.0,
                         np.exp(np.where(np.isneginf(M), 0.0, M - m_tot)))
            l_tot = a * L + np.exp(sk - m_tot)
            out[bi, mi] = (a / l_tot)[:, None] * O
    return out


def sparse_attn_lse_fp64(q, kv, attn_sink, topk_idxs, scale):
    """float64 ``(o, lse)`` per query on the compacted slots.

    ``lse[b, m, h] = ln(sum_t exp(s_t) + exp(sink[h]))`` over the valid slots,
    computed as ``zmax + ln(sum exp(z - zmax))`` with ``z`` the scores and the
    sink; ``o`` is ``sparse_attn_fp64``'s. No mass (no slot, sink = -inf):
    ``o = 0``, ``lse = -inf``. Returns float64 ``[b, m, h, d]`` and ``[b, m, h]``.
    """
    qn = _as_f64(q)
    kvn = _as_f64(kv)
    sk = _as_f64(attn_sink)
    idx = np.asarray(topk_idxs.numpy() if isinstance(topk_idxs, torch.Tensor)
                     else topk_idxs, dtype=np.int64)
    b, m, h, d = qn.shape
    kv_len = kvn.shape[1]
    if ((idx < -1) | (idx >= kv_len)).any():
        raise RuntimeError("sparse_attn: index out of bounds")
    out = np.zeros((b, m, h, d), dtype=np.float64)
    lse = np.full((b, m, h), -np.inf, dtype=np.float64)
    for bi in range(b):
        for mi in range(m):
            rows = idx[bi, mi]
            rows = rows[rows != -1]
            K = kvn[bi, rows]                        # [n, d]
            s = (qn[bi, mi] @ K.T) * float(scale)    # [h, n]
            z = np.concatenate([s, sk[:, None]], axis=1)
            zmax = z.max(axis=1)
            live = ~np.isneginf(zmax)
            zm = np.where(live, zmax, 0.0)
            e = np.exp(z - zm[:, None])              # exp(-inf) = 0 for a -inf sink
            den = e.sum(axis=1)
            lse[bi, mi] = np.where(live, zm + np.log(np.where(live, den, 1.0)), -np.inf)
            w = e[:, :-1] / np.where(live, den, 1.0)[:, None]
            out[bi, mi] = np.where(live[:, None], w @ K, 0.0)
    return out, lse


def merge_fp64(o_parts, lse_parts, attn_sink=None):
    """float64 merge of partials ``o_parts [n, b, m, h, d]``, ``lse_parts
    [n, b, m, h]`` with the sink ``[h]`` (None: no sink) folded once:
    ``lse = ln(sum_i exp(lse_i) + exp(sink))``, ``o = sum_i exp(lse_i - lse) o_i``.
    A part with ``lse_i = -inf`` contributes nothing (its ``o_i`` is ignored).
    Returns float64 ``[b, m, h, d]`` and ``[b, m, h]``."""
    O = _as_f64(o_parts)
    L = _as_f64(lse_parts)
    n, b, m, h = L.shape
    terms = list(L)
    if attn_sink is not None:
        terms.append(np.broadcast_to(_as_f64(attn_sink), (b, m, h)))
    if not terms:
        return np.zeros(O.shape[1:] if O.ndim == 5 else (b, m, h, 0)), np.full((b, m, h), -np.inf)
    T = np.stack(terms)                              # [n(+1), b, m, h]
    mx = T.max(axis=0)
    live = ~np.isneginf(mx)
    mz = np.where(live, mx, 0.0)
    lse = np.where(live, mz + np.log(np.where(live, np.exp(T - mz).sum(axis=0), 1.0)),
                   -np.inf)
    out = np.zeros(O.shape[1:], dtype=np.float64)
    for i in range(n):
        li = L[i]
        use = live & ~np.isneginf(li)
        w = np.where(use, np.exp(np.where(use, li - np.where(live, lse, 0.0), 0.0)), 0.0)
        out += np.where(use[..., None], w[..., None] * O[i], 0.0)
    return out, lse


def sparse_attn_bruteforce_lse(q, kv, attn_sink, topk_idxs, scale) -> np.ndarray:
    """Scalar-loop ``lse[b, m, h] = ln(sum_t exp(s_t) + exp(sink[h]))`` with
    ``math.log`` / ``math.exp`` over an explicit max (tiny shapes only)."""
    qn = _as_f64(q).tolist()
    kvn = _as_f64(kv).tolist()
    sk = _as_f64(attn_sink).tolist()
    idx = (topk_idxs.tolist() if isinstance(topk_idxs, torch.Tensor)
           else np.asarray(topk_idxs).tolist())
    b = len(qn)
    m = len(qn[0]) if b else 0
    h = len(qn[0][0]) if m else 0
    d = len(qn[0][0][0]) if h else 0
    out = np.full((b, m, h), -np.inf, dtype=np.float64)
    for bi in range(b):
        for mi in range(m):
            rows = [r for r in idx[bi][mi] if r != -1]
            for hi in range(h):
                zs = []
                for r in rows:
                    zs.append(sum(qn[bi][mi][hi][di] * kvn[bi][r][di] for di in range(d))
                              * float(scale))
                zs.append(sk[hi])
                mx = max(zs)
                if mx == -math.inf:
                    continue
                out[bi, mi, hi] = mx + math.log(sum(math.exp(z - mx) for z in zs))
    return out
