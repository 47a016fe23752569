"""CPU restatement of the reference ``fused_moe`` oracle (track 03).

TEST INFRASTRUCTURE ONLY. This module is the checker for the HIP path and the
reported CPU baseline; nothing in the product imports it.

Reference being restated (read as text, never imported or run):

* ``track-03/reference/reference.py:10-35`` -- the formula and its order:
  routing weights ``score.softmax(dim=-1, dtype=float32)`` (``:16``), the
  ``topk`` largest with their expert ids (``:17``), optionally divided by
  their sum (``:18-19``), then cast to the input dtype, bf16 (``:20``). The
  output starts as bf16 zeros (``:22``) and, for expert 0, 1, ..., E-1 in
  that order (``:24``), gets ``+= x * token_weight`` (``:35``) where
  ``x = linear(hidden, w1[e])`` (``:28``, bf16 out), ``gate = silu(x[:, :N])``
  (``:29``, the FIRST N rows of w1 are the gate), ``x = x[:, N:] * gate``
  (``:30``, the last N rows are "up"), ``x = linear(x, w2[e])`` (``:31``) and
  ``token_weight`` is the token's routing weight for e, 0 if e was not
  selected (``:25-26``). Every op takes and returns bf16 tensors, so each
  result above is rounded to bf16 (round to nearest even) before the next
  op uses it, and so is each partial sum of the expert loop.
* ``track-03/requirements.md`` ("算子入参说明") -- shapes and dtypes:
  hidden ``[M, K]``, w1 ``[E, 2N, K]``, w2 ``[E, K, N]``, score ``[M, E]``,
  all bf16; output ``[M, K]`` bf16.

Two choices where the reference leaves something open:

* **Ties in the top-k.** ``torch.topk`` does not specify which of equal
  weights it returns (on CPU it does not prefer the lower index). bf16 router
  scores tie often (E = 64, topk = 6: ~1.5 % of tokens have a tie across the
  top-k boundary), and the tie decides which expert a token reaches. This
  oracle -- and the HIP path -- take the expert with the LOWER index first.
  Where no tie crosses the boundary the selected set is the same as
  ``torch.topk``'s (``tests/test_oracle_moe.py`` checks it).
* **Unselected experts.** The reference adds ``x * 0`` for every token an
  expert was not selected by. For finite ``x`` that leaves the running bf16
  sum unchanged, so only selected (token, expert) pairs are computed, summed
  in ascending expert order.

Functions
---------
``route``               routing in torch (fp32 softmax, lower-index tie rule).
``fused_moe_ref``       torch CPU, bf16 ops in the reference's order on the
                        routed tokens of each expert.
``fused_moe_fp64``      NumPy: every product/sum in float64 from the bf16
                        inputs, rounded to bf16 at exactly the reference's
                        rounding points (an exact-rounding model).
``fused_moe_loops``     per-token scalar loops (float64, tiny shapes only).
``bf16_round``          float64/float32 array -> nearest bf16 value, as float64.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def bf16_round(x):
    """Round to the nearest bf16 (ties to even), returned as float64. Goes
    through float32 like a torch fp32 -> bf16 cast; inf/nan pass through."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isfinite(f), out, f).astype(np.float64)


def route(score, topk, renormalize=False):
    """(ids [M, topk] int64 ascending, weights [M, topk] bf16 in ids' order).

    ``reference.py:16-20``: fp32 softmax of the bf16 scores, the topk largest
    (lower expert index first among equal weights), optional renormalisation
    in fp32, then bf16.
    """
    w = score.float().softmax(dim=-1)
    order = torch.sort(w, dim=-1, descending=True, stable=True)
    vals, ids = order.values[:, :topk], order.indices[:, :topk]
    if renormalize:
        vals = vals / vals.sum(dim=-1, keepdim=True)
    ids_sorted, perm = torch.sort(ids, dim=-1)
    return ids_sorted, torch.gather(vals, 1, perm).to(torch.bfloat16)


def fused_moe_ref(hidden, w1, w2, score, topk, renormalize=False):
    """``reference.py:10-35`` in torch (CPU, bf16 ops) on the routed tokens."""
    M, K = hidden.shape
    E, N = w1.shape[0], w2.shape[-1]
    ids, wts = route(score, topk, renormalize)
    out = torch.zeros(M, K, dtype=hidden.dtype)
    for e in range(E):                                   # :24, ascending experts
        tok, slot = torch.nonzero(ids == e, as_tuple=True)
        if tok.numel() == 0:
            continue
        x = torch.nn.functional.linear(hidden[tok], w1[e])          # :28
        gate = torch.nn.functional.silu(x[:, :N])                   # :29
        x = x[:, N:] * gate                                         # :30
        x = torch.nn.functional.linear(x, w2[e])                    # :31
        out[tok] += x * wts[tok, slot][:, None]                     # :35
    return out


def _silu64(x):
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-x))


def _route_np(score64, topk, renormalize):
    """NumPy routing: float64 softmax rounded to fp32 (the reference's dtype),
    stable descending order, fp32 renormalisation, bf16."""
    s = score64 - score64.max(axis=1, keepdims=True)
    e = np.exp(s)
    w = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    order = np.argsort(-w, axis=1, kind="stable")[:, :topk]
    vals = np.take_along_axis(w, order, axis=1)
    if renormalize:
        vals = (vals / vals.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    perm = np.argsort(order, axis=1, kind="stable")
    return np.take_along_axis(order, perm, axis=1), bf16_round(np.take_along_axis(vals, perm, 1))


def fused_moe_fp64(hidden, w1, w2, score, topk, renormalize=False):
    """Exact-rounding model: float64 arithmetic from the bf16 inputs, bf16
    rounding at the reference's points. Returns float64 ``[M, K]``."""
    h = hidden.double().numpy()
    ids, wts = _route_np(score.double().numpy(), topk, renormalize)
    M, K = h.shape
    N = w2.shape[-1]
    out = np.zeros((M, K))
    for e in np.unique(ids):  # only the experts in use are widened to float64
        tok, slot = np.nonzero(ids == e)
        x = bf16_round(h[tok] @ w1[e].double().numpy().T)
        g = bf16_round(_silu64(x[:, :N]))
        u = bf16_round(x[:, N:] * g)
        y = bf16_round(u @ w2[e].double().numpy().T)
        yw = bf16_round(y * wts[tok, slot][:, None])
        out[tok] = bf16_round(out[tok] + yw)
    return out


def fused_moe_loops(hidden, w1, w2, score, topk, renormalize=False):
    """One token at a time, scalar float64 loops over its selected experts in
    ascending order (tiny shapes only)."""
    h = hidden.double().tolist()
    a1 = w1.double().tolist()
    a2 = w2.double().tolist()
    sc = score.double().tolist()
    M, K = hidden.shape
    E, N = w1.shape[0], w2.shape[-1]
    r = lambda v: float(bf16_round(np.float64(v)))  # noqa: E731
    out = []
    for t in range(M):
        mx = max(sc[t])
        ex = [math.exp(v - mx) for v in sc[t]]
        tot = sum(ex)
        w = [float(np.float32(v / tot)) for v in ex]
        chosen = []
        for _ in range(topk):  # repeated argmax, lowest index among equals
            best = None
            for e in range(E):
                if e not in chosen and (best is None or w[e] > w[best]):
                    best = e
            chosen.append(best)
        den = float(np.float32(sum(np.float32(w[e]) for e in chosen)))
        row = [0.0] * K
        for e in sorted(chosen):
            we = r(float(np.float32(w[e] / den)) if renormalize else w[e])
            x = [r(sum(h[t][k] * a1[e][i][k] for k in range(K))) for i in range(2 * N)]
            u = [r(x[N + j] * r(x[j] / (1.0 + math.exp(-x[j])))) for j in range(N)]
            for k in range(K):
                y = r(sum(u[j] * a2[e][k][j] for j in range(N)))
                row[k] = r(row[k] + r(y * we))
        out.append(row)
    return np.array(out)
