"""Pins the CPU oracle (``oracle/sparse_attn_ref.py``) on the CPU.

The reference ships no golden vectors (its only check is a live comparison,
``track-01/test_correctness.py:22-34``), so the oracle is pinned by:

* agreement of three independent restatements (torch fp32 in the reference's
  operation order, NumPy fp64 on compacted slots, scalar Python loops);
* closed forms: q = 0, one valid slot, sink -> +inf, every slot -1;
* a library special case: sink = -inf is plain softmax attention, checked
  against ``torch.nn.functional.scaled_dot_product_attention`` in float64;
* invariances: slot permutation, ``-1`` == deleted slot, (c*q, scale/c),
  per-query slicing;
* planted mistakes: each mutant oracle below must fail at least one check.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import (masked_fold_fp64, sparse_attn_bruteforce, sparse_attn_fp64,
                    sparse_attn_ref)

SCALE = 0.04419417382415922


def tiny(b=2, m=3, h=2, d=8, kv_len=11, topk=6, seed=0, minus1=0.0, scale=0.35):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, h, d, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, d, generator=g).to(torch.bfloat16)
    sink = torch.randn(h, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q, kv, sink, idx, scale


# ---------------------------------------------------------------------------
# agreement of the restatements
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seed,minus1", [(0, 0.0), (1, 0.3), (2, 0.6), (3, 0.0)])
def test_restatements_agree(seed, minus1):
    args = tiny(seed=seed, minus1=minus1)
    bf = sparse_attn_bruteforce(*args)
    f64 = sparse_attn_fp64(*args)
    np.testing.assert_allclose(f64, bf, rtol=1e-12, atol=1e-12)
    ref = sparse_attn_ref(*args).float().numpy().astype(np.float64)
    # ref = bf16(RNE) of an fp32 computation: within one bf16 ulp of fp64
    assert np.all(np.abs(ref - f64) <= 2.0 ** -8 * np.abs(f64) + 1e-5)


def test_ref_chunking_is_exact():
    q, kv, sink, idx, sc = tiny(b=2, m=9, h=3, d=16, kv_len=40, topk=12, seed=5,
                                minus1=0.2)
    a = sparse_attn_ref(q, kv, sink, idx, sc)
    b_ = sparse_attn_ref(q, kv, sink, idx, sc, chunk=2)
    assert torch.equal(a, b_)


def test_ref_full_shape_dtype():
    q, kv, sink, idx, sc = tiny(b=1, m=2, h=16, d=512, kv_len=70, topk=33, seed=9)
    o = sparse_attn_ref(q, kv, sink, idx, sc)
    assert o.shape == (1, 2, 16, 512) and o.dtype == torch.bfloat16
    np.testing.assert_allclose(o.float().numpy(), sparse_attn_fp64(q, kv, sink, idx, sc),
                               rtol=2 ** -8, atol=1e-5)


# ---------------------------------------------------------------------------
# checks, written as functions of an oracle so mutants can be run through them
# ---------------------------------------------------------------------------
def _f64(x):
    return x.to(torch.float64).numpy()


def check_q_zero(fn):
    """q = 0: every valid score is 0, o = sum(rows, with multiplicity)/(n + e^sink)."""
    q, kv, sink, idx, sc = tiny(b=2, m=3, h=3, d=8, kv_len=9, topk=7, seed=11, minus1=0.3)
    idx[0, 0, :3] = 4  # a duplicate-heavy row
    q = torch.zeros_like(q)
    o = np.asarray(fn(q, kv, sink, idx, sc), dtype=np.float64)
    kvn, sk = _f64(kv), _f64(sink)
    for bi in range(2):
        for mi in range(3):
            rows = [r for r in idx[bi, mi].tolist() if r != -1]
            tot = kvn[bi, rows].sum(axis=0) if rows else np.zeros(8)
            for hi in range(3):
                exp = tot / (len(rows) + math.exp(sk[hi]))
                if not np.allclose(o[bi, mi, hi], exp, rtol=1e-9, atol=1e-12):
                    return False
    return True


def check_single_slot(fn):
    """One valid slot with score s: o = kv_row * sigmoid(s - sink)."""
    q, kv, sink, idx, sc = tiny(b=1, m=2, h=4, d=8, kv_len=7, topk=5, seed=12)
    idx[:] = -1
    idx[0, 0, 3] = 5
    idx[0, 1, 0] = 2
    o = np.asarray(fn(q, kv, sink, idx, sc), dtype=np.float64)
    qn, kvn, sk = _f64(q), _f64(kv), _f64(sink)
    for mi, r in ((0, 5), (1, 2)):
        for hi in range(4):
            s = float(qn[0, mi, hi] @ kvn[0, r]) * sc
            exp = kvn[0, r] / (1.0 + math.exp(sk[hi] - s))
            if not np.allclose(o[0, mi, hi], exp, rtol=1e-9, atol=1e-12):
                return False
    return True


def check_sdpa(fn):
    """sink = -inf: plain softmax attention over the gathered rows (library SDPA)."""
    q, kv, sink, idx, sc = tiny(b=2, m=3, h=4, d=16, kv_len=13, topk=6, seed=13)
    sink = torch.full_like(sink, float("-inf"))
    o = np.asarray(fn(q, kv, sink, idx, sc), dtype=np.float64)
    for bi in range(2):
        for mi in range(3):
            K = kv[bi, idx[bi, mi].long()].to(torch.float64)[None]          # [1, n, d]
            Q = q[bi, mi].to(torch.float64)[:, None, :]                     # [h, 1, d]
            exp = F.scaled_dot_product_attention(
                Q, K.expand(4, -1, -1), K.expand(4, -1, -1), scale=sc)[:, 0]
            if not np.allclose(o[bi, mi], exp.numpy(), rtol=1e-9, atol=1e-12):
                return False
    return True


def check_large_sink(fn):
    """sink -> +inf: the sink takes all the mass, o -> 0."""
    q, kv, sink, idx, sc = tiny(seed=14)
    sink = torch.full_like(sink, 80.0)
    o = np.asarray(fn(q, kv, sink, idx, sc), dtype=np.float64)
    return bool(np.abs(o).max() < 1e-25)


def check_all_masked(fn):
    """every slot -1: o = 0 exactly."""
    q, kv, sink, idx, sc = tiny(seed=15)
    idx[1, 2] = -1
    o = np.asarray(fn(q, kv, sink, idx, sc), dtype=np.float64)
    return bool(np.all(o[1, 2] == 0.0)) and bool(np.abs(o[0, 0]).max() > 0)


def check_minus1_is_deletion(fn):
    """a -1 slot anywhere in the row equals the row without that slot."""
    q, kv, sink, idx, sc = tiny(b=1, m=1, h=2, d=8, kv_len=10, topk=6, seed=16)
    base = idx.clone()
    padded = torch.full((1, 1, 9), -1, dtype=torch.int32)
    padded[0, 0, [0, 2, 3, 5, 7, 8]] = base[0, 0]
    a = np.asarray(fn(q, kv, sink, base, sc), dtype=np.float64)
    b_ = np.asarray(fn(q, kv, sink, padded, sc), dtype=np.float64)
    return bool(np.allclose(a, b_, rtol=1e-12, atol=1e-14))


def check_permutation(fn):
    q, kv, sink, idx, sc = tiny(seed=17, minus1=0.2)
    perm = torch.randperm(idx.shape[-1], generator=torch.Generator().manual_seed(1))
    a = np.asarray(fn(q, kv, sink, idx, sc), dtype=np.float64)
    b_ = np.asarray(fn(q, kv, sink, idx[..., perm], sc), dtype=np.float64)
    return bool(np.allclose(a, b_, rtol=1e-12, atol=1e-14))


CHECKS = [check_q_zero, check_single_slot, check_sdpa, check_large_sink,
          check_all_masked, check_minus1_is_deletion, check_permutation]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_fp64_passes(check):
    assert check(sparse_attn_fp64)


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_bruteforce_passes(check):
    assert check(sparse_attn_bruteforce)


@pytest.mark.parametrize("nsplit", [1, 2, 3, 7])
@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_split_fold_passes(check, nsplit):
    assert check(lambda *a: masked_fold_fp64(*a, nsplit=nsplit))


def test_split_fold_equals_direct_with_empty_parts():
    q, kv, sink, idx, sc = tiny(b=2, m=3, h=3, d=8, kv_len=9, topk=12, seed=18)
    idx[0, 0, :8] = -1      # first parts of this row have no valid slot
    idx[1, 2, 4:] = -1
    ref = sparse_attn_fp64(q, kv, sink, idx, sc)
    for ns in (1, 2, 3, 4, 6, 12, 20):
        np.testing.assert_allclose(masked_fold_fp64(q, kv, sink, idx, sc, ns), ref,
                                   rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------------------
# planted mistakes: each must be caught by at least one check
# ---------------------------------------------------------------------------
def _mutant(kind):
    def fn(q, kv, attn_sink, topk_idxs, scale):
        qn, kvn, sk = _f64(q), _f64(kv), _f64(attn_sink)
        idx = topk_idxs.numpy().astype(np.int64)
        b, m, h, d = qn.shape
        out = np.zeros((b, m, h, d))
        for bi in range(b):
            for mi in range(m):
                rows = idx[bi, mi]
                if kind == "minus1_as_row0":
                    rows = np.where(rows == -1, 0, rows)
                else:
                    rows = rows[rows != -1]
                if kind == "off_by_one_index":
                    rows = (rows + 1) % kvn.shape[1]
                if kind == "dedup_indices":
                    rows = np.unique(rows)
                K = kvn[bi, rows]
                sc = {"no_scale": 1.0, "divide_scale": 1.0 / scale}.get(kind, scale)
                s = qn[bi, mi] @ K.T * sc
                if kind == "drop_sink":
                    z = s
                else:
                    z = np.concatenate([s, sk[:, None]], axis=1)
                if kind == "sign_flip":
                    e = np.exp(z.max(axis=1, keepdims=True) - z)
                else:
                    e = np.exp(z - z.max(axis=1, keepdims=True))
                w = e / e.sum(axis=1, keepdims=True)
                if kind == "drop_sink":
                    wk = w
                elif kind == "drop_first_column":
                    wk = w[:, 1:]
                else:
                    wk = w[:, :-1]
                V = qn[bi, mi] if kind == "wrong_operand" else K
                if kind == "wrong_operand":
                    out[bi, mi] = wk @ np.resize(V, (wk.shape[1], d))
                else:
                    out[bi, mi] = wk @ V
        return out
    return fn


MUTANTS = ["drop_sink", "drop_first_column", "no_scale", "divide_scale",
           "minus1_as_row0", "off_by_one_index", "dedup_indices", "sign_flip",
           "wrong_operand"]


@pytest.mark.parametrize("kind", MUTANTS)
def test_planted_mistake_is_caught(kind):
    fn = _mutant(kind)
    failed = []
    for c in CHECKS:
        try:
            ok = c(fn)
        except Exception:
            ok = False
        if not ok:
            failed.append(c.__name__)
    assert failed, f"mutant {kind} passed every check"


def test_unmutated_template_passes_every_check():
    fn = _mutant("none")
    assert all(c(fn) for c in CHECKS)


# ---------------------------------------------------------------------------
# error behaviour, bf16 cast
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bad", [-2, 11, 1000])
def test_out_of_range_raises_like_gather(bad):
    q, kv, sink, idx, sc = tiny()
    idx[0, 1, 2] = bad
    with pytest.raises(RuntimeError):
        sparse_attn_ref(q, kv, sink, idx, sc)
    with pytest.raises(RuntimeError):
        sparse_attn_fp64(q, kv, sink, idx, sc)


def test_bf16_cast_is_round_to_nearest_even():
    x = torch.tensor([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 1 + 2 ** -8 + 2 ** -20])
    y = x.to(torch.bfloat16).float().tolist()
    assert y == [1.0, 1.015625, -1.0, 1.0078125]


def test_sink_fold_algebra_matches_reference_form():
    """m_tot = max(m, sink) form (track-01/notes.md:32-41) equals softmax over [s, sink]."""
    rng = np.random.default_rng(0)
    for _ in range(50):
        s = rng.normal(size=7) * 5
        sink = rng.normal() * 5
        z = np.concatenate([s, [sink]])
        w = np.exp(z - z.max())
        w /= w.sum()
        m = s.max()
        l_ = np.exp(s - m).sum()
        m_tot = max(m, sink)
        alpha = math.exp(m - m_tot)
        l_tot = alpha * l_ + math.exp(sink - m_tot)
        np.testing.assert_allclose(alpha * np.exp(s - m) / l_tot, w[:-1], rtol=1e-12)
