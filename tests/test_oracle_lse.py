"""Pins the (o, lse) and merge restatements of the oracle (CPU only).

* ``sparse_attn_lse_fp64``: its ``o`` is ``sparse_attn_fp64``'s, its ``lse``
  matches the scalar-loop restatement, closed forms (one slot, q = 0, all
  ``-1``, sink = -inf) and the defining identity
  ``o = sum_t exp(s_t - lse) kv[idx_t]``.
* ``merge_fp64``: partials over a random partition of every query's slots,
  each computed with sink = -inf, merge (with the sink folded once) into the
  unsplit result -- also with empty parts. Planted mistakes (sink folded per
  part, sink dropped, unnormalised weights) break that identity.
"""
import math

import numpy as np
import pytest
import torch

from oracle import (merge_fp64, sparse_attn_bruteforce_lse, sparse_attn_fp64,
                    sparse_attn_lse_fp64)


def case(b, m, h, d, kv_len, topk, seed, minus1=0.0, sink_std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, h, d, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, d, generator=g).to(torch.bfloat16)
    sink = torch.randn(h, generator=g) * sink_std
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q, kv, sink, idx, d ** -0.5


def test_o_is_sparse_attn_fp64():
    q, kv, sink, idx, sc = case(2, 3, 4, 16, 30, 12, seed=1, minus1=0.3)
    o, _ = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    np.testing.assert_allclose(o, sparse_attn_fp64(q, kv, sink, idx, sc), rtol=0, atol=1e-15)


def test_lse_matches_scalar_loops():
    q, kv, sink, idx, sc = case(1, 3, 2, 8, 20, 9, seed=2, minus1=0.25)
    _, lse = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    np.testing.assert_allclose(lse, sparse_attn_bruteforce_lse(q, kv, sink, idx, sc),
                               rtol=0, atol=1e-12)


def test_lse_defining_identity():
    """o = sum_t exp(s_t - lse) kv[idx_t], computed from scratch."""
    q, kv, sink, idx, sc = case(1, 2, 3, 8, 15, 6, seed=3, minus1=0.2)
    o, lse = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    qd, kvd = q.double().numpy(), kv.double().numpy()
    for mi in range(2):
        rows = [r for r in idx[0, mi].tolist() if r != -1]
        for hi in range(3):
            acc = np.zeros(8)
            for r in rows:
                s = float(qd[0, mi, hi] @ kvd[0, r]) * sc
                acc += math.exp(s - lse[0, mi, hi]) * kvd[0, r]
            np.testing.assert_allclose(o[0, mi, hi], acc, rtol=0, atol=1e-12)


def test_lse_closed_forms():
    q, kv, sink, idx, sc = case(1, 4, 2, 8, 10, 5, seed=4)
    idx[0, 0] = -1
    idx[0, 0, 2] = 7                                    # one valid slot
    idx[0, 1] = -1                                      # no valid slot
    q[0, 2] = 0                                         # q = 0: every score is 0
    idx[0, 2] = torch.tensor([1, 1, 3, -1, 4], dtype=torch.int32)  # 4 valid (a duplicate)
    _, lse = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    s = (q[0, 0].double() @ kv[0, 7].double()).numpy() * sc
    np.testing.assert_allclose(lse[0, 0], np.logaddexp(s, sink.double().numpy()), atol=1e-13)
    np.testing.assert_allclose(lse[0, 1], sink.double().numpy(), atol=1e-15)
    np.testing.assert_allclose(lse[0, 2], np.log(4 + np.exp(sink.double().numpy())), atol=1e-13)


def test_no_mass_gives_zero_and_neg_inf():
    q, kv, sink, idx, sc = case(1, 2, 3, 8, 10, 4, seed=5)
    sink = torch.full((3,), float("-inf"))
    idx[0, 0] = -1                                      # no slot and no sink
    idx[0, 1] = torch.tensor([2, -1, -1, -1], dtype=torch.int32)  # one slot, no sink
    o, lse = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    assert np.all(o[0, 0] == 0) and np.all(np.isneginf(lse[0, 0]))
    s = (q[0, 1].double() @ kv[0, 2].double()).numpy() * sc
    np.testing.assert_allclose(lse[0, 1], s, atol=1e-13)
    np.testing.assert_allclose(o[0, 1], np.broadcast_to(kv[0, 2].double().numpy(), (3, 8)),
                               atol=1e-15)


def shard(idx, nparts, seed):
    """Random partition of every query's slots into nparts (others -> -1)."""
    g = torch.Generator().manual_seed(seed)
    owner = torch.randint(0, nparts, idx.shape, generator=g)
    return [torch.where(owner == i, idx, torch.full_like(idx, -1)) for i in range(nparts)]


def partials(q, kv, sink, parts, sc, part_sink=None):
    ps = torch.full_like(sink, float("-inf")) if part_sink is None else part_sink
    res = [sparse_attn_lse_fp64(q, kv, ps, p, sc) for p in parts]
    return np.stack([r[0] for r in res]), np.stack([r[1] for r in res])


@pytest.mark.parametrize("nparts,seed", [(1, 10), (2, 11), (3, 12), (5, 13)])
def test_merge_of_shards_is_the_whole(nparts, seed):
    q, kv, sink, idx, sc = case(2, 3, 4, 16, 40, 17, seed=seed, minus1=0.2)
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    O, L = partials(q, kv, sink, shard(idx, nparts, seed), sc)
    o, lse = merge_fp64(O, L, sink)
    np.testing.assert_allclose(o, o_ref, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, lse_ref, rtol=0, atol=1e-12)


def test_merge_with_empty_parts_and_no_parts():
    q, kv, sink, idx, sc = case(1, 2, 2, 8, 20, 6, seed=14)
    parts = shard(idx, 2, 14) + [torch.full_like(idx, -1)]   # third part is empty
    O, L = partials(q, kv, sink, parts, sc)
    assert np.all(np.isneginf(L[2]))
    o, lse = merge_fp64(O, L, sink)
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    np.testing.assert_allclose(o, o_ref, atol=1e-12)
    np.testing.assert_allclose(lse, lse_ref, atol=1e-12)
    o0, lse0 = merge_fp64(np.zeros((0, 1, 2, 2, 8)), np.zeros((0, 1, 2, 2)), sink)
    assert np.all(o0 == 0)
    np.testing.assert_allclose(lse0, np.broadcast_to(sink.double().numpy(), (1, 2, 2)))
    _, lse_none = merge_fp64(np.zeros((0, 1, 2, 2, 8)), np.zeros((0, 1, 2, 2)), None)
    assert np.all(np.isneginf(lse_none))


def test_planted_merge_mistakes_are_caught():
    q, kv, sink, idx, sc = case(1, 3, 4, 16, 40, 17, seed=15, minus1=0.1)
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    parts = shard(idx, 3, 15)
    # the sink folded into every part, then again by the merge
    O, L = partials(q, kv, sink, parts, sc, part_sink=sink)
    o, lse = merge_fp64(O, L, sink)
    assert np.abs(lse - lse_ref).max() > 1e-3 and np.abs(o - o_ref).max() > 1e-4
    # the sink dropped
    O, L = partials(q, kv, sink, parts, sc)
    o, lse = merge_fp64(O, L, None)
    assert np.abs(lse - lse_ref).max() > 1e-3
    # unnormalised weights exp(lse_i)
    wrong = (np.exp(L)[..., None] * O).sum(axis=0)
    assert np.abs(wrong - o_ref).max() > 1e-3
