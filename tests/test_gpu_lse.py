"""GPU parity of the (o, lse) output and of the merge of partials against the
float64 oracle (sparse_attn_lse_fp64, merge_fp64).

Tolerances: o as in test_gpu_parity (max |err| <= 2e-2, mean <= 2e-3,
relative RMS <= 5e-3); lse max |err| <= 2e-3 (natural log; scores are fp32
sums of bf16 products, so lse is good to about 1e-4 at these sizes).
"""
import numpy as np
import pytest
import torch

from oracle import sparse_attn_lse_fp64
from test_gpu_parity import DEV, check, say
import submission
import sa_workloads as wl

pytestmark = pytest.mark.gpu

LSE_TOL = 2e-3


def rand_case(b, m, kv_len, topk, seed, minus1=0.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q, kv, sink, idx, wl.SCALE


def lse_gpu(q, kv, sink, idx, sc):
    o, lse = submission.sparse_attn_with_lse(q.to(DEV), kv.to(DEV), sink.to(DEV),
                                             idx.to(DEV), sc)
    return o, lse


def check_lse(lse, exp, label):
    lse = lse.detach().double().cpu().numpy()
    fin = np.isfinite(exp)
    assert np.array_equal(np.isneginf(lse), np.isneginf(exp)), label
    err = np.abs(lse[fin] - exp[fin]).max() if fin.any() else 0.0
    say(f"  {label}: lse max|err| {err:.2e}")
    assert err <= LSE_TOL, label


@pytest.mark.parametrize("shape,plan", [
    ((1, 64, 300, 64), "tiles"),          # shared-row plan
    ((4, 1, 2048, 512), "split"),         # split-topk plan (combine kernel)
    ((1, 3, 2048, 64), "per query"),      # per-query plan
])
def test_lse_every_plan(gpu_sa, shape, plan):
    q, kv, sink, idx, sc = rand_case(*shape, seed=sum(shape), minus1=0.15)
    o, lse = lse_gpu(q, kv, sink, idx, sc)
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    check(o, o_ref, f"o with lse ({plan})")
    check_lse(lse, lse_ref, plan)
    # asking for lse does not change o
    o_plain = submission.sparse_attn(q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV), sc)
    assert torch.equal(o, o_plain)


def test_lse_causal_config_sampled(gpu_sa):
    q, kv, sink, idx, sc = wl.make_config_inputs("causal_prefill")
    o, lse = lse_gpu(q, kv, sink, idx, sc)
    sel = [0, 1, 7, 2047, 2048, 4095] + torch.randint(
        0, 4096, (10,), generator=torch.Generator().manual_seed(3)).tolist()
    for t in sel:
        o_ref, lse_ref = sparse_attn_lse_fp64(q[:, t:t + 1], kv, sink, idx[:, t:t + 1], sc)
        check(o[:, t:t + 1], o_ref, f"causal t={t}")
        check_lse(lse[:, t:t + 1], lse_ref, f"causal t={t}")


def test_no_mass_gives_zero_and_neg_inf(gpu_sa):
    q, kv, _, idx, sc = rand_case(1, 8, 100, 64, seed=31)
    sink = torch.full((16,), float("-inf"))
    idx[0, 2] = -1
    for flags in (0, submission.FLAG_PER_QUERY):
        submission.set_path_flags(flags)
        try:
            o, lse = lse_gpu(q, kv, sink, idx, sc)
        finally:
            submission.set_path_flags(0)
        o, lse = o.cpu(), lse.cpu()
        assert torch.all(o[0, 2] == 0) and torch.all(torch.isneginf(lse[0, 2]))
        o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
        check(o, o_ref, f"sink -inf, flags {flags}")
        check_lse(lse, lse_ref, f"sink -inf, flags {flags}")


def shard(idx, nparts, seed):
    g = torch.Generator().manual_seed(seed)
    owner = torch.randint(0, nparts, idx.shape, generator=g)
    return [torch.where(owner == i, idx, torch.full_like(idx, -1)) for i in range(nparts)]


@pytest.mark.parametrize("shape,nparts", [((1, 40, 500, 256), 3), ((2, 3, 1000, 300), 4),
                                          ((1, 64, 300, 64), 2)])
def test_merge_of_gpu_shards_equals_whole(gpu_sa, shape, nparts):
    q, kv, sink, idx, sc = rand_case(*shape, seed=nparts * 7 + shape[1], minus1=0.1)
    neg = torch.full_like(sink, float("-inf"))
    parts = [lse_gpu(q, kv, neg, p, sc) for p in shard(idx, nparts, seed=shape[1])]
    o, lse = submission.sparse_attn_merge([p[0] for p in parts], [p[1] for p in parts],
                                          sink.to(DEV))
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    check(o, o_ref, f"merge of {nparts} shards")
    check_lse(lse, lse_ref, f"merge of {nparts} shards")


def test_merge_empty_part_and_no_parts(gpu_sa):
    q, kv, sink, idx, sc = rand_case(1, 16, 200, 64, seed=41)
    neg = torch.full_like(sink, float("-inf"))
    parts = shard(idx, 2, seed=41) + [torch.full_like(idx, -1)]
    res = [lse_gpu(q, kv, neg, p, sc) for p in parts]
    assert torch.all(torch.isneginf(res[2][1])) and torch.all(res[2][0] == 0)
    o, lse = submission.sparse_attn_merge([r[0] for r in res], [r[1] for r in res], sink.to(DEV))
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    check(o, o_ref, "merge with an empty part")
    check_lse(lse, lse_ref, "merge with an empty part")
    empty_o = torch.zeros(0, 1, 16, 16, 512, dtype=torch.bfloat16, device=DEV)
    empty_l = torch.zeros(0, 1, 16, 16, dtype=torch.float32, device=DEV)
    o0, lse0 = submission.sparse_attn_merge(empty_o, empty_l, sink.to(DEV))
    assert torch.all(o0 == 0)
    assert torch.allclose(lse0.cpu(), sink.expand(1, 16, 16), atol=0, rtol=0)
