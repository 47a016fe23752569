"""GPU parity at head counts other than 16.

The reference's kernels take any power-of-two h (track-01/submission.py:1004,
:1233); this build's kernels compute 16 heads at a time. The C-ABI runs
16 k heads as k calls on 16-head slices of q, sink, o and lse, and 1, 2, 4 or
8 heads on a zero-padded 16-head copy in its workspace. Checked against the
float64 oracle on every plan kind (per query, shared-row tiles, split topk),
bit for bit against the equivalent 16-head calls, with an index plan, and
the head counts the library does not run are refused.
"""
import pytest
import torch

from oracle import sparse_attn_fp64
from test_gpu_parity import DEV, check, say
import sa_workloads as wl

pytestmark = pytest.mark.gpu

PER_QUERY, FORCE_TILES = 1, 2


def case(b, m, h, kv_len, topk, seed, minus1=0.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, h, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(h, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q, kv, sink, idx, wl.SCALE


def run(q, kv, sink, idx, scale, flags=0):
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    o, lse = torch.ops.sa_amd.sparse_attn_fwd_lse(q.to(DEV), kv.to(DEV), sink.to(DEV),
                                                  idx.to(DEV), float(scale), err, flags)
    assert int(err.item()) == 0
    return o, lse


# (b, m, kv_len, topk, flags, minus1): a per-query plan, forced shared-row
# tiles with -1 padding, and a split-topk (decode) plan
PLANS = {"per query": (1, 300, 5000, 128, PER_QUERY, 0.0),
         "tiles": (2, 24, 700, 96, FORCE_TILES, 0.2),
         "split": (4, 1, 9000, 1500, 0, 0.1)}


@pytest.mark.parametrize("h", [1, 2, 4, 8, 32, 48])
@pytest.mark.parametrize("plan", list(PLANS))
def test_head_counts_match_oracle(gpu_sa, h, plan):
    b, m, kv_len, topk, flags, minus1 = PLANS[plan]
    q, kv, sink, idx, sc = case(b, m, h, kv_len, topk, seed=60 + h, minus1=minus1)
    say(f"  h={h} {plan}: b,m,kv_len,topk = {b},{m},{kv_len},{topk}")
    o, lse = run(q, kv, sink, idx, sc, flags)
    assert o.shape == (b, m, h, 512) and lse.shape == (b, m, h)
    sel = [(bi, t) for bi in range(b) for t in sorted({0, m // 2, m - 1})]
    exp = torch.from_numpy(sparse_attn_fp64(q[[s[0] for s in sel], [s[1] for s in sel]][:, None],
                                            kv[[s[0] for s in sel]], sink,
                                            idx[[s[0] for s in sel], [s[1] for s in sel]][:, None],
                                            sc))
    got = o.cpu()[[s[0] for s in sel], [s[1] for s in sel]]
    check(got, exp[:, 0].numpy(), f"h={h} {plan}")


@pytest.mark.parametrize("h", [32, 48])
def test_multiple_of_16_equals_its_slices(gpu_sa, h):
    """h = 16 k is k independent 16-head calls: the same bits."""
    q, kv, sink, idx, sc = case(1, 64, h, 3000, 200, seed=70, minus1=0.1)
    o, lse = run(q, kv, sink, idx, sc)
    for g in range(h // 16):
        sl = slice(16 * g, 16 * g + 16)
        o_g, l_g = run(q[:, :, sl].contiguous(), kv, sink[sl].contiguous(), idx, sc)
        assert torch.equal(o[:, :, sl], o_g) and torch.equal(lse[:, :, sl], l_g)


@pytest.mark.parametrize("h", [1, 2, 4, 8])
@pytest.mark.parametrize("flags", [PER_QUERY, FORCE_TILES])
def test_fewer_heads_equal_padded_16(gpu_sa, h, flags):
    """h < 16 runs on a zero-padded 16-head copy: its heads equal the first h
    heads of the 16-head call on that padded q, bit for bit (the heads of a
    query are independent)."""
    q, kv, sink, idx, sc = case(1, 40, h, 1200, 150, seed=80 + h, minus1=0.1)
    o, lse = run(q, kv, sink, idx, sc, flags)
    q16 = torch.zeros(1, 40, 16, 512, dtype=torch.bfloat16)
    q16[:, :, :h] = q
    s16 = torch.zeros(16)
    s16[:h] = sink
    o16, l16 = run(q16, kv, s16, idx, sc, flags)
    assert torch.equal(o, o16[:, :, :h]) and torch.equal(lse, l16[:, :, :h])


def test_fewer_heads_with_index_plan_and_drop_in(gpu_sa):
    """The drop-in with 8 heads, plain and with a reused index plan."""
    import submission
    q, kv, sink, idx, sc = case(1, 64, 8, 2048, 256, seed=90, minus1=0.05)
    qd, kvd, sd, idd = (t.to(DEV) for t in (q, kv, sink, idx))
    o = submission.sparse_attn(qd, kvd, sd, idd, sc)
    plan = submission.sparse_attn_plan(qd, kvd, idd)
    o_p = submission.sparse_attn(qd, kvd, sd, idd, sc, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(o, o_p)
    check(o.cpu()[:, :8], sparse_attn_fp64(q[:, :8], kv, sink, idx[:, :8], sc), "h=8 drop-in")


@pytest.mark.parametrize("h", [3, 12, 24])
def test_unsupported_head_counts_raise(gpu_sa, h):
    q, kv, sink, idx, sc = case(1, 8, h, 256, 32, seed=95)
    with pytest.raises(ValueError):
        run(q, kv, sink, idx, sc)
