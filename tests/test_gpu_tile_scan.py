"""The tile launch of short-query tile plans (topk <= 384, whose per-query
queries run one wave each): one work-group per CU walks the tiles t = b,
b + G, ... and runs those the index kernel made shared. It must equal the
ordered launch (SA_FLAG_TILE_ORDERED: the order kernel's tile order, one
work-group per tile) bit for bit in o, lse and the error word, with several
shared tiles per work-group, per-query tiles between them, an aborted tile
in the middle of a work-group's walk and ragged last tiles; samples are
checked against the float64 oracle.
"""
import numpy as np
import pytest
import torch

from oracle import sparse_attn_fp64
from sa_testutil import expect_plan
from test_gpu_parity import DEV, sampled_check, say
import sa_workloads as wl

pytestmark = pytest.mark.gpu

TILE_ORDERED = 32


def cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def run_lse(q, kv, sink, idx, scale, flags):
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    o, lse = torch.ops.sa_amd.sparse_attn_fwd_lse(q.to(DEV), kv.to(DEV), sink.to(DEV),
                                                  idx.to(DEV), float(scale), err, flags)
    return o.cpu(), lse.cpu(), int(err.item())


def base(b, m, kv_len, topk, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    return g, q, kv, sink, idx


def windows_all_shared():
    """Every tile shared (windows of 128 rows, 2 apart), about three tiles per
    CU, a ragged last tile and some -1 slots."""
    m = 8 * 3 * cus() + 5
    g, q, kv, sink, idx = base(1, m, 8192, 128, seed=51)
    t = torch.arange(m)
    idx[0] = ((torch.arange(128)[None] + 2 * t[:, None]) % 8192).to(torch.int32)
    idx[0, ::7, 100:] = -1
    return q, kv, sink, idx, [(0, 0), (0, 9), (0, m // 2), (0, m - 1)]


def mixed_modes():
    """Runs of shared tiles (windows) between per-query tiles (random rows),
    so that a work-group's walk meets both, over two batches."""
    m = 8 * 2 * cus() + 3
    g, q, kv, sink, idx = base(2, m, 4096, 192, seed=52)
    t = torch.arange(m)
    win = ((torch.arange(192)[None] + 3 * t[:, None]) % 4096).to(torch.int32)
    sel = (t // 8) % 5 < 2
    idx[:, sel] = win[sel]
    return q, kv, sink, idx, [(0, 0), (1, 17), (0, 8 * 5 + 2), (1, m - 1)]


def aborted_in_walk():
    """Shared tiles throughout; tile 1 aborts at run time (a last row whose
    score for query 8 is far above everything its first step sees), and its
    work-group has more shared tiles after it."""
    m = 8 * (cus() + 9)
    g, q, kv, sink, idx = base(1, m, 6000, 256, seed=53)
    t = torch.arange(m)
    idx[0] = ((torch.arange(256)[None] + 3 * t[:, None]) % 4096).to(torch.int32)
    idx[0, 8:16, -1] = 5000
    kv[0, 5000] = (q[0, 8].float().mean(0) * 60).to(torch.bfloat16)
    return q, kv, sink, idx, [(0, 0), (0, 20), (0, m - 1)]


def bad_index():
    """Shared tiles with one out-of-range index and a tile of -1 rows only:
    the same error word and the same outputs from both launches."""
    m = 8 * cus() + 8 * 4 + 6
    g, q, kv, sink, idx = base(1, m, 3000, 64, seed=54)
    t = torch.arange(m)
    idx[0] = ((torch.arange(64)[None] + t[:, None]) % 3000).to(torch.int32)
    idx[0, 40, 7] = 3000
    idx[0, 64:72] = -1
    return q, kv, sink, idx, []


def placed_regime():
    """Between half as many tiles as CUs and as many: the ordered launch
    places the tiles itself (no order kernel), the scan runs one per
    work-group."""
    m = 8 * (cus() - 3) + 2
    g, q, kv, sink, idx = base(1, m, 3000, 96, seed=55)
    t = torch.arange(m)
    idx[0] = ((torch.arange(96)[None] + 2 * t[:, None]) % 3000).to(torch.int32)
    return q, kv, sink, idx, [(0, 1), (0, m - 1)]


CASES = {"windows, all shared": windows_all_shared, "mixed modes": mixed_modes,
         "aborted tile in a walk": aborted_in_walk, "bad index": bad_index,
         "placed regime": placed_regime}


@pytest.mark.parametrize("name", list(CASES))
def test_tile_scan_equals_ordered(gpu_sa, name):
    q, kv, sink, idx, sel = CASES[name]()
    say(f"tile scan vs ordered: {name} b={q.shape[0]} m={q.shape[1]} "
        f"kv={kv.shape[1]} topk={idx.shape[2]}")
    expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    o_s, lse_s, err_s = run_lse(q, kv, sink, idx, wl.SCALE, 0)
    o_o, lse_o, err_o = run_lse(q, kv, sink, idx, wl.SCALE, TILE_ORDERED)
    assert err_s == err_o
    assert (err_s != 0) == (name == "bad index")
    assert torch.equal(o_s, o_o) and torch.equal(lse_s, lse_o)
    if name == "aborted tile in a walk":
        # row 5000 dominates queries 8..15 (|o| up to ~20): relative RMS
        # against float64 there, the sampled check elsewhere
        exp = sparse_attn_fp64(q[:, 8:16], kv, sink, idx[:, 8:16], wl.SCALE)
        err = o_s[:, 8:16].double().numpy() - exp
        rel = float(np.sqrt((err ** 2).mean() / (exp ** 2).mean()))
        say(f"  aborted tile: rel_rms={rel:.3e}")
        assert rel <= 5e-3
    if sel:
        sampled_check(o_s, q, kv, sink, idx, wl.SCALE, sel, f"tile scan: {name}")


def test_tile_scan_planned_equals_plain(gpu_sa):
    """An index plan (which holds a tile order) and the plain call, both with
    the scanning tile launch, against the ordered launch of the planned call."""
    q, kv, sink, idx = (x.to(DEV) for x in mixed_modes()[:4])
    plan = gpu_sa.sparse_attn_plan(q, kv, idx)
    o_plain = gpu_sa.sparse_attn(q, kv, sink, idx, wl.SCALE)
    o_plan = gpu_sa.sparse_attn(q, kv, sink, idx, wl.SCALE, plan=plan)
    gpu_sa.set_path_flags(gpu_sa.FLAG_TILE_ORDERED)
    try:
        plan_o = gpu_sa.sparse_attn_plan(q, kv, idx)
        o_ord = gpu_sa.sparse_attn(q, kv, sink, idx, wl.SCALE, plan=plan_o)
    finally:
        gpu_sa.set_path_flags(0)
    assert torch.equal(o_plain, o_plan) and torch.equal(o_plan, o_ord)
