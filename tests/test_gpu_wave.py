"""GPU parity of the one-wave-per-query kernel (sa_fwd_wave_kernel): short
unsplit queries (topk <= 384) of per-query plans and of the per-query tiles
of shared-row plans, checked against the float64 oracle on every query, with
the launched-kernel mask of sa_forward_events naming the kernel that ran.

Tolerance as in test_gpu_parity: max |err| <= 2e-2, mean |err| <= 2e-3,
relative RMS <= 5e-3 against float64; lse max |err| <= 2e-3; exact zeros for
queries without a valid slot.
"""

import numpy as np
import pytest
import torch

from oracle import sparse_attn_fp64, sparse_attn_lse_fp64
from sa_testutil import expect_plan
from test_gpu_parity import DEV, check, say
import sa_capi
import sa_workloads as wl

pytestmark = pytest.mark.gpu

PER_QUERY = 1
INDEX, QUERY, TILE, WAVE = (1 << sa_capi.KERNELS.index(k) for k in ("index", "query", "tile",
                                                                    "wave"))

def case(b, m, kv_len, topk, seed, minus1=0.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q, kv, sink, idx, wl.SCALE

def run(q, kv, sink, idx, sc, flags=0, o=None, with_lse=False):
    """One call through the C-ABI's event hook: (o, lse or None, launched
    mask, error word, workspace)."""
    lib = sa_capi.load()
    q, kv, sink, idx = (t.to(DEV) for t in (q, kv, sink, idx))
    if o is None:
        o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=DEV) if with_lse else None
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    a = sa_capi.make_args(q, kv, sink, idx, o, sc, flags, err=err, lse=lse)
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    say(f"  wave call b,m,kv,topk={tuple(q.shape[:2]) + (kv.shape[1], idx.shape[2])} "
        f"flags={flags}")
    mask = sa_capi.forward_events(lib, a, torch.cuda.current_stream().cuda_stream,
                                  [None] * (2 * sa_capi.SA_KERNEL_COUNT))
    torch.cuda.synchronize()
    return o, lse, mask, int(err.item()), ws

def per_query_queries(ws, b, m):
    """[b, m] bool: the queries of the tiles the index kernel made per query
    (tile meta at workspace offset 0: union size, mode, valid slots,
    overflow per tile; mode 1 = shared)."""
    tpb = -(-m // 8)
    meta = ws[:16 * b * tpb].view(torch.int32).view(b * tpb, 4).cpu()
    per_tile = (meta[:, 1] != 1).view(b, tpb)
    return per_tile.repeat_interleave(8, dim=1)[:, :m]

# At least as many queries as CUs (256 here) where topk > 64, so that the
# plan does not split them (asserted first).
@pytest.mark.parametrize("b,m,kv_len,topk,minus1", [
    (2, 160, 1024, 128, 0.0),    # contest-like prefill: every tile per query
    (1, 261, 4096, 100, 0.2),    # ragged last tile (5 queries: a one-query work-group)
    (3, 89, 2048, 384, 0.1),     # the largest list; tiles of 8 + 1
    (1, 24, 600, 17, 0.0),       # one 16-row and one 1-row step (tiles shared here)
    # a batch's kv above 4 MiB: each query's rows sorted ascending (2, 4 and
    # 8 keys per lane)
    (1, 300, 8192, 128, 0.1),
    (1, 280, 6000, 256, 0.05),
    (2, 133, 5000, 384, 0.1),
])
def test_wave_tiles_full(gpu_sa, b, m, kv_len, topk, minus1):
    """Per-query tiles of a shared-row plan run one wave per query; every
    query matches the oracle, and the plain per-query plan (every query one
    wave) matches the oracle too and equals the per-query tiles' queries bit
    for bit (the same kernel computes each query the same way)."""
    q, kv, sink, idx, sc = case(b, m, kv_len, topk, seed=b * 1000 + m + topk, minus1=minus1)
    expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    o, _, mask, err, ws = run(q, kv, sink, idx, sc)
    assert err == 0
    assert mask & WAVE and mask & INDEX and mask & TILE
    sel = per_query_queries(ws, b, m)
    say(f"  {int(sel.sum())} of {b * m} queries in per-query tiles")
    if kv_len == 1024:
        assert sel.all()  # 128 random rows of 1024: 8 queries share few
    exp = sparse_attn_fp64(q, kv, sink, idx, sc)
    check(o, exp, f"wave tiles {b}x{m} topk {topk}")
    o_p, _, mask_p, _, _ = run(q, kv, sink, idx, sc, flags=PER_QUERY)
    if expect_plan(q, kv, idx, PER_QUERY)["nsplit"] == 1:
        assert mask_p == WAVE
        check(o_p, exp, f"wave plain {b}x{m} topk {topk}")
        assert torch.equal(o.cpu()[sel], o_p.cpu()[sel])

@pytest.mark.parametrize("b,m", [(3, 99), (5, 61)])
def test_wave_plain_plan_across_batches(gpu_sa, b, m):
    """The plain per-query plan: work-group i runs queries 2i and 2i + 1 of
    b x m, which straddle batches when m is odd; the last work-group has one
    query. Different kv per batch, so a query gathered from the wrong batch
    fails the oracle check."""
    q, kv, sink, idx, sc = case(b, m, 777, 200, seed=b + m, minus1=0.05)
    p = expect_plan(q, kv, idx, PER_QUERY, tiles=False)
    if p["nsplit"] != 1:
        pytest.skip(f"{b * m} queries split on this device")
    o, lse, mask, err, _ = run(q, kv, sink, idx, sc, flags=PER_QUERY, with_lse=True)
    assert err == 0 and mask == WAVE
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    check(o, o_ref, f"wave plain {b}x{m}")
    d = np.abs(lse.double().cpu().numpy() - lse_ref).max()
    say(f"  lse max|err| {d:.2e}")
    assert d <= 2e-3

def test_wave_masked_duplicates_and_sink(gpu_sa):
    """Queries with no valid slot give exact zeros (lse = the sink's), all-
    duplicate queries weigh one row by its count, and -1 slots anywhere are
    skipped, all within one two-query work-group's stream."""
    q, kv, sink, idx, sc = case(1, 16, 512, 48, seed=3)
    idx[0, 0] = -1                                      # nothing valid
    idx[0, 1, :] = 7                                    # one row, 48 times
    idx[0, 2, ::2] = -1                                 # every other slot
    idx[0, 3, :40] = -1                                 # a short tail only
    idx[0, 5] = -1                                      # second of a pair empty
    o, lse, mask, err, _ = run(q, kv, sink, idx, sc, with_lse=True)
    assert err == 0 and mask & WAVE
    o_ref, lse_ref = sparse_attn_lse_fp64(q, kv, sink, idx, sc)
    check(o, o_ref, "wave masked/duplicates")
    oc = o.cpu()
    assert torch.all(oc[0, 0] == 0) and torch.all(oc[0, 5] == 0)
    d = np.abs(lse.double().cpu().numpy() - lse_ref).max()
    assert d <= 2e-3

def test_wave_bad_index_reported(gpu_sa):
    """An index outside [-1, kv_len) sets the error word; the other slots of
    the query still count."""
    q, kv, sink, idx, sc = case(1, 32, 256, 64, seed=9)
    idx[0, 17, 5] = 256
    idx[0, 30, 63] = -7
    o, _, mask, err, _ = run(q, kv, sink, idx, sc)
    assert mask & WAVE and err == 1
    ok = idx.clone()
    ok[0, 17, 5] = -1
    ok[0, 30, 63] = -1
    check(o, sparse_attn_fp64(q, kv, sink, ok, sc), "wave bad index")

def test_wave_topk_cap(gpu_sa):
    """topk 384 (the list's capacity) runs one wave per query; topk 385 runs
    the 4-wave per-query kernel. Both match the oracle."""
    for topk, want in ((384, WAVE), (385, QUERY)):
        q, kv, sink, idx, sc = case(1, 260, 3000, topk, seed=topk, minus1=0.1)
        if expect_plan(q, kv, idx, PER_QUERY, tiles=False)["nsplit"] != 1:
            pytest.skip("260 queries split on this device")
        o, _, mask, err, _ = run(q, kv, sink, idx, sc, flags=PER_QUERY)
        assert err == 0 and mask == want
        check(o, sparse_attn_fp64(q, kv, sink, idx, sc), f"topk {topk}")

def test_wave_sorted_rows_past_2gib(gpu_sa):
    """A batch's kv of 2.3 GiB: the 32-bit row offsets of the wave kernel's
    lists reach past 2^31, and each query's rows are sorted as unsigned
    offsets. Half of every query's slots name rows beyond the 2^31-byte mark
    (kv_len is above the shared-row limit: a per-query plan). Sampled queries
    match the oracle on a compacted copy of the rows they name."""
    kv_len = (1 << 21) + 300_000
    b, m, topk = 1, 300, 128
    g = torch.Generator().manual_seed(77)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    lo = torch.randint(0, 1 << 21, (b, m, topk // 2), generator=g, dtype=torch.int32)
    hi = torch.randint(1 << 21, kv_len, (b, m, topk // 2), generator=g, dtype=torch.int32)
    idx = torch.cat([hi, lo], dim=2)  # high offsets first: the sort must move them
    idx[:, ::9, 5] = -1
    gd = torch.Generator(device=DEV).manual_seed(78)
    kv = torch.randn(b, kv_len, 512, generator=gd, device=DEV).to(torch.bfloat16)
    p = expect_plan(q, kv, idx, 0, tiles=False)
    if p["nsplit"] != 1:
        pytest.skip(f"{m} queries split on this device")
    o, _, mask, err, _ = run(q, kv, sink, idx, wl.SCALE)
    assert err == 0 and mask == WAVE
    sel = [0, 1, 9, 150, 299]
    rows = torch.unique(idx[0, sel][idx[0, sel] >= 0])
    remap = torch.full((kv_len,), -1, dtype=torch.int32)
    remap[rows.long()] = torch.arange(rows.numel(), dtype=torch.int32)
    idx_c = idx[:, sel].clone()
    idx_c[idx_c >= 0] = remap[idx_c[idx_c >= 0].long()]
    kv_c = kv[:, rows.to(DEV).long()].cpu()
    exp = sparse_attn_fp64(q[:, sel], kv_c, sink, idx_c, wl.SCALE)
    check(o.cpu()[:, sel], exp, "wave rows past 2^31")

@pytest.mark.parametrize("topk", [128, 400])
def test_index_long_cache_many_tiles(gpu_sa, topk):
    """kv_len 9 000 (the index kernel's 1 024-thread form, one work-group per
    CU by its count table) with three tiles per CU: every third tile takes
    windows (shared), the others random rows (per query). The modes come out
    as built, per-query tiles equal the plain per-query plan bit for bit,
    shared tiles agree within the tolerance, and samples match the oracle.
    topk 128 runs the per-query tiles one wave each, 400 in the 4-wave
    kernel."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    m = 8 * 3 * cus + 3
    q, kv, sink, idx, sc = case(1, m, 9000, topk, seed=topk + 5, minus1=0.02)
    t = torch.arange(m)
    win = ((torch.arange(topk)[None] + 2 * t[:, None]) % 9000).to(torch.int32)
    sel = (t // 8) % 3 == 0
    idx[0, sel] = win[sel]
    expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    o, _, mask, err, ws = run(q, kv, sink, idx, sc)
    assert err == 0 and mask & INDEX and mask & TILE
    pq = per_query_queries(ws, 1, m)[0]
    # full tiles come out as built (the ragged last tile of 3 window queries
    # is cheaper per query by the mode rule)
    full = torch.arange(m) < m // 8 * 8
    assert not pq[sel & full].any() and pq[~sel & full].all(), "modes as built"
    o_p, _, _, _, _ = run(q, kv, sink, idx, sc, flags=PER_QUERY)
    oc, opc = o.cpu(), o_p.cpu()
    assert torch.equal(oc[0, pq], opc[0, pq])
    d = (oc.float() - opc.float()).abs()
    say(f"  long-cache index kernel, topk {topk}: shared vs per query max {d.max().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3
    s = [0, 9, 8 * 3 * 5, m // 2, m - 1]
    check(oc[:, s], sparse_attn_fp64(q[:, s], kv, sink, idx[:, s], sc), f"long-cache index {topk}")

def test_index_bitmap_mode_bad_index(gpu_sa):
    """kv_len 12 000, topk 64: the index kernel decides each tile's mode from
    a bitmap of its rows before it counts them. An out-of-range index in a
    shared tile and one in a per-query tile set the error word; every other
    slot counts, as in the oracle with those two slots masked."""
    m = 8 * 40
    q, kv, sink, idx, sc = case(1, m, 12000, 64, seed=91, minus1=0.05)
    t = torch.arange(m)
    win = ((torch.arange(64)[None] + t[:, None]) % 12000).to(torch.int32)
    sel = (t // 8) % 2 == 0
    idx[0, sel] = win[sel]
    idx[0, 3, 10] = 12000            # a shared tile (tile 0)
    idx[0, 9, 20] = -5               # a per-query tile (tile 1)
    o, _, mask, err, ws = run(q, kv, sink, idx, sc)
    assert err == 1 and mask & INDEX
    pq = per_query_queries(ws, 1, m)[0]
    assert not pq[:8].any() and pq[8:16].all()
    ok = idx.clone()
    ok[0, 3, 10] = -1
    ok[0, 9, 20] = -1
    check(o, sparse_attn_fp64(q, kv, sink, ok, sc), "bitmap mode, bad index")
