"""GPU parity of the shared-row tile path (index kernel + tile kernel) against
the float64 oracle and against the per-query path on the same inputs.

Tolerance as in test_gpu_parity: max |err| <= 2e-2, mean |err| <= 2e-3,
relative RMS <= 5e-3 against float64; exact zeros for all -1 rows.
"""
import numpy as np
import pytest
import torch

from oracle import sparse_attn_fp64
from sa_testutil import expect_plan
from test_gpu_parity import DEV, check, config, sampled_check, say
import sa_workloads as wl

pytestmark = pytest.mark.gpu

PER_QUERY, FORCE_TILES = 1, 2


def run(q, kv, sink, idx, scale, flags=0, check_err=True):
    err = torch.zeros(1, dtype=torch.int32, device=DEV) if check_err else None
    o = torch.ops.sa_amd.sparse_attn_fwd(q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV),
                                         float(scale), err, flags)
    if err is not None:
        assert int(err.item()) == 0
    return o


def rand_case(b, m, kv_len, topk, seed, minus1=0.0, sink_std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g) * sink_std
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q, kv, sink, idx, wl.SCALE


def test_causal_prefill_tiles_vs_per_query(gpu_sa):
    """Full config through both paths: sampled oracle check of the default
    (tile) path, and every query of the two paths against each other."""
    q, kv, sink, idx, sc = config("causal_prefill")
    o_t = run(q, kv, sink, idx, sc)
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY)
    ts = [0, 1, 2, 3, 4, 5, 6, 7, 2044, 2045, 2046, 2047, 2048, 2049, 4092, 4093, 4094, 4095]
    ts += torch.randint(0, 4096, (30,), generator=torch.Generator().manual_seed(9)).tolist()
    sampled_check(o_t, q, kv, sink, idx, sc, [(0, t) for t in ts], "causal tiles")
    d = (o_t.float() - o_p.float()).abs()
    say(f"  tiles vs per-query: max {d.max().item():.3e} mean {d.mean().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3


def test_high_locality_tiles_vs_per_query(gpu_sa):
    q, kv, sink, idx, sc = config("high_locality")
    o_t = run(q, kv, sink, idx, sc)
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY)
    d = (o_t.float() - o_p.float()).abs()
    say(f"  tiles vs per-query: max {d.max().item():.3e} mean {d.mean().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3
    sel = [(0, 0), (0, 1), (1, 2), (2, 3), (3, 508), (3, 511)]
    sampled_check(o_t, q, kv, sink, idx, sc, sel, "high locality tiles")


@pytest.mark.parametrize("m", [4, 5, 7, 8, 9, 13, 16, 23])
def test_forced_tiles_ragged_m(gpu_sa, m):
    q, kv, sink, idx, sc = rand_case(2, m, 300, 64, seed=100 + m, minus1=0.2)
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    check(o, sparse_attn_fp64(q, kv, sink, idx, sc), f"forced tiles m={m}")


def test_forced_tiles_many_queries_long_topk(gpu_sa):
    # 260 queries >= CUs: no split, so topk > 64 can take the tile path
    q, kv, sink, idx, sc = rand_case(1, 260, 5000, 700, seed=7, minus1=0.1)
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    sel = [(0, m) for m in (0, 1, 2, 3, 100, 255, 256, 257, 258, 259)]
    sampled_check(o, q, kv, sink, idx, sc, sel, "forced tiles topk=700")
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY)
    assert (o.float() - o_p.float()).abs().max().item() <= 2e-2


def test_tile_duplicates_multiplicity(gpu_sa):
    """Duplicates inside a query and shared rows across queries of a tile."""
    q, kv, sink, idx, sc = rand_case(1, 8, 40, 64, seed=21)  # 64 draws from 40 rows
    idx[0, 0, :32] = 5       # one row 32 times
    idx[0, 1, ::2] = 7
    idx[0, 2] = 9            # every slot the same row: 64-fold
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    check(o, sparse_attn_fp64(q, kv, sink, idx, sc), "tile duplicates")


def test_tile_reference_jump_falls_back(gpu_sa):
    """A column whose scores jump far above its first step's max makes the tile
    hand itself to the per-query code (the tile kernel never rescales O): that
    tile's queries then match the plain per-query plan (one wave per query:
    same math, other summation order) and the oracle."""
    # 256 queries: the plan must not split them, so the tile path runs
    q, kv, sink, idx, sc = rand_case(1, 256, 200, 128, seed=28)
    expect_plan(q, kv, idx, FORCE_TILES, tiles=True, nsplit=1)
    kv[0, 150] = (q[0, 2].float().mean(0) * 60).to(torch.bfloat16)  # a row matching query 2
    idx[0, 2, :64] = torch.arange(64, dtype=torch.int32)   # first step: ordinary rows
    idx[0, 2, 64] = 150                                     # later: a huge score
    o_t = run(q, kv, sink, idx, sc, flags=FORCE_TILES).cpu()
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY).cpu()
    a8, p8 = o_t[0, :8].double(), o_p[0, :8].double()     # tile 0 ran per query
    assert ((a8 - p8).pow(2).mean() / p8.pow(2).mean()).sqrt().item() <= 5e-3
    exp = sparse_attn_fp64(q, kv, sink, idx, sc)
    err = o_t.double().numpy() - exp
    rel = float(np.sqrt((err ** 2).mean() / (exp ** 2).mean()))
    say(f"  reference jump: rel_rms={rel:.3e}")
    assert rel <= 5e-3


def test_tile_count_overflow_falls_back(gpu_sa):
    """A row repeated more than 255 times in one query cannot be counted in a
    byte; that tile runs per query and stays exact."""
    q, kv, sink, idx, sc = rand_case(1, 300, 50, 300, seed=22)
    idx[0, 1] = 3            # 300 copies
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    sel = [(0, 0), (0, 1), (0, 2), (0, 3), (0, 4), (0, 299)]
    sampled_check(o, q, kv, sink, idx, sc, sel, "count overflow")


def test_tile_all_masked_queries(gpu_sa):
    q, kv, sink, idx, sc = rand_case(1, 12, 100, 64, seed=23, minus1=0.3)
    idx[0, 8:12] = -1        # a whole (ragged) tile without valid slots
    idx[0, 3] = -1           # one all -1 query inside a tile
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES).cpu()
    assert torch.all(o[0, 8:12] == 0) and torch.all(o[0, 3] == 0)
    check(o, sparse_attn_fp64(q, kv, sink, idx, sc), "masked tiles")


def test_tile_largest_count_table(gpu_sa):
    """kv_len = 16384 needs the 128 KiB count table (dynamic LDS)."""
    q, kv, sink, idx, sc = rand_case(1, 16, 16384, 64, seed=24)
    idx[0, :, :32] = torch.arange(16384 - 32, 16384, dtype=torch.int32)  # top rows, shared
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    check(o, sparse_attn_fp64(q, kv, sink, idx, sc), "kv_len 16384 tiles")


def test_tile_out_of_range_reported(gpu_sa):
    q, kv, sink, idx, sc = rand_case(1, 8, 100, 64, seed=25)
    idx[0, 5, 10] = 100
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    o = torch.ops.sa_amd.sparse_attn_fwd(q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV),
                                         sc, err, FORCE_TILES)
    assert int(err.item()) == 1
    fixed = idx.clone()
    fixed[0, 5, 10] = -1
    check(o, sparse_attn_fp64(q, kv, sink, fixed, sc), "tile bad index skipped")


def test_tile_sink_visible_and_exact_rows(gpu_sa):
    """q = 0, sink = -inf and a tile whose queries share rows: every query's output
    is exactly the mean of its rows when the rows are duplicates of one row."""
    _, kv, _, _, sc = rand_case(1, 1, 64, 1, seed=26)
    q = torch.zeros(1, 4, 16, 512, dtype=torch.bfloat16)
    sink = torch.full((16,), float("-inf"))
    idx = torch.full((1, 4, 8), -1, dtype=torch.int32)
    idx[0, 0, 0] = 11
    idx[0, 1, [1, 2]] = 11        # same row twice
    idx[0, 2, [0, 3, 5, 7]] = 30  # another row four times
    idx[0, 3, 4] = 30
    o = run(q, kv, sink, idx, sc, flags=FORCE_TILES).cpu()
    for mi, r in ((0, 11), (1, 11), (2, 30), (3, 30)):
        assert torch.equal(o[0, mi], kv[0, r].expand(16, -1)), mi


def test_tiles_deterministic(gpu_sa):
    q, kv, sink, idx, sc = rand_case(1, 260, 2000, 256, seed=27)
    expect_plan(q, kv, idx, FORCE_TILES, tiles=True, nsplit=1)
    a = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    b = run(q, kv, sink, idx, sc, flags=FORCE_TILES)
    assert torch.equal(a, b)


def test_per_query_tiles_match_direct_launch(gpu_sa):
    """A tile plan whose tiles all go per query (low overlap): the per-query
    launch after the shared-row kernel runs them, one work-group per query
    of the plan reading its tile's mode, with a ragged last tile. Each query
    must equal the direct per-query launch bit for bit, and the sampled
    oracle check must pass."""
    q, kv, sink, idx, sc = rand_case(1, 300, 16384, 256, seed=21, minus1=0.1)
    expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    o_l = run(q, kv, sink, idx, sc)
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY)
    # tiles 0..36 (8 random queries each: dense work ~8x the valid slots) run
    # per query; so may the last tile's 4
    assert torch.equal(o_l[:, :296], o_p[:, :296])
    d = (o_l.float() - o_p.float()).abs()
    assert d.max().item() <= 2e-2
    sampled_check(o_l, q, kv, sink, idx, sc, [(0, t) for t in (0, 1, 150, 295, 296, 299)],
                  "per-query tiles")


def mixed_many_tiles(seed):
    """2 x 4400 queries (1100 tiles, more than the order kernel's 1024
    threads), every third tile of overlapping windows (shared), the others
    128 random rows of 4096 (per query), ragged last tiles."""
    q, kv, sink, idx, sc = rand_case(2, 4400, 4096, 128, seed=seed)
    t = torch.arange(4400)
    win = ((torch.arange(128)[None] + 3 * t[:, None]) % 4096).to(torch.int32)
    sel = (t // 8) % 3 == 0
    idx[:, sel] = win[sel]
    return q, kv, sink, idx, sc, sel


def test_per_query_tiles_strided_over_many_tiles(gpu_sa):
    """The per-query launch after the shared-row kernel strides over the
    per-query tiles' queries, which the order kernel lists in tile order after
    the shared tiles: those queries equal the direct per-query launch bit for
    bit, the shared tiles' agree within the tolerance, and a sample matches
    the oracle."""
    q, kv, sink, idx, sc, sel = mixed_many_tiles(seed=31)
    expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    o = run(q, kv, sink, idx, sc).cpu()
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY).cpu()
    assert torch.equal(o[:, ~sel], o_p[:, ~sel])
    d = (o.float() - o_p.float()).abs()
    say(f"  strided per-query tiles: max {d.max().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3
    sampled_check(o, q, kv, sink, idx, sc,
                  [(0, 0), (0, 9), (1, 23), (1, 2401), (0, 4391), (1, 4399)], "strided")


def test_per_query_tiles_mixed_with_aborted_tile(gpu_sa):
    """Shared tiles, per-query tiles from the index kernel and a tile that
    aborts at run time (scores jump far above its reference) in one call: the
    aborted tile's work-group runs its queries per query itself, and the
    per-query tiles' queries run in the per-query launch after the shared-row
    kernel."""
    # 256 queries (the plan must not split them); 512 random rows of 8192 per
    # query leave a tile's dense work ~7.6x its valid slots, so those tiles go
    # to the per-query kernel
    q, kv, sink, idx, sc = rand_case(1, 256, 8192, 512, seed=22)
    expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    # queries 0..31: overlapping windows (shared tiles); 32..255 stay random
    # (per-query tiles from the index kernel)
    for t in range(32):
        idx[0, t] = torch.arange(512, dtype=torch.int32) + 4 * t
    # tile 1 (queries 8..15): a last row whose score for query 8 is far above
    # everything the tile's first step sees
    idx[0, 8:16, -1] = 2000
    kv[0, 2000] = (q[0, 8].float().mean(0) * 60).to(torch.bfloat16)
    o = run(q, kv, sink, idx, sc).cpu()
    o_p = run(q, kv, sink, idx, sc, flags=PER_QUERY).cpu()
    d = (o.float() - o_p.float()).abs()
    d[0, 8:16] = 0  # |o| up to ~20 there: compared by relative RMS below
    say(f"  mixed list: max {d.max().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3
    # the aborted tile ran per query in the tile kernel (the 4-wave per-query
    # code); the plain plan runs its queries one wave each: same math, other
    # summation order
    a8, p8 = o[0, 8:16].double(), o_p[0, 8:16].double()
    assert ((a8 - p8).pow(2).mean() / p8.pow(2).mean()).sqrt().item() <= 5e-3
    assert torch.equal(o[0, 32:], o_p[0, 32:])     # per-query tiles
    sampled_check(o, q, kv, sink, idx, sc, [(0, t) for t in (0, 7, 16, 31, 40, 255)], "mixed")
    # row 2000 dominates queries 8..15 (|o| up to ~20, bf16 ulp 0.125 there):
    # relative RMS against float64 instead of the absolute bound
    exp = sparse_attn_fp64(q[:, 8:16], kv, sink, idx[:, 8:16], sc)
    err = o[:, 8:16].double().numpy() - exp
    rel = float(np.sqrt((err ** 2).mean() / (exp ** 2).mean()))
    say(f"  aborted tile: rel_rms={rel:.3e}")
    assert rel <= 5e-3


TILE_SKIP, TILE_DENSE = 8, 16


def run_lse(q, kv, sink, idx, scale, flags):
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    o, lse = torch.ops.sa_amd.sparse_attn_fwd_lse(q.to(DEV), kv.to(DEV), sink.to(DEV),
                                                  idx.to(DEV), float(scale), err, flags)
    assert int(err.item()) == 0
    return o, lse


def windows_case(b, m, kv_len, nwin, seed, keep=0.75):
    """High-locality-style indices: each query takes nwin 64-row windows,
    keeping the previous query's starts with probability `keep`."""
    q, kv, sink, idx, sc = rand_case(b, m, kv_len, 64 * nwin, seed)
    g = torch.Generator().manual_seed(seed + 1)
    for bi in range(b):
        starts = 64 * torch.randperm(kv_len // 64, generator=g)[:nwin]
        for t in range(m):
            if t and torch.rand(1, generator=g).item() >= keep:
                starts = 64 * torch.randperm(kv_len // 64, generator=g)[:nwin]
            s = torch.sort(starts).values
            idx[bi, t] = (s[:, None] + torch.arange(64)[None]).reshape(-1).to(torch.int32)
    return q, kv, sink, idx, sc


def skip_cases():
    cases = {"windows": windows_case(2, 64, 8192, 6, seed=41),
             "dense random": rand_case(1, 64, 512, 256, seed=42, minus1=0.3),
             "ragged m": rand_case(1, 13, 2048, 64, seed=43, minus1=0.1)}
    # duplicates, -1 padding in the middle of rows, an all-masked tile and a
    # tile whose union ends inside a 64-row step
    q, kv, sink, idx, sc = windows_case(1, 40, 4096, 3, seed=44)
    idx[0, 3, 5:20] = idx[0, 3, 0]        # one row named 16 times
    idx[0, 9, ::3] = -1
    idx[0, 16:24] = -1                    # tile 2: no valid slot
    idx[0, 32:40, 100:] = -1              # tile 4: 100 slots per query
    cases["edge"] = (q, kv, sink, idx, sc)
    return cases


@pytest.mark.parametrize("name", ["windows", "dense random", "ragged m", "edge"])
def test_tile_forms_bit_identical(gpu_sa, name):
    """The pair-skipping and the dense form of the shared-row step give the
    same bits (o and lse): per accumulator they run the same MFMAs in the same
    order, and a skipped block would only add zeros. Both are also held to
    the float64 oracle on a sample."""
    q, kv, sink, idx, sc = skip_cases()[name]
    o_s, l_s = run_lse(q, kv, sink, idx, sc, FORCE_TILES | TILE_SKIP)
    o_d, l_d = run_lse(q, kv, sink, idx, sc, FORCE_TILES | TILE_DENSE)
    assert torch.equal(o_s, o_d) and torch.equal(l_s, l_d)
    b, m = idx.shape[:2]
    sel = sorted({(bi, t) for bi in range(b) for t in (0, 1, 7, 8, 17, m - 1) if t < m})
    sampled_check(o_s, q, kv, sink, idx, sc, sel, f"tile skip form, {name}")


def test_tile_forms_aborted_tile(gpu_sa):
    """A tile whose scores jump above its reference aborts to the per-query
    code in both forms; the outputs agree bit for bit."""
    q, kv, sink, idx, sc = windows_case(1, 16, 4096, 4, seed=45)
    idx[0, 8:16, -1] = 2000
    kv[0, 2000] = (q[0, 8].float().mean(0) * 60).to(torch.bfloat16)
    o_s = run(q, kv, sink, idx, sc, flags=FORCE_TILES | TILE_SKIP)
    o_d = run(q, kv, sink, idx, sc, flags=FORCE_TILES | TILE_DENSE)
    assert torch.equal(o_s, o_d)


def test_tile_form_flags_refused_together(gpu_sa):
    q, kv, sink, idx, sc = rand_case(1, 8, 256, 32, seed=46)
    with pytest.raises((ValueError, RuntimeError)):
        run(q, kv, sink, idx, sc, flags=TILE_SKIP | TILE_DENSE)
