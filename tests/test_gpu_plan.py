"""GPU tests of the index plan (sparse_attn_plan / sa_plan_indices +
SA_FLAG_PLANNED): a planned call equals the unplanned call bit for bit on
every plan kind, one plan serves calls with other q, kv values and sinks, and
the Python layer refuses a plan whose indices changed."""
import ctypes

import pytest
import torch

from test_gpu_parity import DEV, sampled_check, say
import sa_capi
from sa_testutil import expect_plan
import sa_workloads as wl

pytestmark = pytest.mark.gpu

TILE, QUERY, INDEX, ORDER, COMBINE, WAVE = 1 << 2, 1 << 3, 1 << 0, 1 << 1, 1 << 4, 1 << 5


def case(b, m, kv_len, topk, seed, minus1=0.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV), wl.SCALE


def windows(b, m, kv_len, seed, tiles=True):
    """Overlapping windows: shared tiles when b * m is large enough that no
    query is split (asserted unless `tiles` is False)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    idx = torch.stack([torch.arange(256, dtype=torch.int32) + 3 * t for t in range(m)])
    idx = idx[None].repeat(b, 1, 1) % kv_len
    idx[:, ::5, 200:] = -1
    if tiles:
        expect_plan(q, kv, idx, 0, tiles=True, nsplit=1)
    return q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV), wl.SCALE


CASES = {
    "shared tiles": lambda: windows(2, 157, 3000, seed=1),
    "per-query tiles": lambda: case(1, 300, 16384, 256, seed=2, minus1=0.1),
    "split (decode)": lambda: case(8, 1, 32768, 2048, seed=3),
    "per query, no split": lambda: case(1, 400, 20000, 128, seed=4, minus1=0.2),
}


@pytest.mark.parametrize("name", list(CASES))
def test_planned_equals_unplanned(gpu_sa, name):
    q, kv, sink, idx, sc = CASES[name]()
    plan = gpu_sa.sparse_attn_plan(q, kv, idx)
    o0, l0 = gpu_sa.sparse_attn_with_lse(q, kv, sink, idx, sc)
    for rep in range(2):
        o1, l1 = gpu_sa.sparse_attn_with_lse(q, kv, sink, idx, sc, plan=plan)
        assert torch.equal(o0, o1) and torch.equal(l0, l1)
    assert torch.equal(gpu_sa.sparse_attn(q, kv, sink, idx, sc, plan=plan), o0)


def test_plan_serves_other_values(gpu_sa):
    """One plan, three calls with fresh q, kv values and sinks: each equals
    its own unplanned call, and the oracle on sampled queries."""
    q, kv, sink, idx, sc = windows(1, 300, 4096, seed=5)
    plan = gpu_sa.sparse_attn_plan(q, kv, idx)
    g = torch.Generator(device=DEV).manual_seed(6)
    for rep in range(3):
        q2 = torch.randn(q.shape, generator=g, device=DEV).to(torch.bfloat16)
        kv2 = torch.randn(kv.shape, generator=g, device=DEV).to(torch.bfloat16)
        s2 = torch.randn(16, generator=g, device=DEV) * 2
        o_p = gpu_sa.sparse_attn(q2, kv2, s2, idx, sc, plan=plan)
        o_u = gpu_sa.sparse_attn(q2, kv2, s2, idx, sc)
        assert torch.equal(o_p, o_u)
    sampled_check(o_p, q2.cpu(), kv2.cpu(), s2.cpu(), idx.cpu(), sc,
                  [(0, t) for t in (0, 7, 8, 31, 299)], "planned")


def test_plan_refuses_changed_indices(gpu_sa):
    q, kv, sink, idx, sc = windows(1, 16, 1000, seed=7, tiles=False)
    plan = gpu_sa.sparse_attn_plan(q, kv, idx)
    with pytest.raises(ValueError):
        gpu_sa.sparse_attn(q, kv, sink, idx.clone(), sc, plan=plan)      # other tensor
    with pytest.raises(ValueError):
        gpu_sa.sparse_attn(q[:, :8], kv, sink, idx[:, :8], sc, plan=plan)  # other shapes
    idx[0, 0, 0] = 5                                                     # modified in place
    with pytest.raises(ValueError):
        gpu_sa.sparse_attn(q, kv, sink, idx, sc, plan=plan)
    say("  stale plans refused")


def test_plan_reports_bad_index(gpu_sa):
    q, kv, sink, idx, sc = windows(1, 300, 1000, seed=8)   # a tile plan: checked there
    idx[0, 3, 10] = 1000                                   # == kv_len: out of range
    with pytest.raises(RuntimeError):
        gpu_sa.sparse_attn_plan(q, kv, idx)


def test_plan_of_an_aborting_tile(gpu_sa):
    """A tile whose scores jump far above its reference runs per query inside
    the shared-row kernel; planned, it does so again on every call."""
    q, kv, sink, idx, sc = case(1, 256, 200, 128, seed=28)
    expect_plan(q, kv, idx, gpu_sa.FLAG_FORCE_TILES, tiles=True, nsplit=1)
    kv[0, 150] = (q[0, 2].float().mean(0) * 60).to(torch.bfloat16)
    idx[0, 2, :64] = torch.arange(64, dtype=torch.int32, device=DEV)
    idx[0, 2, 64] = 150
    gpu_sa.set_path_flags(gpu_sa.FLAG_FORCE_TILES)
    try:
        plan = gpu_sa.sparse_attn_plan(q, kv, idx)
        o_u = gpu_sa.sparse_attn(q, kv, sink, idx, sc)
        o_p = gpu_sa.sparse_attn(q, kv, sink, idx, sc, plan=plan)
        o_p2 = gpu_sa.sparse_attn(q, kv, sink, idx, sc, plan=plan)
    finally:
        gpu_sa.set_path_flags(0)
    assert torch.equal(o_u, o_p) and torch.equal(o_p, o_p2)


@pytest.mark.parametrize("shape,plain,planned", [
    # short queries: one wave each; neither call launches ORDER (the tile
    # launch walks the tiles' modes)
    ((1, 64, 300, 64), INDEX | WAVE | TILE, WAVE | TILE),
    ((1, 300, 2048, 700), INDEX | QUERY | TILE, QUERY | TILE),
    ((4, 1, 2048, 512), QUERY | COMBINE, QUERY | COMBINE),
    ((1, 3, 2048, 64), WAVE, WAVE),
])
def test_capi_planned_launches(gpu_sa, shape, plain, planned):
    q, kv, sink, idx, sc = case(*shape, seed=sum(shape))
    lib = sa_capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    a = sa_capi.make_args(q, kv, sink, idx, o, sc)
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    none = [None] * (2 * sa_capi.SA_KERNEL_COUNT)
    assert sa_capi.forward_events(lib, a, stream, none) == plain
    ref = o.clone()
    o.fill_(float("nan"))
    ws2 = torch.full((max(n, 1),), 0xAB, dtype=torch.uint8, device=DEV)  # a fresh workspace
    a.workspace = ws2.data_ptr()
    sa_capi.check(lib, lib.sa_plan_indices(ctypes.byref(a), ctypes.c_void_p(stream)), "plan")
    a.flags = sa_capi.SA_FLAG_PLANNED
    assert sa_capi.forward_events(lib, a, stream, none) == planned
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


def mixed_long(m, seed):
    """topk 448 (above the one-wave kernel's): every third tile of windows
    (shared), the others random rows of 8192 (per query), -1 slots."""
    q, kv, sink, idx, sc = case(1, m, 8192, 448, seed=seed, minus1=0.05)
    t = torch.arange(m, device=DEV)
    win = ((torch.arange(448, device=DEV)[None] + 5 * t[:, None]) % 8192).to(torch.int32)
    sel = (t // 8) % 3 == 0
    idx[0, sel] = win[sel]
    return q, kv, sink, idx, sc


def placed_cases():
    """Shapes whose tiles number between half the CUs and the CUs: the plain
    call places them itself (no order kernel)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    m = 8 * cus  # cus tiles
    return {
        "high locality": lambda: (*[x.to(DEV) for x in wl.make_config_inputs("high_locality")[:4]],
                                  wl.SCALE),
        "windows, ragged": lambda: windows(1, m - 5, 3000, seed=12),
        "per-query tiles": lambda: case(1, m // 2 + 8, 16384, 256, seed=13, minus1=0.1),
        "mixed, bad index": lambda: case(2, m // 2, 700, 128, seed=14, minus1=0.3),
        "per-query tiles, long topk": lambda: case(1, m // 2 + 8, 16384, 512, seed=15,
                                                   minus1=0.1),
        "mixed, long topk": lambda: mixed_long(m - 11, seed=16),
    }


@pytest.mark.parametrize("name", ["high locality", "windows, ragged", "per-query tiles",
                                  "mixed, bad index", "per-query tiles, long topk",
                                  "mixed, long topk"])
def test_placed_tiles_match_ordered(gpu_sa, name):
    """A plain call in the placed regime equals the planned call, whose tiles
    run in the tile order's placement, bit for bit (o, lse and the error
    word). The plain call makes no tile order; with topk up to 384 the short
    queries run one wave each and the tile launch scans for shared tiles."""
    q, kv, sink, idx, sc = placed_cases()[name]()
    if name == "mixed, bad index":
        idx[1, 17, 3] = kv.shape[1] + 5
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lib = sa_capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for planned in (False, True):
        o = torch.full_like(q, float("nan"))
        lse = torch.full(q.shape[:3], float("nan"), device=DEV)
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        a = sa_capi.make_args(q, kv, sink, idx, o, sc, err=err, lse=lse)
        n = sa_capi.workspace_bytes(lib, a)
        ws = torch.full((max(n, 1),), 0xAB, dtype=torch.uint8, device=DEV)
        a.workspace, a.workspace_bytes = ws.data_ptr(), n
        if planned:
            sa_capi.check(lib, lib.sa_plan_indices(ctypes.byref(a), ctypes.c_void_p(stream)),
                          "plan")
            a.flags = sa_capi.SA_FLAG_PLANNED
        none = [None] * (2 * sa_capi.SA_KERNEL_COUNT)
        launched = sa_capi.forward_events(lib, a, stream, none)
        torch.cuda.synchronize()
        outs.append((o, lse, int(err.item()), launched))
    (o1, l1, e1, k1), (o2, l2, e2, k2) = outs
    expect_plan(q, kv, idx, tiles=True)
    ntiles = q.shape[0] * -(-q.shape[1] // 8)
    assert 2 * ntiles >= cus and ntiles <= cus, "the shape must be in the placed regime"
    # topk <= 384: the per-query tiles run one wave per query; above, in the
    # QUERY launch (a placed call has no order to make)
    pq = WAVE if idx.shape[2] <= 384 else QUERY
    assert k1 == INDEX | pq | TILE and k2 == pq | TILE
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert e1 == e2 == (1 if name == "mixed, bad index" else 0)
    samples = {"high locality": [(0, 0), (1, 129), (2, 300), (3, 511)],
               "per-query tiles, long topk": [(0, 0), (0, q.shape[1] - 1)],
               "mixed, long topk": [(0, 1), (0, 9), (0, q.shape[1] - 1)]}
    if name in samples:  # and the values themselves, on a sample
        sampled_check(o1, q.cpu(), kv.cpu(), sink.cpu(), idx.cpu(), sc, samples[name],
                      f"placed {name}")
