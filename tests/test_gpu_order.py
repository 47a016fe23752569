"""GPU test of the tile order that the index plan writes (sa_plan_indices,
read back from the workspace): it is a permutation of the tiles; the shared
tiles come first, each with key 1 + its step count, and the per-query tiles
after them with key 0. When
the shared tiles outnumber the CUs they run longest first. When every one
starts at once (at most one per CU) each XCD gets one contiguous run of them
in tile order: work-group i runs on XCD i % 8, so slot i holds the
(first_x + i // 8)-th shared tile of XCD x = i % 8."""
import ctypes
import os

import pytest
import torch

import sa_capi
import sa_workloads as wl
from test_gpu_parity import DEV, say
from test_gpu_plan import case, windows

pytestmark = pytest.mark.gpu

TILE_BITS = 22
MODE_SHARED = 1
XCDS = 8
PLAN_KEYS = ["nsplit", "split_len", "tiles", "tiles_per_b", "ntiles", "tile_cap", "ws",
             "meta_off", "order_off", "rows_off", "cnts_off", "part_off"]


def host_plan(a, cus):
    """The launch plan (workspace offsets) the library makes for these args."""
    host = ctypes.CDLL(os.path.join(os.path.dirname(sa_capi.LIB_PATH), "libsa_host_test.so"))
    host.sa_host_plan_full.argtypes = [ctypes.c_void_p, ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_int64)]
    out = (ctypes.c_int64 * len(PLAN_KEYS))()
    assert host.sa_host_plan_full(ctypes.addressof(a), cus, out) == 0
    return dict(zip(PLAN_KEYS, list(out)))


def causal(m, kv_len, topk, seed):
    """Causal indices: query t names min(t + 1, topk) distinct rows of [0, t]."""
    g = torch.Generator().manual_seed(seed)
    idx = torch.full((1, m, topk), -1, dtype=torch.int32)
    for t in range(m):
        n = min(t + 1, topk)
        idx[0, t, :n] = torch.randperm(t + 1, generator=g)[:n].to(torch.int32)
    q = torch.randn(1, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(1, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    return q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV), wl.SCALE


def high_locality():
    q, kv, sink, idx, sc = wl.make_config_inputs("high_locality", seed=0)
    return q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV), sc


def mixed_many():
    """1100 tiles, every third of overlapping windows (shared), the others
    random (per query): the sorted order over several passes."""
    q, kv, sink, idx, sc = case(2, 4400, 4096, 128, seed=3)
    t = torch.arange(4400)
    win = ((torch.arange(128)[None] + 3 * t[:, None]) % 4096).to(torch.int32)
    sel = ((t // 8) % 3 == 0).to(DEV)
    idx[:, sel] = win.to(DEV)[sel]
    return q, kv, sink, idx, sc


CASES = {
    "causal, more shared tiles than CUs": lambda: causal(2560, 2560, 1024, seed=5),
    "high locality, one tile per CU": high_locality,
    "shared tiles, few": lambda: windows(2, 157, 3000, seed=1),
    "per-query tiles": lambda: case(1, 300, 16384, 256, seed=2, minus1=0.1),
    "mixed, more tiles than the order kernel's threads": lambda: mixed_many(),
}


@pytest.mark.parametrize("name", list(CASES))
def test_tile_order(name):
    say(f"tile order: {name}")
    q, kv, sink, idx, sc = CASES[name]()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lib = sa_capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    a = sa_capi.make_args(q, kv, sink, idx, o, sc)
    p = host_plan(a, cus)
    assert p["tiles"] == 1
    n = sa_capi.workspace_bytes(lib, a)
    assert n == p["ws"]
    ws = torch.full((n,), 0xAB, dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    sa_capi.check(lib, lib.sa_plan_indices(ctypes.byref(a), ctypes.c_void_p(stream)), "plan")
    torch.cuda.synchronize()
    nt = p["ntiles"]
    meta = ws[p["meta_off"]:p["meta_off"] + 16 * nt].view(torch.int32).view(nt, 4).cpu()
    order = ws[p["order_off"]:p["order_off"] + 4 * nt].view(torch.int32).cpu()

    shared = meta[:, 1] == MODE_SHARED
    want_key = torch.where(shared, (meta[:, 0] + 63) // 64 + 1, torch.zeros_like(meta[:, 0]))
    tiles = order & ((1 << TILE_BITS) - 1)
    keys = order >> TILE_BITS
    assert torch.equal(torch.sort(tiles).values, torch.arange(nt, dtype=torch.int32))
    assert torch.equal(keys, want_key[tiles.long()])
    ns = int(shared.sum())
    assert bool((keys[:ns] > 0).all()) and bool((keys[ns:] == 0).all())
    # up to the 16 384 tiles whose keys the order keeps in LDS, the per-query
    # tiles are placed by rank (no atomics): in tile order
    assert bool((tiles[ns:][1:] > tiles[ns:][:-1]).all()), "per-query tiles in tile order"
    if ns > cus:
        assert bool((keys[:ns][1:] <= keys[:ns][:-1]).all()), "longest first"
    else:
        ids = torch.nonzero(shared).flatten().tolist()  # shared tiles in tile order
        counts = [(ns - x + XCDS - 1) // XCDS for x in range(XCDS)]
        first = [sum(counts[:x]) for x in range(XCDS)]
        want = [ids[first[s % XCDS] + s // XCDS] for s in range(ns)]
        assert tiles[:ns].tolist() == want


def test_tile_order_beyond_key_cache():
    """More tiles (16 400) than the order keeps keys for in LDS (16 384): the
    keys are loaded again in the second pass and per-query tiles are placed
    by one LDS atomic per wave. Tiles alternate in runs between 32 shared
    rows (every query of the tile names the same window: shared) and 32
    random rows of 4 096 per query (union about 250 rows: per query). Only
    the plan runs (sa_plan_indices); q and o are allocated, never read."""
    b, m, kv_len, topk = 1, 8 * 16400, 4096, 32
    say(f"tile order beyond the key cache: {m // 8} tiles")
    g = torch.Generator().manual_seed(21)
    t = torch.arange(m)
    win = ((torch.arange(topk)[None] + 64 * ((t // 8) % 60)[:, None]) % kv_len).to(torch.int32)
    rnd = torch.randint(0, kv_len, (m, topk), generator=g, dtype=torch.int32)
    sel = (((t // 8) // 7) % 2 == 0)[:, None]
    idx = torch.where(sel, win, rnd)[None].to(DEV)
    q = torch.empty(b, m, 16, 512, dtype=torch.bfloat16, device=DEV)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16).to(DEV)
    sink = torch.zeros(16, device=DEV)
    o = torch.empty_like(q)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lib = sa_capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    a = sa_capi.make_args(q, kv, sink, idx, o, wl.SCALE)
    p = host_plan(a, cus)
    assert p["tiles"] == 1 and p["ntiles"] == 16400
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.full((n,), 0xAB, dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    sa_capi.check(lib, lib.sa_plan_indices(ctypes.byref(a), ctypes.c_void_p(stream)), "plan")
    torch.cuda.synchronize()
    nt = p["ntiles"]
    meta = ws[p["meta_off"]:p["meta_off"] + 16 * nt].view(torch.int32).view(nt, 4).cpu()
    order = ws[p["order_off"]:p["order_off"] + 4 * nt].view(torch.int32).cpu()
    shared = meta[:, 1] == MODE_SHARED
    ns = int(shared.sum())
    assert 0 < ns < nt, "the case needs shared and per-query tiles"
    want_key = torch.where(shared, (meta[:, 0] + 63) // 64 + 1, torch.zeros_like(meta[:, 0]))
    tiles = order & ((1 << TILE_BITS) - 1)
    keys = order >> TILE_BITS
    assert torch.equal(torch.sort(tiles).values, torch.arange(nt, dtype=torch.int32))
    assert torch.equal(keys, want_key[tiles.long()])
    assert bool((keys[:ns] > 0).all()) and bool((keys[ns:] == 0).all())
    assert bool((keys[:ns][1:] <= keys[:ns][:-1]).all()), "longest first"
