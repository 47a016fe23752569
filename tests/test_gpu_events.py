"""GPU tests of the C-ABI's per-kernel event hook (sa_forward_events) through
the ctypes binding: same output as the torch operator, the expected kernels
launched for each plan, and timed events."""
import ctypes

import pytest
import torch

from test_gpu_parity import DEV
import sa_capi

pytestmark = pytest.mark.gpu

TILE, QUERY, INDEX, ORDER, COMBINE, WAVE = 1 << 2, 1 << 3, 1 << 0, 1 << 1, 1 << 4, 1 << 5


def case(b, m, kv_len, topk, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16).to(DEV)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16).to(DEV)
    sink = torch.randn(16, generator=g).to(DEV)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32).to(DEV)
    return q, kv, sink, idx, 512 ** -0.5


@pytest.mark.parametrize("shape,expect", [
    ((1, 64, 300, 64), INDEX | WAVE | TILE),            # shared-row plan, short queries
    ((1, 300, 2048, 700), INDEX | QUERY | TILE),        # topk above the wave kernel's
    ((4, 1, 2048, 512), QUERY | COMBINE),               # split-topk plan
    ((1, 3, 2048, 64), WAVE),                           # per query, no split
])
def test_events_hook_matches_operator(gpu_sa, shape, expect):
    q, kv, sink, idx, sc = case(*shape, seed=sum(shape))
    ref = torch.ops.sa_amd.sparse_attn_fwd(q, kv, sink, idx, sc, None, 0)
    lib = sa_capi.load()
    o = torch.full_like(q, float("nan"))
    a = sa_capi.make_args(q, kv, sink, idx, o, sc)
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    stream = torch.cuda.current_stream()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * sa_capi.SA_KERNEL_COUNT)]
    for e in evs:
        e.record(stream)
    torch.cuda.synchronize()
    mask = sa_capi.forward_events(lib, a, stream.cuda_stream, evs)
    torch.cuda.synchronize()
    assert mask == expect
    assert torch.equal(o, ref)
    for k in range(sa_capi.SA_KERNEL_COUNT):
        if (mask >> k) & 1:
            assert evs[2 * k].elapsed_time(evs[2 * k + 1]) > 0.0


def test_events_hook_without_events_still_reports_kernels(gpu_sa):
    q, kv, sink, idx, sc = case(1, 16, 500, 128, seed=5)
    ref = torch.ops.sa_amd.sparse_attn_fwd(q, kv, sink, idx, sc, None, 0)
    lib = sa_capi.load()
    o = torch.empty_like(q)
    a = sa_capi.make_args(q, kv, sink, idx, o, sc)
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    launched = ctypes.c_uint32(0)
    rc = lib.sa_forward_events(ctypes.byref(a),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                               None, ctypes.byref(launched))
    assert rc == sa_capi.SA_OK
    torch.cuda.synchronize()
    assert launched.value == QUERY | COMBINE   # 16 queries < CUs: split plan, reported
    assert torch.equal(o, ref)
