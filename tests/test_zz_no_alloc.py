"""GPU tests of the allocation-free entry point sa_forward_noalloc
(lib/libsa_noalloc_gfx950.so), through the C-ABI (ctypes): its output must
equal sa_forward's (with a caller workspace)
bit for bit, since both run the same kernels, on two calls in a row where the
second input is smaller (the library's scratch array then holds the first
call's contents). Each plan kind is covered: shared-row tiles, split-topk,
per query, and short queries over a long cache. A call that needs more
scratch than the array holds is refused
with SA_ESCRATCH before any device work.
"""
import ctypes

import pytest
import torch

import sa_capi
import sa_workloads as wl

pytestmark = pytest.mark.gpu

DEV = "cuda"


def case(b, m, kv_len, topk, seed, minus1=0.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    if minus1:
        idx[torch.rand(b, m, topk, generator=g) < minus1] = -1
    return [t.to(DEV) for t in (q, kv, sink, idx)] + [wl.SCALE]


def with_workspace(lib, q, kv, sink, idx, sc):
    """sa_forward with a workspace the caller allocates: the reference result."""
    o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=DEV)
    a = sa_capi.make_args(q, kv, sink, idx, o, sc, lse=lse)
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sa_capi.check(lib, lib.sa_forward(ctypes.byref(a), stream), "sa_forward")
    torch.cuda.synchronize()
    return o, lse, n


def noalloc(lib, q, kv, sink, idx, sc, flags=0):
    o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=DEV)
    a = sa_capi.make_args(q, kv, sink, idx, o, sc, flags=flags, lse=lse)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = sa_capi.noalloc_load().sa_forward_noalloc(ctypes.byref(a), stream)
    torch.cuda.synchronize()
    return rc, o, lse


CASES = {
    # (first call, second call with a smaller input)
    "tiles": ((1, 512, 2048, 1024, 1, 0.1), (1, 64, 700, 256, 2, 0.0)),
    "split": ((8, 1, 32768, 2048, 3, 0.0), (4, 1, 9000, 1000, 4, 0.05)),
    "per query": ((1, 300, 20000, 128, 5, 0.2), (1, 40, 3000, 64, 6, 0.0)),
    # short queries over a long cache: the index kernel's bitmap-first mode,
    # the scanning tile launch and sorted rows in the wave kernel
    "short queries, long cache": ((1, 300, 9000, 128, 10, 0.05), (1, 80, 8192, 64, 11, 0.0)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_equals_forward_twice(name):
    lib = sa_capi.load()
    for shape in CASES[name]:
        q, kv, sink, idx, sc = case(*shape)
        print(f"  {name}: b,m,kv_len,topk = {shape[:4]}", flush=True)
        o_ref, lse_ref, n = with_workspace(lib, q, kv, sink, idx, sc)
        assert n <= sa_capi.SA_NOALLOC_SCRATCH_BYTES
        rc, o, lse = noalloc(lib, q, kv, sink, idx, sc)
        assert rc == sa_capi.SA_OK, lib.sa_strerror(rc)
        assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)


def test_noalloc_causal_prefill_config():
    """The headline configuration (40 MiB of tile workspace) fits the array."""
    lib = sa_capi.load()
    qc, kvc, sinkc, idxc, sc = wl.make_config_inputs("causal_prefill")
    q, kv, sink, idx = (t.to(DEV) for t in (qc, kvc, sinkc, idxc))
    o_ref, lse_ref, n = with_workspace(lib, q, kv, sink, idx, sc)
    assert 32 << 20 < n <= sa_capi.SA_NOALLOC_SCRATCH_BYTES
    rc, o, lse = noalloc(lib, q, kv, sink, idx, sc)
    assert rc == sa_capi.SA_OK
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)
    # a smaller call right after, then the full one again
    q2, kv2, sink2, idx2, _ = case(1, 100, 1500, 300, 7)
    o2_ref, _, _ = with_workspace(lib, q2, kv2, sink2, idx2, sc)
    rc, o2, _ = noalloc(lib, q2, kv2, sink2, idx2, sc)
    assert rc == sa_capi.SA_OK and torch.equal(o2, o2_ref)
    rc, o, _ = noalloc(lib, q, kv, sink, idx, sc)
    assert rc == sa_capi.SA_OK and torch.equal(o, o_ref)


def test_noalloc_refuses_oversized_and_planned():
    lib = sa_capi.load()
    # 1024 tiles with 16384-entry unions: ~320 MiB of workspace
    q, kv, sink, idx, sc = case(1, 8192, 16384, 2048, 8)
    a = sa_capi.make_args(q, kv, sink, idx, torch.empty_like(q), sc)
    assert sa_capi.workspace_bytes(lib, a) > sa_capi.SA_NOALLOC_SCRATCH_BYTES
    rc, o, _ = noalloc(lib, q, kv, sink, idx, sc)
    assert rc == sa_capi.SA_ESCRATCH
    assert sa_capi.noalloc_load().sa_noalloc_scratch_bytes() == sa_capi.SA_NOALLOC_SCRATCH_BYTES
    assert "sa_forward_noalloc" in lib.sa_strerror(rc).decode()
    assert torch.isnan(o).all()  # nothing was launched
    q, kv, sink, idx, sc = case(1, 64, 700, 256, 9)
    rc, o, _ = noalloc(lib, q, kv, sink, idx, sc, flags=sa_capi.SA_FLAG_PLANNED)
    assert rc == sa_capi.SA_EINVAL and torch.isnan(o).all()
