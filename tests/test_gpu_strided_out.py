"""GPU tests: o and lse written into strided views through the C-ABI. Each
kernel's epilogue addresses an output row from its (query, head) strides; here
the views hold every other head of wider buffers, so a wrong stride shows up
as a mismatch with the contiguous call or as a write into the gaps. Covered:
shared-row tiles (ordered and placed), per-query parts, and the split-topk
combine."""
import ctypes

import pytest
import torch

from test_gpu_parity import DEV
import sa_capi

pytestmark = pytest.mark.gpu


def case(b, m, kv_len, topk, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16).to(DEV)
    kv = torch.randn(b, kv_len, 512, generator=g).to(torch.bfloat16).to(DEV)
    sink = torch.randn(16, generator=g).to(DEV)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32).to(DEV)
    return q, kv, sink, idx, 512 ** -0.5


def forward(lib, q, kv, sink, idx, o, lse, sc, flags):
    a = sa_capi.make_args(q, kv, sink, idx, o, sc, flags=flags, lse=lse)
    n = sa_capi.workspace_bytes(lib, a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    sa_capi.check(lib, lib.sa_forward(ctypes.byref(a),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                  "sa_forward")
    torch.cuda.synchronize()


@pytest.mark.parametrize("shape,flags,label", [
    ((2, 13, 300, 64), sa_capi.SA_FLAG_FORCE_TILES, "shared-row tiles, ordered"),
    ((1, 1600, 2048, 64), sa_capi.SA_FLAG_FORCE_TILES, "shared-row tiles, placed"),
    ((2, 13, 300, 64), sa_capi.SA_FLAG_PER_QUERY, "per-query parts"),
    ((4, 1, 2048, 512), 0, "split-topk combine"),
])
def test_strided_o_and_lse(gpu_sa, shape, flags, label):
    q, kv, sink, idx, sc = case(*shape, seed=sum(shape))
    b, m = shape[0], shape[1]
    lib = sa_capi.load()
    o_ref = torch.empty_like(q)
    lse_ref = torch.empty(b, m, 16, dtype=torch.float32, device=DEV)
    forward(lib, q, kv, sink, idx, o_ref, lse_ref, sc, flags)
    # every other head of a [b, m, 32, 576] buffer: strides (m*32*576, 32*576, 1152, 1)
    o_base = torch.full((b, m, 32, 576), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse_base = torch.full((b, m, 32), float("nan"), dtype=torch.float32, device=DEV)
    o = o_base[:, :, ::2, :512]
    lse = lse_base[:, :, ::2]
    assert not o.is_contiguous() and not lse.is_contiguous()
    forward(lib, q, kv, sink, idx, o, lse, sc, flags)
    print(f"  {label}: o {tuple(o.stride())}, lse {tuple(lse.stride())}", flush=True)
    assert torch.equal(o, o_ref), label
    assert torch.equal(lse, lse_ref), label
    assert torch.isnan(o_base[:, :, 1::2]).all() and torch.isnan(o_base[..., 512:]).all(), label
    assert torch.isnan(lse_base[:, :, 1::2]).all(), label
