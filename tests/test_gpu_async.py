"""The drop-in's default index check is asynchronous ("deferred").

A call neither allocates an error word nor reads one back: it returns while
the stream is still busy, and a bad index is reported by the next call on the
device or by ``check_index_errors()`` (which synchronizes), once the call
that met it has run. The modes "sync" and "off" are covered by
test_gpu_parity.py::test_out_of_range_raises.
"""
import pytest
import torch

from test_gpu_parity import DEV, check, small
from oracle import sparse_attn_fp64

pytestmark = pytest.mark.gpu

SLEEP_CYCLES = 50_000_000  # a bounded spin kernel queued ahead of the call


@pytest.fixture
def deferred(gpu_sa):
    gpu_sa.set_index_check("deferred")
    gpu_sa.check_index_errors()  # start from a clear flag
    yield gpu_sa
    gpu_sa.set_index_check(True)


def inputs(bad=None, seed=31):
    q, kv, sink, idx, sc = small(1, 3, 700, 100, seed=seed)
    if bad is not None:
        idx[0, 1, 50] = bad
    return q.to(DEV), kv.to(DEV), sink.to(DEV), idx.to(DEV), sc


def test_call_returns_while_stream_busy(deferred):
    q, kv, sink, idx, sc = inputs(bad=9999)
    torch.cuda.synchronize()
    torch.cuda._sleep(SLEEP_CYCLES)
    o = deferred.sparse_attn(q, kv, sink, idx, sc)
    busy = not torch.cuda.current_stream().query()
    assert busy, "the call waited for the stream"
    with pytest.raises(RuntimeError):
        deferred.check_index_errors()
    deferred.check_index_errors()  # reported once, then clear
    # the bad slot was skipped (never read): the same as deleting it
    fixed = idx.cpu().clone()
    fixed[0, 1, 50] = -1
    check(o, sparse_attn_fp64(q.cpu(), kv.cpu(), sink.cpu(), fixed, sc), "deferred, skipped")


@pytest.mark.parametrize("bad", [-2, 700])
def test_next_call_reports(deferred, bad):
    q, kv, sink, idx, sc = inputs(bad=bad)
    deferred.sparse_attn(q, kv, sink, idx, sc)
    torch.cuda.synchronize()  # the flagged call has run
    qg, kvg, sinkg, idxg, _ = inputs()
    with pytest.raises(RuntimeError):
        deferred.sparse_attn(qg, kvg, sinkg, idxg, sc)
    o = deferred.sparse_attn(qg, kvg, sinkg, idxg, sc)  # reported once
    torch.cuda.synchronize()
    check(o, sparse_attn_fp64(qg.cpu(), kvg.cpu(), sinkg.cpu(), idxg.cpu(), sc), "after report")


def test_good_calls_never_report(deferred):
    q, kv, sink, idx, sc = inputs()
    for _ in range(3):
        deferred.sparse_attn(q, kv, sink, idx, sc)
        deferred.sparse_attn_with_lse(q, kv, sink, idx, sc)
    deferred.check_index_errors()


def test_plan_reports_deferred(deferred):
    """An index plan that keeps index state (tiles) validates in the plan call."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 64, 16, 512, generator=g).to(torch.bfloat16).to(DEV)
    kv = torch.randn(1, 300, 512, generator=g).to(torch.bfloat16).to(DEV)
    idx = torch.randint(0, 300, (1, 64, 64), generator=g, dtype=torch.int32)
    idx[0, 5, 3] = 300
    deferred.sparse_attn_plan(q, kv, idx.to(DEV))
    with pytest.raises(RuntimeError):
        deferred.check_index_errors()
