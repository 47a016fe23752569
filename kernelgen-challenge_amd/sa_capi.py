"""ctypes binding of the C-ABI declared in ``include/sparse_attn.h``.

The HIP library ``lib/libsparse_attn_gfx950.so`` is plain C: a Python caller
of the reference's ``sparse_attn`` (track-01/submission.py:975) can reach it
with this binding alone, without the torch operator. ``bench.py`` uses it for
the per-kernel event hook ``sa_forward_events``.

Tensors are torch tensors on the current HIP device; only their data pointers,
shapes and strides cross the boundary.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libsparse_attn_gfx950.so")
# sa_forward_noalloc and its device array (include/sparse_attn_noalloc.h)
NOALLOC_LIB_PATH = os.path.join(_HERE, "lib", "libsa_noalloc_gfx950.so")

SA_OK, SA_EINVAL, SA_EUNSUPPORTED, SA_EWORKSPACE, SA_EHIP, SA_ESCRATCH = range(6)
SA_NOALLOC_SCRATCH_BYTES = 48 << 20
SA_FLAG_PER_QUERY, SA_FLAG_FORCE_TILES, SA_FLAG_PLANNED = 1, 2, 4
SA_FLAG_TILE_SKIP, SA_FLAG_TILE_DENSE, SA_FLAG_TILE_ORDERED = 8, 16, 32
KERNELS = ("index", "order", "tile", "query", "combine", "wave")  # SA_KERNEL_* order
SA_KERNEL_COUNT = len(KERNELS)


class SaArgs(ctypes.Structure):
    """``struct sa_args`` (include/sparse_attn.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("kv", ctypes.c_void_p), ("sink", ctypes.c_void_p),
        ("idx", ctypes.c_void_p), ("o", ctypes.c_void_p),
        ("b", ctypes.c_int64), ("m", ctypes.c_int64), ("h", ctypes.c_int64),
        ("d", ctypes.c_int64), ("kv_len", ctypes.c_int64), ("topk", ctypes.c_int64),
        ("sq", ctypes.c_int64 * 4), ("skv", ctypes.c_int64 * 3),
        ("sidx", ctypes.c_int64 * 3), ("so", ctypes.c_int64 * 4),
        ("scale", ctypes.c_float), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t), ("err_word", ctypes.c_void_p),
        ("flags", ctypes.c_uint32), ("lse", ctypes.c_void_p), ("slse", ctypes.c_int64 * 3),
    ]


class SaMergeArgs(ctypes.Structure):
    """``struct sa_merge_args`` (include/sparse_attn.h)."""
    _fields_ = [
        ("o_parts", ctypes.c_void_p), ("lse_parts", ctypes.c_void_p),
        ("sink", ctypes.c_void_p), ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("n", ctypes.c_int64), ("b", ctypes.c_int64), ("m", ctypes.c_int64),
        ("h", ctypes.c_int64), ("d", ctypes.c_int64),
        ("sop", ctypes.c_int64 * 5), ("slp", ctypes.c_int64 * 4),
        ("so", ctypes.c_int64 * 4), ("slse", ctypes.c_int64 * 3),
    ]


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library and declare every entry point's signature."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    args_p = ctypes.POINTER(SaArgs)
    lib.sa_abi_version.restype = ctypes.c_int
    lib.sa_abi_version.argtypes = []
    lib.sa_workspace_bytes.argtypes = [args_p, ctypes.POINTER(ctypes.c_size_t)]
    lib.sa_forward.argtypes = [args_p, ctypes.c_void_p]
    lib.sa_forward_events.argtypes = [args_p, ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_uint32)]
    lib.sa_merge.argtypes = [ctypes.POINTER(SaMergeArgs), ctypes.c_void_p]
    lib.sa_plan_indices.argtypes = [args_p, ctypes.c_void_p]
    lib.sa_strerror.restype = ctypes.c_char_p
    lib.sa_strerror.argtypes = [ctypes.c_int]
    return lib


def noalloc_load(path: str = NOALLOC_LIB_PATH) -> ctypes.CDLL:
    """Load the allocation-free entry point's library. Loading it reserves
    SA_NOALLOC_SCRATCH_BYTES on each GPU the process uses it on."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    lib.sa_forward_noalloc.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_void_p]
    lib.sa_noalloc_scratch_bytes.restype = ctypes.c_int
    lib.sa_noalloc_scratch_bytes.argtypes = []
    return lib


def make_args(q, kv, sink, idx, o, scale: float, flags: int = 0, err=None, lse=None) -> SaArgs:
    """sa_args for torch tensors q [b,m,h,d], kv [b,n,d], sink [h], idx [b,m,k], o like q,
    and optionally lse fp32 [b,m,h]."""
    a = SaArgs()
    a.q, a.kv, a.sink = q.data_ptr(), kv.data_ptr(), sink.data_ptr()
    a.idx, a.o = idx.data_ptr(), o.data_ptr()
    a.b, a.m, a.h, a.d = q.shape
    a.kv_len, a.topk = kv.shape[1], idx.shape[2]
    a.sq[:] = list(q.stride())
    a.skv[:] = list(kv.stride())
    a.sidx[:] = list(idx.stride())
    a.so[:] = list(o.stride())
    a.scale = float(scale)
    a.err_word = err.data_ptr() if err is not None else None
    a.flags = flags
    if lse is not None:
        a.lse = lse.data_ptr()
        a.slse[:] = list(lse.stride())
    return a


def check(lib: ctypes.CDLL, rc: int, what: str) -> None:
    if rc != SA_OK:
        raise RuntimeError(f"{what}: {lib.sa_strerror(rc).decode()} (code {rc})")


def workspace_bytes(lib: ctypes.CDLL, a: SaArgs) -> int:
    n = ctypes.c_size_t(0)
    check(lib, lib.sa_workspace_bytes(ctypes.byref(a), ctypes.byref(n)), "sa_workspace_bytes")
    return n.value


def forward_events(lib: ctypes.CDLL, a: SaArgs, stream: int, events) -> int:
    """sa_forward_events with 2 * SA_KERNEL_COUNT torch.cuda.Event objects
    (or None entries); returns the bit mask of launched kernels."""
    handles = (ctypes.c_void_p * (2 * SA_KERNEL_COUNT))(
        *[(ev.cuda_event if ev is not None else None) for ev in events])
    launched = ctypes.c_uint32(0)
    check(lib, lib.sa_forward_events(ctypes.byref(a), ctypes.c_void_p(stream), handles,
                                     ctypes.byref(launched)), "sa_forward_events")
    return launched.value


# ---------------------------------------------------------------------------
# track-02 hc_split_sinkhorn (include/hc_sinkhorn.h)
# ---------------------------------------------------------------------------
HC_LIB_PATH = os.path.join(_HERE, "lib", "libhc_sinkhorn_gfx950.so")
HC_OK, HC_EINVAL, HC_EUNSUPPORTED, HC_EHIP = range(4)
HC_FLAG_LANES16, HC_FLAG_LANES1 = 1, 2


class HcArgs(ctypes.Structure):
    """``struct hc_args`` (include/hc_sinkhorn.h)."""
    _fields_ = [
        ("mixes", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("base", ctypes.c_void_p),
        ("pre", ctypes.c_void_p), ("post", ctypes.c_void_p), ("comb", ctypes.c_void_p),
        ("n", ctypes.c_int64), ("hc_mult", ctypes.c_int32), ("iters", ctypes.c_int32),
        ("eps", ctypes.c_float), ("flags", ctypes.c_uint32),
    ]


def hc_load(path: str = HC_LIB_PATH) -> ctypes.CDLL:
    """Load the track-02 library and declare its entry points."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    lib.hc_abi_version.restype = ctypes.c_int
    lib.hc_abi_version.argtypes = []
    lib.hc_strerror.restype = ctypes.c_char_p
    lib.hc_strerror.argtypes = [ctypes.c_int]
    lib.hc_split_sinkhorn.argtypes = [ctypes.POINTER(HcArgs), ctypes.c_void_p]
    return lib


def check_hc(lib, rc: int, what: str = "hc_split_sinkhorn") -> None:
    if rc != HC_OK:
        raise RuntimeError(f"{what}: {lib.hc_strerror(rc).decode()} (code {rc})")


def hc_make_args(mixes, scale, base, pre, post, comb, iters=20, eps=1e-6, flags=0,
                 hc_mult=4) -> HcArgs:
    """hc_args for contiguous fp32 torch tensors mixes [..., 24], scale [3],
    base [24], pre / post [..., 4], comb [..., 4, 4]."""
    a = HcArgs()
    a.mixes, a.scale, a.base = mixes.data_ptr(), scale.data_ptr(), base.data_ptr()
    a.pre, a.post, a.comb = pre.data_ptr(), post.data_ptr(), comb.data_ptr()
    a.n = mixes.numel() // 24
    a.hc_mult, a.iters, a.eps, a.flags = hc_mult, iters, eps, flags
    return a


# ---------------------------------------------------------------------------
# track-03 fused_moe (include/fused_moe.h)
# ---------------------------------------------------------------------------
FM_LIB_PATH = os.path.join(_HERE, "lib", "libfused_moe_gfx950.so")
FM_OK, FM_EINVAL, FM_EUNSUPPORTED, FM_EWORKSPACE, FM_EHIP = range(5)
FM_FLAG_LARGE_TILES, FM_FLAG_SMALL_TILES, FM_FLAG_BIG_TILES, FM_FLAG_ORDERED_SUM = 1, 2, 4, 8
FM_KERNELS = ("route", "plan", "gateup", "down", "reduce")  # FM_KERNEL_* order
FM_KERNEL_COUNT = len(FM_KERNELS)


class FmArgs(ctypes.Structure):
    """``struct fm_args`` (include/fused_moe.h)."""
    _fields_ = [
        ("hidden", ctypes.c_void_p), ("w1", ctypes.c_void_p), ("w2", ctypes.c_void_p),
        ("score", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("M", ctypes.c_int64), ("K", ctypes.c_int64), ("N", ctypes.c_int64),
        ("E", ctypes.c_int64), ("topk", ctypes.c_int64),
        ("s_hidden", ctypes.c_int64), ("s_score", ctypes.c_int64), ("s_out", ctypes.c_int64),
        ("renormalize", ctypes.c_int32), ("flags", ctypes.c_uint32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


def fm_load(path: str = FM_LIB_PATH) -> ctypes.CDLL:
    """Load the track-03 library and declare its entry points."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    args_p = ctypes.POINTER(FmArgs)
    lib.fm_abi_version.restype = ctypes.c_int
    lib.fm_abi_version.argtypes = []
    lib.fm_strerror.restype = ctypes.c_char_p
    lib.fm_strerror.argtypes = [ctypes.c_int]
    lib.fm_workspace_bytes.argtypes = [args_p, ctypes.POINTER(ctypes.c_size_t)]
    lib.fm_forward.argtypes = [args_p, ctypes.c_void_p]
    lib.fm_forward_events.argtypes = [args_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_uint32)]
    return lib


def fm_make_args(hidden, w1, w2, score, out, topk, renormalize=False, flags=0) -> FmArgs:
    """fm_args for torch tensors hidden [M, K], w1 [E, 2N, K], w2 [E, K, N],
    score [M, E], out [M, K] (rows with unit inner stride)."""
    a = FmArgs()
    a.hidden, a.w1, a.w2 = hidden.data_ptr(), w1.data_ptr(), w2.data_ptr()
    a.score, a.out = score.data_ptr(), out.data_ptr()
    a.M, a.K = hidden.shape
    a.E, a.N = w1.shape[0], w2.shape[2]
    a.topk = topk
    a.s_hidden, a.s_score, a.s_out = hidden.stride(0), score.stride(0), out.stride(0)
    a.renormalize = 1 if renormalize else 0
    a.flags = flags
    return a


def fm_check(lib, rc: int, what: str = "fused_moe") -> None:
    if rc != FM_OK:
        raise RuntimeError(f"{what}: {lib.fm_strerror(rc).decode()} (code {rc})")


def fm_workspace_bytes(lib, a: FmArgs) -> int:
    n = ctypes.c_size_t(0)
    fm_check(lib, lib.fm_workspace_bytes(ctypes.byref(a), ctypes.byref(n)), "fm_workspace_bytes")
    return n.value


def fm_forward_events(lib, a: FmArgs, stream: int, events) -> int:
    """fm_forward_events with 2 * FM_KERNEL_COUNT torch.cuda.Event objects (or
    None entries); returns the bit mask of launched kernels."""
    handles = (ctypes.c_void_p * (2 * FM_KERNEL_COUNT))(
        *[(ev.cuda_event if ev is not None else None) for ev in events])
    launched = ctypes.c_uint32(0)
    fm_check(lib, lib.fm_forward_events(ctypes.byref(a), ctypes.c_void_p(stream), handles,
                                        ctypes.byref(launched)), "fm_forward_events")
    return launched.value
