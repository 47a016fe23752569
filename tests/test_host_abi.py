"""CPU tests of the C-ABI boundary (no GPU, no compute calls).

* the HIP library loads and exports every function ``include/sparse_attn.h``
  declares;
* argument errors come back as return codes before any device work;
* the g++ build of the host-side validation and split-topk planning
  (``csrc/sa_plan.h``) behaves as documented;
* the Python drop-in refuses CPU tensors (there is no CPU fallback).
"""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "kernelgen-challenge_amd")
LIB = os.path.join(PKG, "lib")
HEADER = os.path.join(REPO, "include", "sparse_attn.h")
NOALLOC_HEADER = os.path.join(REPO, "include", "sparse_attn_noalloc.h")
NOALLOC_LIB = os.path.join(LIB, "libsa_noalloc_gfx950.so")

SA_OK, SA_EINVAL, SA_EUNSUPPORTED, SA_EWORKSPACE, SA_EHIP, SA_ESCRATCH = range(6)


class SaArgs(ctypes.Structure):
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
    _fields_ = [
        ("o_parts", ctypes.c_void_p), ("lse_parts", ctypes.c_void_p),
        ("sink", ctypes.c_void_p), ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("n", ctypes.c_int64), ("b", ctypes.c_int64), ("m", ctypes.c_int64),
        ("h", ctypes.c_int64), ("d", ctypes.c_int64),
        ("sop", ctypes.c_int64 * 5), ("slp", ctypes.c_int64 * 4),
        ("so", ctypes.c_int64 * 4), ("slse", ctypes.c_int64 * 3),
    ]


def _libs_built():
    return all(os.path.exists(os.path.join(LIB, f)) for f in
               ("libsparse_attn_gfx950.so", "sa_torch_ext.so", "libsa_host_test.so"))


@pytest.fixture(scope="module")
def libs():
    if not _libs_built():  # build in-tree (hipcc cross-compiles without a GPU)
        import importlib.util
        spec = importlib.util.spec_from_file_location("sa_build", os.path.join(PKG, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    hip = ctypes.CDLL(os.path.join(LIB, "libsparse_attn_gfx950.so"))
    host = ctypes.CDLL(os.path.join(LIB, "libsa_host_test.so"))
    for lib in (hip,):
        lib.sa_forward.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_void_p]
        lib.sa_workspace_bytes.argtypes = [ctypes.POINTER(SaArgs),
                                           ctypes.POINTER(ctypes.c_size_t)]
        lib.sa_strerror.restype = ctypes.c_char_p
    host.sa_host_validate.argtypes = [ctypes.POINTER(SaArgs)]
    host.sa_host_validate_merge.argtypes = [ctypes.POINTER(SaMergeArgs)]
    hip.sa_merge.argtypes = [ctypes.POINTER(SaMergeArgs), ctypes.c_void_p]
    host.sa_host_plan_full.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_int64)]
    host.sa_host_plan.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_int,
                                  ctypes.POINTER(ctypes.c_int64),
                                  ctypes.POINTER(ctypes.c_int64),
                                  ctypes.POINTER(ctypes.c_size_t)]
    return hip, host


def good_args(b=1, m=4, kv_len=100, topk=64):
    a = SaArgs()
    a.q, a.kv, a.sink, a.idx, a.o = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    a.b, a.m, a.h, a.d, a.kv_len, a.topk = b, m, 16, 512, kv_len, topk
    a.sq[:] = [m * 16 * 512, 16 * 512, 512, 1]
    a.so[:] = [m * 16 * 512, 16 * 512, 512, 1]
    a.skv[:] = [kv_len * 512, 512, 1]
    a.sidx[:] = [m * topk, topk, 1]
    a.scale = 512 ** -0.5
    return a


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(sa_\w+)\s*\(", text, re.M)))


def test_header_declares_expected_api():
    assert declared_functions() == ["sa_abi_version", "sa_forward", "sa_forward_events",
                                    "sa_merge", "sa_plan_indices",
                                    "sa_strerror", "sa_workspace_bytes"]
    text = open(NOALLOC_HEADER).read()
    assert sorted(set(re.findall(r"^\s*\w+\s*\*?\s*(sa_\w+)\s*\(", text, re.M))) == \
        ["sa_forward_noalloc", "sa_noalloc_scratch_bytes"]


def test_plan_indices_rejects_bad_args_without_device_work(libs):
    hip, host = libs
    hip.sa_plan_indices.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_void_p]
    assert hip.sa_plan_indices(None, None) == SA_EINVAL
    a = good_args()
    a.d = 256
    assert hip.sa_plan_indices(ctypes.byref(a), None) == SA_EUNSUPPORTED
    a = good_args()
    a.flags = 64
    assert hip.sa_plan_indices(ctypes.byref(a), None) == SA_EINVAL
    a.flags = 8 | 16                           # both tile forms at once
    assert hip.sa_plan_indices(ctypes.byref(a), None) == SA_EINVAL
    a = good_args(b=0)                         # empty: nothing to plan
    assert hip.sa_plan_indices(ctypes.byref(a), None) == SA_OK
    a = good_args()
    a.flags = 4                                # SA_FLAG_PLANNED is a valid bit
    assert host.sa_host_validate(ctypes.byref(a)) == SA_OK
    a.flags = 32 | 8                           # SA_FLAG_TILE_ORDERED (version 9), with a form
    assert host.sa_host_validate(ctypes.byref(a)) == SA_OK


def test_ctypes_binding_matches_header_layout():
    """The package's ctypes binding (sa_capi) lays sa_args out like this
    test's own transcription of the header."""
    import sys
    sys.path.insert(0, PKG)
    import sa_capi
    for mine, theirs in ((SaArgs, sa_capi.SaArgs), (SaMergeArgs, sa_capi.SaMergeArgs)):
        assert ctypes.sizeof(theirs) == ctypes.sizeof(mine)
        assert len(theirs._fields_) == len(mine._fields_)
        for (n1, _), (n2, _) in zip(theirs._fields_, mine._fields_):
            assert n1 == n2 and getattr(theirs, n1).offset == getattr(mine, n2).offset
    assert sa_capi.KERNELS == ("index", "order", "tile", "query", "combine", "wave")
    text = open(HEADER).read()
    assert "SA_KERNEL_COUNT = 6" in text


def test_forward_events_rejects_bad_args_without_device_work(libs):
    hip, _ = libs
    hip.sa_forward_events.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_uint32)]
    launched = ctypes.c_uint32(7)
    a = good_args()
    a.h = 12
    assert hip.sa_forward_events(ctypes.byref(a), None, None, ctypes.byref(launched)) == \
        SA_EUNSUPPORTED
    assert launched.value == 0
    a = good_args()
    a.b = 0                                     # empty: nothing launched, no events
    assert hip.sa_forward_events(ctypes.byref(a), None, None, ctypes.byref(launched)) == SA_OK
    assert launched.value == 0


def test_library_exports_every_declared_symbol(libs):
    hip, _ = libs
    for name in declared_functions():
        assert hasattr(hip, name), f"{name} not exported"
    assert hip.sa_abi_version() == 9
    # the allocation-free entry point and its device array live in their own
    # library, so sa_forward's callers do not carry the array
    assert not hasattr(hip, "sa_forward_noalloc")
    noalloc = ctypes.CDLL(NOALLOC_LIB)
    for name in ("sa_forward_noalloc", "sa_noalloc_scratch_bytes"):
        assert hasattr(noalloc, name), f"{name} not exported"
    src = open(os.path.join(PKG, "csrc", "sparse_attn_gfx950.hip")).read()
    assert "static __device__" not in src


def test_strerror_covers_codes(libs):
    hip, _ = libs
    msgs = [hip.sa_strerror(c).decode() for c in range(6)]
    assert msgs[0] == "ok" and len(set(msgs)) == 6
    assert hip.sa_strerror(99).decode() == "unknown error"


def test_noalloc_rejects_bad_args_without_device_work(libs):
    """sa_forward_noalloc validates like sa_forward and refuses a planned call
    (an index plan lives in a caller's workspace) before any device work."""
    hip = ctypes.CDLL(NOALLOC_LIB)
    hip.sa_forward_noalloc.argtypes = [ctypes.POINTER(SaArgs), ctypes.c_void_p]
    assert hip.sa_forward_noalloc(None, None) == SA_EINVAL
    a = good_args()
    a.d = 256
    assert hip.sa_forward_noalloc(ctypes.byref(a), None) == SA_EUNSUPPORTED
    a = good_args()
    a.flags = 4
    assert hip.sa_forward_noalloc(ctypes.byref(a), None) == SA_EINVAL
    a = good_args(b=0)
    assert hip.sa_forward_noalloc(ctypes.byref(a), None) == SA_OK
    assert hip.sa_noalloc_scratch_bytes() == 48 << 20
    text = open(NOALLOC_HEADER).read()
    assert "#define SA_NOALLOC_SCRATCH_BYTES (48u << 20)" in text


def test_forward_rejects_null_args(libs):
    hip, host = libs
    assert hip.sa_forward(None, None) == SA_EINVAL
    assert host.sa_host_validate(None) == SA_EINVAL
    ws = ctypes.c_size_t(0)
    assert hip.sa_workspace_bytes(None, ctypes.byref(ws)) == SA_EINVAL
    assert hip.sa_workspace_bytes(ctypes.byref(good_args()), None) == SA_EINVAL


@pytest.mark.parametrize("field,value,code", [
    ("h", 12, SA_EUNSUPPORTED), ("h", 0, SA_EUNSUPPORTED), ("h", 24, SA_EUNSUPPORTED),
    ("h", 3, SA_EUNSUPPORTED), ("d", 256, SA_EUNSUPPORTED),
    ("b", -1, SA_EINVAL), ("topk", -3, SA_EINVAL), ("kv_len", -1, SA_EINVAL),
    ("q", 0, SA_EINVAL), ("o", 0, SA_EINVAL), ("sink", 0, SA_EINVAL),
    ("idx", 0, SA_EINVAL), ("kv", 0, SA_EINVAL),
    ("q", 0x10008, SA_EINVAL), ("o", 0x50002, SA_EINVAL), ("kv", 0x20004, SA_EINVAL),
    ("scale", float("nan"), SA_EINVAL), ("flags", 64, SA_EINVAL), ("flags", 8 | 16, SA_EINVAL),
    ("flags", 1 << 31, SA_EINVAL), ("workspace", 0x70008, SA_EINVAL),
])
def test_forward_argument_errors(libs, field, value, code):
    hip, host = libs
    a = good_args()
    setattr(a, field, value)
    assert host.sa_host_validate(ctypes.byref(a)) == code
    assert hip.sa_forward(ctypes.byref(a), None) == code


@pytest.mark.parametrize("arr,i,value", [
    ("sq", 3, 2), ("so", 3, 2), ("skv", 2, 2), ("sidx", 2, 2),
    ("sq", 2, 500), ("so", 1, 12), ("skv", 1, 516), ("sq", 0, -8),
])
def test_forward_stride_errors(libs, arr, i, value):
    hip, host = libs
    a = good_args()
    getattr(a, arr)[i] = value
    assert host.sa_host_validate(ctypes.byref(a)) == SA_EINVAL
    assert hip.sa_forward(ctypes.byref(a), None) == SA_EINVAL


def test_empty_shapes_are_ok_without_device_work(libs):
    hip, host = libs
    for b, m in ((0, 4), (3, 0)):
        a = good_args(b=b, m=m)
        a.q = a.o = a.kv = a.idx = a.sink = 0
        assert host.sa_host_validate(ctypes.byref(a)) == SA_OK
        assert hip.sa_forward(ctypes.byref(a), None) == SA_OK


def test_optional_pointers(libs):
    _, host = libs
    a = good_args(topk=0)
    a.idx = 0
    assert host.sa_host_validate(ctypes.byref(a)) == SA_OK  # no slots, no idx needed
    a = good_args(kv_len=0)
    a.kv = 0
    assert host.sa_host_validate(ctypes.byref(a)) == SA_OK  # only -1 slots possible


def plan(host, a, cus):
    ns, sl, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_size_t()
    rc = host.sa_host_plan(ctypes.byref(a), cus, ctypes.byref(ns), ctypes.byref(sl),
                           ctypes.byref(ws))
    assert rc == SA_OK
    return ns.value, sl.value, ws.value


PART_BYTES = 2 * 16 * 4 + 16 * 512 * 4


def plan_full(host, a, cus):
    out = (ctypes.c_int64 * 12)()
    assert host.sa_host_plan_full(ctypes.byref(a), cus, out) == SA_OK
    keys = ["nsplit", "split_len", "tiles", "tiles_per_b", "ntiles", "tile_cap", "ws",
            "meta_off", "order_off", "rows_off", "cnts_off", "part_off"]
    return dict(zip(keys, list(out)))


@pytest.mark.parametrize("b,m,kv_len,topk,flags,tiles", [
    (1, 4096, 4096, 2048, 0, True),      # causal prefill: shared-row tiles
    (4, 512, 16384, 512, 0, True),       # high locality
    (1, 1024, 131072, 2048, 0, False),   # long context: count table too big
    (32, 1, 32768, 2048, 0, False),      # decode: one query per batch, split
    (1, 4096, 4096, 2048, 1, False),     # SA_FLAG_PER_QUERY
    (1, 8, 16384, 64, 2, True),          # largest count table, no split
    (1, 8, 16385, 64, 2, False),
    (1, 4, 100, 64, 2, True),            # half a tile
    (1, 3, 100, 64, 2, False),           # fewer queries than half a tile
    (1, 300, 100, 0, 0, False),          # no slots
    (1, 256, 16384, 2 ** 27, 2, True),   # the largest topk the index kernel counts in 32 bits
    (1, 256, 16384, 2 ** 27 + 1, 2, False),
    (1, 256, 16384, 2 ** 31 - 1, 0, False),
])
def test_tile_plan(libs, b, m, kv_len, topk, flags, tiles):
    _, host = libs
    a = good_args(b=b, m=m, topk=topk, kv_len=kv_len)
    a.flags = flags
    p = plan_full(host, a, 256)
    assert bool(p["tiles"]) == tiles
    if tiles:
        assert p["nsplit"] == 1
        assert p["tiles_per_b"] == -(-m // 8) and p["ntiles"] == b * p["tiles_per_b"]
        assert p["tile_cap"] % 64 == 0 and p["tile_cap"] >= min(kv_len, 8 * topk)
        # per tile: meta, its slot in the launch order, a 32-bit offset per
        # union row and an fp16 log2 multiplicity per (query, union row)
        assert p["ws"] >= p["ntiles"] * (16 + 4 + (4 + 2 * 8) * p["tile_cap"])
        regions = [(p["meta_off"], 16 * p["ntiles"]), (p["order_off"], 4 * p["ntiles"]),
                   (p["rows_off"], 4 * p["ntiles"] * p["tile_cap"]),
                   (p["cnts_off"], 2 * 8 * p["ntiles"] * p["tile_cap"])]
        for (o0, n0), (o1, _) in zip(regions, regions[1:]):
            assert o0 % 256 == 0 and o0 + n0 <= o1           # aligned, disjoint, in order
        assert regions[-1][0] + regions[-1][1] <= p["ws"]


@pytest.mark.parametrize("b,m,topk,cus,expect_ns,expect_len", [
    (32, 1, 2048, 256, 8, 256),      # decode: 32 queries -> 8 parts of 4 tiles
    (1, 4096, 2048, 256, 1, 2048),   # causal prefill: enough queries
    (1, 64, 256, 256, 4, 64),        # plumbing: 4 parts of one tile
    (1, 1024, 2048, 256, 1, 2048),   # long context
    (64, 1, 128, 256, 2, 64),        # contest decode, topk 128
    (1, 1, 640, 256, 10, 64),        # one query: one tile per part
    (1, 1, 60, 256, 1, 60),          # shorter than a tile: never split
    (1, 1, 4000, 80, 63, 64),
])
def test_split_plan(libs, b, m, topk, cus, expect_ns, expect_len):
    _, host = libs
    a = good_args(b=b, m=m, topk=topk, kv_len=5000)
    ns, sl, ws = plan(host, a, cus)
    assert (ns, sl) == (expect_ns, expect_len)
    assert (ns - 1) * sl < topk <= ns * sl           # parts cover topk exactly
    if ns > 1:
        assert ws == b * m * ns * PART_BYTES


def test_python_dropin_refuses_cpu_tensors():
    import torch
    import submission
    q = torch.zeros(1, 2, 16, 512, dtype=torch.bfloat16)
    kv = torch.zeros(1, 8, 512, dtype=torch.bfloat16)
    sink = torch.zeros(16)
    idx = torch.zeros(1, 2, 4, dtype=torch.int32)
    with pytest.raises(ValueError):
        submission.sparse_attn(q, kv, sink, idx, 0.1)
    with pytest.raises(ValueError):
        submission.sparse_attn(q[0], kv, sink, idx, 0.1)


def test_index_check_modes(monkeypatch):
    """Default "deferred" (asynchronous); "sync" / "off" by name, by the
    legacy booleans and by SPARSE_ATTN_CHECK=1 / 0; anything else refused."""
    import importlib
    import submission
    try:
        for env, mode in ((None, "deferred"), ("1", "sync"), ("0", "off"), ("sync", "sync"),
                          ("deferred", "deferred")):
            if env is None:
                monkeypatch.delenv("SPARSE_ATTN_CHECK", raising=False)
            else:
                monkeypatch.setenv("SPARSE_ATTN_CHECK", env)
            assert importlib.reload(submission).index_check_mode() == mode, env
        for value, mode in ((True, "sync"), (False, "off"), ("deferred", "deferred")):
            submission.set_index_check(value)
            assert submission.index_check_mode() == mode
            assert submission.index_check_enabled() == (mode != "off")
        with pytest.raises(ValueError):
            submission.set_index_check("sometimes")
    finally:
        monkeypatch.delenv("SPARSE_ATTN_CHECK", raising=False)
        importlib.reload(submission)


def test_torch_operator_registers(libs):
    import torch
    import submission
    submission.load_extension()
    assert hasattr(torch.ops.sa_amd, "sparse_attn_fwd")
    schema = str(torch.ops.sa_amd.sparse_attn_fwd.default._schema)
    assert "Tensor q" in schema and "float scale" in schema


def test_lse_argument_checks(libs):
    hip, host = libs
    a = good_args()
    a.lse = 0x60002                      # not 4-byte aligned
    assert host.sa_host_validate(ctypes.byref(a)) == SA_EINVAL
    a.lse = 0x60000
    a.slse[:] = [64, 16, -1]
    assert host.sa_host_validate(ctypes.byref(a)) == SA_EINVAL
    a.slse[:] = [64, 16, 1]
    assert host.sa_host_validate(ctypes.byref(a)) == SA_OK


def good_merge(n=3, b=1, m=2, h=16, d=512):
    a = SaMergeArgs()
    a.o_parts, a.lse_parts, a.sink, a.o, a.lse = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    a.n, a.b, a.m, a.h, a.d = n, b, m, h, d
    a.sop[:] = [b * m * h * d, m * h * d, h * d, d, 1]
    a.slp[:] = [b * m * h, m * h, h, 1]
    a.so[:] = [m * h * d, h * d, d, 1]
    a.slse[:] = [m * h, h, 1]
    return a


@pytest.mark.parametrize("field,value,code", [
    ("n", -1, SA_EINVAL), ("d", 12, SA_EINVAL), ("o", 0, SA_EINVAL),
    ("o_parts", 0, SA_EINVAL), ("lse_parts", 0, SA_EINVAL), ("o", 0x40008, SA_EINVAL),
    ("lse", 0x50002, SA_EINVAL), ("sink", 0x30001, SA_EINVAL),
])
def test_merge_argument_errors(libs, field, value, code):
    hip, host = libs
    a = good_merge()
    setattr(a, field, value)
    assert host.sa_host_validate_merge(ctypes.byref(a)) == code
    assert hip.sa_merge(ctypes.byref(a), None) == code


@pytest.mark.parametrize("arr,i,value", [("sop", 4, 2), ("sop", 2, 7), ("so", 3, 2),
                                         ("so", 1, -8), ("slp", 0, -1), ("slse", 2, -1)])
def test_merge_stride_errors(libs, arr, i, value):
    hip, host = libs
    a = good_merge()
    getattr(a, arr)[i] = value
    assert host.sa_host_validate_merge(ctypes.byref(a)) == SA_EINVAL


def test_merge_optional_and_empty(libs):
    hip, host = libs
    a = good_merge()
    a.sink = None
    a.lse = None
    assert host.sa_host_validate_merge(ctypes.byref(a)) == SA_OK
    a = good_merge(n=0)
    a.o_parts = None                    # no parts: only o (and lse) are written
    a.lse_parts = None
    assert host.sa_host_validate_merge(ctypes.byref(a)) == SA_OK
    a = good_merge(b=0)
    a.o = None                          # empty output: nothing to check or run
    assert hip.sa_merge(ctypes.byref(a), None) == SA_OK


@pytest.mark.parametrize("h", [1, 2, 4, 8, 16, 32, 48, 64])
def test_supported_head_counts_validate(libs, h):
    """Powers of two up to 8 (padded to 16 in the workspace) and multiples of
    16 (16-head slices) pass the host checks; the workspace of a call with
    fewer than 16 heads holds a 16-head copy of q and o beyond the plan."""
    hip, host = libs
    a = good_args()
    a.h = h
    a.sq[:] = [a.m * h * 512, h * 512, 512, 1]
    a.so[:] = list(a.sq)
    assert host.sa_host_validate(ctypes.byref(a)) == SA_OK
    ws = ctypes.c_int64(0)
    assert host.sa_host_workspace_bytes(ctypes.byref(a), 256, ctypes.byref(ws)) == SA_OK
    a16 = good_args()
    ws16 = ctypes.c_int64(0)
    assert host.sa_host_workspace_bytes(ctypes.byref(a16), 256, ctypes.byref(ws16)) == SA_OK
    if h < 16:
        assert ws.value >= ws16.value + 2 * a.b * a.m * 16 * 512 * 2
    else:
        assert ws.value == ws16.value
