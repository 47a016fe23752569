"""CPU tests of the track-03 fused_moe C-ABI (include/fused_moe.h): no GPU,
no compute calls.

* the HIP library loads and exports every function the header declares;
* the ctypes binding lays fm_args out field for field as the header does;
* argument errors come back as return codes before any device work;
* the workspace size covers the buffers the kernels use;
* the Python drop-in keeps the reference wrapper's asserts and refuses CPU
  tensors (there is no CPU fallback).
"""
import ctypes
import os
import re
import sys

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "kernelgen-challenge_amd")
HEADER = os.path.join(REPO, "include", "fused_moe.h")
sys.path.insert(0, PKG)

import sa_capi  # noqa: E402


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(sa_capi.FM_LIB_PATH):
        import importlib.util
        spec = importlib.util.spec_from_file_location("sa_build", os.path.join(PKG, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return sa_capi.fm_load()


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fm_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_function(lib):
    assert declared() == ["fm_abi_version", "fm_forward", "fm_forward_events", "fm_strerror",
                          "fm_workspace_bytes"]
    for name in declared():
        assert hasattr(lib, name)
    assert lib.fm_abi_version() == 4


def test_binding_matches_header_struct():
    text = open(HEADER).read()
    body = re.search(r"typedef struct fm_args \{(.*?)\} fm_args;", text, re.S).group(1)
    names = []
    for line in body.splitlines():
        line = re.sub(r"/\*.*?\*/", "", line).strip()
        if not line:
            continue
        decl = line.rstrip(";").replace("*", " ")
        for part in decl.split(","):
            names.append(part.split()[-1])
    assert names == [f for f, _ in sa_capi.FmArgs._fields_]
    # 5 pointers, 8 int64, two 32-bit fields, a pointer and a size_t: no padding
    assert ctypes.sizeof(sa_capi.FmArgs) == 5 * 8 + 8 * 8 + 4 + 4 + 8 + 8


def args(M=4, K=256, N=128, E=8, topk=2):
    a = sa_capi.FmArgs()
    a.hidden, a.w1, a.w2, a.score, a.out = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    a.M, a.K, a.N, a.E, a.topk = M, K, N, E, topk
    a.s_hidden, a.s_score, a.s_out = K, E, K
    return a


@pytest.mark.parametrize("field,value,code", [
    ("K", 200, sa_capi.FM_EUNSUPPORTED), ("N", 100, sa_capi.FM_EUNSUPPORTED),
    ("E", 257, sa_capi.FM_EUNSUPPORTED), ("topk", 33, sa_capi.FM_EINVAL),
    ("topk", 9, sa_capi.FM_EINVAL), ("topk", 0, sa_capi.FM_EINVAL), ("M", -1, sa_capi.FM_EINVAL),
    ("hidden", 0, sa_capi.FM_EINVAL), ("out", 0x50008, sa_capi.FM_EINVAL),
    ("score", 0x40001, sa_capi.FM_EINVAL), ("s_hidden", 100, sa_capi.FM_EINVAL),
    ("s_score", 4, sa_capi.FM_EINVAL), ("flags", 3, sa_capi.FM_EINVAL),
    ("flags", 5, sa_capi.FM_EINVAL), ("flags", 6, sa_capi.FM_EINVAL),
    ("flags", 16, sa_capi.FM_EINVAL), ("flags", 8 | 3, sa_capi.FM_EINVAL),
])
def test_argument_errors_before_device_work(lib, field, value, code):
    a = args()
    setattr(a, field, value)
    assert lib.fm_forward(ctypes.byref(a), None) == code
    n = ctypes.c_size_t(0)
    assert lib.fm_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == code


def test_topk_limit(lib):
    a = args(E=64, topk=33)
    assert lib.fm_forward(ctypes.byref(a), None) == sa_capi.FM_EUNSUPPORTED
    a = args(E=64, topk=32)
    assert lib.fm_forward(ctypes.byref(a), None) == sa_capi.FM_EWORKSPACE  # valid, no workspace


def test_null_and_empty(lib):
    assert lib.fm_forward(None, None) == sa_capi.FM_EINVAL
    assert lib.fm_workspace_bytes(ctypes.byref(args()), None) == sa_capi.FM_EINVAL
    a = args(M=0)
    assert lib.fm_forward(ctypes.byref(a), None) == sa_capi.FM_OK  # nothing to do
    assert sa_capi.fm_workspace_bytes(lib, a) == 0
    a = args()
    assert lib.fm_forward(ctypes.byref(a), None) == sa_capi.FM_EWORKSPACE  # no workspace
    assert "workspace" in lib.fm_strerror(sa_capi.FM_EWORKSPACE).decode()


@pytest.mark.parametrize("M,E,topk", [(1, 8, 2), (64, 64, 6), (4096, 64, 6), (4096, 8, 2)])
def test_workspace_covers_the_buffers(lib, M, E, topk):
    K, N = 2048, 1024
    n = sa_capi.fm_workspace_bytes(lib, args(M=M, K=K, N=N, E=E, topk=topk))
    P = M * topk
    # routing (ids, weights), sorted pairs, the intermediate and the weighted
    # expert outputs, in bf16
    assert n >= P * 12 + P * (N + K) * 2
    assert n <= P * 12 + P * (N + K) * 2 + 16 * (P + E) + 16 * 1024


def test_dropin_asserts_and_refuses_cpu():
    import submission
    h = torch.zeros(4, 256, dtype=torch.bfloat16)
    w1 = torch.zeros(8, 256, 256, dtype=torch.bfloat16)
    w2 = torch.zeros(8, 256, 128, dtype=torch.bfloat16)
    sc = torch.zeros(4, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        submission.fused_moe(h, w1, w2, sc, 2)
    with pytest.raises(AssertionError):
        submission.fused_moe(h, w1[:, :100], w2, sc, 2)
    with pytest.raises(AssertionError):
        submission.fused_moe(h[None], w1, w2, sc, 2)
