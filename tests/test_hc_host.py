"""CPU tests of the track-02 boundary (no GPU needed):

* ``lib/libhc_sinkhorn_gfx950.so`` loads and exports every function
  ``include/hc_sinkhorn.h`` declares;
* ``hc_split_sinkhorn`` rejects bad arguments with the documented codes before
  it touches the device, and does nothing for zero tokens;
* the Python drop-in keeps the reference's checks
  (``track-02/submission.py:340-346``: ``assert`` on a 3-D ``mixes``,
  ``hc_mult == 4`` and a last dim of 24) and refuses CPU tensors, since there
  is no CPU path.
"""
import ctypes
import os
import re

import pytest
import torch

import sa_capi
from hc_sinkhorn import hc_split_sinkhorn

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "hc_sinkhorn.h")


def declared_functions():
    text = open(HEADER).read()
    return re.findall(r"^(?:int|const char\*)\s+(\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def hc():
    if not os.path.exists(sa_capi.HC_LIB_PATH):
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "sa_build", os.path.join(REPO, "kernelgen-challenge_amd", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return sa_capi.hc_load()


def test_exports_every_declared_function(hc):
    names = declared_functions()
    assert set(names) == {"hc_abi_version", "hc_strerror", "hc_split_sinkhorn"}
    for name in names:
        assert hasattr(hc, name), f"{name} not exported"
    assert hc.hc_abi_version() == 1


def test_strerror(hc):
    for rc in range(4):
        assert len(hc.hc_strerror(rc)) > 0
    assert hc.hc_strerror(99) == b"unknown error"


def args(n=1, ptr=0x100000, **kw):
    a = sa_capi.HcArgs()
    a.mixes = a.scale = a.base = a.pre = a.post = a.comb = ptr
    a.n, a.hc_mult, a.iters, a.eps, a.flags = n, 4, 20, 1e-6, 0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,rc", [
    (dict(n=-1), sa_capi.HC_EINVAL),
    (dict(hc_mult=3), sa_capi.HC_EUNSUPPORTED),
    (dict(hc_mult=8), sa_capi.HC_EUNSUPPORTED),
    (dict(flags=3), sa_capi.HC_EINVAL),            # both lane layouts
    (dict(flags=4), sa_capi.HC_EINVAL),            # unknown bit
    (dict(n=1 << 31), sa_capi.HC_EUNSUPPORTED),
    (dict(mixes=None), sa_capi.HC_EINVAL),
    (dict(comb=None), sa_capi.HC_EINVAL),
    (dict(mixes=0x100004), sa_capi.HC_EINVAL),     # 16-byte rows
    (dict(pre=0x100008), sa_capi.HC_EINVAL),
])
def test_rejects_bad_arguments(hc, kw, rc):
    a = args(**kw)
    assert hc.hc_split_sinkhorn(ctypes.byref(a), None) == rc


def test_null_args_and_zero_tokens(hc):
    assert hc.hc_split_sinkhorn(None, None) == sa_capi.HC_EINVAL
    a = args(n=0, ptr=0)  # nothing to read or write: no launch, null pointers allowed
    assert hc.hc_split_sinkhorn(ctypes.byref(a), None) == sa_capi.HC_OK


def test_drop_in_checks():
    mixes, sc, base = torch.randn(2, 3, 24), torch.randn(3), torch.randn(24)
    with pytest.raises(AssertionError, match="3D"):
        hc_split_sinkhorn(mixes[0], sc, base)
    with pytest.raises(AssertionError, match="hc_mult=4"):
        hc_split_sinkhorn(mixes, sc, base, hc_mult=3)
    with pytest.raises(AssertionError, match="last dim must be 24"):
        hc_split_sinkhorn(mixes[..., :20], sc, base)
    with pytest.raises(ValueError, match="GPU only"):
        hc_split_sinkhorn(mixes, sc, base)


def test_submission_exports_track02_entry():
    import submission
    assert submission.hc_split_sinkhorn is hc_split_sinkhorn
    assert "hc_split_sinkhorn" in submission.__all__
