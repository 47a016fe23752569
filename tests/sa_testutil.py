"""Helpers shared by the GPU tests: the launch plan the library will choose.

Several tests exercise one kernel path (shared-row tiles, no split) and pick
their shapes for it. The plan depends on the device's compute-unit count, so
they assert the plan first, through the g++ build of the host-side planner
(``libsa_host_test.so``, the same ``sa_plan.h`` the HIP library compiles),
instead of assuming a count.
"""
import ctypes
import os

import torch

import sa_capi

_LIB = os.path.join(os.path.dirname(sa_capi.LIB_PATH), "libsa_host_test.so")
_host = None
_KEYS = ["nsplit", "split_len", "tiles", "tiles_per_b", "ntiles", "tile_cap", "ws",
         "meta_off", "order_off", "rows_off", "cnts_off", "part_off"]


def device_cus() -> int:
    return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count


def plan_of(q, kv, idx, flags=0) -> dict:
    """The plan sa_forward makes for these tensors on the current device."""
    global _host
    if _host is None:
        _host = ctypes.CDLL(_LIB)
        _host.sa_host_plan_full.argtypes = [ctypes.POINTER(sa_capi.SaArgs), ctypes.c_int,
                                            ctypes.POINTER(ctypes.c_int64)]
    o = q  # only its strides and pointer alignment are read
    a = sa_capi.make_args(q, kv, q.new_zeros(16, dtype=torch.float32), idx, o, 1.0, flags)
    out = (ctypes.c_int64 * len(_KEYS))()
    rc = _host.sa_host_plan_full(ctypes.byref(a), device_cus(), out)
    assert rc == sa_capi.SA_OK, f"plan: code {rc}"
    return dict(zip(_KEYS, list(out)))


def expect_plan(q, kv, idx, flags=0, tiles=None, nsplit=None) -> dict:
    """Assert the plan these tests rely on (shared-row tiles, no split, ...)."""
    p = plan_of(q, kv, idx, flags)
    if tiles is not None:
        assert bool(p["tiles"]) == tiles, f"plan has tiles={bool(p['tiles'])} on " \
                                          f"{device_cus()} CUs; the test needs {tiles}"
    if nsplit is not None:
        assert p["nsplit"] == nsplit, f"plan splits {p['nsplit']} ways on {device_cus()} CUs"
    return p
