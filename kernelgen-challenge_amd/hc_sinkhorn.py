"""Drop-in ``hc_split_sinkhorn`` for MI355X (track 02 of the reference).

Same signature, argument meaning and error behaviour as the reference entry
point ``track-02/submission.py:316-444``: ``mixes`` must be 3-D with
``hc_mult = 4`` (last dim 24), checked by ``assert`` as there (``:340-346``);
inputs are made contiguous (``:349-351``, in the operator) and ``pre``,
``post``, ``comb`` are new contiguous tensors of ``mixes``' dtype and device
(``:353-355``; here three slices of one allocation). The arithmetic is
``track-02/reference/reference.py:38-51``. One HIP kernel launch does it all
(``csrc/hc_sinkhorn_gfx950.hip`` behind ``include/hc_sinkhorn.h``), on the
current stream, with no synchronisation. There is no CPU path: CPU tensors
raise ``ValueError``.
"""
from __future__ import annotations

import torch

__all__ = ["hc_split_sinkhorn", "FLAG_LANES16", "FLAG_LANES1"]

# Lanes per token (hc_args.flags in include/hc_sinkhorn.h); 0 lets the
# library choose from the token count.
FLAG_LANES16 = 1
FLAG_LANES1 = 2

_op = None  # the extension's hc_split_sinkhorn once it is loaded


def _load():
    global _op
    from submission import load_extension  # lazy: submission re-exports this module
    # the module function, not torch.ops.sa_amd.hc_split_sinkhorn: the same
    # operator without the dispatcher's per-call boxing
    _op = load_extension().hc_split_sinkhorn
    return _op


def hc_split_sinkhorn(mixes: torch.Tensor, hc_scale: torch.Tensor, hc_base: torch.Tensor,
                      hc_mult: int = 4, sinkhorn_iters: int = 20, eps: float = 1e-6,
                      flags: int = 0):
    """
    Args:
        mixes:          [b, s, (2 + hc_mult) * hc_mult]   fp32
        hc_scale:       [3]                               fp32
        hc_base:        [(2 + hc_mult) * hc_mult]         fp32
        hc_mult:        number of streams (4 only, as the reference's kernel)
        sinkhorn_iters: Sinkhorn rounds (row + column) after the softmax
        eps:            numerical-stability constant
        flags:          lanes-per-token choice (this build only; 0 = automatic)

    Returns:
        pre  [b, s, hc_mult], post [b, s, hc_mult], comb [b, s, hc_mult, hc_mult]
    """
    assert mixes.dim() == 3, f"mixes must be 3D, got shape {tuple(mixes.shape)}"
    assert hc_mult == 4, f"this kernel is specialized for hc_mult=4, got {hc_mult}"
    hc3 = 2 * hc_mult + hc_mult * hc_mult
    assert mixes.shape[2] == hc3, f"mixes last dim must be {hc3}, got {mixes.shape[2]}"
    if not (mixes.is_cuda and hc_scale.is_cuda and hc_base.is_cuda):
        raise ValueError("hc_split_sinkhorn runs on the GPU only; move all inputs to the device")
    op = _op or _load()
    # the operator makes the inputs contiguous (track-02/submission.py:349-351)
    return op(mixes, hc_scale, hc_base, int(hc_mult), int(sinkhorn_iters), float(eps),
              int(flags))
