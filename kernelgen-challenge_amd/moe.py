"""Drop-in ``fused_moe`` for MI355X (track 03 of the reference).

Same signature, argument meaning and error behaviour as the reference entry
point ``track-03/submission.py:274-306``: 2-D ``hidden_states`` and
``score``, 3-D ``w1`` / ``w2`` with matching E, K and ``2N``, checked by
``assert`` as there (``:279-291``); inputs are made contiguous (``:293-296``,
in the operator) and the output is a new ``[M, K]`` tensor of
``hidden_states``' dtype and device. The arithmetic is
``track-03/reference/reference.py:10-35`` with its bf16 rounding points,
including ``renormalize`` (which the reference's Triton submission ignores,
``:276-277``). Ties in the top-k go to the lower expert index (the
reference leaves them to ``torch.topk``). Five HIP kernel launches
(``csrc/fused_moe_gfx950.hip`` behind ``include/fused_moe.h``) on the
current stream, with no synchronisation; the workspace comes from torch's
caching allocator. There is no CPU path: CPU tensors raise ``ValueError``.
"""
from __future__ import annotations

import torch

__all__ = ["fused_moe", "FLAG_LARGE_TILES", "FLAG_SMALL_TILES", "FLAG_BIG_TILES",
           "FLAG_ORDERED_SUM"]

# Tile choice (fm_args.flags in include/fused_moe.h); 0 lets the library
# choose from the tokens per expert.
FLAG_LARGE_TILES = 1
FLAG_SMALL_TILES = 2
FLAG_BIG_TILES = 4
# The final sum always as its own launch, never as atomic adds of the down
# GEMM (same bits); combines with one tile flag.
FLAG_ORDERED_SUM = 8

_op = None  # the extension's fused_moe once it is loaded


def _load():
    global _op
    from submission import load_extension  # lazy: submission re-exports this module
    # the module function, not torch.ops.sa_amd.fused_moe: the same operator
    # without the dispatcher's per-call boxing
    _op = load_extension().fused_moe
    return _op


def fused_moe(hidden_states, w1, w2, score, topk, renormalize=False, flags=0):
    """
    Args:
        hidden_states:  [M, K]       bf16
        w1:             [E, 2N, K]   bf16 (gate rows 0..N-1, up rows N..2N-1)
        w2:             [E, K, N]    bf16
        score:          [M, E]       bf16 router logits
        topk:           experts per token
        renormalize:    divide the selected weights by their sum
        flags:          tile choice (this build only; 0 = automatic)

    Returns:
        [M, K] bf16
    """
    assert hidden_states.dim() == 2
    assert w1.dim() == 3
    assert w2.dim() == 3
    assert score.dim() == 2
    M, K = hidden_states.shape
    E_w1, two_N, K_w1 = w1.shape
    E_w2, K_w2, N = w2.shape
    M_s, E_s = score.shape
    assert E_w1 == E_w2 == E_s
    assert K == K_w1 == K_w2
    assert two_N == 2 * N
    assert M_s == M
    if not (hidden_states.is_cuda and w1.is_cuda and w2.is_cuda and score.is_cuda):
        raise ValueError("fused_moe runs on the GPU only; move all inputs to the device")
    op = _op or _load()
    return op(hidden_states, w1, w2, score, int(topk), bool(renormalize), int(flags))
