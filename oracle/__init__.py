"""CPU oracle for the sparse_attn hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the reported CPU
baseline. The product path (``kernelgen-challenge_amd/submission.py``) never
imports it and has no CPU fallback.
"""
from .sparse_attn_ref import (  # noqa: F401
    sparse_attn_ref,
    sparse_attn_fp64,
    sparse_attn_bruteforce,
    masked_fold_fp64,
    sparse_attn_lse_fp64,
    merge_fp64,
    sparse_attn_bruteforce_lse,
)
