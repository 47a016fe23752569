"""Write the small golden fixtures in this directory.

The reference holds no golden vectors for this path (its only check is a live
comparison with unseeded indices, ``track-01/test_correctness.py:22-34``), so
these fixtures come from this repository's float64 oracle
(``oracle.sparse_attn_fp64``), which ``tests/test_oracle.py`` pins. Each
``.npz`` holds the inputs (bf16 as uint16 bit patterns), the float64 oracle
output and the bf16 output of the torch-CPU restatement. Load with
``numpy.load(path)`` (no pickles).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import sparse_attn_fp64, sparse_attn_ref  # noqa: E402

SCALE = 0.04419417382415922


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def case(name, b, m, kv_len, topk, seed, pattern, sink_std=1.0, kv_std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, 16, 512, generator=g).to(torch.bfloat16)
    kv = (torch.randn(b, kv_len, 512, generator=g) * kv_std).to(torch.bfloat16)
    sink = torch.randn(16, generator=g) * sink_std
    if pattern == "sorted_perm":
        idx = torch.stack([torch.stack([torch.randperm(kv_len, generator=g)[:topk].sort().values
                                        for _ in range(m)]) for _ in range(b)]).to(torch.int32)
    elif pattern == "uniform":  # with replacement: duplicates occur
        idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    elif pattern == "padded":   # -1 slots interleaved, one all -1 row, one single-slot row
        idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
        idx[torch.rand(b, m, topk, generator=g) < 0.4] = -1
        idx[0, 0] = -1
        idx[0, 1] = -1
        idx[0, 1, topk // 2] = 7
    elif pattern == "causal":
        idx = torch.full((b, m, topk), -1, dtype=torch.int32)
        for t in range(m):
            n = min(t + 1, topk)
            idx[0, t, :n] = torch.randperm(t + 1, generator=g)[:n].to(torch.int32)
    else:
        raise ValueError(pattern)
    f64 = sparse_attn_fp64(q, kv, sink, idx, SCALE)
    ref = sparse_attn_ref(q, kv, sink, idx, SCALE)
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        q=bf16_bits(q), kv=bf16_bits(kv), sink=sink.numpy(), idx=idx.numpy(),
        scale=np.float64(SCALE), expected_f64=f64.astype(np.float32),
        expected_ref_bf16=bf16_bits(ref))


CASES = [
    # name, b, m, kv_len, topk, seed, pattern, extra
    ("plumbing_slice", 1, 4, 256, 64, 0, "sorted_perm", {}),
    ("duplicates_ragged", 2, 2, 200, 150, 1, "uniform", {}),
    ("padded_sink_visible", 1, 3, 96, 80, 2, "padded", {"sink_std": 3.0}),
    ("causal_head", 1, 6, 64, 4, 3, "causal", {"kv_std": 0.5}),
]

if __name__ == "__main__":
    for name, b, m, kv_len, topk, seed, pattern, extra in CASES:
        case(name, b, m, kv_len, topk, seed, pattern, **extra)
        print("wrote", name)
