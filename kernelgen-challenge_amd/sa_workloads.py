"""Seeded input generators for the sparse_attn hot path.

Two families of shapes:

* ``CONFIGS``: the five measurement configurations of this build (plumbing,
  decode, causal prefill, long context, high locality), each generated on the
  CPU from ``torch.Generator().manual_seed(seed)`` in the fixed draw order
  q, kv, attn_sink, indices, so the CPU oracle and the GPU see the same bits.
* ``CONTEST_WORKLOADS``: the ten contest shapes of the reference harness
  (``track-01/workloads.py:15-26``), with the same dtypes, h=16, d=512 and
  ``SCALE`` (``track-01/workloads.py:7-11``). The reference draws their
  indices from the unseeded global RNG (``track-01/workloads.py:36``); here
  they come from the same seeded CPU generator, uniform with replacement as
  in the reference, so duplicates can occur.

Floats are drawn as fp32 ``randn * std`` and rounded to bf16 with
``.to(torch.bfloat16)`` (round to nearest even). "N(0, s)" means std s.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

DTYPE = torch.bfloat16
SINK_DTYPE = torch.float32
HEAD_DIM = 512
NUM_HEADS = 16
SCALE = 0.04419417382415922          # 512 ** -0.5, track-01/workloads.py:11


@dataclass(frozen=True)
class Config:
    name: str
    b: int
    m: int
    kv_len: int
    topk: int
    pattern: str          # "sorted_perm" | "perm" | "causal" | "windows"
    q_std: float = 1.0
    kv_std: float = 1.0
    sink_std: float = 1.0


CONFIGS = {
    "plumbing": Config("plumbing", 1, 64, 2048, 256, "sorted_perm"),
    "decode": Config("decode", 32, 1, 32768, 2048, "perm"),
    "causal_prefill": Config("causal_prefill", 1, 4096, 4096, 2048, "causal"),
    "long_context": Config("long_context", 1, 1024, 131072, 2048, "perm",
                           kv_std=0.5),
    "high_locality": Config("high_locality", 4, 512, 16384, 512, "windows",
                            sink_std=2.0),
}

# (label, kind, batch, seq_len, kv_len, topk): track-01/workloads.py:15-26
CONTEST_WORKLOADS = [
    ("prefill-64x1024-1024-128", "Prefill", 64, 1024, 1024, 128),
    ("prefill-64x1024-1280-384", "Prefill", 64, 1024, 1280, 384),
    ("prefill-16x4096-4096-128", "Prefill", 16, 4096, 4096, 128),
    ("prefill-1x16384-16384-128", "Prefill", 1, 16384, 16384, 128),
    ("prefill-1x16384-20480-640", "Prefill", 1, 16384, 20480, 640),
    ("decode-64x1-128-128", "Decode", 64, 1, 128, 128),
    ("decode-64x1-400-392", "Decode", 64, 1, 400, 392),
    ("decode-64x1-640-640", "Decode", 64, 1, 640, 640),
    ("decode-16x1-1408-640", "Decode", 16, 1, 1408, 640),
    ("decode-1x1-4480-640", "Decode", 1, 1, 4480, 640),
]


def _randn_bf16(g, shape, std):
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std).to(DTYPE)


def _indices(cfg: Config, g: torch.Generator) -> torch.Tensor:
    b, m, kv_len, topk = cfg.b, cfg.m, cfg.kv_len, cfg.topk
    idx = torch.empty(b, m, topk, dtype=torch.int32)
    if cfg.pattern in ("sorted_perm", "perm"):
        for bi in range(b):
            for mi in range(m):
                row = torch.randperm(kv_len, generator=g)[:topk]
                if cfg.pattern == "sorted_perm":
                    row = row.sort().values
                idx[bi, mi] = row.to(torch.int32)
    elif cfg.pattern == "causal":
        # query t draws min(t+1, topk) distinct indices from [0, t]; the rest
        # of its slots are the -1 sentinel.
        idx.fill_(-1)
        for bi in range(b):
            for t in range(m):
                n = min(t + 1, topk, kv_len)
                row = torch.randperm(min(t + 1, kv_len), generator=g)[:n]
                idx[bi, t, :n] = row.to(torch.int32)
    elif cfg.pattern == "windows":
        # 8 aligned windows of 64 tokens per query (topk = 8 * 64). Query 0
        # draws 8 distinct window starts; every later query keeps each of the
        # previous query's starts with probability 0.75 and replaces the
        # others with fresh starts not already in its set. Indices are the
        # windows concatenated in ascending start order.
        win = 64
        nwin = topk // win
        nstarts = kv_len // win
        for bi in range(b):
            starts = torch.randperm(nstarts, generator=g)[:nwin].tolist()
            for mi in range(m):
                if mi > 0:
                    keep = torch.rand(nwin, generator=g) < 0.75
                    kept = [s for s, k in zip(starts, keep.tolist()) if k]
                    fresh = torch.randperm(nstarts, generator=g).tolist()
                    pool = [s for s in fresh if s not in kept]
                    starts = kept + pool[: nwin - len(kept)]
                row = torch.cat([torch.arange(s * win, s * win + win)
                                 for s in sorted(starts)])
                idx[bi, mi] = row.to(torch.int32)
    else:
        raise ValueError(f"unknown index pattern {cfg.pattern!r}")
    return idx


def make_config_inputs(name: str, seed: int = 0, h: int = NUM_HEADS,
                       d: int = HEAD_DIM):
    """CPU inputs ``(q, kv, attn_sink, topk_idxs, scale)`` for ``CONFIGS[name]``."""
    cfg = CONFIGS[name]
    g = torch.Generator().manual_seed(seed)
    q = _randn_bf16(g, (cfg.b, cfg.m, h, d), cfg.q_std)
    kv = _randn_bf16(g, (cfg.b, cfg.kv_len, d), cfg.kv_std)
    sink = torch.randn(h, generator=g, dtype=torch.float32) * cfg.sink_std
    idx = _indices(cfg, g)
    return q, kv, sink, idx, SCALE


def make_inputs(b, m, kv_len, topk, h=NUM_HEADS, d=HEAD_DIM, seed=0):
    """Seeded CPU counterpart of ``track-01/workloads.py:29-37``.

    q, kv ~ N(0, 1) bf16, sink ~ N(0, 1) fp32, indices uniform in
    ``[0, kv_len)`` with replacement.
    """
    g = torch.Generator().manual_seed(seed)
    q = _randn_bf16(g, (b, m, h, d), 1.0)
    kv = _randn_bf16(g, (b, kv_len, d), 1.0)
    sink = torch.randn(h, generator=g, dtype=torch.float32)
    idx = torch.randint(0, kv_len, (b, m, topk), generator=g, dtype=torch.int32)
    return q, kv, sink, idx, SCALE


def count_valid(topk_idxs: torch.Tensor) -> int:
    """Number of non-sentinel slots (N_valid)."""
    return int((topk_idxs != -1).sum())


def unique_rows(topk_idxs: torch.Tensor) -> int:
    """Number of distinct (batch, row) pairs referenced by valid slots."""
    total = 0
    for bi in range(topk_idxs.shape[0]):
        v = topk_idxs[bi].flatten()
        v = v[v != -1]
        total += int(torch.unique(v).numel())
    return total
