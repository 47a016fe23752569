"""Pins of the track-03 fused_moe oracle (CPU only).

The reference ships no golden vectors (its test compares live against the
torch oracle at atol = rtol = 5e-2, track-03/test_correctness.py:24-35), so
the oracle in ``oracle/fused_moe_ref.py`` is pinned by:

* agreement of its three restatements (torch bf16 ops, the NumPy
  exact-rounding model, per-token scalar loops);
* routing against ``torch.topk`` wherever no tie crosses the top-k boundary,
  and the documented tie rule (lower expert index first) where one does;
* closed forms: one expert with topk = 1 is the plain gated MLP
  ``down(silu(gate) * up)`` with gate = the first N rows of w1; hidden = 0
  gives 0; with identical experts, ``renormalize`` gives that MLP and no
  renormalisation scales it by the top-k softmax mass; topk = E weighs every
  expert by its softmax weight;
* invariance under permuting the experts together with their score columns;
* planted mistakes: each mutant below fails at least one check.
"""
import math

import numpy as np
import pytest
import torch

from oracle.fused_moe_ref import (bf16_round, fused_moe_fp64, fused_moe_loops,
                                  fused_moe_ref, route)


def make(M, K, N, E, seed, wstd=0.02):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * N, K, generator=g) * wstd).to(torch.bfloat16)
    w2 = (torch.randn(E, K, N, generator=g) * wstd).to(torch.bfloat16)
    score = torch.randn(M, E, generator=g).to(torch.bfloat16)
    return hidden, w1, w2, score


def _np(x):
    return np.asarray(x.double().numpy() if torch.is_tensor(x) else x, dtype=np.float64)


def mlp64(h, w1e, w2e):
    """The gated MLP of one expert in float64 (no rounding): gate = rows :N."""
    N = w2e.shape[-1]
    x = _np(h) @ _np(w1e).T
    g = x[:, :N] / (1.0 + np.exp(-x[:, :N]))
    return (x[:, N:] * g) @ _np(w2e).T


def close(a, b, rel=0.02, atol=1e-6):
    """Within the drift of a few bf16 roundings, measured against the scale of
    the output: intermediate roundings (2^-9 relative each) cancel in the
    down projection, so small outputs carry errors of the large ones' size."""
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return bool(np.abs(a - b).max() <= atol + rel * np.abs(b).max())


# ---------------------------------------------------------------------------
# restatements agree
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("renorm", [False, True])
@pytest.mark.parametrize("M,K,N,E,topk,seed", [(5, 32, 16, 6, 3, 1), (7, 48, 24, 4, 4, 2),
                                                (3, 16, 8, 8, 1, 3)])
def test_restatements_agree_tiny(M, K, N, E, topk, seed, renorm):
    args = make(M, K, N, E, seed, wstd=0.3)
    a = fused_moe_loops(*args, topk, renorm)
    b = fused_moe_fp64(*args, topk, renorm)
    c = fused_moe_ref(*args, topk, renorm).double().numpy()
    assert np.abs(a).max() > 0.1
    assert np.array_equal(a, b)
    # torch's bf16 GEMMs accumulate in float32: at most a rare one-ulp step
    assert close(c, b, rel=2 ** -8)


def test_ref_and_model_agree_at_contest_decode_shape():
    args = make(64, 2048, 1024, 8, seed=0)
    b = fused_moe_fp64(*args, 2)
    c = fused_moe_ref(*args, 2).double().numpy()
    d = np.abs(b - c)
    assert c.dtype == np.float64 and np.abs(b).max() > 0.2
    assert d.max() <= 2 ** -8 * np.abs(b).max() and d.mean() <= 1e-5


def test_bf16_round_is_torch_cast():
    x = np.random.default_rng(0).standard_normal(200_000) * np.exp(
        np.random.default_rng(1).uniform(-20, 20, 200_000))
    x = np.concatenate([x, [0.0, -0.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, np.inf, -np.inf]])
    t = torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    assert np.array_equal(bf16_round(x), t)


# ---------------------------------------------------------------------------
# routing: torch.topk agreement and the tie rule
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("E,topk", [(8, 2), (64, 6), (64, 1), (16, 16)])
def test_route_matches_torch_topk_without_boundary_ties(E, topk):
    score = torch.randn(4096, E, generator=torch.Generator().manual_seed(E + topk)).to(
        torch.bfloat16)
    ids, wts = route(score, topk)
    w = score.float().softmax(dim=-1)
    tv, ti = w.topk(topk, dim=-1)
    srt = torch.sort(w, dim=-1, descending=True).values
    tie = (srt[:, topk - 1] == srt[:, topk]) if topk < E else torch.zeros(4096, dtype=torch.bool)
    ok = ~tie
    assert ok.sum() > 3000
    assert torch.equal(torch.sort(ti, dim=1).values[ok], ids[ok])
    ref_w = torch.gather(tv, 1, torch.argsort(ti, dim=1)).to(torch.bfloat16)
    assert torch.equal(ref_w[ok], wts[ok])


def test_tie_rule_lower_index_first():
    score = torch.tensor([[1.0, 2.0, 2.0, 0.0, 2.0], [3.0, 3.0, 3.0, 3.0, 3.0],
                          [0.5, 0.5, -1.0, 2.0, 0.5]]).to(torch.bfloat16)
    ids, _ = route(score, 2)
    assert ids.tolist() == [[1, 2], [0, 1], [0, 3]]


# ---------------------------------------------------------------------------
# checks, written as functions of an oracle so mutants can be run through them
# ---------------------------------------------------------------------------
def check_single_expert(fn):
    """E = 1, topk = 1: weight 1, the output is the gated MLP (gate = w1[:N])."""
    h, w1, w2, s = make(4, 32, 16, 1, seed=11, wstd=0.3)
    out = np.asarray(fn(h, w1, w2, s, 1), dtype=np.float64)
    return close(out, mlp64(h, w1[0], w2[0]))


def check_zero_hidden(fn):
    h, w1, w2, s = make(3, 32, 16, 4, seed=12, wstd=0.3)
    out = np.asarray(fn(torch.zeros_like(h), w1, w2, s, 2), dtype=np.float64)
    return bool(np.all(out == 0.0))


def check_renormalize_identical_experts(fn):
    """Identical experts: renormalised weights sum to 1 (the MLP itself);
    without renormalisation the MLP is scaled by the top-k softmax mass."""
    h, w1, w2, s = make(5, 32, 16, 1, seed=13, wstd=0.3)
    E = 6
    w1e, w2e = w1.expand(E, -1, -1).contiguous(), w2.expand(E, -1, -1).contiguous()
    score = torch.randn(5, E, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    y = mlp64(h, w1[0], w2[0])
    mass = torch.sort(score.double().softmax(-1), dim=-1, descending=True).values[:, :3].sum(-1)
    ok_r = close(np.asarray(fn(h, w1e, w2e, score, 3, True), dtype=np.float64), y)
    ok_n = close(np.asarray(fn(h, w1e, w2e, score, 3, False), dtype=np.float64),
                 y * mass.numpy()[:, None])
    return ok_r and ok_n


def check_topk_all(fn):
    """topk = E: every expert, weighted by its softmax weight."""
    h, w1, w2, s = make(4, 32, 16, 3, seed=14, wstd=0.3)
    p = s.double().softmax(-1).numpy()
    exp = sum(p[:, e:e + 1] * mlp64(h, w1[e], w2[e]) for e in range(3))
    return close(np.asarray(fn(h, w1, w2, s, 3), dtype=np.float64), exp)


def check_selection(fn):
    """Scores with a clear order: the two largest experts, by softmax weight."""
    h, w1, w2, _ = make(4, 32, 16, 5, seed=15, wstd=0.3)
    s = torch.tensor([[3.0, 0.0, 1.0, -2.0, 2.0], [0.0, 1.0, 2.0, 3.0, 4.0],
                      [4.0, 3.0, 2.0, 1.0, 0.0], [-1.0, 2.5, -1.0, 1.5, -3.0]]).to(torch.bfloat16)
    p = s.double().softmax(-1).numpy()
    exp = np.zeros((4, 32))
    for t, sel in enumerate(([0, 4], [3, 4], [0, 1], [1, 3])):
        for e in sel:
            exp[t] += p[t, e] * mlp64(h[t:t + 1], w1[e], w2[e])[0]
    return close(np.asarray(fn(h, w1, w2, s, 2), dtype=np.float64), exp)


def check_tie_rule(fn):
    """A tie across the top-1 boundary goes to the lower expert index."""
    h, w1, w2, _ = make(2, 32, 16, 4, seed=16, wstd=0.3)
    s = torch.tensor([[0.0, 2.0, 2.0, 1.0], [1.0, -1.0, 1.0, 1.0]]).to(torch.bfloat16)
    p = s.double().softmax(-1).numpy()
    exp = np.stack([p[0, 1] * mlp64(h[:1], w1[1], w2[1])[0],
                    p[1, 0] * mlp64(h[1:], w1[0], w2[0])[0]])
    return close(np.asarray(fn(h, w1, w2, s, 1), dtype=np.float64), exp)


def check_permutation(fn):
    """Permuting experts together with their score columns changes nothing
    but the order of the bf16 sums."""
    h, w1, w2, s = make(6, 32, 16, 5, seed=17, wstd=0.3)
    perm = torch.tensor([3, 0, 4, 1, 2])
    a = np.asarray(fn(h, w1, w2, s, 2), dtype=np.float64)
    b = np.asarray(fn(h, w1[perm], w2[perm], s[:, perm], 2), dtype=np.float64)
    return close(a, b)


CHECKS = [check_single_expert, check_zero_hidden, check_renormalize_identical_experts,
          check_topk_all, check_selection, check_tie_rule, check_permutation]


def _as_np(fn):
    return lambda *a: np.asarray(fn(*a).double().numpy() if torch.is_tensor(fn(*a))
                                 else fn(*a), dtype=np.float64)


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
@pytest.mark.parametrize("oracle", ["ref", "fp64", "loops"])
def test_oracle_passes(check, oracle):
    fn = {"ref": lambda *a: fused_moe_ref(*a).double().numpy(),
          "fp64": fused_moe_fp64, "loops": fused_moe_loops}[oracle]
    assert check(fn)


# ---------------------------------------------------------------------------
# planted mistakes: each must be caught by at least one check
# ---------------------------------------------------------------------------
def _mutant(kind):
    def fn(hidden, w1, w2, score, topk, renormalize=False):
        h, a1, a2 = _np(hidden), _np(w1), _np(w2)
        s = _np(score)
        M, E, N = h.shape[0], a1.shape[0], a2.shape[-1]
        ax = 0 if kind == "softmax_over_tokens" else 1
        z = np.exp(s - s.max(axis=ax, keepdims=True))
        p = (z / z.sum(axis=ax, keepdims=True)).astype(np.float32)
        out = np.zeros((M, a2.shape[1]))
        for t in range(M):
            key = p[t] if kind != "ascending_topk" else -p[t]
            if kind == "higher_index_ties":
                order = np.lexsort((-np.arange(E), -key))
            else:
                order = np.lexsort((np.arange(E), -key))
            sel = order[:topk]
            w = p[t, sel].astype(np.float64)
            if (renormalize and kind != "ignore_renormalize") or kind == "always_renormalize":
                w = w / w.sum()
            if kind == "no_weight":
                w = np.ones_like(w)
            for e, we in sorted(zip(sel, w)):
                x = h[t] @ a1[e].T
                gate, up = (x[N:], x[:N]) if kind == "gate_up_swapped" else (x[:N], x[N:])
                act = gate if kind == "no_silu" else gate / (1.0 + np.exp(-gate))
                out[t] += bf16_round(we) * ((up * act) @ a2[e].T)
        return out
    return fn


MUTANTS = ["gate_up_swapped", "no_silu", "ascending_topk", "softmax_over_tokens",
           "ignore_renormalize", "always_renormalize", "no_weight", "higher_index_ties"]


def test_unmutated_template_passes_every_check():
    fn = _mutant("none")
    failed = [c.__name__ for c in CHECKS if not c(fn)]
    assert not failed, failed


@pytest.mark.parametrize("kind", MUTANTS)
def test_planted_mistake_is_caught(kind):
    fn = _mutant(kind)
    failed = []
    for c in CHECKS:
        try:
            ok = c(fn)
        except Exception:
            ok = False
        if not ok:
            failed.append(c.__name__)
    assert failed, f"mutant {kind} passed every check"


def test_shapes_and_dtype():
    args = make(3, 64, 32, 4, seed=20)
    out = fused_moe_ref(*args, 2)
    assert out.shape == (3, 64) and out.dtype == torch.bfloat16
    assert math.isfinite(float(out.float().abs().max()))
