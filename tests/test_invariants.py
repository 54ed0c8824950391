"""The full-size invariant checks (tests/attn_checks.py) must accept correct
results rounded to bf16 and reject plausible mistakes.

The honest results are the oracle's fp64 closed forms and brute force
(oracle/attention.py), rounded to bf16 as the kernels' outputs are.  Each
mistake is planted in a throw-away copy of the oracle's source, on the CPU.
"""
from __future__ import annotations

import types
from pathlib import Path

import numpy as np
import pytest
import torch

import attn_checks

REPO = Path(__file__).resolve().parents[1]
SOURCE = (REPO / "oracle" / "attention.py").read_text()


def variant(old: str | None = None, new: str | None = None) -> types.ModuleType:
    src = SOURCE
    if old is not None:
        assert src.count(old) == 1, f"mutation anchor not found once: {old!r}"
        src = src.replace(old, new)
    mod = types.ModuleType("oracle_variant")
    exec(compile(src, "oracle_variant", "exec"), mod.__dict__)
    return mod


def bf16(x) -> torch.Tensor:
    return torch.as_tensor(np.asarray(x)).to(torch.bfloat16).float()


def ratios(mod, window, T=200, H=2, D=16, seed=0) -> dict:
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(1, T, H, D, generator=g, dtype=torch.float64) for _ in range(4))
    q, k, v, do = (t.bfloat16().double() for t in (q, k, v, do))
    o, _ = mod.brute_force_forward(q.numpy(), k.numpy(), v.numpy(), window)
    _, dk, dv = mod.closed_form_backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), window)
    return attn_checks.invariant_ratios(bf16(o), bf16(dk), bf16(dv), v, do, window)


@pytest.mark.parametrize("window", [None, 1, 5, 24, 199])
def test_correct_results_in_bf16_pass(window):
    r = ratios(variant(), window)
    print(r)
    assert attn_checks.invariants_hold(r), r


def test_grouped_query_heads_pass():
    """Hkv < H: dv_sum sums dO over the query heads of each kv head."""
    from oracle import attention as oracle

    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 150, 4, 16, generator=g).bfloat16()
    k, v = (torch.randn(2, 150, 2, 16, generator=g).bfloat16() for _ in range(2))
    do = torch.randn(2, 150, 4, 16, generator=g).bfloat16()
    o, _ = oracle.forward(q, k, v, 20, dtype=torch.float64)
    _, dk, dv = oracle.backward(q, k, v, do, 20, dtype=torch.float64)
    r = attn_checks.invariant_ratios(o.bfloat16(), dk.bfloat16(), dv.bfloat16(), v, do, 20)
    assert attn_checks.invariants_hold(r), r


def test_window_extreme_matches_brute_force():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 37, 3, 5, generator=g)
    for w in (1, 2, 3, 7, 8, 9, 36, 37, 50):
        mx = attn_checks._window_extreme(x, w, True)
        mn = attn_checks._window_extreme(x, w, False)
        for t in range(37):
            lo = max(0, t - w + 1)
            assert torch.equal(mx[:, t], x[:, lo : t + 1].amax(dim=1))
            assert torch.equal(mn[:, t], x[:, lo : t + 1].amin(dim=1))


MUTANTS = {
    # caught by dk_sum: the rows of dS no longer sum to zero
    "dropped delta term": ("dS = P * (dP - (dO * O).sum(axis=1, keepdims=True))", "dS = P * dP", "dk_sum"),
    "transposed dS in dK": ("dk[b, :, h] = scale * dS.T @ Q", "dk[b, :, h] = scale * dS @ Q", "dk_sum"),
    # caught by dv_sum: P from a mask one key wider at both ends (the next key
    # past the diagonal, one more at the window edge) than the lse that
    # normalises it
    "mask off by one between P and lse": (
        "P = np.exp(S - S.max(axis=1, keepdims=True))\n            P /= P.sum(axis=1, keepdims=True)",
        "S1 = np.where((i - j >= -1) & (i - j < w + 1), scale * Q @ K.T, -np.inf)\n"
        "            P = np.exp(S1 - S.max(axis=1, keepdims=True))\n"
        "            P /= np.exp(S - S.max(axis=1, keepdims=True)).sum(axis=1, keepdims=True)",
        "dv_sum",
    ),
    "stale row sum (P rows sum to 0.95)": (
        "P /= P.sum(axis=1, keepdims=True)", "P /= 1.05 * P.sum(axis=1, keepdims=True)", "dv_sum",
    ),
    # caught by o_hull: O normalised by a wrong sum
    "O normalised by 0.95 of its row sum": ("o[b, i, h] = acc / z", "o[b, i, h] = acc / (0.95 * z)", "o_hull"),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
@pytest.mark.parametrize("window", [None, 24])
def test_mutant_is_caught(name, window):
    old, new, check = MUTANTS[name]
    r = ratios(variant(old, new), window)
    tol = {"dk_sum": attn_checks.DK_SUM_TOL, "dv_sum": attn_checks.DV_SUM_TOL, "o_hull": attn_checks.O_HULL_TOL}
    assert r[check] > tol[check], (name, r)
    assert not attn_checks.invariants_hold(r)
