"""The oracle's pins must catch plausible mistakes.

Each case plants one mistake in a copy of oracle/attention.py (on the CPU,
in a throw-away module) and checks that the independent pins used by
tests/test_oracle.py -- fp64 brute force, closed forms, the committed golden
vectors -- reject the mutant while accepting the real oracle.
"""
from __future__ import annotations

import math
import types
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
SOURCE = (REPO / "oracle" / "attention.py").read_text()
GOLDEN = np.load(Path(__file__).with_name("golden") / "attention_small.npz")


def load_variant(old: str | None = None, new: str | None = None) -> types.ModuleType:
    src = SOURCE
    if old is not None:
        assert src.count(old) >= 1, f"mutation anchor not found: {old!r}"
        src = src.replace(old, new)
    mod = types.ModuleType("oracle_variant")
    exec(compile(src, "oracle_variant", "exec"), mod.__dict__)
    return mod


def pins_hold(mod) -> bool:
    """True when `mod` passes the pins: brute force (forward), the GQA case,
    closed forms of the special cases, and the golden vectors (fwd + bwd)."""
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(2, 23, 2, 8, generator=g, dtype=torch.float64) for _ in range(3))
    ref = types.ModuleType("ref")
    exec(compile(SOURCE, "ref", "exec"), ref.__dict__)
    for W in (None, 4):
        o, lse = mod.forward(q, k, v, W, dtype=torch.float64)
        bo, blse = ref.brute_force_forward(q.numpy(), k.numpy(), v.numpy(), W)
        if not (np.allclose(o.numpy(), bo, atol=2e-6) and np.allclose(lse.numpy(), blse, atol=1e-10)):
            return False
    # grouped-query heads: 4 query heads over 2 kv heads (head h reads kv head h // 2)
    q4 = torch.randn(2, 23, 4, 8, generator=g, dtype=torch.float64)
    o, _ = mod.forward(q4, k, v, 6, dtype=torch.float64)
    bo, _ = ref.brute_force_forward(q4.numpy(), k.numpy(), v.numpy(), 6)
    if not np.allclose(o.numpy(), bo, atol=2e-6):
        return False
    qz = torch.zeros_like(q)
    _, lse = mod.forward(qz, k, v, 5, dtype=torch.float64)
    expect = torch.tensor([math.log(min(i + 1, 5)) for i in range(23)], dtype=torch.float64)
    if not torch.allclose(lse, expect.expand_as(lse), atol=1e-10):
        return False
    for name in ("ragged_w5", "gqa_full"):
        c = {key: torch.from_numpy(GOLDEN[f"{name}/{key}"]) for key in ("q", "k", "v", "do", "o", "dq", "dk", "dv")}
        W = int(GOLDEN[f"{name}/window"]) or None
        o, _ = mod.forward(c["q"], c["k"], c["v"], W, dtype=torch.float64)
        dq, dk, dv = mod.backward(c["q"], c["k"], c["v"], c["do"], W, dtype=torch.float64)
        for got, key in ((o, "o"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
            if not torch.allclose(got, c[key].double(), atol=2e-5):
                return False
        if name == "ragged_w5":
            Hq = c["q"].shape[2]
            cq, ck, cv = mod.closed_form_backward(c["q"].numpy(), c["k"].numpy(), c["v"].numpy(), c["do"].numpy(), W)
            for got, key in ((cq, "dq"), (ck, "dk"), (cv, "dv")):
                if not np.allclose(got, c[key].numpy(), atol=1e-9):
                    return False
            assert Hq == 2
    return True


def test_real_oracle_passes_the_pins():
    assert pins_hold(load_variant())


MUTANTS = {
    "window off by one (mask)": ("return ((distance >= 0) & (distance < window))",
                                 "return ((distance >= 0) & (distance <= window))"),
    "window off by one (scores)": ("ok = (dist >= 0) & (dist < w)\n    return s.masked_fill",
                                   "ok = (dist >= 0) & (dist <= w)\n    return s.masked_fill"),
    "scale 1/D instead of 1/sqrt(D)": ("scale = 1.0 / math.sqrt(q.shape[-1])\n    attn =",
                                       "scale = 1.0 / q.shape[-1]\n    attn ="),
    "anti-causal mask": ("causal = torch.ones((q_len, kv_len), dtype=torch.bool).tril()",
                         "causal = torch.ones((q_len, kv_len), dtype=torch.bool).triu()"),
    "softmax over the wrong axis": ("attn = torch.softmax(attn.float(), dim=-1)",
                                    "attn = torch.softmax(attn.float(), dim=-2)"),
    "gqa heads tiled instead of interleaved": ("kh = kh.repeat_interleave(rep, dim=1)\n        vh = vh.repeat_interleave(rep, dim=1)",
                                               "kh = kh.repeat(1, rep, 1, 1)\n        vh = vh.repeat(1, rep, 1, 1)"),
    "dropped delta term in dS": ("dS = P * (dP - (dO * O).sum(axis=1, keepdims=True))", "dS = P * dP"),
    "transposed operand in dK": ("dk[b, :, h] = scale * dS.T @ Q", "dk[b, :, h] = scale * dS @ Q"),
    "dQ sign error": ("dq[b, :, h] = scale * dS @ K", "dq[b, :, h] = -scale * dS @ K"),
    "lse without the max shift": ("lse[b, h, i] = m + math.log(z)", "lse[b, h, i] = math.log(z)"),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_mutant_is_caught(name):
    old, new = MUTANTS[name]
    mod = load_variant(old, new)
    if name == "lse without the max shift":
        # brute force is the pin itself here: the torch restatement must disagree with it
        g = torch.Generator().manual_seed(9)
        q, k, v = (torch.randn(1, 9, 1, 8, generator=g, dtype=torch.float64) for _ in range(3))
        _, lse = load_variant().forward(q, k, v, 4, dtype=torch.float64)
        _, blse = mod.brute_force_forward(q.numpy(), k.numpy(), v.numpy(), 4)
        assert not np.allclose(lse.numpy(), blse, atol=1e-6)
        return
    assert not pins_hold(mod), f"mutant {name!r} slipped through the pins"
