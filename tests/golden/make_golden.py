"""Writes tests/golden/attention_small.npz: seeded causal sliding-window
attention cases with fp64 expected outputs.

Expected values come from the oracle's per-query brute-force loops (forward,
lse) and its textbook closed-form gradients (numpy), not from torch autograd,
so the fixtures pin the oracle's torch restatement independently.  Inputs are
bf16-representable (rounded through bfloat16), so the same fixtures also feed
the GPU kernels.  Run from the repo root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
from oracle import attention as oracle  # noqa: E402

CASES = {
    # name: (B, T, H, Hkv, D, window (0 = full causal), seed)
    "ragged_w5": (1, 29, 2, 2, 64, 5, 101),
    "gqa_full": (1, 24, 4, 2, 64, 0, 102),
    "d128_w8": (1, 20, 1, 1, 128, 8, 103),
}


def main() -> None:
    out = {}
    for name, (B, T, H, Hkv, D, W, seed) in CASES.items():
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(B, T, H, D, generator=g).bfloat16().double().numpy()
        k = torch.randn(B, T, Hkv, D, generator=g).bfloat16().double().numpy()
        v = torch.randn(B, T, Hkv, D, generator=g).bfloat16().double().numpy()
        do = torch.randn(B, T, H, D, generator=g).bfloat16().double().numpy()
        win = W if W > 0 else None
        o, lse = oracle.brute_force_forward(q, k, v, win)
        rep = H // Hkv
        kr, vr = np.repeat(k, rep, axis=2), np.repeat(v, rep, axis=2)
        dq, dk, dv = oracle.closed_form_backward(q, kr, vr, do, win)
        dk = dk.reshape(B, T, Hkv, rep, D).sum(3)
        dv = dv.reshape(B, T, Hkv, rep, D).sum(3)
        for key, val in (("q", q), ("k", k), ("v", v), ("do", do)):
            out[f"{name}/{key}"] = val.astype(np.float32)  # exact: bf16 values
        for key, val in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            out[f"{name}/{key}"] = val
        out[f"{name}/window"] = np.array(W)
    path = Path(__file__).with_name("attention_small.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
