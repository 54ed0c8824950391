"""Size-independent checks of attention outputs over every (batch, head) slice.

Used by the GPU parity tests at BASELINE's full sizes, where the exact oracle
covers only bands of a few slices; tests/test_invariants.py pins these checks
on the CPU (they accept the oracle's bf16-rounded results and reject planted
mistakes).  All three follow from the math of the `torch` backend
(kernels.py:785-800), whatever the inputs:

  dk_sum   sum_j dS_ij = sum_j P_ij (dP_ij - delta_i) = 0 for every query row
           i, because delta_i = sum_d dO_id O_id = sum_j P_ij dP_ij.  Hence
           sum_j dK_j = scale sum_i (sum_j dS_ij) q_i = 0 per (batch, kv head).
  dv_sum   rows of P sum to 1, so sum_j dV_j = sum_j sum_i P_ij dO_i =
           sum_i dO_i, summed over the query heads of each kv head.
  o_hull   O_i is a convex combination of the V rows in its window, so every
           component of O_i lies in [min_j V_jd, max_j V_jd] over that window.

Ratios are scale-free: dk_sum = ||sum_j dK_j|| / sqrt(sum_j ||dK_j||^2) (and
the same for dV after subtracting sum_i dO_i); o_hull = the largest excess of
O beyond the window's [min, max] in units of the window's max |V|.  Rounding
the results to bf16 keeps dk_sum and dv_sum near 2^-8 / sqrt(3) (random
rounding errors of 2^-8 relative size add in quadrature in both numerator and
denominator) and o_hull below 2^-7 (the P weights rounded to bf16 sum to
1 +- 2^-8, then O itself is rounded); a dropped delta term, a transposed
operand, a window off by one between forward and backward or a missing
normalisation give ratios of order 0.1 to 1.
"""
from __future__ import annotations

import torch

DK_SUM_TOL = 0.02
DV_SUM_TOL = 0.02
O_HULL_TOL = 2.0 ** -7 + 1e-6


def _window_extreme(x: torch.Tensor, w: int, largest: bool) -> torch.Tensor:
    """max (or min) of x over the last w positions (inclusive) along dim 1 of
    (B, T, ...), by doubling: O(T log w)."""
    T = x.shape[1]
    w = min(w, T)
    op = torch.maximum if largest else torch.minimum
    fill = float("-inf") if largest else float("inf")

    def shifted(y: torch.Tensor, s: int) -> torch.Tensor:
        out = torch.full_like(y, fill)
        if s < T:
            out[:, s:] = y[:, : T - s]
        return out

    m, span = x, 1
    while 2 * span <= w:
        m = op(m, shifted(m, span))
        span *= 2
    # m[t] covers [t - span + 1, t]; cover [t - w + 1, t] with two such spans
    return op(m, shifted(m, w - span)) if w > span else m


def invariant_ratios(o, dk, dv, v, do, window: int | None) -> dict:
    """Worst ratio of each invariant over all slices, as Python floats.

    o, do: (B, T, H, D); dk, dv, v: (B, T, Hkv, D); any float dtype, any
    device (computed in fp32 there).  window None or >= T means causal."""
    B, T, H, D = o.shape
    Hkv = v.shape[2]
    G = H // Hkv
    o, dk, dv, v, do = (t.float() for t in (o, dk, dv, v, do))
    # dk_sum per (b, kv head)
    s = dk.sum(dim=1)                                     # (B, Hkv, D)
    den = dk.pow(2).sum(dim=(1, 3)).sqrt().clamp_min(1e-30)  # (B, Hkv)
    dk_sum = (s.norm(dim=-1) / den).max().item()
    # dv_sum per (b, kv head): sum_j dV_j - sum_i,g dO_i
    sdo = do.view(B, T, Hkv, G, D).sum(dim=(1, 3))        # (B, Hkv, D)
    den = dv.pow(2).sum(dim=(1, 3)).sqrt().clamp_min(1e-30)
    dv_sum = ((dv.sum(dim=1) - sdo).norm(dim=-1) / den).max().item()
    # o_hull per element
    w = T if window is None else min(window, T)
    vmax = _window_extreme(v, w, True).repeat_interleave(G, dim=2)
    vmin = _window_extreme(v, w, False).repeat_interleave(G, dim=2)
    scale = torch.maximum(vmax.abs(), vmin.abs()).clamp_min(1e-30)
    excess = torch.clamp(o - vmax, min=0) + torch.clamp(vmin - o, min=0)
    o_hull = (excess / scale).max().item()
    return {"dk_sum": dk_sum, "dv_sum": dv_sum, "o_hull": o_hull}


def invariants_hold(r: dict) -> bool:
    return r["dk_sum"] <= DK_SUM_TOL and r["dv_sum"] <= DV_SUM_TOL and r["o_hull"] <= O_HULL_TOL
