"""CPU oracle for hackable-lm's residual add + RMSNorm (no weight).

TEST INFRASTRUCTURE ONLY.  Only tests/ may import this module, and only as
the checker.  The library in hackable-lm_amd/hlm_attn never imports it.

What it restates:
  residual_rms_norm           model.py:73-75 with rms_norm_torch (model.py:14-16):
                              out = residual + branch in the inputs' dtype (one
                              rounding, as the bf16 add rounds), then
                              normed = out * rsqrt(mean(out^2) + eps) evaluated
                              in `compute` precision from that out
  residual_rms_norm_backward  the gradient autograd takes through the two
                              lines above, in closed form: both inputs receive
                              grad_out + r (grad_normed - z mean(grad_normed z))

How they are pinned (tests/test_oracle_residual_norm.py): residual_rms_norm by
a brute-force loop over rows; the backward by fp64 autograd of the reference
formula and by central finite differences; invariants (a row's normed RMS is
1 up to eps, scaling a row leaves normed unchanged); planted mistakes (a sum
in place of the mean, a missing grad_out term, r in place of r^3) rejected.
"""
from __future__ import annotations

import torch


def residual_rms_norm(residual: torch.Tensor, branch: torch.Tensor, eps: float,
                      compute: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """model.py:73-75: (out in the inputs' dtype, normed in `compute`)."""
    out = residual + branch
    o = out.to(compute)
    return out, o * torch.rsqrt(o.pow(2).mean(dim=-1, keepdim=True) + eps)


def residual_rms_norm_backward(out: torch.Tensor, grad_out: torch.Tensor, grad_normed: torch.Tensor,
                               eps: float, compute: torch.dtype = torch.float32) -> torch.Tensor:
    """Closed-form gradient of (out, normed) with respect to residual (and
    equally branch), from the forward's out."""
    o = out.to(compute)
    gn = grad_normed.to(compute)
    r = torch.rsqrt(o.pow(2).mean(dim=-1, keepdim=True) + eps)
    mean_gz = (gn * o * r).mean(dim=-1, keepdim=True)
    return grad_out.to(compute) + r * (gn - o * r * mean_gz)
