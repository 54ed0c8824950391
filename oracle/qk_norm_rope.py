"""CPU oracle for hackable-lm's fused q/k RMSNorm + partial rotary embedding.

TEST INFRASTRUCTURE ONLY.  Only tests/ may import this module, and only as
the checker.  The library in hackable-lm_amd/hlm_attn never imports it.

What it restates (each function cites the reference lines it follows):
  rms_norm                 kernels.py:245-248 (model.py:14-16): x * rsqrt(mean(x^2) + eps)
  apply_partial_rope       kernels.py:670-676: the first R = cos.shape[-1] dims
                           rotate in pairs (d, d + R/2) with cos/sin[..., :R/2];
                           the rest pass through
  qk_norm_rope             kernels.py:756-771 CPU branch (= QKVProjection.fwd_torch,
                           model.py:101-115): norm, then rope, for q and k
  qk_norm_rope_backward    kernels.py:703-741 CPU branch: the gradient rotated
                           back (apply_partial_rope with -sin), then the
                           weightless RMSNorm backward in closed form
  rotary_tables            model.py:50-70 RotaryEmbedding tables (cos, sin of
                           positions x inverse frequencies, duplicated halves)

How each one is pinned (tests/test_oracle_qk.py): qk_norm_rope against the
reference test's own closed form on its own shapes (tests/test_kernels.py:
265-299: q (2,5,3,8), k (2,5,2,8), R = 4, atol 1e-6); qk_norm_rope_backward
against autograd of qk_norm_rope (and the reference test's autograd check) and
against central finite differences in fp64; invariants: the rotation keeps
every row's norm (|out| = |x| * rsqrt(mean(x^2) + eps)), R = 0 reduces to
plain RMSNorm, and the rotation of the pair (d, d + h) is the 2-D rotation by
the angle whose cos/sin are given; rotary_tables against model.py's formula
for a few entries computed by hand.
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    """kernels.py:245-248 without a weight."""
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)


def _as_bt1r(t: torch.Tensor, T: int) -> torch.Tensor:
    """cos / sin given as (T, R), (1, T, 1, R) or (1, 1, T, R) -> (1, T, 1, R)."""
    R = t.shape[-1]
    return t.reshape(T, R)[None, :, None, :]


def apply_partial_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """kernels.py:670-676 on x (B, T, heads, D) with cos/sin broadcastable to it."""
    rotary_dim = cos.shape[-1]
    half = rotary_dim // 2
    cos_half = cos[..., :half]
    sin_half = sin[..., :half]
    x1, x2, x_pass = x[..., :half], x[..., half:rotary_dim], x[..., rotary_dim:]
    return torch.cat((x1 * cos_half - x2 * sin_half, x2 * cos_half + x1 * sin_half, x_pass), dim=-1)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """kernels.py:756-771 (CPU branch), computed in the inputs' dtype (use fp32
    or fp64 inputs for a reference)."""
    T = q.shape[1]
    c, s = _as_bt1r(cos, T).to(q.dtype), _as_bt1r(sin, T).to(q.dtype)
    return apply_partial_rope(rms_norm(q, eps), c, s), apply_partial_rope(rms_norm(k, eps), c, s)


def _norm_backward_no_weight(x: torch.Tensor, grad: torch.Tensor, eps: float) -> torch.Tensor:
    """kernels.py:703-708: d/dx of x * rsqrt(mean(x^2) + eps) applied to grad."""
    inv = torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    dot = (grad * x).mean(dim=-1, keepdim=True)
    return grad * inv - x * inv.pow(3) * dot


def qk_norm_rope_backward(q: torch.Tensor, k: torch.Tensor, grad_q: torch.Tensor, grad_k: torch.Tensor,
                          cos: torch.Tensor, sin: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """kernels.py:711-741 (CPU branch): rotate the gradient back, then the norm
    backward."""
    T = q.shape[1]
    c, s = _as_bt1r(cos, T).to(q.dtype), _as_bt1r(sin, T).to(q.dtype)
    gq = apply_partial_rope(grad_q.to(q.dtype), c, -s)
    gk = apply_partial_rope(grad_k.to(q.dtype), c, -s)
    return _norm_backward_no_weight(q, gq, eps), _norm_backward_no_weight(k, gk, eps)


def rotary_tables(T: int, dim: int, theta: float = 1_000_000.0, fraction: float = 0.25,
                  dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """model.py:50-70 RotaryEmbedding: (T, R) cos and sin tables, R = the rotary
    width int(dim * fraction) rounded down to even; both halves repeat the
    R / 2 frequencies."""
    rotary_dim = int(dim * fraction)
    rotary_dim -= rotary_dim % 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2).float() / rotary_dim))
    t = torch.arange(T, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)
