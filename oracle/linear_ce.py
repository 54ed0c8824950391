"""CPU oracle for hackable-lm's LM-head fused linear + cross-entropy.

TEST INFRASTRUCTURE ONLY.  Only tests/ may import
this module, and only as the checker.  The library in hackable-lm_amd/hlm_attn
never imports it.

What it restates (each function cites the reference lines it follows):
  ce_rows                     kernels.py:292-316 (_linear_ce_kernel): per row,
                              loss = (logsumexp(x) - x_t) / n_tokens and the
                              row overwritten with (softmax(x) - onehot_t) / n_tokens;
                              plus F.cross_entropy's ignore_index rule (a
                              target of -100 gives a zero row), which the
                              reference's torch path (model.py:324-339) applies
  fused_linear_cross_entropy  kernels.py:878-942: the chunked loop; returns the
                              mean loss and the gradients of hidden, W and b
  lm_head_torch_loss          model.py:324-339 (LMHeadProjection.fwd_torch):
                              chunked F.cross_entropy(reduction="sum") / n_tokens

How each one is pinned (tests/test_oracle_ce.py): lm_head_torch_loss by the
reference test's own closed form on its own shapes (tests/test_kernels.py:
11-26: vocab 33, (3, 7) tokens, dense F.cross_entropy, atol 1e-6); ce_rows by
autograd of F.cross_entropy in fp64 (with ignored rows), by uniform logits
(loss = log V / n), by gradient rows summing to zero, and by planted mistakes
it must reject; fused_linear_cross_entropy by autograd of the dense loss in
fp64 for all three gradients and by chunked == unchunked.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

IGNORE_INDEX = -100


def ce_rows(logits: torch.Tensor, targets: torch.Tensor, n_tokens: int,
            ignore_index: int = IGNORE_INDEX) -> tuple[torch.Tensor, torch.Tensor]:
    """kernels.py:292-316 in fp64: (per-row loss, gradient rows) for (rows, V)
    logits; rows whose target is ignore_index are zero in both."""
    x = logits.to(torch.float64)
    t = targets.to(torch.int64)
    m = x.max(dim=-1, keepdim=True).values
    e = torch.exp(x - m)
    d = e.sum(dim=-1, keepdim=True)
    lse = (m + torch.log(d)).squeeze(-1)
    valid = t != ignore_index
    safe_t = torch.where(valid, t, torch.zeros_like(t))
    target_logit = x.gather(1, safe_t[:, None]).squeeze(1)
    loss = torch.where(valid, (lse - target_logit) / n_tokens, torch.zeros_like(lse))
    grad = e / d
    grad[torch.arange(x.shape[0]), safe_t] -= 1.0
    grad = torch.where(valid[:, None], grad / n_tokens, torch.zeros_like(grad))
    return loss, grad


def fused_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                               targets: torch.Tensor, chunk_size: int) -> tuple[torch.Tensor, ...]:
    """kernels.py:878-942 in fp64: (mean loss, grad_hidden, grad_weight,
    grad_bias or None), chunk by chunk of `chunk_size` rows."""
    h = hidden.reshape(-1, hidden.shape[-1]).to(torch.float64)
    w = weight.to(torch.float64)
    b = None if bias is None else bias.to(torch.float64)
    t = targets.reshape(-1)
    n_tokens = h.shape[0]
    grad_h = torch.zeros_like(h)
    grad_w = torch.zeros_like(w)
    grad_b = None if b is None else torch.zeros_like(b)
    loss = torch.zeros((), dtype=torch.float64)
    for start in range(0, n_tokens, chunk_size):
        end = min(start + chunk_size, n_tokens)
        logits = h[start:end] @ w.t()
        if b is not None:
            logits = logits + b
        rows, g = ce_rows(logits, t[start:end], n_tokens)
        loss = loss + rows.sum()
        grad_h[start:end] = g @ w
        grad_w += g.t() @ h[start:end]
        if grad_b is not None:
            grad_b += g.sum(dim=0)
    return loss, grad_h, grad_w, grad_b


def lm_head_torch_loss(hidden: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                       targets: torch.Tensor, chunk_size: int | None) -> torch.Tensor:
    """model.py:324-339: chunked F.cross_entropy(reduction="sum") / n_tokens."""
    h = hidden.reshape(-1, hidden.shape[-1])
    t = targets.reshape(-1)
    n_tokens = t.numel()
    step = chunk_size if chunk_size else n_tokens
    total = h.new_zeros((), dtype=torch.float32)
    for start in range(0, n_tokens, step):
        end = min(start + step, n_tokens)
        logits = F.linear(h[start:end], weight, bias)
        total = total + F.cross_entropy(logits.float(), t[start:end], reduction="sum")
    return total / n_tokens
