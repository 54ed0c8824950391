"""Pins of the LM-head cross-entropy oracle (oracle/linear_ce.py), CPU only."""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import linear_ce as co


def test_reference_test_dense_equals_chunked():
    """tests/test_kernels.py:11-26: vocab 33, hidden (3, 7, n_embd), targets in
    [0, 33), dense F.cross_entropy == the chunked torch head at atol 1e-6."""
    torch.manual_seed(0)
    n_embd = 64
    weight = torch.randn(33, n_embd) * 0.02
    hidden = torch.randn(3, 7, n_embd)
    targets = torch.randint(0, 33, (3, 7))
    dense = F.cross_entropy(F.linear(hidden, weight).float().reshape(-1, 33), targets.reshape(-1))
    for chunk in (None, 4, 5, 21):
        assert torch.allclose(co.lm_head_torch_loss(hidden, weight, None, targets, chunk), dense, atol=1e-6)


def test_ce_rows_match_autograd_with_ignored_rows():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(9, 40, generator=g, dtype=torch.float64) * 3
    targets = torch.randint(0, 40, (9,), generator=g)
    targets[2] = -100
    targets[5] = 39
    n_tokens = 23  # the mean runs over all tokens, not over this chunk's rows
    x = logits.clone().requires_grad_(True)
    ref = F.cross_entropy(x, targets, reduction="sum") / n_tokens
    ref.backward()
    loss, grad = co.ce_rows(logits, targets, n_tokens)
    assert torch.allclose(loss.sum(), ref.detach(), atol=1e-12)
    assert torch.allclose(grad, x.grad, atol=1e-12)
    assert loss[2] == 0 and torch.count_nonzero(grad[2]) == 0


def test_ce_rows_closed_forms():
    V, n = 50, 7
    loss, grad = co.ce_rows(torch.zeros(3, V), torch.tensor([0, 10, V - 1]), n)
    assert torch.allclose(loss, torch.full((3,), math.log(V) / n, dtype=torch.float64))
    assert torch.allclose(grad.sum(dim=-1), torch.zeros(3, dtype=torch.float64), atol=1e-15)
    assert math.isclose(grad[1, 10].item(), (1 / V - 1) / n)
    # shift invariance and no overflow for large logits
    big = torch.randn(4, V, dtype=torch.float64) + 1e4
    l1, g1 = co.ce_rows(big, torch.tensor([1, 2, 3, 4]), n)
    l2, g2 = co.ce_rows(big - 1e4, torch.tensor([1, 2, 3, 4]), n)
    assert torch.isfinite(l1).all() and torch.allclose(l1, l2, atol=1e-9) and torch.allclose(g1, g2, atol=1e-12)


def test_fused_linear_cross_entropy_matches_autograd():
    g = torch.Generator().manual_seed(2)
    hidden = torch.randn(37, 16, generator=g, dtype=torch.float64)
    weight = torch.randn(29, 16, generator=g, dtype=torch.float64) * 0.3
    bias = torch.randn(29, generator=g, dtype=torch.float64) * 0.1
    targets = torch.randint(0, 29, (37,), generator=g)
    targets[3] = -100
    h, w, b = (t.clone().requires_grad_(True) for t in (hidden, weight, bias))
    ref = F.cross_entropy(F.linear(h, w, b), targets, reduction="sum") / 37
    ref.backward()
    for chunk in (37, 8, 5):
        loss, gh, gw, gb = co.fused_linear_cross_entropy(hidden, weight, bias, targets, chunk)
        assert torch.allclose(loss, ref.detach(), atol=1e-12)
        assert torch.allclose(gh, h.grad, atol=1e-12)
        assert torch.allclose(gw, w.grad, atol=1e-12)
        assert torch.allclose(gb, b.grad, atol=1e-12)


# --- planted mistakes must be caught ------------------------------------------

def _mutant(kind):
    def ce_rows(logits, targets, n_tokens, ignore_index=-100):
        x = logits.to(torch.float64)
        t = targets.to(torch.int64)
        e = torch.exp(x) if kind == "no_max" else torch.exp(x - x.max(dim=-1, keepdim=True).values)
        p = e / e.sum(dim=-1, keepdim=True)
        n = x.shape[0] if kind == "per_chunk_mean" else n_tokens
        tt = (t + 1) % x.shape[1] if kind == "off_by_one" else t
        grad = p.clone()
        if kind != "no_onehot":
            grad[torch.arange(x.shape[0]), tt] -= 1.0
        loss = -torch.log(p.gather(1, tt[:, None]).squeeze(1))
        return loss / n, grad / n
    return ce_rows


@pytest.mark.parametrize("kind", ["no_max", "per_chunk_mean", "off_by_one", "no_onehot"])
def test_ce_mutants_are_caught(kind):
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(6, 30, generator=g, dtype=torch.float64) * 2 + (800 if kind == "no_max" else 0)
    targets = torch.randint(0, 30, (6,), generator=g)
    x = logits.clone().requires_grad_(True)
    ref = F.cross_entropy(x, targets, reduction="sum") / 11
    ref.backward()
    loss, grad = _mutant(kind)(logits, targets, 11)
    bad = not (torch.isfinite(loss).all() and torch.allclose(loss.sum(), ref.detach(), atol=1e-9)
               and torch.allclose(grad, x.grad, atol=1e-9))
    assert bad
