"""Pins of the residual add + RMSNorm oracle (oracle/residual_norm.py), CPU only."""
from __future__ import annotations

import math

import torch

from oracle import residual_norm as ro


def _brute(residual, branch, eps):
    out = residual + branch
    normed = torch.empty(out.shape, dtype=torch.float64)
    for idx in range(out.shape[0]):
        row = [float(v) for v in out[idx]]
        inv = 1.0 / math.sqrt(sum(v * v for v in row) / len(row) + eps)
        normed[idx] = torch.tensor([v * inv for v in row], dtype=torch.float64)
    return out, normed


def test_forward_matches_brute_force_and_bf16_add():
    g = torch.Generator().manual_seed(0)
    res = torch.randn(6, 24, generator=g).bfloat16()
    br = torch.randn(6, 24, generator=g).bfloat16()
    out, normed = ro.residual_rms_norm(res, br, 1e-6, compute=torch.float64)
    assert out.dtype == torch.bfloat16 and torch.equal(out, (res.float() + br.float()).bfloat16())
    _, bn = _brute(out.double(), torch.zeros_like(out, dtype=torch.float64), 1e-6)
    assert torch.allclose(normed, bn, atol=1e-12)


def test_invariants():
    x = torch.randn(5, 32, dtype=torch.float64) * 7
    _, n1 = ro.residual_rms_norm(x, torch.zeros_like(x), 0.0, compute=torch.float64)
    assert torch.allclose(n1.pow(2).mean(dim=-1), torch.ones(5, dtype=torch.float64), atol=1e-12)
    _, n2 = ro.residual_rms_norm(3 * x, torch.zeros_like(x), 0.0, compute=torch.float64)
    assert torch.allclose(n1, n2, atol=1e-12)


def test_backward_matches_autograd_and_finite_differences():
    g = torch.Generator().manual_seed(1)
    res = torch.randn(4, 16, generator=g, dtype=torch.float64, requires_grad=True)
    br = torch.randn(4, 16, generator=g, dtype=torch.float64, requires_grad=True)
    g_out = torch.randn(4, 16, generator=g, dtype=torch.float64)
    g_norm = torch.randn(4, 16, generator=g, dtype=torch.float64)
    out = res + br
    normed = out * torch.rsqrt(out.pow(2).mean(dim=-1, keepdim=True) + 1e-6)  # model.py:14-16, 73-75
    ((out * g_out).sum() + (normed * g_norm).sum()).backward()
    got = ro.residual_rms_norm_backward(out.detach(), g_out, g_norm, 1e-6, compute=torch.float64)
    assert torch.allclose(got, res.grad, atol=1e-12) and torch.allclose(got, br.grad, atol=1e-12)
    x0 = res.detach()
    step = 1e-6
    for idx in ((0, 0), (2, 7), (3, 15)):
        e = torch.zeros_like(x0)
        e[idx] = step

        def loss(x):
            o, n = ro.residual_rms_norm(x, br.detach(), 1e-6, compute=torch.float64)
            return (o * g_out).sum() + (n * g_norm).sum()

        fd = (loss(x0 + e) - loss(x0 - e)).item() / (2 * step)
        assert abs(fd - got[idx].item()) < 1e-6


def test_mutants_are_caught():
    g = torch.Generator().manual_seed(2)
    o = torch.randn(3, 8, generator=g, dtype=torch.float64)
    go = torch.randn(3, 8, generator=g, dtype=torch.float64)
    gn = torch.randn(3, 8, generator=g, dtype=torch.float64)
    good = ro.residual_rms_norm_backward(o, go, gn, 1e-6, compute=torch.float64)
    r = torch.rsqrt(o.pow(2).mean(dim=-1, keepdim=True) + 1e-6)
    mutants = [
        r * (gn - o * r * (gn * o * r).mean(dim=-1, keepdim=True)),            # grad_out dropped
        go + r * (gn - o * (gn * o * r).mean(dim=-1, keepdim=True)),           # r^3 -> r^2
        go + r * (gn - o * r * (gn * o * r).sum(dim=-1, keepdim=True)),        # sum for mean
    ]
    for bad in mutants:
        assert not torch.allclose(bad, good, atol=1e-6)
    _, n_sum = ro.residual_rms_norm(o, torch.zeros_like(o), 1e-6, compute=torch.float64)
    wrong = o * torch.rsqrt(o.pow(2).sum(dim=-1, keepdim=True) + 1e-6)
    assert not torch.allclose(wrong, n_sum, atol=1e-6)
