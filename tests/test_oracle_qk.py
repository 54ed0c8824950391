"""Pins of the q/k RMSNorm + partial RoPE oracle (oracle/qk_norm_rope.py), CPU only.

Checks that do not restate the oracle's own formula: the reference test's
closed form on its shapes (tests/test_kernels.py:265-299), the 2-D rotation
identity written with complex numbers, norm preservation, R = 0 reducing to a
brute-force RMSNorm loop, autograd and finite differences for the backward,
hand-computed RotaryEmbedding entries, and planted mistakes that these pins
must reject.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import qk_norm_rope as qo


def _inputs(B=2, T=5, H=3, Hkv=2, D=8, R=4, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g, dtype=dtype)
    k = torch.randn(B, T, Hkv, D, generator=g, dtype=dtype)
    freqs = torch.randn(T, R // 2, generator=g, dtype=dtype)
    cos = torch.cat((freqs.cos(), freqs.cos()), dim=-1)
    sin = torch.cat((freqs.sin(), freqs.sin()), dim=-1)
    return q, k, cos, sin, freqs


def test_reference_test_closed_form():
    """tests/test_kernels.py:265-299: q (2,5,3,8), k (2,5,2,8), 2 frequencies,
    cos/sin shaped (1, T, 1, 4), eps 1e-6, compared at atol 1e-6."""
    torch.manual_seed(0)
    q = torch.randn(2, 5, 3, 8)
    k = torch.randn(2, 5, 2, 8)
    freqs = torch.randn(5, 2)
    cos = torch.cat((freqs.cos(), freqs.cos()), dim=-1)[None, :, None, :]
    sin = torch.cat((freqs.sin(), freqs.sin()), dim=-1)[None, :, None, :]

    def ref(x):
        x_norm = x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + 1e-6)
        x1, x2, x_pass = x_norm[..., :2], x_norm[..., 2:4], x_norm[..., 4:]
        c = cos[..., :2]
        s = sin[..., :2]
        return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s, x_pass), dim=-1)

    q_out, k_out = qo.qk_norm_rope(q, k, cos, sin, 1e-6)
    assert torch.allclose(q_out, ref(q), atol=1e-6)
    assert torch.allclose(k_out, ref(k), atol=1e-6)


def _rms_brute(x: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty_like(x)
    for idx in np.ndindex(x.shape[:-1]):
        row = x[idx]
        ms = sum(float(v) * float(v) for v in row) / len(row)
        out[idx] = row / math.sqrt(ms + eps)
    return out


def test_rotation_is_complex_multiplication_and_keeps_norms():
    q, k, cos, sin, freqs = _inputs(D=16, R=8, seed=1)
    q_out, k_out = qo.qk_norm_rope(q, k, cos, sin, 1e-6)
    h = 4
    for x, out in ((q, q_out), (k, k_out)):
        z = torch.from_numpy(_rms_brute(x.numpy(), 1e-6))
        zc = torch.complex(z[..., :h], z[..., h:2 * h])
        rot = torch.polar(torch.ones_like(freqs), freqs)[None, :, None, :]  # e^{i theta}
        want = zc * rot
        assert torch.allclose(out[..., :h], want.real, atol=1e-12)
        assert torch.allclose(out[..., h:2 * h], want.imag, atol=1e-12)
        assert torch.allclose(out[..., 2 * h:], z[..., 2 * h:], atol=1e-12)
        assert torch.allclose(out.norm(dim=-1), z.norm(dim=-1), atol=1e-12)


def test_zero_rotary_width_is_plain_rmsnorm():
    q, k, _, _, _ = _inputs(D=8, R=4, seed=2)
    empty = torch.zeros(q.shape[1], 0, dtype=q.dtype)
    q_out, k_out = qo.qk_norm_rope(q, k, empty, empty, 1e-5)
    assert np.allclose(q_out.numpy(), _rms_brute(q.numpy(), 1e-5), atol=1e-12)
    assert np.allclose(k_out.numpy(), _rms_brute(k.numpy(), 1e-5), atol=1e-12)


def test_backward_matches_autograd_and_finite_differences():
    q, k, cos, sin, _ = _inputs(D=8, R=4, seed=3)
    q.requires_grad_(True)
    k.requires_grad_(True)
    g = torch.Generator().manual_seed(9)
    gq = torch.randn(q.shape, generator=g, dtype=q.dtype)
    gk = torch.randn(k.shape, generator=g, dtype=k.dtype)
    q_out, k_out = qo.qk_norm_rope(q, k, cos, sin, 1e-6)
    ((q_out * gq).sum() + (k_out * gk).sum()).backward()
    dq, dk = qo.qk_norm_rope_backward(q.detach(), k.detach(), gq, gk, cos, sin, 1e-6)
    assert torch.allclose(dq, q.grad, atol=1e-12)
    assert torch.allclose(dk, k.grad, atol=1e-12)
    # central differences on a few entries of q
    qd = q.detach()
    step = 1e-6
    for idx in ((0, 0, 0, 0), (1, 4, 2, 3), (0, 2, 1, 7)):
        e = torch.zeros_like(qd)
        e[idx] = step
        lp = (qo.qk_norm_rope(qd + e, k.detach(), cos, sin, 1e-6)[0] * gq).sum()
        lm = (qo.qk_norm_rope(qd - e, k.detach(), cos, sin, 1e-6)[0] * gq).sum()
        assert abs((lp - lm).item() / (2 * step) - dq[idx].item()) < 1e-6


def test_rotary_tables_match_hand_computed_entries():
    cos, sin = qo.rotary_tables(T=6, dim=64, theta=10000.0, fraction=0.25)
    assert cos.shape == (6, 16)
    # R = 16, frequencies theta^(-2j/16); entry (t, j) and its duplicate (t, j + 8)
    for t, j in ((0, 0), (3, 1), (5, 7)):
        ang = t * 10000.0 ** (-2 * j / 16)
        assert abs(cos[t, j].item() - math.cos(ang)) < 1e-6
        assert abs(sin[t, j + 8].item() - math.sin(ang)) < 1e-6
    c2, _ = qo.rotary_tables(T=2, dim=10, fraction=0.25)  # int(2.5) = 2 -> R = 2
    assert c2.shape == (2, 2)


# --- planted mistakes must be caught ------------------------------------------

def _mutant_rope(kind):
    def apply(x, cos, sin):
        R = cos.shape[-1]
        h = R // 2
        c, s = cos[..., :h], sin[..., :h]
        x1, x2, xp = x[..., :h], x[..., h:R], x[..., R:]
        if kind == "sign":
            return torch.cat((x1 * c + x2 * s, x2 * c - x1 * s, xp), dim=-1)
        if kind == "second_half_table":
            return torch.cat((x1 * cos[..., h:R] - x2 * sin[..., :h], x2 * cos[..., h:R] + x1 * sin[..., :h], xp), dim=-1)
        if kind == "adjacent_pairs":
            xe, xo = x[..., 0:R:2], x[..., 1:R:2]
            return torch.cat((xe * c - xo * s, xo * c + xe * s, xp), dim=-1)
        raise ValueError(kind)
    return apply


@pytest.mark.parametrize("kind", ["sign", "adjacent_pairs"])
def test_rope_mutants_are_caught(kind, monkeypatch):
    q, k, cos, sin, freqs = _inputs(D=16, R=8, seed=4)
    monkeypatch.setattr(qo, "apply_partial_rope", _mutant_rope(kind))
    q_out, _ = qo.qk_norm_rope(q, k, cos, sin, 1e-6)
    z = torch.from_numpy(_rms_brute(q.numpy(), 1e-6))
    want = torch.complex(z[..., :4], z[..., 4:8]) * torch.polar(torch.ones_like(freqs), freqs)[None, :, None, :]
    assert not torch.allclose(q_out[..., :4], want.real, atol=1e-6)


def test_norm_mutants_are_caught(monkeypatch):
    q, k, cos, sin, _ = _inputs(D=8, R=0 + 4, seed=5)
    empty = torch.zeros(q.shape[1], 0, dtype=q.dtype)
    brute = _rms_brute(q.numpy(), 1e-5)
    for bad in (lambda x, eps: x * torch.rsqrt(x.pow(2).sum(dim=-1, keepdim=True) + eps),
                lambda x, eps: x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True)) + eps):
        monkeypatch.setattr(qo, "rms_norm", bad)
        q_out, _ = qo.qk_norm_rope(q, k, empty, empty, 1e-5)
        assert not np.allclose(q_out.numpy(), brute, atol=1e-8)


def test_backward_mutant_is_caught(monkeypatch):
    """Rotating the gradient forward instead of back must fail the autograd pin."""
    q, k, cos, sin, _ = _inputs(D=8, R=4, seed=6)
    g = torch.Generator().manual_seed(1)
    gq = torch.randn(q.shape, generator=g, dtype=q.dtype)
    gk = torch.randn(k.shape, generator=g, dtype=k.dtype)
    qr = q.clone().requires_grad_(True)
    q_out, k_out = qo.qk_norm_rope(qr, k, cos, sin, 1e-6)
    ((q_out * gq).sum() + (k_out * gk).sum()).backward()
    real = qo.apply_partial_rope
    monkeypatch.setattr(qo, "apply_partial_rope", lambda x, c, s: real(x, c, s.abs()))
    dq, _ = qo.qk_norm_rope_backward(q, k, gq, gk, cos, sin, 1e-6)
    assert not torch.allclose(dq, qr.grad, atol=1e-6)
