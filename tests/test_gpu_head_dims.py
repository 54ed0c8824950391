"""Head dims beyond the kernels' native (64, 64) / (128, 128) on the GPU: Dv !=
Dqk and other sizes up to 128 run zero-padded (GPU only).  Tolerances are the
attention parity tests': O within 1e-2 + 2e-2 |ref|, gradients within a
norm-relative 3e-2, against the fp32 evaluation of the same bf16 inputs."""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oracle

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def _close_o(got, ref):
    err = (got.float().cpu() - ref).abs()
    assert bool((err <= 1e-2 + 2e-2 * ref.abs()).all()), f"max err {err.max().item():.3e}"


def _close_grad(name, got, ref):
    rel = ((got.float().cpu() - ref).norm() / ref.norm()).item()
    assert rel <= 3e-2, f"{name}: norm-relative error {rel:.3e}"


def test_reference_dv_ne_dqk_closed_form():
    """tests/test_kernels.py:98-130: q, k (2, 3, 5, 7), v (2, 3, 5, 9), causal
    with a 3-key window, softmax(QK^T / sqrt(7)) V; gradients exist."""
    import hlm_attn

    dev = _dev()
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 3, 5, 7, generator=g).bfloat16().float()
    k = torch.randn(2, 3, 5, 7, generator=g).bfloat16().float()
    v = torch.randn(2, 3, 5, 9, generator=g).bfloat16().float()
    mask = torch.ones(5, 5, dtype=torch.bool).tril() & ((torch.arange(5)[:, None] - torch.arange(5)[None, :]) < 3)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    scores = torch.matmul(qr, kr.transpose(-2, -1)) / math.sqrt(7)
    ref = torch.matmul(torch.softmax(scores.masked_fill(~mask, float("-inf")), dim=-1), vr)
    do = torch.randn(ref.shape, generator=g).bfloat16().float()
    ref.backward(do)
    # the hip path takes (B, T, H, D)
    qd, kd, vd = (t.transpose(1, 2).to(dev).bfloat16().requires_grad_(True) for t in (q, k, v))
    out = hlm_attn.attention(qd, kd, vd, window_size=3)
    assert out.shape == (2, 5, 3, 9)
    out.backward(do.transpose(1, 2).to(dev).bfloat16())
    torch.cuda.synchronize()
    _close_o(out.detach().transpose(1, 2), ref.detach())
    for name, got, want in (("dq", qd.grad, qr.grad), ("dk", kd.grad, kr.grad), ("dv", vd.grad, vr.grad)):
        assert got is not None and got.shape == want.transpose(1, 2).shape
        _close_grad(name, got.transpose(1, 2), want)


@pytest.mark.parametrize("dqk,dv", [(64, 128), (128, 64), (32, 32), (96, 96), (80, 48), (7, 9)])
@pytest.mark.parametrize("window", [None, 40])
def test_padded_head_dims_match_oracle(dqk, dv, window):
    import hlm_attn

    dev = _dev()
    print(f"head dims ({dqk}, {dv}) window {window}", flush=True)
    B, T, H = 1, 150, 2
    g = torch.Generator().manual_seed(dqk * 1000 + dv)
    q = torch.randn(B, T, H, dqk, generator=g).bfloat16()
    k = torch.randn(B, T, H, dqk, generator=g).bfloat16()
    v = torch.randn(B, T, H, dv, generator=g).bfloat16()
    do = torch.randn(B, T, H, dv, generator=g).bfloat16()
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = hlm_attn.attention(qd, kd, vd, window_size=window)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    ro, _ = oracle.forward(q, k, v, window)
    _close_o(out.detach(), ro)
    rdq, rdk, rdv = oracle.backward(q, k, v, do, window)
    for name, got, ref in (("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv)):
        _close_grad(name, got, ref)
