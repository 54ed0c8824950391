"""The single-pass backward (hlm_attn_bwd_fused, selected by HLM_ATTN_BWD=fused)
against the two-kernel backward and the fp32 oracle (GPU only).

dK and dV must equal the two-kernel path's bit for bit (same loop arithmetic,
same workspace values); dQ, summed from bf16 partials of the 128-key tiles,
must meet the gradient tolerances against the oracle (3e-2 norm-relative and
elementwise, as in test_gpu_parity) and stay within 1e-2 norm-relative of
the two-kernel dQ.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oracle
from test_gpu_parity import assert_grad, make_inputs

pytestmark = pytest.mark.gpu

DQ_VS_TWO_KERNEL = 1e-2


def _device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def _both_backwards(q, k, v, do, window, dev, monkeypatch):
    """Forward once, then the two-kernel and the single-pass backward on the
    same device tensors; returns (two-kernel dq, dk, dv), (fused dq, dk, dv)."""
    from hlm_attn import ops

    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    w = 0 if window is None else window
    scale = 1.0 / math.sqrt(q.shape[-1])
    o, lse = ops.hip_attn_fwd(qd, kd, vd, w, scale)
    monkeypatch.delenv("HLM_ATTN_BWD", raising=False)
    two = ops.hip_attn_bwd(dod, qd, kd, vd, o, lse, w, scale)
    monkeypatch.setenv("HLM_ATTN_BWD", "fused")
    assert ops.fused_backward_selected()
    fused = ops.hip_attn_bwd(dod, qd, kd, vd, o, lse, w, scale)
    torch.cuda.synchronize()
    return two, fused


def _compare_paths(two, fused):
    assert torch.equal(two[1], fused[1]), "dk differs from the two-kernel backward"
    assert torch.equal(two[2], fused[2]), "dv differs from the two-kernel backward"
    a, b = two[0].float(), fused[0].float()
    rel = ((a - b).norm() / a.norm()).item() if a.norm() > 0 else (a - b).abs().max().item()
    print(f"  dq fused vs two-kernel: norm-rel {rel:.2e} (<= {DQ_VS_TWO_KERNEL}), max|d| "
          f"{(a - b).abs().max().item():.2e}", flush=True)
    assert rel <= DQ_VS_TWO_KERNEL


CASES = [
    # B, T, H, Hkv, D=64, window, seed
    (1, 1, 2, 2, None, 0),       # single token
    (2, 37, 3, 3, 5, 1),         # ragged T, tiny window
    (1, 128, 2, 2, 1, 2),        # W = 1: dQ = 0
    (2, 200, 2, 2, 64, 3),
    (2, 300, 4, 2, 77, 5),       # grouped-query heads: one workgroup covers two query heads
    (1, 333, 4, 1, 129, 7),      # MQA, ragged, W not tile aligned
    (2, 1024, 6, 6, 256, 8),     # BASELINE configs[0] shape
    (1, 700, 2, 2, None, 9),     # plain causal: up to 6 partials per row
    (1, 640, 2, 2, 513, 10),     # W = 4 * 128 + 1: the most partials per row for its window
]


@pytest.mark.parametrize("B,T,H,Hkv,window,seed", CASES)
def test_fused_backward_matches_oracle_and_two_kernel_path(B, T, H, Hkv, window, seed, monkeypatch):
    dev = _device()
    print(f"case fused B={B} T={T} H={H} Hkv={Hkv} D=64 W={window} seed={seed}", flush=True)
    q, k, v, do = make_inputs(B, T, H, Hkv, 64, seed)
    two, fused = _both_backwards(q, k, v, do, window, dev, monkeypatch)
    _compare_paths(two, fused)
    rdq, rdk, rdv = oracle.backward(q, k, v, do, window)
    assert_grad("dq", fused[0].float().cpu(), rdq)
    assert_grad("dk", fused[1].float().cpu(), rdk)
    assert_grad("dv", fused[2].float().cpu(), rdv)


@pytest.mark.parametrize("name,B,T,H,window", [("cfg2", 8, 2048, 12, 512), ("cfg3", 8, 2048, 12, None)])
def test_fused_backward_full_size(name, B, T, H, window, monkeypatch):
    """BASELINE's D = 64 configs: the two paths agree (dK, dV exactly), and
    the fused dQ of slice (b, h) = (0, 0) and (B - 1, H - 1) meets the
    oracle's tolerances."""
    dev = _device()
    print(f"case fused full size {name}", flush=True)
    q, k, v, do = make_inputs(B, T, H, H, 64, 42)
    two, fused = _both_backwards(q, k, v, do, window, dev, monkeypatch)
    _compare_paths(two, fused)
    for b, h in ((0, 0), (B - 1, H - 1)):
        sl = slice(h, h + 1)
        rdq, _, _ = oracle.backward(q[b:b + 1, :, sl], k[b:b + 1, :, sl], v[b:b + 1, :, sl], do[b:b + 1, :, sl], window)
        assert_grad(f"dq[{b},{h}]", fused[0][b:b + 1, :, sl].float().cpu(), rdq)


def test_fused_switch_keeps_two_kernel_path_at_head_dim_128(monkeypatch):
    """HLM_ATTN_BWD=fused only applies at D = 64: D = 128 runs the two-kernel
    backward, bit-identical to the default."""
    dev = _device()
    q, k, v, do = make_inputs(1, 300, 2, 2, 128, 11)
    two, fused = _both_backwards(q, k, v, do, 100, dev, monkeypatch)
    for a, b in zip(two, fused):
        assert torch.equal(a, b)


def test_fused_backward_through_autograd(monkeypatch):
    """hlm_attn.attention's autograd with the switch on: gradients vs the oracle."""
    import hlm_attn

    dev = _device()
    monkeypatch.setenv("HLM_ATTN_BWD", "fused")
    q, k, v, do = make_inputs(2, 400, 4, 2, 64, 12)
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = hlm_attn.attention(qd, kd, vd, window_size=150)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    rdq, rdk, rdv = oracle.backward(q, k, v, do, 150)
    assert_grad("dq", qd.grad.float().cpu(), rdq)
    assert_grad("dk", kd.grad.float().cpu(), rdk)
    assert_grad("dv", vd.grad.float().cpu(), rdv)


def test_fused_backward_with_strided_views_and_expanded_grad(monkeypatch):
    """Strides the model hands the backward: q, k, v as views of one fused
    projection (row stride 3 H D) and an expanded upstream gradient
    (o.sum().backward(): all strides 0); the switch changes dK/dV by nothing
    and dQ by the rounding of its partials."""
    import hlm_attn

    dev = _device()
    B, T, H, D = 2, 260, 4, 64
    g = torch.Generator().manual_seed(31)
    fused = torch.randn(B, T, 3 * H * D, generator=g).bfloat16().to(dev)
    grads = {}
    for mode in ("two", "fused"):
        if mode == "fused":
            monkeypatch.setenv("HLM_ATTN_BWD", "fused")
        else:
            monkeypatch.delenv("HLM_ATTN_BWD", raising=False)
        leaf = fused.clone().requires_grad_(True)
        q, k, v = (t.view(B, T, H, D) for t in leaf.split((H * D, H * D, H * D), dim=-1))
        assert not v.is_contiguous()
        hlm_attn.attention(q, k, v, window_size=70).float().sum().backward()
        torch.cuda.synchronize()
        grads[mode] = leaf.grad.view(B, T, 3, H, D)
    two, one = grads["two"], grads["fused"]
    assert torch.equal(two[:, :, 1:], one[:, :, 1:]), "dk/dv differ"
    a, b = two[:, :, 0].float(), one[:, :, 0].float()
    assert ((a - b).norm() / a.norm()).item() <= DQ_VS_TWO_KERNEL
    qf, kf, vf = (t.reshape(B, T, H, D).cpu() for t in fused.split((H * D, H * D, H * D), dim=-1))
    rdq, _, _ = oracle.backward(qf, kf, vf, torch.ones(B, T, H, D), 70)
    assert_grad("dq", b.cpu(), rdq)
