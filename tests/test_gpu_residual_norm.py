"""Parity of the HIP residual add + RMSNorm with oracle/residual_norm.py (GPU only).

  out        bit-exact: bf16(residual + branch), as the bf16 add rounds it
  normed     |hip - ref| <= 2^-7 |ref| + 1e-5, and >= 99% of entries equal
             to the fp32 value rounded to bf16 (one rounding of an fp32 result)
  grad_in    |hip - ref| <= 2^-7 |ref| + 1e-4 (fp32 math, one bf16 rounding)
"""
from __future__ import annotations

import pytest
import torch

from oracle import residual_norm as ro

pytestmark = pytest.mark.gpu

RTOL = 2.0 ** -7


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def _check(name, got, ref, atol, exact_frac=None):
    err = (got.float().cpu() - ref).abs()
    bound = atol + RTOL * ref.abs()
    assert bool((err <= bound).all()), f"{name}: max err {err.max().item():.3e}"
    if exact_frac is not None:
        frac = (got.cpu() == ref.bfloat16()).float().mean().item()
        assert frac >= exact_frac, f"{name}: {frac:.4f} exact"


@pytest.mark.parametrize("shape", [(1, 1, 8), (2, 37, 768), (3, 5, 1152), (1, 9, 4096), (2, 3, 8192), (4, 100, 520)],
                         ids=lambda s: "x".join(map(str, s)))
def test_forward_and_backward_match_oracle(shape):
    from hlm_attn import ops

    dev = _dev()
    print(f"residual_rms_norm {shape}", flush=True)
    g = torch.Generator().manual_seed(shape[-1] + shape[1])
    res = torch.randn(*shape, generator=g).bfloat16()
    br = (torch.randn(*shape, generator=g) * 0.3).bfloat16()
    g_out = torch.randn(*shape, generator=g).bfloat16()
    g_norm = torch.randn(*shape, generator=g).bfloat16()
    out, normed = ops.hip_residual_rms_norm(res.to(dev), br.to(dev), 1e-6)
    grad = ops.hip_residual_rms_norm_backward(out, g_out.to(dev), g_norm.to(dev), 1e-6)
    torch.cuda.synchronize()
    r_out, r_normed = ro.residual_rms_norm(res, br, 1e-6)
    assert torch.equal(out.cpu(), r_out)
    _check("normed", normed, r_normed, 1e-5, exact_frac=0.99)
    r_grad = ro.residual_rms_norm_backward(r_out, g_out, g_norm, 1e-6)
    _check("grad_in", grad, r_grad, 1e-4)


def test_autograd_through_output_projection():
    """OutputProjection.fwd_hip (model.py:253-264): both outputs used, the
    gradient reaches the residual and o_proj's weight."""
    from hlm_attn import AttentionConfig, OutputProjection

    dev = _dev()
    cfg = AttentionConfig(n_layer=1, n_head=4, n_kv_head=4, n_embd=256, head_dim=64)
    torch.manual_seed(0)
    mod = OutputProjection(cfg).to(dev)
    for p in mod.parameters():
        p.data = p.data.to(torch.bfloat16)
    g = torch.Generator().manual_seed(3)
    y = torch.randn(2, 33, 4, 64, generator=g).bfloat16().to(dev).requires_grad_(True)
    res = torch.randn(2, 33, 256, generator=g).bfloat16().to(dev).requires_grad_(True)
    g_out = torch.randn(2, 33, 256, generator=g).bfloat16().to(dev)
    g_norm = torch.randn(2, 33, 256, generator=g).bfloat16().to(dev)
    out, normed = mod(y, res)
    ((out.float() * g_out.float()).sum() + (normed.float() * g_norm.float()).sum()).backward()
    torch.cuda.synchronize()
    branch = mod.o_proj(y.detach().reshape(2, 33, 256)).detach()
    r_out, r_normed = ro.residual_rms_norm(res.detach().cpu(), branch.cpu(), cfg.norm_eps)
    assert torch.equal(out.detach().cpu(), r_out)
    _check("normed", normed.detach(), r_normed, 1e-5)
    r_grad = ro.residual_rms_norm_backward(r_out, g_out.cpu(), g_norm.cpu(), cfg.norm_eps)
    _check("grad residual", res.grad, r_grad, 1e-4)
    assert mod.o_proj.weight.grad is not None and torch.isfinite(mod.o_proj.weight.grad.float()).all()


def test_direct_path_equals_the_custom_op():
    import hlm_attn
    from hlm_attn import ops

    dev = _dev()
    res = torch.randn(8, 2048, 768, device=dev).bfloat16()
    br = torch.randn(8, 2048, 768, device=dev).bfloat16()
    with torch.no_grad():
        a = hlm_attn.residual_rms_norm_hip(res, br, 1e-6)
    b = ops.hip_residual_rms_norm(res, br, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
