"""Parity of the HIP q/k RMSNorm + partial RoPE producer with its oracle (GPU only).

The oracle (oracle/qk_norm_rope.py) evaluates the reference's CPU branch
(kernels.py:756-771 forward, :703-741 backward) in fp32 on the same
bf16-rounded inputs and bf16-rounded rotary tables the kernel reads.  The
kernel computes in fp32 and rounds each output once to bf16, so:
  forward / backward   |hip - ref| <= 2^-7 |ref| + 1e-5 (forward) or 1e-4 (backward)
                       elementwise, i.e. within two bf16 half-ulps of the fp32
                       value, and at least 99% of the entries equal the fp32
                       value rounded to bf16 exactly.
Rotary tables are bf16 (what RotaryEmbedding hands the producer, model.py:62-70)
or fp32, each read in its own type.  Cases cover q/k read in place as strided views of one fused (B, T, (H+2Hkv)D)
projection (model.py:92-99), contiguous q/k, MQA, rotary widths 0, 16, 32, 48,
64 and D, D = 64 and 128, ragged row counts and the benchmark shape.
"""
from __future__ import annotations

import pytest
import torch

from oracle import qk_norm_rope as qo

pytestmark = pytest.mark.gpu

FWD_ATOL, BWD_ATOL, RTOL = 1e-5, 1e-4, 2.0 ** -7
EPS = 1e-6


def _device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def make_inputs(B, T, H, Hkv, D, R, layout, seed):
    """q, k (bf16, as views of a fused projection or contiguous), bf16 rotary
    tables (1, T, 1, R) as model.py:117-126 passes them, and upstream grads."""
    g = torch.Generator().manual_seed(seed)
    if layout == "fused":
        qkv = torch.randn(B, T, (H + 2 * Hkv) * D, generator=g).bfloat16()
        q = qkv[..., : H * D].view(B, T, H, D)
        k = qkv[..., H * D : (H + Hkv) * D].view(B, T, Hkv, D)
    else:
        q = torch.randn(B, T, H, D, generator=g).bfloat16()
        k = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    cos, sin = qo.rotary_tables(T, D, fraction=R / D, dtype=torch.bfloat16)
    cos, sin = cos[None, :, None, :], sin[None, :, None, :]
    gq = torch.randn(B, T, H, D, generator=g).bfloat16()
    gk = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    return q, k, cos, sin, gq, gk


def to_dev(t, dev):
    """Copies a (possibly strided) CPU view to the device keeping its strides."""
    if t.is_contiguous():
        return t.to(dev)
    base = t._base if t._base is not None else t
    return torch.as_strided(base.to(dev), t.shape, t.stride(), t.storage_offset())


def check(name, got, ref, atol):
    err = (got.float() - ref).abs()
    bound = atol + RTOL * ref.abs()
    assert bool((err <= bound).all()), (
        f"{name}: max err {err.max().item():.3e}, worst excess {(err - bound).max().item():.3e}"
    )
    exact = (got == ref.bfloat16()).float().mean().item()
    assert exact >= 0.99, f"{name}: only {exact:.4f} of entries equal the rounded fp32 value"


CASES = [
    # B, T, H, Hkv, D, R, layout, seed
    (1, 1, 1, 1, 64, 16, "contig", 0),       # one row per tensor
    (2, 37, 3, 3, 64, 16, "fused", 1),       # the model's layout, ragged T
    (1, 129, 4, 1, 64, 0, "contig", 2),      # MQA, R = 0: plain RMSNorm
    (2, 65, 2, 2, 64, 64, "fused", 3),       # R = D
    (1, 33, 3, 3, 128, 32, "fused", 4),      # D = 128 at its default R
    (2, 17, 2, 1, 128, 128, "contig", 5),    # D = 128, R = D, MQA
    (1, 300, 2, 2, 128, 48, "fused", 6),     # R / 2 not a power of two
    (3, 100, 5, 5, 64, 32, "fused", 7),      # rows not a multiple of a block
]
FULL = (8, 2048, 12, 12, 64, 16, "fused", 0)  # the attention benchmark's shape


def _ids(c):
    return "B{}_T{}_H{}_Hkv{}_D{}_R{}_{}".format(*c[:7])


def _run_case(case, fp32_tables=False):
    from hlm_attn import ops

    dev = _device()
    B, T, H, Hkv, D, R, layout, seed = case
    print(f"qk_norm_rope case {_ids(case)} fp32_tables={fp32_tables}", flush=True)
    q, k, cos, sin, gq, gk = make_inputs(B, T, H, Hkv, D, R, layout, seed)
    if fp32_tables:  # full-precision fp32 tables, read as fp32 (HLM_TABLE_F32)
        cos, sin = qo.rotary_tables(T, D, fraction=R / D, dtype=torch.float32)
        cos, sin = cos[None, :, None, :], sin[None, :, None, :]
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    assert qd.stride() == q.stride()
    cd, sd = cos.to(dev), sin.to(dev)
    q_out, k_out = ops.hip_qk_norm_rope(qd, kd, cd, sd, EPS)
    dq, dk = ops.hip_qk_norm_rope_backward(qd, kd, gq.to(dev), gk.to(dev), cd, sd, EPS)
    torch.cuda.synchronize()
    assert q_out.is_contiguous() and k_out.is_contiguous() and q_out.dtype == torch.bfloat16
    rq, rk = qo.qk_norm_rope(q.float(), k.float(), cos.float(), sin.float(), EPS)
    check("q_out", q_out.cpu(), rq, FWD_ATOL)
    check("k_out", k_out.cpu(), rk, FWD_ATOL)
    rdq, rdk = qo.qk_norm_rope_backward(q.float(), k.float(), gq.float(), gk.float(), cos.float(), sin.float(), EPS)
    check("grad_q", dq.cpu(), rdq, BWD_ATOL)
    check("grad_k", dk.cpu(), rdk, BWD_ATOL)


@pytest.mark.parametrize("case", CASES + [FULL], ids=_ids)
def test_forward_and_backward_match_oracle(case):
    """bf16 rotary tables, as the model passes them."""
    _run_case(case)


@pytest.mark.parametrize("case", [CASES[1], CASES[4], CASES[6]], ids=_ids)
def test_fp32_tables_match_oracle(case):
    _run_case(case, fp32_tables=True)


def test_full_size_properties():
    """At the benchmark shape: each output row of the forward has the norm of
    the normalised row (the rotation is orthogonal), sqrt(D) up to eps and bf16
    rounding, and two calls agree bit for bit."""
    from hlm_attn import qk_norm_rope_hip

    dev = _device()
    B, T, H, Hkv, D, R, layout, seed = FULL
    q, k, cos, sin, _, _ = make_inputs(B, T, H, Hkv, D, R, layout, seed)
    qd, kd, cd, sd = to_dev(q, dev), to_dev(k, dev), cos.to(dev), sin.to(dev)
    a = qk_norm_rope_hip(qd, kd, cd, sd, EPS)
    b = qk_norm_rope_hip(qd, kd, cd, sd, EPS)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    for x, out in ((qd, a[0]), (kd, a[1])):
        n = out.float().norm(dim=-1)
        want = x.float().norm(dim=-1) * torch.rsqrt(x.float().pow(2).mean(dim=-1) + EPS)
        assert ((n - want).abs() <= 4e-3 * want + 1e-4).all()


def test_autograd_through_fused_projection_views():
    """Gradients flow back into the fused projection tensor through the
    strided q / k views; an unused k output contributes a zero gradient
    (the reference's None-gradient rule, kernels.py:716-719)."""
    from hlm_attn import qk_norm_rope_hip

    dev = _device()
    B, T, H, Hkv, D, R = 2, 50, 3, 1, 64, 16
    g = torch.Generator().manual_seed(11)
    qkv_cpu = torch.randn(B, T, (H + 2 * Hkv) * D, generator=g).bfloat16()
    gq = torch.randn(B, T, H, D, generator=g).bfloat16()
    cos, sin = qo.rotary_tables(T, D, fraction=R / D, dtype=torch.bfloat16)
    qkv = qkv_cpu.to(dev).requires_grad_(True)
    q = qkv[..., : H * D].view(B, T, H, D)
    k = qkv[..., H * D : (H + Hkv) * D].view(B, T, Hkv, D)
    q_out, _ = qk_norm_rope_hip(q, k, cos.to(dev)[None, :, None], sin.to(dev)[None, :, None], EPS)
    (q_out.float() * gq.to(dev).float()).sum().backward()
    grad = qkv.grad.cpu()
    rq = qkv_cpu[..., : H * D].view(B, T, H, D).float()
    rk = qkv_cpu[..., H * D : (H + Hkv) * D].view(B, T, Hkv, D).float()
    rdq, _ = qo.qk_norm_rope_backward(rq, rk, gq.float(), torch.zeros_like(rk), cos.float(), sin.float(), EPS)
    check("grad_q via view", grad[..., : H * D].view(B, T, H, D), rdq, BWD_ATOL)
    assert torch.count_nonzero(grad[..., H * D :]) == 0


def test_projection_module_fwd_hip():
    """QKVProjection (model.py:76-126) with qkv_backend='hip' equals the
    reference's fwd_torch math on the module's own projection output."""
    from hlm_attn import AttentionConfig, QKVProjection

    dev = _device()
    cfg = AttentionConfig(n_layer=1, n_head=4, n_kv_head=4, n_embd=256, head_dim=64)
    torch.manual_seed(0)
    mod = QKVProjection(cfg, 0).to(dev)
    # the reference's bf16 policy casts parameters only (kernels.py:960-966);
    # the rotary inverse frequencies stay fp32
    for p in mod.parameters():
        p.data = p.data.to(torch.bfloat16)
    x = torch.randn(2, 40, 256, generator=torch.Generator().manual_seed(1)).bfloat16().to(dev)
    with torch.no_grad():
        q, k, v = mod(x)
        proj = mod.qkv_proj(x).cpu()
        # the module's own tables, computed on the device as model.py:62-69 does
        # (their fp32 cos / sin may differ from a CPU evaluation in the last bit,
        # which can move a bf16 rounding)
        cos, sin = (t.cpu() for t in mod.rope(40, dev, torch.bfloat16))
    torch.cuda.synchronize()
    assert cos.shape == (1, 1, 40, 16) and cos.dtype == torch.bfloat16
    ref_cos, _ = qo.rotary_tables(40, 64)
    assert (cos[0, 0].float() - ref_cos).abs().max() <= 2.0 ** -8
    pq = proj[..., :256].view(2, 40, 4, 64).float()
    pk = proj[..., 256:512].view(2, 40, 4, 64).float()
    rq, rk = qo.qk_norm_rope(pq, pk, cos.float(), sin.float(), cfg.norm_eps)
    check("module q", q.cpu(), rq, FWD_ATOL)
    check("module k", k.cpu(), rk, FWD_ATOL)
    assert torch.equal(v.cpu(), proj[..., 512:].view(2, 40, 4, 64))


@pytest.mark.parametrize("D,R,msg", [(64, 8, "rotary_dim"), (32, 16, "head_dim")])
def test_unsupported_shapes_raise(D, R, msg):
    from hlm_attn import ops

    dev = _device()
    q = torch.zeros(1, 4, 2, D, dtype=torch.bfloat16, device=dev)
    cos = torch.zeros(4, R, device=dev)
    with pytest.raises(RuntimeError, match=msg):
        ops.hip_qk_norm_rope(q, q, cos, cos, EPS)
