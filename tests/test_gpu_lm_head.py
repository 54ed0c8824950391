"""Parity of the LM head's HIP cross-entropy rows and the fused linear +
cross-entropy built on them, against oracle/linear_ce.py (GPU only).

Tolerances (the kernel computes in fp32 from bf16 or fp32 logits and
rounds each gradient once to the logits' type):
  per-row loss * n_tokens   |hip - ref| <= 1e-4 + 1e-5 |ref|
  gradient * n_tokens       bf16: |hip - ref| <= 2^-8 |ref| + 1e-6
                            fp32: |hip - ref| <= 1e-5 |ref| + 1e-7
  fused linear CE (fp32 hidden/weights, fp32 GEMMs): loss within 1e-5
  relative, gradients within 1e-4 of their max entry; (bf16) loss within
  1e-2 relative, gradients norm-relative 3e-2.
"""
from __future__ import annotations

import pytest
import torch

from oracle import linear_ce as co

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


CASES = [
    # rows, V, dtype, note
    (5, 33, torch.bfloat16),      # V not a multiple of 8: the generic path
    (7, 1000, torch.bfloat16),    # one 16-byte chunk per thread
    (3, 2048, torch.float32),
    (64, 32768, torch.bfloat16),  # the reference Triton kernel's largest block
    (4, 50257, torch.bfloat16),   # odd V (GPT-2 sized): generic path
    (4, 65536, torch.bfloat16),   # the largest register-resident row
    (4, 70000, torch.bfloat16),   # beyond it: generic path
    (6, 32768, torch.float32),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"rows{c[0]}_V{c[1]}_{str(c[2]).split('.')[-1]}")
def test_ce_rows_match_oracle(case):
    from hlm_attn import ops

    dev = _dev()
    rows, V, dtype = case
    print(f"ce rows {case}", flush=True)
    g = torch.Generator().manual_seed(V)
    logits = (torch.randn(rows, V, generator=g) * 3).to(dtype)
    targets = torch.randint(0, V, (rows,), generator=g)
    targets[0] = 0
    targets[-1] = V - 1
    if rows > 2:
        targets[1] = -100  # ignored
    n_tokens = 3 * rows + 1
    ref_loss, ref_grad = co.ce_rows(logits, targets, n_tokens)
    ld = logits.to(dev)
    loss = ops.hip_linear_ce(ld, targets.to(dev), n_tokens)
    torch.cuda.synchronize()
    err = (loss.cpu().double() - ref_loss).abs() * n_tokens
    assert bool((err <= 1e-4 + 1e-5 * (ref_loss.abs() * n_tokens)).all()), f"loss err {err.max().item():.3e}"
    got = ld.cpu().double() * n_tokens
    want = ref_grad * n_tokens
    rtol, atol = (2.0 ** -8, 1e-6) if dtype == torch.bfloat16 else (1e-5, 1e-7)
    gerr = (got - want).abs()
    assert bool((gerr <= rtol * want.abs() + atol).all()), f"grad err {gerr.max().item():.3e}"
    if rows > 2:
        assert loss[1].item() == 0.0 and torch.count_nonzero(ld[1]) == 0


def test_out_of_range_target_gives_nan_row():
    from hlm_attn import ops

    dev = _dev()
    logits = torch.randn(3, 64, device=dev).bfloat16()
    loss = ops.hip_linear_ce(logits, torch.tensor([1, 64, -5], device=dev), 3)
    torch.cuda.synchronize()
    assert torch.isfinite(loss[0]) and torch.isnan(loss[1]) and torch.isnan(loss[2])
    assert torch.isfinite(logits[0].float()).all() and torch.isnan(logits[1].float()).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("chunk", [None, 2048])
def test_fused_linear_cross_entropy_matches_oracle(dtype, chunk):
    import hlm_attn

    dev = _dev()
    n_tokens, hidden_size, vocab = 5000, 128, 1000  # 5000 = 2048 + 2048 + 904 with chunk 2048
    g = torch.Generator().manual_seed(7)
    hidden = torch.randn(n_tokens, hidden_size, generator=g).to(dtype)
    weight = (torch.randn(vocab, hidden_size, generator=g) * 0.05).to(dtype)
    targets = torch.randint(0, vocab, (n_tokens,), generator=g)
    h = hidden.to(dev).requires_grad_(True)
    w = weight.to(dev).requires_grad_(True)
    loss = hlm_attn.fused_linear_cross_entropy_with_weight(h, w, None, targets.to(dev), backend="hip", chunk_size=chunk)
    (loss * 2.0).backward()  # the backward scales the saved gradients by the incoming one
    torch.cuda.synchronize()
    ref_loss, ref_gh, ref_gw, _ = co.fused_linear_cross_entropy(hidden, weight, None, targets, chunk or n_tokens)
    rel = abs(loss.item() - ref_loss.item()) / ref_loss.item()
    if dtype == torch.float32:
        assert rel <= 1e-5
        for name, got, ref in (("hidden", h.grad, ref_gh), ("weight", w.grad, ref_gw)):
            err = (got.double().cpu() / 2 - ref).abs().max().item()
            assert err <= 1e-4 * ref.abs().max().item(), name
    else:
        assert rel <= 1e-2
        for name, got, ref in (("hidden", h.grad, ref_gh), ("weight", w.grad, ref_gw)):
            diff = got.double().cpu() / 2 - ref
            assert (diff.norm() / ref.norm()).item() <= 3e-2, name


def test_lm_head_projection_matches_dense_cross_entropy():
    """LMHeadProjection.fwd_hip against the reference test's dense closed form
    (tests/test_kernels.py:11-26), fp32 parameters as that test uses."""
    import torch.nn.functional as F

    from hlm_attn import AttentionConfig, LMHeadProjection

    dev = _dev()
    cfg = AttentionConfig(n_layer=1, n_head=1, n_kv_head=1, n_embd=64, vocab_size=33)
    torch.manual_seed(0)
    head = LMHeadProjection(cfg).to(dev)
    hidden = torch.randn(3, 7, 64, device=dev)
    targets = torch.randint(0, 33, (3, 7), device=dev)
    dense = F.cross_entropy(F.linear(hidden, head.lm_head.weight).float().reshape(-1, 33), targets.reshape(-1))
    logits, loss = head(hidden, targets)
    assert logits is None
    assert torch.allclose(loss, dense, atol=1e-5)
    out, none = head(hidden)
    assert none is None and out.shape == (3, 7, 33)
