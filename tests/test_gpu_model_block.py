"""A transformer block's attention half built from the hip modules (GPU only):
QKVProjection (hip q/k producer) -> AttentionCore (hip attention) ->
OutputProjection (hip residual add + RMSNorm), then the LM head's hip fused
linear + cross-entropy: eager against the fp32 CPU evaluation of the
reference's torch formulas (loss within 2e-2 relative, gradients
norm-relative 5e-2: bf16 weights and activations through five ops), and
torch.compile(fullgraph=True) (kernels.py:126-137) against eager.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as attn_oracle
from oracle import qk_norm_rope as qk_oracle
from oracle import residual_norm as res_oracle

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


class Block(torch.nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        from hlm_attn import AttentionCore, LMHeadProjection, OutputProjection, QKVProjection

        self.qkv = QKVProjection(cfg, layer_idx)
        self.attention = AttentionCore(cfg, layer_idx)
        self.out = OutputProjection(cfg)
        self.head = LMHeadProjection(cfg)

    def forward(self, x_norm, residual, targets):
        q, k, v = self.qkv(x_norm)
        y = self.attention(q, k, v)
        x, x_norm = self.out(y, residual)
        _, loss = self.head(x_norm, targets)
        return loss


def _make(dev):
    from hlm_attn import AttentionConfig

    cfg = AttentionConfig(n_layer=2, n_head=4, n_kv_head=4, n_embd=256, head_dim=64, vocab_size=512,
                          attention_window=64, loss_chunk_size=None)
    torch.manual_seed(0)
    block = Block(cfg, 0).to(dev)
    for p in block.parameters():  # the reference's bf16 policy: parameters only (kernels.py:960-966)
        p.data = p.data.to(torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 96, 256, generator=g).bfloat16()
    res = torch.randn(2, 96, 256, generator=g).bfloat16()
    targets = torch.randint(0, 512, (2, 96), generator=g)
    return cfg, block, x, res, targets


def _reference_loss(cfg, block, x, res, targets):
    """The reference's torch formulas in fp32 on the CPU, same bf16 weights."""
    w_qkv = block.qkv.qkv_proj.weight.detach().float().cpu().requires_grad_(True)
    w_o = block.out.o_proj.weight.detach().float().cpu()
    w_head = block.head.lm_head.weight.detach().float().cpu()
    xf, rf = x.float(), res.float()
    qkv = xf @ w_qkv.t()
    q, k, v = qkv.split((256, 256, 256), dim=-1)
    q, k, v = (t.reshape(2, 96, 4, 64) for t in (q, k, v))
    cos, sin = qk_oracle.rotary_tables(96, 64, dtype=torch.bfloat16)
    q, k = qk_oracle.qk_norm_rope(q, k, cos.float(), sin.float(), cfg.norm_eps)
    y = attn_oracle.attention_core_torch(q, k, v, 64)
    out, normed = res_oracle.residual_rms_norm(rf, y.reshape(2, 96, 256) @ w_o.t(), cfg.norm_eps)
    loss = F.cross_entropy((normed @ w_head.t()).reshape(-1, 512), targets.reshape(-1))
    loss.backward()
    return loss.detach(), w_qkv.grad


def test_block_matches_reference_formulas_and_compiles():
    dev = _dev()
    cfg, block, x, res, targets = _make(dev)
    ref_loss, ref_gw = _reference_loss(cfg, block, x, res, targets)

    results = []
    for fn in (block, torch.compile(block, fullgraph=True, dynamic=False)):
        block.zero_grad(set_to_none=True)
        xd = x.to(dev).requires_grad_(True)
        loss = fn(xd, res.to(dev), targets.to(dev))
        loss.backward()
        torch.cuda.synchronize()
        results.append((loss.detach().float().cpu(), block.qkv.qkv_proj.weight.grad.float().cpu().clone(),
                        xd.grad.float().cpu().clone()))
    (l_e, gw_e, gx_e), (l_c, gw_c, gx_c) = results
    assert abs(l_e.item() - ref_loss.item()) <= 2e-2 * ref_loss.item(), (l_e.item(), ref_loss.item())
    rel = ((gw_e - ref_gw).norm() / ref_gw.norm()).item()
    assert rel <= 5e-2, f"qkv weight gradient: norm-relative {rel:.3e}"
    # compiled against eager: the same kernels, torch's own ops may fuse differently
    assert abs(l_c.item() - l_e.item()) <= 1e-2 * abs(l_e.item())
    assert ((gw_c - gw_e).norm() / gw_e.norm()).item() <= 2e-2
    assert ((gx_c - gx_e).norm() / gx_e.norm()).item() <= 2e-2
