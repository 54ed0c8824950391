"""AttentionCore with the hip backend, mirroring hackable-lm's model.py:129-250.

The reference picks `fwd_<attention_backend>` per call (model.py:169-174);
this class carries the same per-layer window (model.py:136), the same
window-or-None rule at call time (model.py:155-159) and the same
(B, T, H, D) in / (B, T, H, D) out layout as `fwd_flash_attn_2`
(model.py:216-226).  `fwd_hip` is the method the reference's AttentionCore
gains when the backend is registered there.

The reference routes CPU tensors to its own `torch` backend
(model.py:170); this library has no CPU path and raises instead.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import kernels
from .config import attention_window_size, layer_attention_window, normalize_attention_backend


@dataclass
class AttentionConfig:
    """The ModelConfig fields AttentionCore reads (config.py:213-232)."""

    n_layer: int
    n_head: int
    n_kv_head: int
    attention_window: int | None = 512
    attention_full_every: int | None = 4
    attention_backend: str = "hip"
    dropout: float = 0.0


class AttentionCore(nn.Module):
    def __init__(self, config: AttentionConfig, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.n_head = config.n_head
        self.n_kv_head = config.n_kv_head
        self.attention_window = layer_attention_window(
            layer_idx, config.n_layer, config.attention_window, config.attention_full_every
        )
        self.dropout = config.dropout

    def _attention_window_size(self, seq_len: int) -> int | None:
        return attention_window_size(self.attention_window, seq_len)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        backend = normalize_attention_backend(self.config.attention_backend)
        fwd_backend = getattr(self, f"fwd_{backend}", None)
        if fwd_backend is None:
            raise RuntimeError(f"{type(self).__name__} does not support backend {backend!r}")
        return fwd_backend(q, k, v)

    def fwd_hip(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return kernels.scaled_dot_product_attention(
            q,
            k,
            v,
            self.dropout if self.training else 0.0,
            is_causal=True,
            attn_mask=None,
            window_size=self._attention_window_size(q.shape[1]),
            backend="hip",
        )
