"""AttentionCore, QKVProjection, OutputProjection, DownProjection and
LMHeadProjection with the hip backend, mirroring hackable-lm's
model.py:129-250, :50-126, :253-264, :295-304 and :317-352.

The reference picks `fwd_<attention_backend>` per call (model.py:169-174);
this class carries the same per-layer window (model.py:136), the same
window-or-None rule at call time (model.py:155-159) and the same
(B, T, H, D) in / (B, T, H, D) out layout as `fwd_flash_attn_2`
(model.py:216-226).  `fwd_hip` is the method the reference's AttentionCore
gains when the backend is registered there, next to `fwd_flash_attn_2`.

QKVProjection mirrors model.py:76-126: the fused q/k/v projection, then the
q/k RMSNorm + partial RoPE producer; `fwd_hip` is `fwd_triton` with the HIP
producer in place of the Triton one, fed the same views and rotary tables.

AttentionCore routes CPU tensors to `fwd_torch`, the reference's dense math
(model.py:170, :176-196 with kernels.py:785-800), as the reference does;
attention_backend="torch" selects it on any device.  The hip backend never
falls back to it: a ROCm tensor without libhlm_attn.so raises.  The other
modules have no CPU path and raise on CPU tensors.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import kernels
from .config import (
    attention_window_size,
    layer_attention_window,
    normalize_attention_backend,
    normalize_module_backend,
)


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
    # QKVProjection's fields (config.py:213-232)
    n_embd: int = 0
    head_dim: int = 64
    rope_theta: float = 1_000_000.0
    rope_fraction: float = 0.25
    norm_eps: float = 1e-6
    qkv_backend: str = "hip"
    # LMHeadProjection's fields (config.py:213-232)
    vocab_size: int = 0
    loss_chunk_size: int | None = 4096
    lm_head_backend: str = "hip"
    # OutputProjection / DownProjection fields (config.py:213-232)
    mlp_hidden: int = 0
    output_backend: str = "hip"
    down_backend: str = "hip"


class RotaryEmbedding(nn.Module):
    """model.py:50-70: cos / sin tables (1, 1, T, R) over R = int(dim * fraction)
    rounded down to even, both halves repeating the R / 2 frequencies
    theta^(-2j/R); cached for the longest sequence seen, returned in `dtype`."""

    def __init__(self, dim: int, theta: float = 1_000_000.0, fraction: float = 0.25) -> None:
        super().__init__()
        rotary_dim = int(dim * fraction)
        self.rotary_dim = rotary_dim - rotary_dim % 2
        exponents = torch.arange(0, self.rotary_dim, 2).float() / self.rotary_dim
        self.register_buffer("inv_freq", 1.0 / (theta ** exponents), persistent=False)
        self._cached_len = 0
        self._cos: torch.Tensor | None = None
        self._sin: torch.Tensor | None = None

    def forward(self, seq_len: int, device: torch.device, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        if self._cos is None or seq_len > self._cached_len or self._cos.device != device:
            positions = torch.arange(seq_len, device=device, dtype=torch.float32)
            angles = torch.outer(positions, self.inv_freq.to(device))
            angles = torch.cat((angles, angles), dim=-1)
            self._cos, self._sin = angles.cos()[None, None], angles.sin()[None, None]
            self._cached_len = seq_len
        return self._cos[:, :, :seq_len].to(dtype=dtype), self._sin[:, :, :seq_len].to(dtype=dtype)


class QKVProjection(nn.Module):
    """model.py:76-126 with the hip producer.  The projection's q and k are
    views of one (B, T, (H + 2 Hkv) D) tensor; the producer reads them in
    place through their strides and writes contiguous normalised, rotated
    q and k; v stays the view."""

    def __init__(self, config: AttentionConfig, layer_idx: int) -> None:
        super().__init__()
        del layer_idx
        self.config = config
        self.n_head = config.n_head
        self.n_kv_head = config.n_kv_head
        self.head_dim = config.head_dim
        self.q_dim = config.n_head * config.head_dim
        self.kv_dim = config.n_kv_head * config.head_dim
        self.qkv_proj = nn.Linear(config.n_embd, self.q_dim + 2 * self.kv_dim, bias=False)
        self.rope = RotaryEmbedding(config.head_dim, config.rope_theta, config.rope_fraction)

    def _project(self, x: torch.Tensor):
        bsz, seq_len, _ = x.shape
        q, k, v = self.qkv_proj(x).split((self.q_dim, self.kv_dim, self.kv_dim), dim=-1)
        q = q.view(bsz, seq_len, self.n_head, self.head_dim)
        k = k.view(bsz, seq_len, self.n_kv_head, self.head_dim)
        v = v.view(bsz, seq_len, self.n_kv_head, self.head_dim)
        cos, sin = self.rope(seq_len, x.device, q.dtype)
        return q, k, v, cos, sin

    def forward(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        backend = normalize_module_backend("qkv_backend", self.config.qkv_backend)
        fwd_backend = getattr(self, f"fwd_{backend}", None)
        if fwd_backend is None:
            raise RuntimeError(f"{type(self).__name__} does not support backend {backend!r}")
        return fwd_backend(x)

    def fwd_hip(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        q, k, v, cos, sin = self._project(x)
        q, k = kernels.qk_norm_rope_hip(q, k, cos.transpose(1, 2), sin.transpose(1, 2), self.config.norm_eps)
        return q, k, v


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
        self._mask_cache: torch.Tensor | None = None

    def _attention_window_size(self, seq_len: int) -> int | None:
        return attention_window_size(self.attention_window, seq_len)

    def _sliding_window_mask(self, seq_len: int, device: torch.device) -> torch.Tensor | None:
        """model.py:141-151: bool (1, 1, T, T), True where 0 <= i - j < window,
        None when the layer has no window or it covers the sequence; kept for
        the last (T, device)."""
        if self._attention_window_size(seq_len) is None:
            return None
        cached = self._mask_cache
        if cached is None or cached.shape[-1] != seq_len or cached.device != device:
            pos = torch.arange(seq_len, device=device)
            lag = pos[:, None] - pos[None, :]
            cached = ((lag >= 0) & (lag < self.attention_window))[None, None]
            self._mask_cache = cached
        return cached

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        backend = normalize_attention_backend(self.config.attention_backend)
        if q.device.type == "cpu":  # model.py:170
            backend = "torch"
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

    def fwd_torch(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """model.py:176-196: heads first, k/v heads repeated for GQA, the window
        as an explicit mask (plain causal without one), the reference's dense
        math, (B, T, H, D) back."""
        seq_len = q.shape[1]
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if self.n_kv_head != self.n_head:
            group = self.n_head // self.n_kv_head
            k = k.repeat_interleave(group, dim=1)
            v = v.repeat_interleave(group, dim=1)
        mask = self._sliding_window_mask(seq_len, q.device)
        y = kernels.scaled_dot_product_attention(
            q,
            k,
            v,
            self.dropout if self.training else 0.0,
            is_causal=mask is None,
            attn_mask=mask,
            window_size=self._attention_window_size(seq_len),
            backend="torch",
        )
        return y.transpose(1, 2)


class LMHeadProjection(nn.Module):
    """model.py:317-352 with the hip fused linear + cross-entropy: without
    targets the logits; with targets (None, mean loss) through
    kernels.fused_linear_cross_entropy_with_weight(backend="hip")."""

    def __init__(self, config: AttentionConfig) -> None:
        super().__init__()
        self.config = config
        self.lm_head = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self.chunk_size = config.loss_chunk_size

    def forward(self, hidden: torch.Tensor, targets: torch.Tensor | None = None):
        backend = normalize_module_backend("lm_head_backend", self.config.lm_head_backend)
        fwd_backend = getattr(self, f"fwd_{backend}", None)
        if fwd_backend is None:
            raise RuntimeError(f"{type(self).__name__} does not support backend {backend!r}")
        return fwd_backend(hidden, targets)

    def fwd_hip(self, hidden: torch.Tensor, targets: torch.Tensor | None = None):
        if targets is None:
            return self.lm_head(hidden), None
        loss = kernels.fused_linear_cross_entropy_with_weight(
            hidden, self.lm_head.weight, self.lm_head.bias, targets, backend="hip", chunk_size=self.chunk_size
        )
        return None, loss


class _ResidualNormProjection(nn.Module):
    """A projection followed by residual_rms_norm, dispatched on a module
    backend field like the reference's AcceleratedModule (model.py:19-38)."""

    backend_field = ""

    def forward(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        backend = normalize_module_backend(self.backend_field, getattr(self.config, self.backend_field))
        fwd_backend = getattr(self, f"fwd_{backend}", None)
        if fwd_backend is None:
            raise RuntimeError(f"{type(self).__name__} does not support backend {backend!r}")
        return fwd_backend(x, residual)


class OutputProjection(_ResidualNormProjection):
    """model.py:253-264 with the hip residual add + RMSNorm."""

    backend_field = "output_backend"

    def __init__(self, config: AttentionConfig) -> None:
        super().__init__()
        self.config = config
        self.norm_eps = config.norm_eps
        self.o_proj = nn.Linear(config.n_head * config.head_dim, config.n_embd, bias=False)

    def fwd_hip(self, y: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        bsz, seq_len, n_head, head_dim = y.shape
        y = y.reshape(bsz, seq_len, n_head * head_dim)
        return kernels.residual_rms_norm_hip(residual, self.o_proj(y), self.norm_eps)


class DownProjection(_ResidualNormProjection):
    """model.py:295-304 with the hip residual add + RMSNorm."""

    backend_field = "down_backend"

    def __init__(self, config: AttentionConfig) -> None:
        super().__init__()
        self.config = config
        self.norm_eps = config.norm_eps
        self.down_proj = nn.Linear(config.mlp_hidden, config.n_embd, bias=False)

    def fwd_hip(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return kernels.residual_rms_norm_hip(residual, self.down_proj(x), self.norm_eps)
