"""MI355X (gfx950) causal sliding-window attention backend for hackable-lm.

Public surface:
  attention(q, k, v, window_size=None)        differentiable (B,T,H,D) bf16 attention
  scaled_dot_product_attention(...)           the reference's dispatch signature, backend="hip"
  AttentionCore                               model.py's attention module with fwd_hip
  QKVProjection, RotaryEmbedding              model.py's projection + tables, fwd_hip producer
  ATTENTION_BACKENDS, layer_attention_window  config.py's names and layer pattern
  hip_attention_available, resolve_attention_backend
  qk_norm_rope_hip                            the fused q/k RMSNorm + partial RoPE producer
  fused_linear_cross_entropy_with_weight      the LM head's chunked linear + cross-entropy (backend="hip")
  LMHeadProjection                            model.py's LM head with fwd_hip
  residual_rms_norm_hip                       residual add + RMSNorm (OutputProjection / DownProjection)
  OutputProjection, DownProjection            model.py's projections with fwd_hip
The kernels live in libhlm_attn.so (built by hlm_attn.build), reached through
the C ABI in include/hlm_attn.h.
"""
from .config import (
    ATTENTION_BACKENDS,
    HIP_BACKEND,
    MODULE_BACKENDS,
    attention_window_size,
    layer_attention_window,
    normalize_attention_backend,
    normalize_attention_full_every,
    normalize_attention_window,
    normalize_module_backend,
)
from .kernels import (
    attention,
    fused_linear_cross_entropy_with_weight,
    hip_attention_available,
    qk_norm_rope_hip,
    residual_rms_norm_hip,
    resolve_attention_backend,
    scaled_dot_product_attention,
)
from .model import (
    AttentionConfig,
    AttentionCore,
    DownProjection,
    LMHeadProjection,
    OutputProjection,
    QKVProjection,
    RotaryEmbedding,
)

__all__ = [
    "ATTENTION_BACKENDS",
    "HIP_BACKEND",
    "MODULE_BACKENDS",
    "AttentionConfig",
    "AttentionCore",
    "attention",
    "fused_linear_cross_entropy_with_weight",
    "LMHeadProjection",
    "attention_window_size",
    "hip_attention_available",
    "layer_attention_window",
    "normalize_attention_backend",
    "normalize_attention_full_every",
    "normalize_attention_window",
    "normalize_module_backend",
    "QKVProjection",
    "RotaryEmbedding",
    "qk_norm_rope_hip",
    "residual_rms_norm_hip",
    "OutputProjection",
    "DownProjection",
    "resolve_attention_backend",
    "scaled_dot_product_attention",
]
