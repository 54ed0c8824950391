"""The hip branch of hackable-lm's attention dispatch.

`scaled_dot_product_attention` keeps the signature of
/root/reference/kernels.py:774-784 and behaves like its FlashAttention branch
(kernels.py:816-841): an explicit mask is rejected, q/k/v are cast to bf16,
the window becomes the kernels' causal look-back, the scale is 1/sqrt(D) and
the result is bf16 in (B, T, H, D).  Like the FlashAttention-3/4 branches
(kernels.py:842-843) it rejects dropout.

`hip_attention_available` and `resolve_attention_backend` mirror the probe and
fallback rules of resolve_kernel_backends (kernels.py:146-242) for the
attention field.

`qk_norm_rope_hip` is the producer step before attention, with the signature
and semantics of the reference's `qk_norm_rope_triton` (kernels.py:756-771):
RMSNorm of each q and k row, then the partial rotary embedding.
"""
from __future__ import annotations

import math
from typing import Any

import torch

from . import _lib
from .config import HIP_BACKEND, normalize_attention_backend


def hip_attention_available() -> bool:
    """True when a ROCm device is visible and libhlm_attn.so loads."""
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    try:
        _lib.load()
    except (_lib.HipAttentionUnavailable, OSError):
        return False
    return True


def resolve_attention_backend(attention_backend: str, allow_torch_backend: bool = False) -> str:
    """Resolves a requested attention backend the way the reference resolves
    flash_attn_2 (kernels.py:177-181, :221-228): raise when the hip library is
    unusable, unless the caller allows the reference's torch backend."""
    backend = normalize_attention_backend(attention_backend)
    if backend != HIP_BACKEND:
        return backend
    if hip_attention_available():
        return HIP_BACKEND
    if allow_torch_backend:
        return "torch"
    raise RuntimeError(
        "attention_backend=hip needs a ROCm GPU and libhlm_attn.so; "
        "build it with `python -m hlm_attn.build`."
    )


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    window_size: int | None = None,
    scale: float | None = None,
) -> torch.Tensor:
    """Causal (sliding-window) attention on (B, T, H, D) tensors through the HIP
    kernels.  window_size=None is plain causal; window_size=W lets query i see
    keys i-W+1..i.  Differentiable in q, k and v."""
    from . import ops  # registers the custom ops on first use

    if q.dtype != torch.bfloat16:
        q = q.to(torch.bfloat16)
    if k.dtype != torch.bfloat16:
        k = k.to(torch.bfloat16)
    if v.dtype != torch.bfloat16:
        v = v.to(torch.bfloat16)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if window_size is not None and window_size < 1:
        raise RuntimeError(f"window_size must be >= 1 or None, got {window_size}")
    window = 0 if window_size is None else int(window_size)
    if ops.direct_call_ok(q, k, v):  # inference: same kernels, without the dispatcher's host cost
        out, _ = ops.attn_fwd_impl(q, k, v, window, float(scale))
        return out
    out, _ = ops.hip_attn_fwd(q, k, v, window, float(scale))
    return out


def scaled_dot_product_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dropout_p: float,
    is_causal: bool = True,
    attn_mask: torch.Tensor | None = None,
    block_mask: Any | None = None,
    window_size: int | None = None,
    backend: str = HIP_BACKEND,
) -> torch.Tensor:
    """Dispatch entry with the reference's signature; implements backend="hip"."""
    if backend != HIP_BACKEND:
        raise RuntimeError(
            f"unsupported attention backend {backend!r}: this library implements only {HIP_BACKEND!r}; "
            "the other backends stay in the host model's kernels.py"
        )
    if attn_mask is not None or block_mask is not None:
        raise RuntimeError(f"{backend} path expects window_size instead of an explicit attention mask")
    if dropout_p:
        raise RuntimeError(f"{backend} backend does not support dropout")
    if not is_causal:
        raise RuntimeError(f"{backend} backend implements causal attention only")
    return attention(q, k, v, window_size=window_size)


def qk_norm_rope_hip(
    q: torch.Tensor,
    k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused q/k RMSNorm + partial RoPE on the GPU (kernels.py:756-771).

    q (B, T, H, D) and k (B, T, Hkv, D) as QKVProjection._project makes them
    (model.py:92-99: views of the fused projection, bf16); cos / sin as
    QKVProjection.fwd_triton passes them (model.py:117-126: the rotary tables
    transposed to (1, T, 1, R)), or (T, R).  Returns contiguous bf16 q and k.
    Differentiable.  There is no CPU path: a CPU tensor raises (the reference
    routes CPU runs to its torch math instead)."""
    from . import ops

    if q.device.type != "cuda":
        raise RuntimeError("qk_norm_rope_hip runs on ROCm devices only; use the torch path on the CPU")
    if ops.direct_call_ok(q, k, cos, sin):  # inference: same kernel, without the dispatcher's host cost
        return ops.qk_norm_rope_impl(q, k, cos, sin, float(eps))
    return ops.hip_qk_norm_rope(q, k, cos, sin, float(eps))
