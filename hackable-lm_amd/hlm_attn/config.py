"""Attention-backend names and the per-layer window pattern.

Mirrors the attention part of hackable-lm's config.py so the hip backend is
selected and configured exactly like the existing ones:
  ATTENTION_BACKENDS / normalize_attention_backend   config.py:11, :71-77
  MODULE_BACKENDS / normalize_module_backend         config.py:10, :62-68
                                                     (qkv_backend picks the q/k producer)
  normalize_attention_window / _full_every           config.py:172-181
  layer_attention_window                             config.py:184-191
"""
from __future__ import annotations

HIP_BACKEND = "hip"
REFERENCE_ATTENTION_BACKENDS = frozenset(
    {"torch", "flex_attention", "flash_attn_2", "flash_attn_3", "flash_attn_4"}
)
# The reference's set plus the one backend this library adds.
ATTENTION_BACKENDS = REFERENCE_ATTENTION_BACKENDS | {HIP_BACKEND}


# config.py:10 plus "hip": the fused q/k RMSNorm + RoPE producer of this library.
REFERENCE_MODULE_BACKENDS = frozenset({"torch", "triton"})
MODULE_BACKENDS = REFERENCE_MODULE_BACKENDS | {HIP_BACKEND}


def normalize_module_backend(name: str, backend: str) -> str:
    """Lower-cases and validates a module backend such as qkv_backend (config.py:62-68)."""
    if not isinstance(backend, str):
        raise ValueError(f"unknown {name} {backend!r}")
    backend = backend.lower()
    if backend not in MODULE_BACKENDS:
        raise ValueError(f"unknown {name} {backend!r}")
    return backend


def normalize_attention_backend(backend: str) -> str:
    """Lower-cases and validates a backend name (config.py:71-77)."""
    if not isinstance(backend, str):
        raise ValueError(f"unknown attention_backend {backend!r}")
    backend = backend.lower()
    if backend not in ATTENTION_BACKENDS:
        raise ValueError(f"unknown attention_backend {backend!r}")
    return backend


def normalize_attention_window(attention_window: int | None) -> int | None:
    """0 or None disables the window (config.py:172-175)."""
    if attention_window is None or attention_window == 0:
        return None
    return int(attention_window)


def normalize_attention_full_every(attention_full_every: int | None) -> int | None:
    """0 or None disables periodic full layers (config.py:178-181)."""
    if attention_full_every is None or attention_full_every == 0:
        return None
    return int(attention_full_every)


def layer_attention_window(
    layer_idx: int, n_layer: int, attention_window: int | None, attention_full_every: int | None
) -> int | None:
    """Window of one layer, or None for full causal attention (config.py:184-191):
    no window configured, the last layer, and every `attention_full_every`-th
    layer (1-based) are full."""
    if attention_window is None:
        return None
    if layer_idx == n_layer - 1:
        return None
    if attention_full_every is not None and (layer_idx + 1) % attention_full_every == 0:
        return None
    return attention_window


def attention_window_size(window: int | None, seq_len: int) -> int | None:
    """A window at least as long as the sequence is plain causal (model.py:155-159)."""
    if window is None or window >= seq_len:
        return None
    return window
