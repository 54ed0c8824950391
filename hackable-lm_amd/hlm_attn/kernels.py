"""The hip branch of hackable-lm's attention dispatch.

`scaled_dot_product_attention` keeps the signature of
/root/reference/kernels.py:774-784 and behaves like its FlashAttention branch
(kernels.py:816-841): an explicit mask is rejected, q/k/v are cast to bf16,
the window becomes the kernels' causal look-back, the scale is 1/sqrt(D) and
the result is bf16 in (B, T, H, D).  Like the FlashAttention-3/4 branches
(kernels.py:842-843) it rejects dropout.  backend="torch" is the reference's
dense math on (B, H, T, D) tensors (kernels.py:785-800), which the mirrored
AttentionCore runs for CPU tensors as the reference's does (model.py:170).

`hip_attention_available` and `resolve_attention_backend` mirror the probe and
fallback rules of resolve_kernel_backends (kernels.py:146-242) for the
attention field.

`qk_norm_rope_hip` is the producer step before attention, with the signature
and semantics of the reference's `qk_norm_rope_triton` (kernels.py:756-771):
RMSNorm of each q and k row, then the partial rotary embedding.

`fused_linear_cross_entropy_with_weight(..., backend="hip")` is the LM head's
chunked linear + cross-entropy with the signature and result of
kernels.py:945-959: the HIP cross-entropy rows in place of the Triton
`linear_ce` op, inside this package's own chunk loop (`_LMHeadLoss`).
"""
from __future__ import annotations

import math
from typing import Any

import torch

from . import _lib
from .config import HIP_BACKEND, normalize_attention_backend


def hip_attention_available() -> bool:
    """True when a ROCm device is visible and every module the forward and
    backward need loads: libhlm_attn.so (the kernels and the C ABI) and its
    CPython binding.  The torch extension of the forward is optional (a host
    fast path) and is not required here."""
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    try:
        _lib.load()
        _lib.load_pycall()
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
    keys i-W+1..i.  Differentiable in q, k and v.

    The kernels take head dims 64 and 128 with Dv = Dqk.  Other head dims up
    to 128, and Dv != Dqk (model.py:181-184 allows it; the reference test
    uses Dqk = 7, Dv = 9, tests/test_kernels.py:103-105), run on them with
    the head dims zero-padded to the next of 64 / 128: zero columns of q and
    k leave q.k unchanged, zero columns of v only add zero output columns
    (sliced off), and the scale stays 1/sqrt(Dqk).  Gradients flow back
    through the padding exactly."""
    ops = _ops or _load_ops()
    bf16 = torch.bfloat16
    if q.dtype is not bf16:
        q = q.to(bf16)
    if k.dtype is not bf16:
        k = k.to(bf16)
    if v.dtype is not bf16:
        v = v.to(bf16)
    dqk, dv = q.shape[-1], v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(dqk)
    if window_size is not None and window_size < 1:
        raise RuntimeError(f"window_size must be >= 1 or None, got {window_size}")
    window = 0 if window_size is None else int(window_size)
    if k.shape[-1] != dqk:
        raise RuntimeError(f"q head dim {dqk} and k head dim {k.shape[-1]} differ")
    d_kernel = dqk if dqk == dv and (dqk == 64 or dqk == 128) else padded_head_dim(dqk, dv)
    if d_kernel != dqk or d_kernel != dv:
        pad = torch.nn.functional.pad
        q, k = pad(q, (0, d_kernel - dqk)), pad(k, (0, d_kernel - dqk))
        v = pad(v, (0, d_kernel - dv))
    if ops.direct_call_ok(q, k, v):  # inference: same kernels, without the dispatcher's host cost
        out, _ = ops.attn_fwd_impl(q, k, v, window, float(scale))
    else:
        out, _ = ops.hip_attn_fwd(q, k, v, window, float(scale))
    return out if d_kernel == dv else out[..., :dv]


_ops = None


def _load_ops():
    """hlm_attn.ops, imported (which registers the custom ops) on first use."""
    global _ops
    from . import ops

    _ops = ops
    return ops


def padded_head_dim(dqk: int, dv: int) -> int:
    """The kernel head dim that (Dqk, Dv) run at: 64 or 128."""
    d = max(dqk, dv)
    if d < 1 or d > 128:
        raise RuntimeError(f"head dims ({dqk}, {dv}) are not supported: the kernels take at most 128")
    return 64 if d <= 64 else 128


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
    """Dispatch entry with the reference's signature; implements backend="hip"
    and the reference's backend="torch" math."""
    if backend == "torch":
        return _torch_sdpa(q, k, v, dropout_p, is_causal, attn_mask)
    if backend != HIP_BACKEND:
        raise RuntimeError(
            f"unsupported attention backend {backend!r}: this library implements only {HIP_BACKEND!r} "
            "and the reference's 'torch' math; the other backends stay in the host model's kernels.py"
        )
    if attn_mask is not None or block_mask is not None:
        raise RuntimeError(f"{backend} path expects window_size instead of an explicit attention mask")
    if dropout_p:
        raise RuntimeError(f"{backend} backend does not support dropout")
    if not is_causal:
        raise RuntimeError(f"{backend} backend implements causal attention only")
    return attention(q, k, v, window_size=window_size)


def _torch_sdpa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dropout_p: float,
    is_causal: bool,
    attn_mask: torch.Tensor | None,
) -> torch.Tensor:
    """The reference's backend="torch" (kernels.py:785-800) on (B, H, T, D):
    scores q.k^T / sqrt(D) in the inputs' dtype, the causal triangle and a bool
    mask filled with -inf (a float mask is added), softmax in fp32 cast back,
    optional dropout, then P @ v.  Plain torch operators on any device; the
    right operand of each product (k transposed, v) is made contiguous first,
    since bf16 batched products on ROCm have faulted on strided right operands."""
    scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(q.shape[-1]))
    if is_causal:
        n_q, n_k = scores.shape[-2], scores.shape[-1]
        keep = torch.ones((n_q, n_k), dtype=torch.bool, device=q.device).tril()
        scores = scores.masked_fill(~keep, float("-inf"))
    if attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            scores = scores.masked_fill(~attn_mask, float("-inf"))
        else:
            scores = scores + attn_mask
    probs = torch.softmax(scores.float(), dim=-1).to(dtype=q.dtype)
    if dropout_p:
        probs = torch.nn.functional.dropout(probs, p=dropout_p, training=True)
    return torch.matmul(probs, v.contiguous())


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


# --- the LM head's fused linear + cross-entropy -----------------------------------

LINEAR_CE_MIN_CHUNK_SIZE = 2048  # kernels.py:252


def _next_power_of_2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def linear_ce_chunk_size(n_tokens: int, hidden_size: int, vocab_size: int, requested: int | None) -> int:
    """Rows per chunk, by the reference's rule (kernels.py:897-903): a requested
    size (at least 2048), or enough rows that one chunk's logits are about the
    size of the hidden states; never more than n_tokens."""
    if requested is not None and requested < 0:
        raise RuntimeError(f"loss_chunk_size must be nonnegative, got {requested}")
    if requested:
        return min(n_tokens, max(requested, LINEAR_CE_MIN_CHUNK_SIZE))
    inc_factor = -(-vocab_size // hidden_size)
    chunk = _next_power_of_2(-(-n_tokens // inc_factor))
    return min(n_tokens, max(chunk, LINEAR_CE_MIN_CHUNK_SIZE))


class _LMHeadLoss(torch.autograd.Function):
    """Mean cross-entropy of hidden @ W^T (+ b), differentiable in hidden, W
    and b, without ever holding more than one chunk of logits.

    The rows are processed in chunks (`linear_ce_chunk_size`).  One logits
    workspace of chunk x V is allocated once and every chunk's GEMM writes
    into it; the HIP row kernel (hackable_lm::hip_linear_ce) turns it in
    place into the gradient of the mean loss and returns the rows' losses.
    The three gradient products are formed in the forward, straight into
    their destinations: dhidden rows by a GEMM whose output is the chunk's
    slice of the dhidden buffer, dW accumulated inside the GEMM (addmm_, one
    rounding per chunk), db by an in-place add.  The backward only scales the
    three by the incoming gradient.  The results match the reference's
    chunked loop (kernels.py:878-942), which this replaces."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, bias, requested_chunk_size):
        from . import ops

        hidden = hidden.contiguous()
        weight = weight.contiguous()
        targets = targets.contiguous()
        n, d = hidden.shape
        vocab = weight.shape[0]
        rows = linear_ce_chunk_size(n, d, vocab, requested_chunk_size)
        want_h, want_w = hidden.requires_grad, weight.requires_grad
        want_b = bias is not None and bias.requires_grad
        d_hidden = torch.empty_like(hidden) if want_h else None
        d_weight = torch.zeros_like(weight) if want_w else None
        d_bias = torch.zeros_like(bias) if want_b else None
        losses = torch.empty(n, dtype=torch.float32, device=hidden.device)
        work = hidden.new_empty((rows, vocab))
        w_t = weight.t()
        for r0 in range(0, n, rows):
            r1 = min(r0 + rows, n)
            h = hidden[r0:r1]
            g = work[: r1 - r0]
            if bias is None:
                torch.mm(h, w_t, out=g)
            else:
                torch.addmm(bias, h, w_t, out=g)
            losses[r0:r1] = ops.hip_linear_ce(g, targets[r0:r1], n)
            if want_h:
                torch.mm(g, weight, out=d_hidden[r0:r1])
            if want_w:
                d_weight.addmm_(g.t(), h)
            if want_b:
                d_bias.add_(g.sum(dim=0).to(d_bias.dtype))
        ctx.save_for_backward(d_hidden, d_weight, d_bias)
        return losses.sum()

    @staticmethod
    def backward(ctx, grad_output):
        d_hidden, d_weight, d_bias = ctx.saved_tensors
        out = []
        for need, t in ((ctx.needs_input_grad[0], d_hidden), (ctx.needs_input_grad[1], d_weight)):
            out.append(t * grad_output.to(t.dtype) if need and t is not None else None)
        out.append(None)
        need_b = ctx.needs_input_grad[3] and d_bias is not None
        out.append(d_bias * grad_output.to(d_bias.dtype) if need_b else None)
        out.append(None)
        return tuple(out)


def fused_linear_cross_entropy_with_weight(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    targets: torch.Tensor,
    backend: str = HIP_BACKEND,
    chunk_size: int | None = None,
) -> torch.Tensor:
    """The reference's entry (kernels.py:945-959) with backend="hip": the mean
    cross-entropy of hidden @ W^T (+ b) against targets, differentiable in
    hidden, W and b.  There is no CPU path (the reference's own torch branch
    serves CPU tensors)."""
    if backend != HIP_BACKEND:
        raise RuntimeError(f"unsupported fused linear cross entropy backend {backend!r}")
    hidden_flat = hidden.reshape(-1, hidden.size(-1))
    targets_flat = targets.reshape(-1).contiguous()
    if hidden_flat.device.type != "cuda":
        raise RuntimeError("the hip fused linear cross entropy runs on ROCm devices only")
    return _LMHeadLoss.apply(hidden_flat, weight, targets_flat, bias, chunk_size)


# --- residual add + RMSNorm (OutputProjection / DownProjection) --------------------


def residual_rms_norm_hip(residual: torch.Tensor, branch: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """residual_rms_norm (model.py:73-75) on the GPU: (out, normed), bf16,
    out = residual + branch and normed = RMSNorm(out) without weight.
    Differentiable in residual and branch.  No CPU path."""
    from . import ops

    if residual.device.type != "cuda":
        raise RuntimeError("residual_rms_norm_hip runs on ROCm devices only; use the torch path on the CPU")
    if ops.direct_call_ok(residual, branch):  # inference: same kernel, without the dispatcher's host cost
        return ops.residual_rms_norm_impl(residual, branch, float(eps))
    return ops.hip_residual_rms_norm(residual, branch, float(eps))
