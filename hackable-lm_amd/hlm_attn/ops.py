"""torch custom ops over the C ABI: hackable_lm::hip_attn_fwd / hip_attn_bwd.

They are registered the way the reference registers its Triton ops
(torch.library.custom_op + register_fake + register_autograd,
/root/reference/kernels.py:320,388,505 and :738-740), so a model that runs
under torch.compile(fullgraph=True) and CUDA-graph capture
(/root/reference/kernels.py:126-143) can trace and capture them: the fake
implementations only describe shapes, and the real ones allocate through
torch's caching allocator, launch on torch's current stream and never
synchronise.  There is no CPU implementation: on a tensor that is not on a
ROCm device, or without libhlm_attn.so, the ops raise.

The backward runs the two-kernel path (hlm_attn_bwd: dq, then dkdv) unless
HLM_ATTN_BWD=fused selects the single-pass one (hlm_attn_bwd_fused, head
dim 64 only; other head dims keep the two-kernel path).
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import torch

from . import _lib

_BF16 = torch.bfloat16


def _layout_ok(t: torch.Tensor, s: tuple) -> bool:
    """t (strides s) fits the kernels: unit D stride, (batch, time, head)
    strides multiples of 8 elements, non-overlapping rows, 16-byte aligned."""
    return s[3] == 1 and not (s[0] | s[1] | s[2]) & 7 and s[1] >= t.shape[3] and not t.data_ptr() & 15


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Returns t if its layout fits the kernels, else a contiguous copy."""
    return t if _layout_ok(t, t.stride()) else t.contiguous()


def _check_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    qs, ks = q.shape, k.shape
    if (q.is_cuda and q.dtype is _BF16 and k.dtype is _BF16 and v.dtype is _BF16 and len(qs) == 4
            and len(ks) == 4 and ks == v.shape and qs[0] == ks[0] and qs[1] == ks[1] and qs[3] == ks[3]
            and ks[2] > 0 and qs[2] % ks[2] == 0 and q.get_device() == k.get_device() == v.get_device()):
        return  # the common case, checked without building device objects
    dev = q.device
    if dev.type != "cuda":
        raise RuntimeError(f"hip attention runs on ROCm devices only, got a tensor on {dev}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != _BF16:
            raise RuntimeError(f"hip attention expects bfloat16 {name}, got {t.dtype}")
        if t.dim() != 4:
            raise RuntimeError(f"hip attention expects {name} shaped (B, T, H, D), got {tuple(t.shape)}")
    if k.device != dev or v.device != dev:
        raise RuntimeError("q, k and v must be on the same device")
    if k.shape != v.shape:
        raise RuntimeError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must have the same shape")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise RuntimeError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree on B, T or D")
    if k.shape[2] == 0 or q.shape[2] % k.shape[2] != 0:
        raise RuntimeError(f"query heads {q.shape[2]} are not a multiple of kv heads {k.shape[2]}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device) -> ctypes.c_void_p:
    """torch's current stream on `device` (a capture stream inside graph
    capture), as the hipStream_t the kernels launch on."""
    if _raw_stream is not None:  # the same handle without building a Stream object
        return ctypes.c_void_p(_raw_stream(device.index if device.index is not None else torch.cuda.current_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _raw_stream_of(index: int) -> int:
    """_stream_handle's value as a Python int, for a device index."""
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def _on_device(device: torch.device):
    """Makes `device` current for the launch; a no-op (and no device guard's
    cost) when it already is."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _on_index(index: int):
    """_on_device for a device index (tensor.get_device())."""
    if index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(index)


def direct_call_ok(*tensors: torch.Tensor) -> bool:
    """True when a call may skip torch's op dispatcher and run the kernels'
    Python implementation directly: plain tensors (not fake or traced), no
    torch.compile tracing in progress, and no input that needs a gradient
    (inference, e.g. the evaluation harness's no-grad forwards).  The
    dispatcher and autograd wrapper cost far more host time than the launch."""
    if torch.compiler.is_compiling():
        return False
    grad = torch.is_grad_enabled()
    for t in tensors:
        if type(t) is not torch.Tensor or (grad and t.requires_grad):
            return False
    return True


def attn_fwd_impl(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int, scale: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """The forward launch behind hackable_lm::hip_attn_fwd (o, lse).  Inputs
    are checked, copied to the kernels' layout where needed, and launched
    through the CPython binding of the C ABI.  When the optional torch
    extension is present, inputs already in the kernels' layout take it
    instead: it checks, allocates and launches in one C++ call, which matters
    at batch 1 and short T, where the kernel takes a few us.  Without it (not
    built, built against another torch, or disabled) the results are the
    same: both paths launch the same kernels through the same C entry points."""
    ext = _lib._torch_fwd
    if ext is None:
        ext = _lib.torch_fwd()
    if ext and q.is_cuda:
        res = ext.fwd(q, k, v, int(window), float(scale), _raw_stream_of(q.get_device()))
        if res:
            return res[0], res[1]
    _check_inputs(q, k, v)
    pycall = _lib._pycall or _lib.load_pycall()
    sq, sk, sv = q.stride(), k.stride(), v.stride()
    if not _layout_ok(q, sq):
        q = q.contiguous()
        sq = q.stride()
    if not _layout_ok(k, sk):
        k = k.contiguous()
        sk = k.stride()
    if not _layout_ok(v, sv):
        v = v.contiguous()
        sv = v.stride()
    B, T, H, D = q.shape
    o = q.new_empty((B, T, H, D))
    lse = q.new_empty((B, H, T), dtype=torch.float32)
    window = int(window)
    nsplit = _split_cache.get((B, T, H, D, window)) or split_count(B, T, H, D, window)
    # small grid: split each query tile's keys, then merge (evaluation-sized calls)
    ws = q.new_empty(nsplit * B * H * T * (D + 2), dtype=torch.float32) if nsplit > 1 else None
    idx = q.get_device()
    with _on_index(idx):
        rc = pycall.fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            0 if ws is None else ws.data_ptr(), nsplit, B, T, H, k.shape[2], D,
            sq[0], sq[1], sq[2], sk[0], sk[1], sk[2], sv[0], sv[1], sv[2], T * H * D, H * D, D,
            window, float(scale), _raw_stream_of(idx),
        )
    if rc != 0:
        _lib.check(rc, _lib.load())
    return o, lse


_split_cache: dict = {}


def split_count(B: int, T: int, H: int, D: int, window: int) -> int:
    """hlm_attn_fwd_split_count, memoised per shape."""
    key = (B, T, H, D, window)
    n = _split_cache.get(key)
    if n is None:
        if len(_split_cache) > 4096:
            _split_cache.clear()
        n = _split_cache[key] = _lib.load().hlm_attn_fwd_split_count(B, T, H, D, window)
    return n


@torch.library.custom_op("hackable_lm::hip_attn_fwd", mutates_args=())
def hip_attn_fwd(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int, scale: float
) -> tuple[torch.Tensor, torch.Tensor]:
    return attn_fwd_impl(q, k, v, window, scale)


@hip_attn_fwd.register_fake
def _(q, k, v, window, scale):
    B, T, H, D = q.shape
    return q.new_empty((B, T, H, D), dtype=_BF16), q.new_empty((B, H, T), dtype=torch.float32)


@torch.library.custom_op("hackable_lm::hip_attn_bwd", mutates_args=())
def hip_attn_bwd(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    window: int,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    _check_inputs(q, k, v)
    lib = _lib.load()
    if dout.shape != q.shape or o.shape != q.shape:
        raise RuntimeError("dout and o must have the shape of q")
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    o = _kernel_ready(o)
    dout = _kernel_ready(dout.to(_BF16))
    lse = lse.contiguous()
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    dq = torch.empty((B, T, H, D), dtype=_BF16, device=q.device)
    dk = torch.empty((B, T, Hkv, D), dtype=_BF16, device=q.device)
    dv = torch.empty((B, T, Hkv, D), dtype=_BF16, device=q.device)
    delta = torch.empty((2, B, H, T), dtype=torch.float32, device=q.device)  # -lse*log2(e), -rowsum(dO*O)
    strides = (_lib.strides3(q), _lib.strides3(k), _lib.strides3(v), _lib.strides3(o),
               _lib.strides3(dout), _lib.strides3(dq), _lib.strides3(dk), _lib.strides3(dv))
    with _on_device(q.device):
        if D == 64 and fused_backward_selected():
            nbytes = lib.hlm_attn_bwd_fused_workspace_bytes(B, T, H, D, int(window))
            if nbytes < 0:
                _lib.check(int(nbytes), lib)
            part = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=q.device)
            rc = lib.hlm_attn_bwd_fused(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dout.data_ptr(), lse.data_ptr(),
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), part.data_ptr(), int(nbytes),
                B, T, H, Hkv, D, *strides, int(window), float(scale), _stream_handle(q.device),
            )
        else:
            rc = lib.hlm_attn_bwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dout.data_ptr(), lse.data_ptr(),
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(),
                B, T, H, Hkv, D, *strides, int(window), float(scale), _stream_handle(q.device),
            )
    _lib.check(rc, lib)
    return dq, dk, dv


def fused_backward_selected() -> bool:
    """True when HLM_ATTN_BWD=fused asks for the single-pass backward."""
    return os.environ.get("HLM_ATTN_BWD", "").lower() == "fused"


@hip_attn_bwd.register_fake
def _(dout, q, k, v, o, lse, window, scale):
    return (
        q.new_empty(q.shape, dtype=_BF16),
        k.new_empty(k.shape, dtype=_BF16),
        v.new_empty(v.shape, dtype=_BF16),
    )


def _setup_context(ctx, inputs, output):
    q, k, v, window, scale = inputs
    o, lse = output
    ctx.save_for_backward(q, k, v, o, lse)
    ctx.window = window
    ctx.scale = scale


def _backward(ctx, dout, _dlse):
    # lse is an auxiliary output for the backward; gradients flowing into it
    # are not propagated (attention() never exposes it).
    q, k, v, o, lse = ctx.saved_tensors
    dq, dk, dv = hip_attn_bwd(dout, q, k, v, o, lse, ctx.window, ctx.scale)
    return dq, dk, dv, None, None


hip_attn_fwd.register_autograd(_backward, setup_context=_setup_context)


# --- the producer step: fused q/k RMSNorm + partial rotary embedding ---------------
#
# hackable_lm::hip_qk_norm_rope mirrors the reference's Triton op
# hackable_lm::qk_norm_rope (/root/reference/kernels.py:505-535, autograd
# :679-741): same inputs (q, k, cos, sin, eps), outputs contiguous in q's and
# k's shapes, backward through the fused kernel.


def _rope_table(t: torch.Tensor, T: int) -> tuple[torch.Tensor, int]:
    """cos / sin in any of the reference's broadcast shapes ((T, R),
    (1, T, 1, R) after its transpose, (1, 1, T, R)) as a contiguous (T, R)
    table and its HLM_TABLE_* code: bf16 tables (the model's, model.py:62-70)
    and fp32 tables are read as they are, other types are converted to fp32."""
    R = t.shape[-1]
    if t.numel() != T * R:
        raise RuntimeError(f"rotary table of shape {tuple(t.shape)} does not hold {T} rows of {R}")
    if t.dtype not in (_BF16, torch.float32):
        t = t.to(torch.float32)
    code = _lib.TABLE_BF16 if t.dtype == _BF16 else _lib.TABLE_F32
    t = t.reshape(T, R).contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t, code


def _check_qk(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor) -> None:
    if q.device.type != "cuda":
        raise RuntimeError(f"hip qk_norm_rope runs on ROCm devices only, got a tensor on {q.device}")
    for name, t in (("q", q), ("k", k)):
        if t.dtype != _BF16:
            raise RuntimeError(f"hip qk_norm_rope expects bfloat16 {name}, got {t.dtype}")
        if t.dim() != 4:
            raise RuntimeError(f"hip qk_norm_rope expects {name} shaped (B, T, heads, D), got {tuple(t.shape)}")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise RuntimeError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree on B, T or D")
    if k.device != q.device or cos.device != q.device:
        raise RuntimeError("q, k, cos and sin must be on the same device")


def qk_norm_rope_impl(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """The forward launch behind hackable_lm::hip_qk_norm_rope."""
    _check_qk(q, k, cos)
    lib = _lib.load()
    q, k = _kernel_ready(q), _kernel_ready(k)
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    c, code = _rope_table(cos, T)
    s, _ = _rope_table(sin.to(c.dtype), T)
    q_out = torch.empty((B, T, H, D), dtype=_BF16, device=q.device)
    k_out = torch.empty((B, T, Hkv, D), dtype=_BF16, device=q.device)
    with _on_device(q.device):
        rc = lib.hlm_qk_norm_rope_fwd(
            q.data_ptr(), k.data_ptr(), c.data_ptr(), s.data_ptr(), code, q_out.data_ptr(), k_out.data_ptr(),
            B, T, H, Hkv, D, c.shape[1], _lib.strides3(q), _lib.strides3(k), float(eps),
            _stream_handle(q.device),
        )
    _lib.check(rc, lib)
    return q_out, k_out


@torch.library.custom_op("hackable_lm::hip_qk_norm_rope", mutates_args=())
def hip_qk_norm_rope(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    return qk_norm_rope_impl(q, k, cos, sin, eps)


@hip_qk_norm_rope.register_fake
def _(q, k, cos, sin, eps):
    return q.new_empty(q.shape, dtype=_BF16), k.new_empty(k.shape, dtype=_BF16)


@torch.library.custom_op("hackable_lm::hip_qk_norm_rope_backward", mutates_args=())
def hip_qk_norm_rope_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    grad_q: torch.Tensor,
    grad_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    _check_qk(q, k, cos)
    lib = _lib.load()
    q, k = _kernel_ready(q), _kernel_ready(k)
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    gq = grad_q.to(_BF16).contiguous()
    gk = grad_k.to(_BF16).contiguous()
    c, code = _rope_table(cos, T)
    s, _ = _rope_table(sin.to(c.dtype), T)
    dq = torch.empty((B, T, H, D), dtype=_BF16, device=q.device)
    dk = torch.empty((B, T, Hkv, D), dtype=_BF16, device=q.device)
    with _on_device(q.device):
        rc = lib.hlm_qk_norm_rope_bwd(
            q.data_ptr(), k.data_ptr(), gq.data_ptr(), gk.data_ptr(), c.data_ptr(), s.data_ptr(), code,
            dq.data_ptr(), dk.data_ptr(), B, T, H, Hkv, D, c.shape[1],
            _lib.strides3(q), _lib.strides3(k), float(eps), _stream_handle(q.device),
        )
    _lib.check(rc, lib)
    return dq, dk


@hip_qk_norm_rope_backward.register_fake
def _(q, k, grad_q, grad_k, cos, sin, eps):
    return q.new_empty(q.shape, dtype=_BF16), k.new_empty(k.shape, dtype=_BF16)


def _qk_setup_context(ctx, inputs, output):
    q, k, cos, sin, eps = inputs
    ctx.save_for_backward(q, k, cos, sin)
    ctx.eps = eps


def _qk_backward(ctx, grad_q, grad_k):
    q, k, cos, sin = ctx.saved_tensors
    if grad_q is None:
        grad_q = torch.zeros_like(q, memory_format=torch.contiguous_format)
    if grad_k is None:
        grad_k = torch.zeros_like(k, memory_format=torch.contiguous_format)
    dq, dk = hip_qk_norm_rope_backward(q, k, grad_q, grad_k, cos, sin, ctx.eps)
    return dq, dk, None, None, None


hip_qk_norm_rope.register_autograd(_qk_backward, setup_context=_qk_setup_context)


# --- the LM head: cross-entropy rows of the fused linear + cross-entropy ----------
#
# hackable_lm::hip_linear_ce mirrors the reference's Triton op
# hackable_lm::linear_ce (/root/reference/kernels.py:320-336): it overwrites
# `logits` in place with the gradient of the mean loss and returns the
# per-row losses (already divided by n_tokens).

IGNORE_INDEX = -100  # F.cross_entropy's default ignore_index


def linear_ce_impl(logits: torch.Tensor, targets: torch.Tensor, n_tokens: int) -> torch.Tensor:
    """The launch behind hackable_lm::hip_linear_ce."""
    if logits.device.type != "cuda":
        raise RuntimeError(f"hip linear_ce runs on ROCm devices only, got a tensor on {logits.device}")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise RuntimeError(f"hip linear_ce expects (rows, vocab) logits with unit column stride, got {tuple(logits.shape)}")
    if logits.dtype not in (_BF16, torch.float32):
        raise RuntimeError(f"hip linear_ce expects bfloat16 or float32 logits, got {logits.dtype}")
    if targets.shape != (logits.shape[0],):
        raise RuntimeError(f"targets {tuple(targets.shape)} do not match {logits.shape[0]} logit rows")
    lib = _lib.load()
    targets = targets.to(device=logits.device, dtype=torch.int64).contiguous()
    loss = torch.empty(logits.shape[0], dtype=torch.float32, device=logits.device)
    code = _lib.DTYPE_BF16 if logits.dtype == _BF16 else _lib.DTYPE_F32
    with _on_device(logits.device):
        rc = lib.hlm_ce_rows(
            logits.data_ptr(), code, logits.stride(0), targets.data_ptr(), loss.data_ptr(),
            logits.shape[0], logits.shape[1], int(n_tokens), IGNORE_INDEX, _stream_handle(logits.device),
        )
    _lib.check(rc, lib)
    return loss


@torch.library.custom_op("hackable_lm::hip_linear_ce", mutates_args=("logits",))
def hip_linear_ce(logits: torch.Tensor, targets: torch.Tensor, n_tokens: int) -> torch.Tensor:
    return linear_ce_impl(logits, targets, n_tokens)


@hip_linear_ce.register_fake
def _(logits, targets, n_tokens):
    return logits.new_empty((logits.shape[0],), dtype=torch.float32)


# --- residual add + RMSNorm after the output / down projections -------------------
#
# hackable_lm::hip_residual_rms_norm computes residual_rms_norm
# (/root/reference/model.py:73-75) on the GPU; the reference leaves its
# backward to autograd, here it is hackable_lm::hip_residual_rms_norm_backward.


def _rows_ready(t: torch.Tensor, n: int) -> torch.Tensor:
    """t as a contiguous, 16-byte aligned bf16 (rows, n) tensor."""
    t = t.to(_BF16).reshape(-1, n)
    if not t.is_contiguous() or t.data_ptr() % 16:
        t = t.contiguous() if not t.is_contiguous() else t.clone()
    return t


def residual_rms_norm_impl(residual: torch.Tensor, branch: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """The launch behind hackable_lm::hip_residual_rms_norm: (out, normed)."""
    if residual.device.type != "cuda":
        raise RuntimeError(f"hip residual_rms_norm runs on ROCm devices only, got a tensor on {residual.device}")
    if residual.shape != branch.shape:
        raise RuntimeError(f"residual {tuple(residual.shape)} and branch {tuple(branch.shape)} differ")
    lib = _lib.load()
    n = residual.shape[-1]
    a, b = _rows_ready(residual, n), _rows_ready(branch, n)
    out = torch.empty(residual.shape, dtype=_BF16, device=residual.device)
    normed = torch.empty(residual.shape, dtype=_BF16, device=residual.device)
    with _on_device(residual.device):
        rc = lib.hlm_residual_rms_norm_fwd(
            a.data_ptr(), b.data_ptr(), out.data_ptr(), normed.data_ptr(), a.shape[0], n, float(eps),
            _stream_handle(residual.device),
        )
    _lib.check(rc, lib)
    return out, normed


@torch.library.custom_op("hackable_lm::hip_residual_rms_norm", mutates_args=())
def hip_residual_rms_norm(residual: torch.Tensor, branch: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    return residual_rms_norm_impl(residual, branch, eps)


@hip_residual_rms_norm.register_fake
def _(residual, branch, eps):
    return residual.new_empty(residual.shape, dtype=_BF16), residual.new_empty(residual.shape, dtype=_BF16)


@torch.library.custom_op("hackable_lm::hip_residual_rms_norm_backward", mutates_args=())
def hip_residual_rms_norm_backward(
    out: torch.Tensor, grad_out: torch.Tensor, grad_normed: torch.Tensor, eps: float
) -> torch.Tensor:
    if out.device.type != "cuda":
        raise RuntimeError(f"hip residual_rms_norm runs on ROCm devices only, got a tensor on {out.device}")
    lib = _lib.load()
    n = out.shape[-1]
    o, go, gn = _rows_ready(out, n), _rows_ready(grad_out, n), _rows_ready(grad_normed, n)
    grad_in = torch.empty(out.shape, dtype=_BF16, device=out.device)
    with _on_device(out.device):
        rc = lib.hlm_residual_rms_norm_bwd(
            o.data_ptr(), go.data_ptr(), gn.data_ptr(), grad_in.data_ptr(), o.shape[0], n, float(eps),
            _stream_handle(out.device),
        )
    _lib.check(rc, lib)
    return grad_in


@hip_residual_rms_norm_backward.register_fake
def _(out, grad_out, grad_normed, eps):
    return out.new_empty(out.shape, dtype=_BF16)


def _res_setup_context(ctx, inputs, output):
    _, _, eps = inputs
    out, _ = output
    ctx.save_for_backward(out)
    ctx.eps = eps


def _res_backward(ctx, grad_out, grad_normed):
    (out,) = ctx.saved_tensors
    if grad_out is None:
        grad_out = torch.zeros_like(out)
    if grad_normed is None:
        grad_normed = torch.zeros_like(out)
    g = hip_residual_rms_norm_backward(out, grad_out, grad_normed, ctx.eps)
    return g, g, None


hip_residual_rms_norm.register_autograd(_res_backward, setup_context=_res_setup_context)
