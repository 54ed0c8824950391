"""CPU oracle for hackable-lm's causal sliding-window attention.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the checker
(or, for the baseline, as the timed stand-in for the reference's CPU path).
The library in hackable-lm_amd/hlm_attn never imports it.

What it restates (each function cites the reference lines it follows):
  layer_attention_window   config.py:184-191
  window_size_at           model.py:155-159
  sliding_window_mask      model.py:143-153
  torch_backend_sdpa       kernels.py:785-800   (the `torch` backend math)
  attention_core_torch     model.py:176-196     ((B,T,H,D) layout, GQA repeat)
  forward / backward       the above in fp32 (or fp64) plus the closed-form
                           logsumexp; backward = autograd of the same graph
  closed_form_backward     textbook gradients of softmax attention (numpy fp64)
  brute_force_forward      per-query Python loops (numpy fp64), tiny sizes only

How each one is pinned (tests/test_oracle.py): torch_backend_sdpa and
attention_core_torch against brute_force_forward and the reference test's
own closed form (tests/test_kernels.py:97-130 shape, Dv != Dqk); the LSE
against brute force and the special cases Q = 0 (log of the window count),
W = 1; backward against closed_form_backward and central finite differences;
the mask and layer pattern against the reference tests' literal values
(tests/test_model.py:58-60, tests/test_config.py:53-56).  Committed fixtures
under tests/golden/ hold fp64 brute-force vectors.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def layer_attention_window(layer_idx: int, n_layer: int, attention_window: int | None,
                           attention_full_every: int | None) -> int | None:
    """config.py:184-191: None (full causal) if no window, for the last layer,
    and for every attention_full_every-th layer."""
    if attention_window is None:
        return None
    if layer_idx == n_layer - 1:
        return None
    if attention_full_every is not None and (layer_idx + 1) % attention_full_every == 0:
        return None
    return attention_window


def window_size_at(window: int | None, seq_len: int) -> int | None:
    """model.py:155-159: a window that covers the sequence is plain causal."""
    if window is None or window >= seq_len:
        return None
    return window


def sliding_window_mask(seq_len: int, window: int | None) -> torch.Tensor | None:
    """model.py:143-153: bool [1,1,T,T], True where 0 <= i - j < window."""
    if window is None or window >= seq_len:
        return None
    pos = torch.arange(seq_len)
    distance = pos[:, None] - pos[None, :]
    return ((distance >= 0) & (distance < window))[None, None, :, :]


def torch_backend_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, is_causal: bool,
                       attn_mask: torch.Tensor | None) -> torch.Tensor:
    """kernels.py:785-800 (dropout 0): (B,H,T,D) layout, scores in the input
    dtype, -inf fill, softmax in fp32, cast back, then P @ V."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    attn = torch.matmul(q, k.transpose(-2, -1)) * scale
    if is_causal:
        q_len, kv_len = q.shape[-2], k.shape[-2]
        causal = torch.ones((q_len, kv_len), dtype=torch.bool).tril()
        attn = attn.masked_fill(~causal, float("-inf"))
    if attn_mask is not None:
        attn = attn.masked_fill(~attn_mask, float("-inf"))
    attn = torch.softmax(attn.float(), dim=-1).to(dtype=q.dtype)
    return torch.matmul(attn, v)


def attention_core_torch(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         window: int | None) -> torch.Tensor:
    """model.py:176-196: (B,T,H,D) in and out, kv heads repeated for GQA."""
    seq_len = q.shape[1]
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if kh.shape[1] != qh.shape[1]:
        rep = qh.shape[1] // kh.shape[1]
        kh = kh.repeat_interleave(rep, dim=1)
        vh = vh.repeat_interleave(rep, dim=1)
    mask = sliding_window_mask(seq_len, window)
    y = torch_backend_sdpa(qh, kh, vh, is_causal=mask is None, attn_mask=mask)
    return y.transpose(1, 2)


def _scores_masked(q: torch.Tensor, k: torch.Tensor, window: int | None) -> torch.Tensor:
    """Scaled scores (B,H,T,T) with -inf outside the causal window."""
    T = q.shape[1]
    qh, kh = q.transpose(1, 2), k.transpose(1, 2)
    if kh.shape[1] != qh.shape[1]:
        kh = kh.repeat_interleave(qh.shape[1] // kh.shape[1], dim=1)
    s = torch.matmul(qh, kh.transpose(-2, -1)) / math.sqrt(q.shape[-1])
    w = T if window is None else min(window, T)
    pos = torch.arange(T)
    dist = pos[:, None] - pos[None, :]
    ok = (dist >= 0) & (dist < w)
    return s.masked_fill(~ok, float("-inf"))


def forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int | None,
            dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of the torch backend evaluated in `dtype` on the CPU.
    O is (B,T,H,D); LSE is (B,H,T), natural log of the masked scaled scores."""
    q, k, v = (t.detach().cpu().to(dtype) for t in (q, k, v))
    o = attention_core_torch(q, k, v, window)
    lse = torch.logsumexp(_scores_masked(q, k, window), dim=-1)
    return o, lse


def backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dout: torch.Tensor,
             window: int | None, dtype: torch.dtype = torch.float32
             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV) by autograd through attention_core_torch in `dtype`."""
    q, k, v = (t.detach().cpu().to(dtype).requires_grad_(True) for t in (q, k, v))
    o = attention_core_torch(q, k, v, window)
    o.backward(dout.detach().cpu().to(dtype))
    return q.grad, k.grad, v.grad


def closed_form_backward(q: np.ndarray, k: np.ndarray, v: np.ndarray, dout: np.ndarray,
                         window: int | None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Textbook softmax-attention gradients in fp64, (B,T,H,D) layout, Hkv == H:
    P = softmax(S), dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dO * O)),
    dQ = scale dS K, dK = scale dS^T Q."""
    q, k, v, dout = (np.asarray(x, dtype=np.float64) for x in (q, k, v, dout))
    B, T, H, D = q.shape
    scale = 1.0 / math.sqrt(D)
    w = T if window is None else min(window, T)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    ok = (i - j >= 0) & (i - j < w)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        for h in range(H):
            Q, K, V, dO = q[b, :, h], k[b, :, h], v[b, :, h], dout[b, :, h]
            S = np.where(ok, scale * Q @ K.T, -np.inf)
            P = np.exp(S - S.max(axis=1, keepdims=True))
            P /= P.sum(axis=1, keepdims=True)
            O = P @ V
            dV = P.T @ dO
            dP = dO @ V.T
            dS = P * (dP - (dO * O).sum(axis=1, keepdims=True))
            dq[b, :, h] = scale * dS @ K
            dk[b, :, h] = scale * dS.T @ Q
            dv[b, :, h] = dV
    return dq, dk, dv


def brute_force_forward(q: np.ndarray, k: np.ndarray, v: np.ndarray, window: int | None
                        ) -> tuple[np.ndarray, np.ndarray]:
    """Per-query loops in fp64 (B,T,H,D); kv heads shared by H/Hkv query heads.
    For each query i: s_j = q_i.k_j/sqrt(D) for j in [max(0, i-W+1), i],
    o_i = sum_j e^{s_j - m} v_j / sum_j e^{s_j - m}, lse_i = m + log sum e^{s_j - m}."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    Dv = v.shape[3]
    scale = 1.0 / math.sqrt(D)
    w = T if window is None else window
    o = np.zeros((B, T, H, Dv))
    lse = np.zeros((B, H, T))
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            for i in range(T):
                js = range(max(0, i - w + 1), i + 1)
                s = [scale * float(np.dot(q[b, i, h], k[b, j, hk])) for j in js]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                acc = np.zeros(Dv)
                for ej, j in zip(e, js):
                    acc += ej * v[b, j, hk]
                o[b, i, h] = acc / z
                lse[b, h, i] = m + math.log(z)
    return o, lse


def causal_window_pairs(T: int, window: int | None) -> int:
    """Number of (query, key) pairs the mask keeps, counted directly."""
    w = T if window is None else min(window, T)
    return sum(min(i + 1, w) for i in range(T))


def band_forward_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dout: torch.Tensor,
                          window: int | None, q_lo: int, q_hi: int,
                          dtype: torch.dtype = torch.float32):
    """The torch-backend math restricted to queries [q_lo, q_hi) of (B,T,H,D)
    tensors, with the mask on absolute positions (model.py:148-150).

    Returns (o, lse, dq, dk, dv, k_lo): o/lse/dq are exact for those queries;
    dk/dv (keys [k_lo, q_hi), k_lo = max(0, q_lo - W + 1)) hold the
    contribution of those queries only, which is the whole gradient for every
    key whose visible queries all lie in [q_lo, q_hi)."""
    T, D = q.shape[1], q.shape[3]
    w = T if window is None else min(window, T)
    k_lo = max(0, q_lo - w + 1)
    qs = q[:, q_lo:q_hi].detach().cpu().to(dtype).requires_grad_(True)
    ks = k[:, k_lo:q_hi].detach().cpu().to(dtype).requires_grad_(True)
    vs = v[:, k_lo:q_hi].detach().cpu().to(dtype).requires_grad_(True)
    dos = dout[:, q_lo:q_hi].detach().cpu().to(dtype)
    qh, kh, vh = qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2)
    if kh.shape[1] != qh.shape[1]:
        rep = qh.shape[1] // kh.shape[1]
        kh, vh = kh.repeat_interleave(rep, dim=1), vh.repeat_interleave(rep, dim=1)
    dist = torch.arange(q_lo, q_hi)[:, None] - torch.arange(k_lo, q_hi)[None, :]
    ok = (dist >= 0) & (dist < w)
    s = (torch.matmul(qh, kh.transpose(-2, -1)) / math.sqrt(D)).masked_fill(~ok, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    o = torch.matmul(torch.softmax(s, dim=-1), vh).transpose(1, 2)
    o.backward(dos)
    return o.detach(), lse.detach(), qs.grad, ks.grad, vs.grad, k_lo
