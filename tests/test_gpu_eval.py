"""The evaluation path on the GPU (GPU only): forward-only calls at batch 1
and ragged T with no KV cache, as the reference's lm-eval adapter makes them
(lm_eval_hackable_lm.py:134-160 loglikelihood batches, :185-207 greedy
generation, one model(idx) per generated token).

Small grids go through the split-key forward (hlm_attn_fwd_split: several
workgroups per query tile's keys, merged by log-sum-exp).  Tolerances are
those of the attention parity tests:
  O    |hip - ref| <= 1e-2 + 2e-2 |ref|     LSE  |hip - ref| <= 1e-3
against the fp32 oracle on the same bf16 inputs; and split against unsplit
O within a few bf16 ulps (|a - b| <= 2^-6 |b| + 4e-3: the two round P to bf16
against different running maxima), LSE within 1e-4.
"""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from oracle import attention as oracle

pytestmark = pytest.mark.gpu

O_ATOL, O_RTOL, LSE_ATOL = 1e-2, 2e-2, 1e-3


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def _inputs(B, T, H, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).bfloat16()
    k = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    v = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    return q, k, v


def _check_o(name, got, ref):
    err = (got.float().cpu() - ref).abs()
    bound = O_ATOL + O_RTOL * ref.abs()
    assert bool((err <= bound).all()), f"{name}: max err {err.max().item():.3e}"


def _run_fwd(q, k, v, window, nsplit):
    """One forward through the C ABI: hlm_attn_fwd (nsplit = 1) or
    hlm_attn_fwd_split with a caller-owned workspace."""
    from hlm_attn import _lib, ops

    lib = _lib.load()
    B, T, H, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=q.device)
    st = [_lib.strides3(t) for t in (q, k, v, o)]
    w = 0 if window is None else window
    stream = ops._stream_handle(q.device)
    if nsplit == 1:
        rc = lib.hlm_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                              B, T, H, k.shape[2], D, *st, w, 1.0 / math.sqrt(D), stream)
    else:
        ws = torch.full((nsplit * B * H * T * (D + 2),), float("nan"), device=q.device)  # no init needed
        rc = lib.hlm_attn_fwd_split(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                    ws.data_ptr(), nsplit, B, T, H, k.shape[2], D, *st, w, 1.0 / math.sqrt(D),
                                    stream)
    _lib.check(rc, lib)
    torch.cuda.synchronize()
    return o, lse


SPLIT_CASES = [
    # B, T, H, Hkv, D, window, nsplit
    (1, 1, 2, 2, 64, None, 2),        # one key tile: the second split is empty
    (1, 37, 3, 3, 64, 5, 3),          # ragged T, tiny window, empty splits
    (1, 300, 4, 4, 64, None, 4),
    (1, 300, 4, 2, 128, 96, 2),       # D = 128, GQA, window not tile-aligned
    (2, 1000, 2, 1, 64, 512, 16),     # MQA, most splits of short rows empty
    (1, 2048, 12, 12, 64, None, 4),   # a full-causal layer at the eval batch
    (1, 2048, 12, 12, 64, 512, 4),    # a local layer at the eval batch
    (1, 777, 2, 2, 128, None, 7),
]


def _ids(c):
    return "B{}_T{}_H{}_Hkv{}_D{}_W{}_S{}".format(*c)


@pytest.mark.parametrize("case", SPLIT_CASES, ids=_ids)
def test_split_forward_matches_oracle_and_unsplit(case):
    B, T, H, Hkv, D, W, ns = case
    dev = _dev()
    print(f"split forward {_ids(case)}", flush=True)
    q, k, v = _inputs(B, T, H, Hkv, D, seed=T + ns)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    o_s, lse_s = _run_fwd(qd, kd, vd, W, ns)
    o_1, lse_1 = _run_fwd(qd, kd, vd, W, 1)
    assert torch.isfinite(o_s).all() and torch.isfinite(lse_s).all()
    ro, rlse = oracle.forward(q, k, v, W)
    _check_o("o (split)", o_s, ro)
    assert (lse_s.cpu() - rlse).abs().max().item() <= LSE_ATOL
    diff = (o_s.float() - o_1.float()).abs()
    assert bool((diff <= 2.0 ** -6 * o_1.float().abs() + 4e-3).all()), f"split vs unsplit {diff.max().item():.3e}"
    assert (lse_s - lse_1).abs().max().item() <= 1e-4


def test_generation_loop_matches_oracle():
    """generate_until's pattern: one no-grad forward per step over the whole
    prefix, T = 1, 2, 3, ... (tile edges included), batch 1."""
    import hlm_attn

    dev = _dev()
    H, D = 12, 64
    q, k, v = _inputs(1, 1030, H, H, D, seed=5)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    lengths = list(range(1, 40)) + [63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513, 700, 1024, 1030]
    with torch.no_grad():
        for T in lengths:
            for W in (64, None):
                out = hlm_attn.attention(qd[:, :T], kd[:, :T], vd[:, :T], window_size=W)
                ro, _ = oracle.forward(q[:, :T], k[:, :T], v[:, :T], None if W is None or W >= T else W)
                _check_o(f"T={T} W={W}", out, ro)


def test_loglikelihood_batch_matches_oracle():
    """_loglikelihood_tokens' pattern: a batch of ragged sequences padded with
    one token id to the longest length minus one, scored in one forward."""
    import hlm_attn

    dev = _dev()
    B, T, H, D = 4, 333, 12, 64
    q, k, v = _inputs(B, T, H, H, D, seed=9)
    q[1, 200:] = q[1, 199]  # padded rows repeat one embedding, as eot padding does
    k[1, 200:] = k[1, 199]
    v[1, 200:] = v[1, 199]
    with torch.no_grad():
        out = hlm_attn.attention(q.to(dev), k.to(dev), v.to(dev), window_size=128)
    ro, _ = oracle.forward(q, k, v, 128)
    _check_o("batch", out, ro)


def test_direct_inference_path_equals_the_custom_op():
    import hlm_attn
    from hlm_attn import ops

    dev = _dev()
    for B, T, W in ((1, 2048, None), (1, 300, 64), (4, 129, None)):
        q, k, v = (t.to(dev) for t in _inputs(B, T, 12, 12, 64, seed=B + T))
        with torch.no_grad():
            direct = hlm_attn.attention(q, k, v, window_size=W)
        via_op, _ = ops.hip_attn_fwd(q, k, v, 0 if W is None else W, 0.125)
        torch.cuda.synchronize()
        assert torch.equal(direct, via_op), (B, T, W)


def test_split_forward_then_backward_matches_oracle():
    """A small-batch training step: the split forward's lse feeds the backward."""
    import hlm_attn

    dev = _dev()
    B, T, H, D, W = 1, 1024, 8, 64, None
    q, k, v = _inputs(B, T, H, H, D, seed=3)
    do = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(4)).bfloat16()
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = hlm_attn.attention(qd, kd, vd, window_size=W)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    ro, _ = oracle.forward(q, k, v, W)
    _check_o("o", out.detach(), ro)
    rdq, rdk, rdv = oracle.backward(q, k, v, do, W)
    for name, got, ref in (("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv)):
        err = (got.float().cpu() - ref).abs()
        assert (err.norm() / ref.norm()).item() <= 3e-2, name
