"""hlm_attn_bwd_noalloc (the backward without a caller workspace) against
hlm_attn_bwd, through the C ABI (GPU only).

Both run the same kernels; the only difference is where the workspace lives
(a fixed device array in the library instead of caller memory), so dq, dk and
dv must agree bit for bit.  Two calls in a row, the second on a smaller
problem (the array keeps the first call's contents), and the results also
against the fp32 oracle at the attention tolerances.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oracle

pytestmark = pytest.mark.gpu


def _device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def _backward_both_ways(B, T, H, Hkv, D, window, seed, dev):
    from hlm_attn import _lib, ops

    lib = _lib.load()
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).bfloat16()
    k = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    v = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    do = torch.randn(B, T, H, D, generator=g).bfloat16()
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    w = 0 if window is None else window
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.hip_attn_fwd(qd, kd, vd, w, scale)
    stream = ops._stream_handle(dev)
    st = _lib.strides3
    out = []
    for noalloc in (False, True):
        dq = torch.full_like(qd, float("nan"))
        dk = torch.full_like(kd, float("nan"))
        dv = torch.full_like(vd, float("nan"))
        common = (B, T, H, Hkv, D, st(qd), st(kd), st(vd), st(o), st(dod), st(dq), st(dk), st(dv), w, scale, stream)
        ptrs = (qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr(), dod.data_ptr(), lse.data_ptr(),
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
        if noalloc:
            rc = lib.hlm_attn_bwd_noalloc(*ptrs, *common)
        else:
            ws = torch.empty(2 * B * H * T, dtype=torch.float32, device=dev)
            rc = lib.hlm_attn_bwd(*ptrs, ws.data_ptr(), *common)
        _lib.check(rc, lib)
        torch.cuda.synchronize()
        out.append((dq, dk, dv))
    return (q, k, v, do), out


def test_noalloc_backward_equals_the_workspace_backward_twice():
    dev = _device()
    cases = [
        # B, T, H, Hkv, D, window, seed: the second call is smaller than the first
        (4, 1024, 8, 4, 64, 256, 1),
        (1, 300, 2, 2, 128, None, 2),
    ]
    for B, T, H, Hkv, D, window, seed in cases:
        print(f"case B={B} T={T} H={H} Hkv={Hkv} D={D} W={window}", flush=True)
        (q, k, v, do), ((dq, dk, dv), (dq2, dk2, dv2)) = _backward_both_ways(B, T, H, Hkv, D, window, seed, dev)
        for name, a, b in (("dq", dq, dq2), ("dk", dk, dk2), ("dv", dv, dv2)):
            assert torch.equal(a, b), f"{name}: noalloc differs from the workspace backward"
        rdq, rdk, rdv = oracle.backward(q, k, v, do, window)
        for name, got, ref in (("dq", dq2, rdq), ("dk", dk2, rdk), ("dv", dv2, rdv)):
            rel = ((got.float().cpu() - ref).norm() / ref.norm()).item()
            print(f"  {name}: norm-rel vs oracle {rel:.2e}", flush=True)
            assert rel <= 3e-2
