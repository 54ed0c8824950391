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


def test_noalloc_backward_captured_in_a_graph_on_its_first_call():
    """The first hlm_attn_bwd_noalloc call of the process (it looks up the
    array's device address) made inside HIP-graph capture on a fresh stream,
    as a caller that cannot allocate would make it; three replays with NaN
    outputs before each and eager work between them each equal
    hlm_attn_bwd bit for bit.  (No other GPU test calls this entry point, so
    the captured call is the first one whether this file runs alone or
    after the rest of the suite.)"""
    from hlm_attn import _lib, ops

    dev = _device()
    lib = _lib.load()
    B, T, H, Hkv, D, w = 2, 640, 4, 2, 64, 200
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, T, H, D, generator=g).bfloat16().to(dev)
    k = torch.randn(B, T, Hkv, D, generator=g).bfloat16().to(dev)
    v = torch.randn(B, T, Hkv, D, generator=g).bfloat16().to(dev)
    do = torch.randn(B, T, H, D, generator=g).bfloat16().to(dev)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.hip_attn_fwd(q, k, v, w, scale)
    st = _lib.strides3
    outs = [tuple(torch.full_like(t, float("nan")) for t in (q, k, v)) for _ in range(2)]

    def call(noalloc, dq, dk, dv):
        common = (B, T, H, Hkv, D, st(q), st(k), st(v), st(o), st(do), st(dq), st(dk), st(dv), w, scale,
                  ops._stream_handle(dev))
        ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
        if noalloc:
            return lib.hlm_attn_bwd_noalloc(*ptrs, *common)
        return lib.hlm_attn_bwd(*ptrs, ws.data_ptr(), *common)

    ws = torch.empty(2 * B * H * T, dtype=torch.float32, device=dev)
    _lib.check(call(False, *outs[0]), lib)
    torch.cuda.synchronize()
    print("eager hlm_attn_bwd done; capturing the first hlm_attn_bwd_noalloc call", flush=True)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        rc = call(True, *outs[1])
    _lib.check(rc, lib)
    for replay in range(3):
        for t in outs[1]:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), outs[0], outs[1]):
            assert torch.equal(a, b), f"replay {replay}: {name} differs from hlm_attn_bwd"
        _ = (q.float() * 2).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
    print("  3 replays equal hlm_attn_bwd bit for bit", flush=True)


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
