"""GPU tests of the hip backend as a model uses it: golden vectors, autograd,
the reference's tensor layouts, torch.compile and HIP-graph capture."""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oracle

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).with_name("golden") / "attention_small.npz"


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def _close(name, got, ref, rtol):
    """|got - ref| <= rtol * (|ref| + max|ref|) + 1e-5 and norm-relative <= rtol."""
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    assert bool((err <= rtol * (ref.abs() + ref.abs().max()) + 1e-5).all()), f"{name}: max err {err.max().item():.3e}"
    if ref.norm() > 0:
        assert (err.norm() / ref.norm()).item() <= rtol, name


def test_golden_vectors_through_the_kernels():
    import hlm_attn

    dev = _dev()
    data = np.load(GOLDEN)
    for name in sorted({k.split("/")[0] for k in data.files}):
        print(f"golden case {name}", flush=True)
        g = lambda key: torch.from_numpy(data[f"{name}/{key}"])  # noqa: E731
        W = int(data[f"{name}/window"]) or None
        q, k, v = (g(x).to(dev).bfloat16().requires_grad_(True) for x in ("q", "k", "v"))
        out = hlm_attn.attention(q, k, v, window_size=W)
        out.backward(g("do").to(dev).bfloat16())
        ref_o = g("o")
        err = (out.detach().float().cpu() - ref_o).abs()
        assert bool((err <= 1e-2 + 2e-2 * ref_o.abs()).all()), f"{name}: o max err {err.max().item():.3e}"
        _close(f"{name} dq", q.grad, g("dq"), 3e-2)
        _close(f"{name} dk", k.grad, g("dk"), 3e-2)
        _close(f"{name} dv", v.grad, g("dv"), 3e-2)


def _qkv_from_fused_projection(B, T, H, D, dev, seed):
    """q, k, v as model.py:92-99 produces them: views of one fused projection
    output (v keeps the projection's row stride)."""
    g = torch.Generator().manual_seed(seed)
    fused = torch.randn(B, T, 3 * H * D, generator=g).bfloat16().to(dev)
    q, k, v = fused.split((H * D, H * D, H * D), dim=-1)
    return q.reshape(B, T, H, D).contiguous(), k.reshape(B, T, H, D).contiguous(), v.view(B, T, H, D)


def test_strided_v_view_matches_contiguous():
    import hlm_attn

    dev = _dev()
    q, k, v = _qkv_from_fused_projection(2, 200, 4, 64, dev, seed=3)
    assert not v.is_contiguous() and v.stride(1) == 3 * 4 * 64
    out_view = hlm_attn.attention(q, k, v, window_size=48)
    out_cont = hlm_attn.attention(q, k, v.contiguous(), window_size=48)
    torch.cuda.synchronize()
    assert torch.equal(out_view, out_cont)


def test_autograd_through_attention_core_layers():
    """A 4-layer pattern (W=64, every 2nd layer full, last full) through the
    AttentionCore mirror, forward and backward, each layer vs the oracle."""
    from hlm_attn import AttentionConfig, AttentionCore

    dev = _dev()
    cfg = AttentionConfig(n_layer=4, n_head=4, n_kv_head=4, attention_window=64, attention_full_every=2)
    B, T, H, D = 2, 160, 4, 64
    for layer in range(4):
        core = AttentionCore(cfg, layer)
        g = torch.Generator().manual_seed(100 + layer)
        q, k, v, do = (torch.randn(B, T, H, D, generator=g).bfloat16() for _ in range(4))
        qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
        out = core(qd, kd, vd)
        out.backward(do.to(dev))
        W = core._attention_window_size(T)
        ro, _ = oracle.forward(q, k, v, W)
        rdq, rdk, rdv = oracle.backward(q, k, v, do, W)
        err = (out.detach().float().cpu() - ro).abs()
        assert bool((err <= 1e-2 + 2e-2 * ro.abs()).all()), f"layer {layer}"
        _close("dq", qd.grad, rdq, 3e-2)
        _close("dk", kd.grad, rdk, 3e-2)
        _close("dv", vd.grad, rdv, 3e-2)


def test_attention_core_backend_switch_on_the_gpu():
    """The drop-in as a model sees it: one AttentionCore, attention_backend
    flipped from the reference's "torch" math (fp32 on the GPU here, so no
    bf16 batched product runs) to "hip", on the same ROCm tensors; outputs
    and gradients agree within the parity tolerances, GQA and a window."""
    from hlm_attn import AttentionConfig, AttentionCore

    dev = _dev()
    B, T, H, Hkv, D = 2, 300, 4, 2, 64
    g = torch.Generator().manual_seed(21)
    q, k, v, do = (torch.randn(B, T, h, D, generator=g).bfloat16() for h in (H, Hkv, Hkv, H))
    grads = {}
    for backend in ("torch", "hip"):
        cfg = AttentionConfig(n_layer=4, n_head=H, n_kv_head=Hkv, attention_window=100, attention_backend=backend)
        core = AttentionCore(cfg, 0).eval()
        dtype = torch.float32 if backend == "torch" else torch.bfloat16
        qd, kd, vd = (t.to(dev, dtype).requires_grad_(True) for t in (q, k, v))
        out = core(qd, kd, vd)
        out.backward(do.to(dev, dtype))
        torch.cuda.synchronize()
        grads[backend] = [t.detach().float().cpu() for t in (out, qd.grad, kd.grad, vd.grad)]
    ref, got = grads["torch"], grads["hip"]
    err = (got[0] - ref[0]).abs()
    assert bool((err <= 1e-2 + 2e-2 * ref[0].abs()).all())
    for name, a, b in zip(("dq", "dk", "dv"), got[1:], ref[1:]):
        _close(name, a, b, 3e-2)


def test_expanded_upstream_gradient():
    """o.sum().backward() hands the backward an expanded dO (all strides 0)."""
    import hlm_attn

    dev = _dev()
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, 96, 2, 64, generator=g).bfloat16() for _ in range(3))
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    hlm_attn.attention(qd, kd, vd, window_size=32).float().sum().backward()
    rdq, rdk, rdv = oracle.backward(q, k, v, torch.ones(1, 96, 2, 64), 32)
    _close("dq", qd.grad, rdq, 3e-2)
    _close("dk", kd.grad, rdk, 3e-2)
    _close("dv", vd.grad, rdv, 3e-2)


def test_results_are_deterministic():
    """No atomics anywhere: two runs give bit-identical outputs and gradients."""
    import hlm_attn

    dev = _dev()
    g = torch.Generator().manual_seed(8)
    q, k, v, do = (torch.randn(2, 700, 4, 64, generator=g).bfloat16().to(dev) for _ in range(4))
    runs = []
    for _ in range(2):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = hlm_attn.attention(qd, kd, vd, window_size=200)
        out.backward(do)
        runs.append([out.detach(), qd.grad, kd.grad, vd.grad])
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_torch_compile_fullgraph_matches_eager():
    """The reference trains under torch.compile(fullgraph=True) (kernels.py:126-137)."""
    import hlm_attn

    dev = _dev()

    def layer(q, k, v):
        return hlm_attn.attention(q, k, v, window_size=64) * 2.0

    compiled = torch.compile(layer, fullgraph=True, dynamic=False)
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (torch.randn(2, 256, 4, 64, generator=g).bfloat16().to(dev) for _ in range(4))
    outs = []
    for fn in (layer, compiled):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = fn(qd, kd, vd)
        out.backward(do)
        outs.append([out.detach(), qd.grad, kd.grad, vd.grad])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_hip_graph_capture_and_replay():
    """fwd + bwd captured in a HIP graph (as CUDA-graph training does,
    kernels.py:140-143), replayed several times with eager work and
    synchronisation in between; every replay must equal the eager result."""
    from hlm_attn import ops

    dev = _dev()
    g = torch.Generator().manual_seed(10)
    q, k, v, do = (torch.randn(2, 512, 4, 64, generator=g).bfloat16().to(dev) for _ in range(4))
    scale = 1 / math.sqrt(64)

    def step():
        o, lse = ops.hip_attn_fwd(q, k, v, 128, scale)
        dq, dk, dv = ops.hip_attn_bwd(do, q, k, v, o, lse, 128, scale)
        return o, lse, dq, dk, dv

    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm up allocations on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for replay in range(3):
        for t in static:
            t.fill_(float("nan")) if t.dtype != torch.bool else None
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(static, eager):
            assert torch.equal(got, want), f"replay {replay} differs from eager"
        _ = (q.float() @ k.float().transpose(-1, -2)).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()


def test_forward_and_backward_without_the_torch_extension(monkeypatch):
    """With the optional torch extension disabled, the forward (training
    custom op and no-grad direct path) runs through the CPython binding of
    the C ABI: outputs and gradients match the oracle, and both paths give
    the same bits as with the extension."""
    import hlm_attn
    from hlm_attn import _lib

    dev = _dev()
    g = torch.Generator().manual_seed(11)
    B, T, H, D, W = 2, 333, 4, 64, 100
    q, k, v, do = (torch.randn(B, T, H, D, generator=g).bfloat16() for _ in range(4))

    def run():
        qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
        out = hlm_attn.attention(qd, kd, vd, window_size=W)
        out.backward(do.to(dev))
        with torch.no_grad():
            direct = hlm_attn.attention(qd.detach(), kd.detach(), vd.detach(), window_size=W)
        torch.cuda.synchronize()
        return [out.detach(), direct, qd.grad, kd.grad, vd.grad]

    with_ext = run()
    monkeypatch.setattr(_lib, "_torch_fwd", False)  # as after a failed import
    assert _lib.torch_fwd() is None
    without = run()
    for a, b in zip(with_ext, without):
        assert torch.equal(a, b)
    ro, _ = oracle.forward(q, k, v, W)
    rdq, rdk, rdv = oracle.backward(q, k, v, do, W)
    for o in without[:2]:
        err = (o.float().cpu() - ro).abs()
        assert bool((err <= 1e-2 + 2e-2 * ro.abs()).all()), f"o max err {err.max().item():.3e}"
    _close("dq", without[2], rdq, 3e-2)
    _close("dk", without[3], rdk, 3e-2)
    _close("dv", without[4], rdv, 3e-2)
