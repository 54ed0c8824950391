"""Parity of the HIP attention kernels with the fp32 oracle (GPU only).

Tolerances (from the build's contract, checked here literally):
  O         |hip - ref| <= 1e-2 + 2e-2 * |ref|    elementwise (bf16 output)
  LSE       |hip - ref| <= 1e-3                   elementwise
  dQ/dK/dV  |hip - ref| <= 3e-2 * (|ref| + max|ref|) + 1e-5  elementwise, i.e.
            relative 3e-2 with the tensor's own scale as the floor for
            near-zero entries (1e-5 absolute when the exact gradient is
            identically zero, as at W = 1), and ||hip - ref|| / ||ref|| <= 3e-2.
The oracle consumes the same bf16-rounded inputs upcast to fp32.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oracle

pytestmark = pytest.mark.gpu

O_ATOL, O_RTOL, LSE_ATOL, GRAD_RTOL, GRAD_ATOL = 1e-2, 2e-2, 1e-3, 3e-2, 1e-5


def _device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


def make_inputs(B, T, H, Hkv, D, seed):
    """q, k, v, dO ~ N(0,1) from one CPU generator, rounded to bf16 (CPU)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).bfloat16()
    k = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    v = torch.randn(B, T, Hkv, D, generator=g).bfloat16()
    do = torch.randn(B, T, H, D, generator=g).bfloat16()
    return q, k, v, do


def run_hip(q, k, v, do, window, dev):
    import hlm_attn
    from hlm_attn import ops

    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    w = 0 if window is None else window
    o, lse = ops.hip_attn_fwd(qd, kd, vd, w, 1.0 / math.sqrt(q.shape[-1]))
    dq, dk, dv = ops.hip_attn_bwd(dod, qd, kd, vd, o, lse, w, 1.0 / math.sqrt(q.shape[-1]))
    torch.cuda.synchronize()
    return [t.float().cpu() for t in (o, lse, dq, dk, dv)]


def assert_out(name, got, ref):
    err = (got - ref).abs()
    bound = O_ATOL + O_RTOL * ref.abs()
    assert bool((err <= bound).all()), f"{name}: max err {err.max().item():.3e}, worst excess {(err - bound).max().item():.3e}"


def assert_lse(got, ref):
    err = (got - ref).abs().max().item()
    assert err <= LSE_ATOL, f"lse: max err {err:.3e}"


def assert_grad(name, got, ref):
    err = (got - ref).abs()
    scale = ref.abs().max()
    assert bool((err <= GRAD_RTOL * (ref.abs() + scale) + GRAD_ATOL).all()), (
        f"{name}: max err {err.max().item():.3e} vs max|ref| {scale.item():.3e}"
    )
    if ref.norm() > 0:
        rel = (err.norm() / ref.norm()).item()
        assert rel <= GRAD_RTOL, f"{name}: norm-relative error {rel:.3e}"


SMALL_CASES = [
    # B, T, H, Hkv, D, window, seed
    (1, 1, 2, 2, 64, None, 0),      # single token: O = V
    (2, 37, 3, 3, 64, 5, 1),        # ragged T, tiny window
    (1, 128, 2, 2, 64, 1, 2),       # W = 1: O = V
    (2, 200, 2, 2, 64, 64, 3),
    (1, 256, 4, 4, 128, 100, 4),
    (2, 300, 4, 2, 64, 77, 5),      # grouped-query heads
    (1, 512, 2, 2, 128, None, 6),   # full causal, D = 128
    (1, 333, 2, 1, 128, 129, 7),    # MQA, ragged, W not tile aligned
    (2, 1024, 6, 6, 64, 256, 8),    # BASELINE configs[0] shape
]


@pytest.mark.parametrize("B,T,H,Hkv,D,window,seed", SMALL_CASES)
def test_fwd_bwd_matches_oracle(B, T, H, Hkv, D, window, seed):
    dev = _device()
    print(f"case B={B} T={T} H={H} Hkv={Hkv} D={D} W={window} seed={seed}", flush=True)
    q, k, v, do = make_inputs(B, T, H, Hkv, D, seed)
    o, lse, dq, dk, dv = run_hip(q, k, v, do, window, dev)
    ro, rlse = oracle.forward(q, k, v, window)
    rdq, rdk, rdv = oracle.backward(q, k, v, do, window)
    assert_out("o", o, ro)
    assert_lse(lse, rlse)
    assert_grad("dq", dq, rdq)
    assert_grad("dk", dk, rdk)
    assert_grad("dv", dv, rdv)


# Shapes around the kernels' tile and ring boundaries: 32-row query blocks,
# 128-row workgroup tiles, 32/64-key tiles and ring depths of 2-6 tiles
# (T and W one below, at and one above those multiples), both head sizes,
# MHA and MQA.
EDGE_CASES = [
    # B, T, H, Hkv, D, window
    (1, 31, 2, 2, 64, None),
    (1, 33, 2, 1, 64, 32),
    (1, 95, 2, 2, 64, 33),
    (1, 97, 2, 2, 128, 64),
    (1, 129, 2, 2, 64, 63),
    (1, 160, 2, 1, 64, 65),
    (1, 191, 2, 2, 128, 127),
    (1, 193, 2, 2, 64, 128),
    (1, 255, 2, 2, 64, 129),
    (1, 257, 2, 1, 128, 191),
    (1, 256, 3, 3, 64, 192),
    (2, 385, 2, 2, 64, 200),
    (1, 640, 2, 2, 64, 320),
    (1, 700, 2, 2, 128, 512),
]


@pytest.mark.parametrize("B,T,H,Hkv,D,window", EDGE_CASES)
def test_tile_edge_shapes_match_oracle(B, T, H, Hkv, D, window):
    dev = _device()
    seed = 100 + T
    print(f"case B={B} T={T} H={H} Hkv={Hkv} D={D} W={window} seed={seed}", flush=True)
    q, k, v, do = make_inputs(B, T, H, Hkv, D, seed)
    o, lse, dq, dk, dv = run_hip(q, k, v, do, window, dev)
    ro, rlse = oracle.forward(q, k, v, window)
    rdq, rdk, rdv = oracle.backward(q, k, v, do, window)
    assert_out("o", o, ro)
    assert_lse(lse, rlse)
    assert_grad("dq", dq, rdq)
    assert_grad("dk", dk, rdk)
    assert_grad("dv", dv, rdv)


FULL_CONFIGS = [
    # name, B, T, H, D, window  (BASELINE.json configs[1..4]; cfg4 = one local and one full layer)
    ("cfg2_local", 8, 2048, 12, 64, 512),
    ("cfg3_full", 8, 2048, 12, 64, None),
    ("cfg4_local", 4, 4096, 12, 128, 1024),
    ("cfg4_full", 4, 4096, 12, 128, None),
    ("cfg5_long", 1, 16384, 16, 128, 2048),
]


@pytest.mark.parametrize("name,B,T,H,D,window", FULL_CONFIGS)
def test_full_size_slices_match_oracle(name, B, T, H, D, window):
    """At BASELINE sizes: exact oracle on query bands of the first and last
    (batch, head), and size-independent invariants on the whole output."""
    dev = _device()
    print(f"case {name} B={B} T={T} H={H} D={D} W={window}", flush=True)
    q, k, v, do = make_inputs(B, T, H, H, D, seed=11)
    o, lse, dq, dk, dv = run_hip(q, k, v, do, window, dev)
    for t in (o, lse, dq, dk, dv):
        assert bool(torch.isfinite(t).all())
    w = T if window is None else window
    band = min(T, w + 256)
    for b, h in ((0, 0), (B - 1, H - 1)):
        sl = lambda t: t[b : b + 1, :, h : h + 1]  # noqa: E731
        for q_lo in sorted({0, min(T // 2 + 3, T - band), T - band}):
            q_hi = q_lo + band
            ro, rlse, rdq, rdk, rdv, k_lo = oracle.band_forward_backward(
                sl(q), sl(k), sl(v), sl(do), window, q_lo, q_hi
            )
            assert_out("o", o[b : b + 1, q_lo:q_hi, h : h + 1], ro)
            assert_lse(lse[b : b + 1, h : h + 1, q_lo:q_hi], rlse)
            assert_grad("dq", dq[b : b + 1, q_lo:q_hi, h : h + 1], rdq)
            # keys whose visible queries all lie in [q_lo, q_hi): [q_lo, q_hi - w + 1) and,
            # for the last band, every key up to T.
            k_end = T if q_hi == T else q_hi - w + 1
            if k_end > q_lo:
                a, z = q_lo - k_lo, k_end - k_lo
                assert_grad("dk", dk[b : b + 1, q_lo:k_end, h : h + 1], rdk[:, a:z])
                assert_grad("dv", dv[b : b + 1, q_lo:k_end, h : h + 1], rdv[:, a:z])
