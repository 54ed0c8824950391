"""Pins the CPU oracle (oracle/attention.py) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: the reference tests' literal values, fp64 brute-force loops, closed
forms that special cases reduce to, finite differences, and the committed
golden vectors.  tests/test_oracle_mutations.py plants plausible mistakes in a
copy of the oracle and shows that these checks catch them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oracle

GOLDEN = __import__("pathlib").Path(__file__).with_name("golden") / "attention_small.npz"
# The reference's torch backend runs its softmax in fp32 whatever the input
# dtype (kernels.py:797), so even fp64 inputs give ~1e-7 accuracy through it.
SOFTMAX_FP32 = 2e-6


def _rand(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


# --- the reference tests' own literal facts --------------------------------

def test_mask_matches_reference_model_test():
    """tests/test_model.py:54-60 of the reference: W=4, T=8."""
    mask = oracle.sliding_window_mask(8, 4)
    assert bool(mask[0, 0, 7, 7])
    assert bool(mask[0, 0, 7, 4])
    assert not bool(mask[0, 0, 7, 3])
    assert mask.shape == (1, 1, 8, 8)


def test_layer_pattern_matches_reference_config_test():
    """tests/test_config.py:53-56 of the reference."""
    assert [oracle.layer_attention_window(i, 8, 512, 4) for i in range(8)] == [512, 512, 512, None, 512, 512, 512, None]
    assert [oracle.layer_attention_window(i, 3, 512, 4) for i in range(3)] == [512, 512, None]
    # BASELINE cfg4: 18 layers, W=1024, every 4th full, plus the last layer.
    pattern = [oracle.layer_attention_window(i, 18, 1024, 4) for i in range(18)]
    assert [i for i, w in enumerate(pattern) if w is None] == [3, 7, 11, 15, 17]
    assert oracle.layer_attention_window(0, 4, None, 4) is None


def test_window_at_least_sequence_is_full_causal():
    """model.py:155-159: W >= T maps to None, and the mask is then not built."""
    assert oracle.window_size_at(8, 8) is None
    assert oracle.window_size_at(9, 8) is None
    assert oracle.window_size_at(7, 8) == 7
    assert oracle.sliding_window_mask(8, 8) is None


def test_torch_backend_matches_reference_closed_form_test():
    """The reference's tests/test_kernels.py:97-130 case (B2 H3 T5, Dqk=7, Dv=9,
    causal & distance<3), seeded, against softmax(QK^T/sqrt(d) masked) V."""
    q, k, v = _rand(2, 3, 5, 7, seed=1), _rand(2, 3, 5, 7, seed=2), _rand(2, 3, 5, 9, seed=3)
    mask = torch.ones(5, 5, dtype=torch.bool).tril()[None, None]
    mask = mask & ((torch.arange(5)[:, None] - torch.arange(5)[None, :]) < 3)[None, None]
    scores = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(7)
    ref = torch.matmul(torch.softmax(scores.masked_fill(~mask, float("-inf")), dim=-1), v)
    out = oracle.torch_backend_sdpa(q.float(), k.float(), v.float(), is_causal=False, attn_mask=mask)
    assert torch.allclose(out.double(), ref, atol=1e-6)  # the reference test's own tolerance
    # and the brute-force loops agree on the same case, (B,T,H,D) layout
    bo, _ = oracle.brute_force_forward(q.transpose(1, 2).numpy(), k.transpose(1, 2).numpy(),
                                       v.transpose(1, 2).numpy(), 3)
    assert np.allclose(bo, ref.transpose(1, 2).numpy(), atol=1e-12)


# --- torch restatement vs brute force --------------------------------------

@pytest.mark.parametrize("T,W,D,H,Hkv", [(1, None, 8, 2, 2), (17, 5, 8, 2, 2), (33, None, 16, 3, 3),
                                         (40, 1, 8, 2, 1), (64, 13, 64, 4, 2), (50, 64, 8, 2, 2)])
def test_forward_matches_brute_force(T, W, D, H, Hkv):
    q, k, v = _rand(2, T, H, D, seed=T), _rand(2, T, Hkv, D, seed=T + 1), _rand(2, T, Hkv, D, seed=T + 2)
    o, lse = oracle.forward(q, k, v, W, dtype=torch.float64)
    bo, blse = oracle.brute_force_forward(q.numpy(), k.numpy(), v.numpy(), W)
    assert np.allclose(o.numpy(), bo, atol=SOFTMAX_FP32)
    assert np.allclose(lse.numpy(), blse, atol=1e-12)


def test_forward_fp32_close_to_fp64():
    q, k, v = (_rand(2, 96, 2, 64, seed=s) for s in (7, 8, 9))
    o32, l32 = oracle.forward(q, k, v, 20, dtype=torch.float32)
    o64, l64 = oracle.forward(q, k, v, 20, dtype=torch.float64)
    assert (o32.double() - o64).abs().max() < 1e-5
    assert (l32.double() - l64).abs().max() < 1e-5


# --- special cases with closed forms ----------------------------------------

def test_window_one_and_single_token_give_v():
    q, k, v = (_rand(1, 12, 2, 8, seed=s) for s in (1, 2, 3))
    o, lse = oracle.forward(q, k, v, 1, dtype=torch.float64)
    assert torch.allclose(o, v, atol=SOFTMAX_FP32)
    # lse of a single key is its own scaled score
    s = (q * k).sum(-1).transpose(1, 2) / math.sqrt(8)
    assert torch.allclose(lse, s, atol=1e-12)
    o1, _ = oracle.forward(q[:, :1], k[:, :1], v[:, :1], None, dtype=torch.float64)
    assert torch.allclose(o1, v[:, :1], atol=SOFTMAX_FP32)


def test_zero_queries_average_the_window():
    """Q = 0: every visible key scores 0, so O_i is the mean of V over the
    window and LSE_i = log(min(i + 1, W))."""
    T, W = 20, 6
    q = torch.zeros(1, T, 1, 8, dtype=torch.float64)
    k, v = _rand(1, T, 1, 8, seed=4), _rand(1, T, 1, 8, seed=5)
    o, lse = oracle.forward(q, k, v, W, dtype=torch.float64)
    for i in range(T):
        lo = max(0, i - W + 1)
        assert torch.allclose(o[0, i, 0], v[0, lo : i + 1, 0].mean(0), atol=SOFTMAX_FP32)
        assert abs(lse[0, 0, i].item() - math.log(i + 1 - lo)) < 1e-12


def test_rows_are_convex_combinations_and_lse_bounds():
    T, W = 30, 7
    q, k, v = (_rand(2, T, 2, 8, seed=s) for s in (11, 12, 13))
    o, lse = oracle.forward(q, k, v, W, dtype=torch.float64)
    for i in range(T):
        lo = max(0, i - W + 1)
        win = v[:, lo : i + 1]
        assert bool((o[:, i] <= win.amax(1) + SOFTMAX_FP32).all())
        assert bool((o[:, i] >= win.amin(1) - SOFTMAX_FP32).all())
        s = torch.einsum("bhd,bjhd->bhj", q[:, i], k[:, lo : i + 1]) / math.sqrt(8)
        smax = s.amax(-1)
        assert bool((lse[:, :, i] >= smax - 1e-12).all())
        assert bool((lse[:, :, i] <= smax + math.log(i + 1 - lo) + 1e-12).all())


def test_slices_are_independent():
    q, k, v = (_rand(2, 24, 3, 8, seed=s) for s in (21, 22, 23))
    o, _ = oracle.forward(q, k, v, 5, dtype=torch.float64)
    o01, _ = oracle.forward(q[1:, :, 1:2], k[1:, :, 1:2], v[1:, :, 1:2], 5, dtype=torch.float64)
    assert torch.allclose(o[1:, :, 1:2], o01, atol=SOFTMAX_FP32)


def test_causality_future_keys_do_not_matter():
    q, k, v = (_rand(1, 16, 2, 8, seed=s) for s in (31, 32, 33))
    o, _ = oracle.forward(q, k, v, None, dtype=torch.float64)
    k2, v2 = k.clone(), v.clone()
    k2[:, 10:] += 5.0
    v2[:, 10:] -= 3.0
    o2, _ = oracle.forward(q, k2, v2, None, dtype=torch.float64)
    assert torch.allclose(o[:, :10], o2[:, :10], atol=SOFTMAX_FP32)
    assert not torch.allclose(o[:, 10:], o2[:, 10:])


# --- backward ------------------------------------------------------------------

@pytest.mark.parametrize("T,W", [(9, None), (21, 4), (32, 1), (40, 40)])
def test_backward_matches_closed_form(T, W):
    q, k, v, do = (_rand(2, T, 2, 8, seed=s) for s in (41, 42, 43, 44))
    dq, dk, dv = oracle.backward(q, k, v, do, W, dtype=torch.float64)
    cq, ck, cv = oracle.closed_form_backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), W)
    assert np.allclose(dq.numpy(), cq, atol=10 * SOFTMAX_FP32)
    assert np.allclose(dk.numpy(), ck, atol=10 * SOFTMAX_FP32)
    assert np.allclose(dv.numpy(), cv, atol=10 * SOFTMAX_FP32)


def test_closed_form_backward_matches_finite_differences():
    """Central differences of the fp64 brute-force forward pin the textbook
    gradient formulas (every element of dQ, dK, dV)."""
    T, W = 7, 3
    q, k, v, do = (_rand(1, T, 1, 4, seed=s).numpy() for s in (51, 52, 53, 54))
    cq, ck, cv = oracle.closed_form_backward(q, k, v, do, W)

    def loss(qq, kk, vv):
        o, _ = oracle.brute_force_forward(qq, kk, vv, W)
        return float((o * do).sum())

    eps = 1e-6
    for grad, which in ((cq, 0), (ck, 1), (cv, 2)):
        for idx in np.ndindex(*grad.shape):
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            up = loss(*args)
            args[which][idx] -= 2 * eps
            dn = loss(*args)
            assert abs((up - dn) / (2 * eps) - grad[idx]) < 1e-7


def test_window_one_gradients():
    """W = 1: O = V, so dV = dO and dQ = dK = 0 exactly."""
    q, k, v, do = (_rand(1, 10, 2, 8, seed=s) for s in (61, 62, 63, 64))
    dq, dk, dv = oracle.backward(q, k, v, do, 1, dtype=torch.float64)
    assert torch.allclose(dv, do, atol=SOFTMAX_FP32)
    assert dq.abs().max() < SOFTMAX_FP32 and dk.abs().max() < SOFTMAX_FP32


def test_gqa_gradients_sum_over_group():
    """Hkv < H: the kv gradient is the sum of the gradients of the repeated heads."""
    q, do = _rand(1, 12, 4, 8, seed=71), _rand(1, 12, 4, 8, seed=72)
    k, v = _rand(1, 12, 2, 8, seed=73), _rand(1, 12, 2, 8, seed=74)
    dq, dk, dv = oracle.backward(q, k, v, do, 5, dtype=torch.float64)
    kr, vr = k.repeat_interleave(2, dim=2), v.repeat_interleave(2, dim=2)
    cq, ck, cv = oracle.closed_form_backward(q.numpy(), kr.numpy(), vr.numpy(), do.numpy(), 5)
    assert np.allclose(dq.numpy(), cq, atol=10 * SOFTMAX_FP32)
    assert np.allclose(dk.numpy(), ck.reshape(1, 12, 2, 2, 8).sum(3), atol=10 * SOFTMAX_FP32)
    assert np.allclose(dv.numpy(), cv.reshape(1, 12, 2, 2, 8).sum(3), atol=10 * SOFTMAX_FP32)


def test_band_oracle_equals_full_oracle():
    T, W = 60, 9
    q, k, v, do = (_rand(2, T, 2, 8, seed=s) for s in (81, 82, 83, 84))
    o, lse = oracle.forward(q, k, v, W, dtype=torch.float64)
    dq, dk, dv = oracle.backward(q, k, v, do, W, dtype=torch.float64)
    bo, blse, bdq, bdk, bdv, k_lo = oracle.band_forward_backward(q, k, v, do, W, 20, 45, dtype=torch.float64)
    assert k_lo == 12
    tol = 10 * SOFTMAX_FP32  # the band evaluates its softmax in fp64, the full path in fp32
    assert torch.allclose(bo, o[:, 20:45], atol=tol)
    assert torch.allclose(blse, lse[:, :, 20:45], atol=1e-12)
    assert torch.allclose(bdq, dq[:, 20:45], atol=tol)
    # keys 20..36 are seen only by queries 20..44
    assert torch.allclose(bdk[:, 20 - k_lo : 37 - k_lo], dk[:, 20:37], atol=tol)
    assert torch.allclose(bdv[:, 20 - k_lo : 37 - k_lo], dv[:, 20:37], atol=tol)
    # a key also seen by a query outside the band gets only part of its gradient
    assert not torch.allclose(bdk[:, 40 - k_lo], dk[:, 40], atol=tol)


def test_pair_count_closed_form():
    """P(T,W) = W(W+1)/2 + (T-W)W, or T(T+1)/2, against the mask itself."""
    for T, W in [(1, None), (10, 3), (64, 64), (100, 7), (128, None)]:
        mask = oracle.sliding_window_mask(T, W)
        count = int(mask.sum()) if mask is not None else T * (T + 1) // 2
        assert oracle.causal_window_pairs(T, W) == count
    assert oracle.causal_window_pairs(2048, 512) == 917760
    assert oracle.causal_window_pairs(16384, 2048) == 31458304


# --- committed golden vectors ---------------------------------------------------

def test_golden_vectors():
    data = np.load(GOLDEN)
    for name in sorted({k.split("/")[0] for k in data.files}):
        g = {k.split("/")[1]: data[k] for k in data.files if k.startswith(name + "/")}
        W = int(g["window"]) if int(g["window"]) > 0 else None
        q, k, v, do = (torch.from_numpy(g[x]) for x in ("q", "k", "v", "do"))
        o, lse = oracle.forward(q, k, v, W, dtype=torch.float64)
        dq, dk, dv = oracle.backward(q, k, v, do, W, dtype=torch.float64)
        for got, key in ((o, "o"), (lse, "lse"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
            tol = 1e-10 if key == "lse" else 10 * SOFTMAX_FP32
            assert np.allclose(got.numpy(), g[key], atol=tol), f"{name}: {key}"
