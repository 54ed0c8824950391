"""CPU tests of the drop-in boundary: the C ABI library and its Python mirror
of the reference's backend interface.  Nothing here launches a kernel.

The dispatch tests follow the reference's own fake-kernel tests
(tests/test_kernels.py:133-226: fake flash_attn_func handles pin the bf16
cast, causal flag, window mapping and bf16 output); here a fake custom op
stands in for the HIP kernels.
"""
from __future__ import annotations

import ctypes
import math
import re
from pathlib import Path

import pytest
import torch

import hlm_attn
from hlm_attn import _lib, config, kernels, model, ops
from oracle import attention as oracle

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "hlm_attn.h"


def declared_symbols() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(hlm_(?:attn|qk|ce|residual)_\w+)\s*\(", text))


# --- the shared library -------------------------------------------------------

def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert {"hlm_attn_fwd", "hlm_attn_bwd", "hlm_attn_last_error", "hlm_attn_abi_version"} <= names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(_lib.SIGNATURES) == names, "ctypes binding and header disagree"
    assert lib.hlm_attn_abi_version() == _lib.ABI_VERSION


def _strides(*s):
    return (ctypes.c_int64 * 3)(*s)


def _fwd(lib, ptr=0x1000, B=1, T=16, H=2, Hkv=2, D=64, strides=(2048, 128, 64), window=0, scale=0.125):
    s = _strides(*strides)
    p = ctypes.c_void_p(ptr) if ptr else None
    lse = ctypes.c_void_p(0x2000)
    return lib.hlm_attn_fwd(p, p, p, p, lse, B, T, H, Hkv, D, s, s, s, s, window, scale, None)


@pytest.mark.parametrize(
    "kwargs,code,msg",
    [
        (dict(D=96), -2, "head_dim 96"),
        (dict(D=32), -2, "head_dim 32"),
        (dict(H=3, Hkv=2), -1, "not a multiple"),
        (dict(H=0), -1, "bad shape"),
        (dict(ptr=None), -1, "null pointer"),
        (dict(ptr=0x1008), -1, "16-byte aligned"),
        (dict(strides=(2048, 100, 64)), -1, "multiple of 8"),
        (dict(strides=(-8, 128, 64)), -1, "multiple of 8"),
        (dict(scale=0.0), -1, "scale"),
        (dict(scale=float("nan")), -1, "scale"),
    ],
)
def test_fwd_rejects_bad_arguments_before_touching_the_device(kwargs, code, msg):
    lib = _lib.load()
    assert _fwd(lib, **kwargs) == code
    assert msg in lib.hlm_attn_last_error().decode()


def test_cpython_binding_passes_the_same_arguments_to_the_c_abi():
    """_pycall.fwd (the no-grad host path) reaches the same validation as the
    ctypes call: same codes, same messages, no device touched; the split
    entry point behind nsplit > 1 too."""
    lib = _lib.load()
    pc = _lib.load_pycall()
    st = (2048, 128, 64) * 4

    def call(ptr=0x1000, nsplit=1, ws=0, D=64, H=2, Hkv=2, window=0, scale=0.125, strides=st):
        return pc.fwd(ptr, ptr, ptr, ptr, 0x2000, ws, nsplit, 1, 16, H, Hkv, D, *strides, window, scale, 0)

    for kwargs, code, msg in [
        (dict(D=96), -2, "head_dim 96"),
        (dict(H=3, Hkv=2), -1, "not a multiple"),
        (dict(ptr=0), -1, "null pointer"),
        (dict(ptr=0x1008), -1, "16-byte aligned"),
        (dict(strides=(2048, 100, 64) * 4), -1, "multiple of 8"),
        (dict(scale=float("nan")), -1, "scale"),
        (dict(nsplit=4, ws=0), -1, "workspace"),
    ]:
        assert call(**kwargs) == code, kwargs
        assert msg in lib.hlm_attn_last_error().decode(), kwargs
    with pytest.raises(TypeError):
        pc.fwd(1, 2, 3)
    with pytest.raises(TypeError):
        call(scale="x")
    with pytest.raises(OverflowError):  # a C int argument out of range raises rather than wrapping
        call(H=2**32 + 2, Hkv=2)


def test_torch_extension_takes_only_kernel_ready_device_inputs():
    """_torch_fwd.fwd (the no-grad fast path) hands back [] for anything it
    does not launch itself -- here CPU tensors, wrong dtypes, wrong ranks or
    mismatched shapes -- so the caller's general path converts or raises."""
    ext = _lib.load_torch_fwd()
    q = torch.zeros(1, 16, 2, 64, dtype=torch.bfloat16)
    assert ext.fwd(q, q, q, 0, 0.125, 0) == []
    assert ext.fwd(q.float(), q.float(), q.float(), 0, 0.125, 0) == []
    assert ext.fwd(q[0], q[0], q[0], 0, 0.125, 0) == []
    assert ext.fwd(q, q[:, :8], q[:, :8], 0, 0.125, 0) == []


def test_empty_problems_are_no_ops():
    lib = _lib.load()
    assert _fwd(lib, B=0) == 0
    assert _fwd(lib, T=0) == 0
    assert lib.hlm_attn_last_error() == b""


def test_bwd_phases_validate_like_bwd():
    lib = _lib.load()
    s = _strides(2048, 128, 64)
    p = ctypes.c_void_p(0x1000)
    for name in ("hlm_attn_bwd", "hlm_attn_bwd_dq", "hlm_attn_bwd_dkdv"):
        fn = getattr(lib, name)
        rc = fn(p, p, p, p, p, p, p, p, p, None, 1, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None)
        assert rc == -1 and b"delta_ws" in lib.hlm_attn_last_error()
        rc = fn(p, p, p, p, p, p, p, p, p, p, 1, 16, 2, 2, 128 + 8, s, s, s, s, s, s, s, s, 0, 0.125, None)
        assert rc == -2


def _partials_per_row_bound(T: int, W: int) -> int:
    """The most 128-key tiles that any query row's keys (q - W + 1 .. q) meet."""
    W = T if W <= 0 or W >= T else W
    return max(q // 128 - max(0, q - W + 1) // 128 + 1 for q in range(T))


@pytest.mark.parametrize("B,T,H,W", [(8, 2048, 12, 512), (8, 2048, 12, 0), (1, 640, 2, 513), (2, 37, 3, 5),
                                     (1, 1, 2, 0), (1, 700, 2, 129)])
def test_fused_backward_workspace_covers_every_partial(B, T, H, W):
    """hlm_attn_bwd_fused_workspace_bytes: one bf16 (B, H, T, 64) plane per
    128-key tile that a row can meet -- W = 512 gives 5, plain causal T / 128."""
    lib = _lib.load()
    R = _partials_per_row_bound(T, W)
    assert lib.hlm_attn_bwd_fused_workspace_bytes(B, T, H, 64, W) == R * B * H * T * 64 * 2
    if (T, W) == (2048, 512):
        assert R == 5
    if W == 0:
        assert R == (T + 127) // 128


def test_fused_backward_validates_before_touching_the_device():
    lib = _lib.load()
    s = _strides(2048, 128, 64)
    p = ctypes.c_void_p(0x1000)
    fn = lib.hlm_attn_bwd_fused
    need = lib.hlm_attn_bwd_fused_workspace_bytes(1, 16, 2, 64, 0)
    assert need == 1 * 1 * 2 * 16 * 64 * 2
    # head dim 128: not implemented by the single pass
    rc = fn(p, p, p, p, p, p, p, p, p, p, p, 1 << 30, 1, 16, 2, 2, 128, s, s, s, s, s, s, s, s, 0, 0.125, None)
    assert rc == -2 and b"head_dim 64 only" in lib.hlm_attn_last_error()
    assert lib.hlm_attn_bwd_fused_workspace_bytes(1, 16, 2, 128, 0) == -2
    # a workspace one byte short, or none
    rc = fn(p, p, p, p, p, p, p, p, p, p, p, need - 1, 1, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None)
    assert rc == -1 and b"needed" in lib.hlm_attn_last_error()
    rc = fn(p, p, p, p, p, p, p, p, p, p, None, need, 1, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None)
    assert rc == -1 and b"partial workspace" in lib.hlm_attn_last_error()
    # the shared argument checks of hlm_attn_bwd come first
    rc = fn(p, p, p, p, p, None, p, p, p, p, p, need, 1, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None)
    assert rc == -1 and b"lse" in lib.hlm_attn_last_error()
    assert fn(p, p, p, p, p, p, p, p, p, p, None, 0, 0, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None) == 0


def test_fused_backward_switch_is_off_by_default(monkeypatch):
    monkeypatch.delenv("HLM_ATTN_BWD", raising=False)
    assert not ops.fused_backward_selected()
    monkeypatch.setenv("HLM_ATTN_BWD", "Fused")
    assert ops.fused_backward_selected()
    monkeypatch.setenv("HLM_ATTN_BWD", "two-kernel")
    assert not ops.fused_backward_selected()


def test_noalloc_backward_validates_and_bounds_its_scratch_before_touching_the_device():
    """hlm_attn_bwd_noalloc: argument errors like hlm_attn_bwd's, and problems
    beyond its fixed scratch (B * H * T > 4,194,304 query rows) rejected with
    a message, all before any device call."""
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    s = _strides(2048, 128, 64)
    fn = lib.hlm_attn_bwd_noalloc
    assert fn(p, p, p, p, p, p, p, p, p, 1, 16, 2, 2, 64 + 8, s, s, s, s, s, s, s, s, 0, 0.125, None) == -2
    assert fn(p, p, p, p, p, None, p, p, p, 1, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None) == -1
    assert b"lse" in lib.hlm_attn_last_error()
    T, H = 65537, 64  # B * H * T = 4,194,368 rows, one row over
    big = _strides(T * H * 64, H * 64, 64)
    rc = fn(p, p, p, p, p, p, p, p, p, 1, T, H, H, 64, *([big] * 8), 0, 0.125, None)
    assert rc == -2 and b"exceeds its fixed scratch" in lib.hlm_attn_last_error()
    assert fn(p, p, p, p, p, p, p, p, p, 0, 16, 2, 2, 64, s, s, s, s, s, s, s, s, 0, 0.125, None) == 0


def test_split_forward_validates_and_its_policy_targets_small_grids():
    lib = _lib.load()
    s = _strides(2048, 128, 64)
    p = ctypes.c_void_p(0x1000)
    lse = ctypes.c_void_p(0x2000)

    def split(ws, nsplit, B=1):
        return lib.hlm_attn_fwd_split(p, p, p, p, lse, ws, nsplit, B, 16, 2, 2, 64, s, s, s, s, 0, 0.125, None)

    for nsplit in (0, 17):
        assert split(ctypes.c_void_p(0x3000), nsplit) == -1
        assert b"nsplit" in lib.hlm_attn_last_error()
    assert split(None, 2) == -1 and b"workspace" in lib.hlm_attn_last_error()
    assert split(ctypes.c_void_p(0x3008), 2) == -1
    assert split(None, 1, B=0) == 0 and split(ctypes.c_void_p(0x3000), 4, B=0) == 0
    # the policy: the training shape is a full grid; batch-1 evaluation calls split
    count = lib.hlm_attn_fwd_split_count
    assert count(8, 2048, 12, 64, 512) == 1
    assert count(1, 2048, 12, 64, 0) == 2  # 33 key tiles in the longest row
    assert count(1, 2048, 12, 64, 512) == 1 and count(1, 1024, 12, 64, 0) == 1  # rows too short to pay
    assert count(1, 8192, 1, 64, 0) == 10  # 129 key tiles; slots allow 12
    assert count(1, 16384, 1, 128, 0) == 4  # bounded by the 512 slots of D = 128
    assert count(1, 128, 12, 64, 0) == 1
    assert count(1, 2048, 12, 96, 0) == 1 and count(0, 2048, 12, 64, 0) == 1
    for B, T, H in ((1, 5000, 1), (1, 16384, 2), (2, 700, 3)):
        assert 1 <= count(B, T, H, 128, 0) <= 16


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.HipAttentionUnavailable, match="build it"):
        _lib.load(tmp_path / "libhlm_attn.so")


# --- torch custom ops --------------------------------------------------------------

def test_ops_refuse_cpu_tensors():
    q = torch.randn(1, 8, 2, 64).bfloat16()
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        ops.hip_attn_fwd(q, q, q, 0, 0.125)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        hlm_attn.attention(q.float(), q.float(), q.float())


def test_fake_implementations_describe_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 40, 8, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 40, 2, 64, dtype=torch.bfloat16)
        o, lse = ops.hip_attn_fwd(q, k, k, 16, 0.125)
        assert o.shape == q.shape and o.dtype == torch.bfloat16
        assert lse.shape == (2, 8, 40) and lse.dtype == torch.float32
        dq, dk, dv = ops.hip_attn_bwd(q, q, k, k, o, lse, 16, 0.125)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape


def test_kernel_ready_keeps_aligned_views_and_copies_the_rest():
    qkv = torch.randn(2, 10, 3 * 4 * 64).bfloat16()
    v = qkv[..., 2 * 256 :].view(2, 10, 4, 64)  # a fused-projection view, as model.py:92-99 makes
    assert ops._kernel_ready(v) is v
    t = torch.randn(2, 10, 4, 64).bfloat16().transpose(2, 3).contiguous().transpose(2, 3)
    assert t.stride(3) != 1 and ops._kernel_ready(t).is_contiguous()
    odd = torch.randn(2, 10, 4, 68).bfloat16()[..., :64]  # row stride 68: not a multiple of 8
    assert ops._kernel_ready(odd).is_contiguous()


# --- dispatch, with a fake op standing in for the kernels ----------------------------

class FakeOp:
    def __init__(self):
        self.calls = []

    def __call__(self, q, k, v, window, scale):
        self.calls.append((q.dtype, k.dtype, v.dtype, q.shape, k.shape, window, scale))
        B, T, H, D = q.shape
        return q.bfloat16(), torch.zeros(B, H, T)


@pytest.fixture()
def fake_op(monkeypatch):
    fake = FakeOp()
    monkeypatch.setattr(ops, "hip_attn_fwd", fake)  # the custom op (autograd / torch.compile)
    monkeypatch.setattr(ops, "attn_fwd_impl", fake)  # the direct inference path
    return fake


def test_direct_path_only_for_plain_inference_calls():
    """Calls skip the dispatcher only when nothing needs autograd or tracing."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    q = torch.randn(1, 4, 2, 64)
    assert ops.direct_call_ok(q, q, q)
    w = q.clone().requires_grad_(True)
    assert not ops.direct_call_ok(q, w, q)
    with torch.no_grad():
        assert ops.direct_call_ok(q, w, q)
    with torch.inference_mode():
        assert ops.direct_call_ok(q, q, q)
    with FakeTensorMode():
        f = torch.empty(1, 4, 2, 64)
        assert not ops.direct_call_ok(f, f, f)


def test_sdpa_casts_to_bf16_and_maps_window(fake_op):
    """The hip branch mirrors the FA2 branch (kernels.py:836-841): bf16 inputs,
    causal, window W means keys i-W+1..i (FA's (W-1, 0)), bf16 output, GQA k."""
    q = torch.randn(2, 4, 3, 64)
    k = torch.randn(2, 4, 1, 64)
    out = kernels.scaled_dot_product_attention(q, k, k, dropout_p=0.0, is_causal=True, window_size=3, backend="hip")
    assert out.dtype == torch.bfloat16
    assert fake_op.calls == [(torch.bfloat16, torch.bfloat16, torch.bfloat16, q.shape, k.shape, 3, 64**-0.5)]
    kernels.scaled_dot_product_attention(q, k, k, dropout_p=0.0, window_size=None, backend="hip")
    assert fake_op.calls[-1][5] == 0  # no window -> plain causal


@pytest.mark.parametrize(
    "kwargs,match",
    [
        (dict(dropout_p=0.1), "dropout"),
        (dict(attn_mask=torch.ones(4, 4, dtype=torch.bool)), "explicit attention mask"),
        (dict(block_mask=object()), "explicit attention mask"),
        (dict(is_causal=False), "causal attention only"),
        (dict(backend="flash_attn_2"), "implements only"),
    ],
)
def test_sdpa_rejects_what_the_kernels_do_not_do(fake_op, kwargs, match):
    q = torch.randn(1, 4, 2, 64)
    args = dict(dropout_p=0.0)
    args.update(kwargs)
    with pytest.raises(RuntimeError, match=match):
        kernels.scaled_dot_product_attention(q, q, q, **args)
    assert fake_op.calls == []


def test_attention_core_uses_layer_pattern(fake_op):
    cfg = model.AttentionConfig(n_layer=8, n_head=2, n_kv_head=2, attention_window=4, attention_full_every=4)
    cores = [model.AttentionCore(cfg, i) for i in range(8)]
    assert [c.attention_window for c in cores] == [4, 4, 4, None, 4, 4, 4, None]
    q = torch.randn(1, 8, 2, 64)
    # CPU tensors take the torch math (model.py:170), so the hip method is called directly here
    out = cores[0].fwd_hip(q, q, q)
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    assert fake_op.calls[-1][5] == 4
    cores[3].fwd_hip(q, q, q)
    assert fake_op.calls[-1][5] == 0
    # W >= T is plain causal (model.py:155-159)
    cores[0].fwd_hip(q[:, :4], q[:, :4], q[:, :4])
    assert fake_op.calls[-1][5] == 0
    cores[0].train()
    cores[0].dropout = 0.1
    with pytest.raises(RuntimeError, match="dropout"):
        cores[0].fwd_hip(q, q, q)


def test_attention_core_rejects_unknown_backend():
    cfg = model.AttentionConfig(n_layer=2, n_head=2, n_kv_head=2, attention_backend="sdpa")
    core = model.AttentionCore(cfg, 0)
    with pytest.raises(ValueError, match="unknown attention_backend"):
        core(torch.zeros(1, 4, 2, 64), torch.zeros(1, 4, 2, 64), torch.zeros(1, 4, 2, 64))
    # a known backend this library does not carry; meta tensors are not routed to the CPU math
    cfg2 = model.AttentionConfig(n_layer=2, n_head=2, n_kv_head=2, attention_backend="flash_attn_2")
    meta = torch.zeros(1, 4, 2, 64, device="meta")
    with pytest.raises(RuntimeError, match="does not support backend"):
        model.AttentionCore(cfg2, 0)(meta, meta, meta)


@pytest.mark.parametrize("backend", ["hip", "torch", "flash_attn_2"])
def test_attention_core_routes_cpu_tensors_to_the_torch_math(fake_op, backend):
    """model.py:169-196: CPU tensors take fwd_torch whatever the configured
    backend; every layer of the 8-layer pattern, with GQA, in fp32 and bf16,
    matches the oracle's restatement of that path (pinned by test_oracle
    against the reference's closed-form test and brute force) and the
    fp64 brute-force loops; the HIP op is never called."""
    cfg = model.AttentionConfig(n_layer=8, n_head=4, n_kv_head=2, attention_window=5,
                                attention_full_every=4, attention_backend=backend)
    gen = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(2, 9, h, 16, generator=gen) for h in (4, 2, 2))
    for layer in (0, 3, 7):
        core = model.AttentionCore(cfg, layer).eval()
        window = None if layer in (3, 7) else 5
        out = core(q, k, v)
        assert out.shape == q.shape and out.dtype == torch.float32
        assert torch.equal(out, oracle.attention_core_torch(q, k, v, window))
        brute, _ = oracle.brute_force_forward(q.double().numpy(), k.double().numpy(), v.double().numpy(), window)
        assert torch.allclose(out.double(), torch.from_numpy(brute), atol=1e-5)
        ob = core(q.bfloat16(), k.bfloat16(), v.bfloat16())
        assert ob.dtype == torch.bfloat16
        assert torch.equal(ob, oracle.attention_core_torch(q.bfloat16(), k.bfloat16(), v.bfloat16(), window))
    assert fake_op.calls == []


def test_attention_core_torch_path_mask_cache_and_dropout():
    """The window mask is built once per sequence length (model.py:141-151);
    training-mode dropout is applied to the probabilities (kernels.py:798-799),
    so p = 1 zeroes the output, and eval mode applies none."""
    cfg = model.AttentionConfig(n_layer=4, n_head=2, n_kv_head=2, attention_window=3, attention_backend="torch")
    core = model.AttentionCore(cfg, 0)
    q = torch.randn(1, 7, 2, 8)
    m1 = core._sliding_window_mask(7, q.device)
    assert core._sliding_window_mask(7, q.device) is m1
    assert torch.equal(m1[0, 0], oracle.sliding_window_mask(7, 3)[0, 0])
    assert core._sliding_window_mask(6, q.device).shape == (1, 1, 6, 6)
    assert core._sliding_window_mask(3, q.device) is None  # W >= T: plain causal
    core.dropout = 1.0
    core.train()
    assert torch.equal(core(q, q, q), torch.zeros_like(q))
    core.eval()
    assert torch.equal(core(q, q, q), oracle.attention_core_torch(q, q, q, 3))


def test_sdpa_torch_branch_matches_reference_closed_form_test(fake_op):
    """kernels.py:785-800 through the dispatcher, on the reference's
    tests/test_kernels.py:97-130 case (B2 H3 T5, Dqk=7, Dv=9, causal and
    distance < 3, (B, H, T, D)) against softmax(QK^T/sqrt(d) masked) V; an
    additive float mask of 0 / -inf gives the same result as the bool mask."""
    gen = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(2, 3, 5, d, generator=gen, dtype=torch.float64) for d in (7, 7, 9))
    lag = torch.arange(5)[:, None] - torch.arange(5)[None, :]
    mask = ((lag >= 0) & (lag < 3))[None, None]
    ref = torch.softmax((q @ k.transpose(-2, -1) / math.sqrt(7)).masked_fill(~mask, float("-inf")), dim=-1) @ v
    out = kernels.scaled_dot_product_attention(q.float(), k.float(), v.float(), 0.0, is_causal=False,
                                               attn_mask=mask, backend="torch")
    assert torch.allclose(out.double(), ref, atol=1e-6)  # the reference test's own tolerance
    additive = torch.zeros(5, 5).masked_fill(~mask[0, 0], float("-inf"))
    out_add = kernels.scaled_dot_product_attention(q.float(), k.float(), v.float(), 0.0, is_causal=True,
                                                   attn_mask=additive, backend="torch")
    assert torch.equal(out_add, out)
    assert fake_op.calls == []


# --- config mirror -----------------------------------------------------------------

def test_backend_names_extend_the_reference_set():
    assert config.REFERENCE_ATTENTION_BACKENDS == {"torch", "flex_attention", "flash_attn_2", "flash_attn_3", "flash_attn_4"}
    assert config.ATTENTION_BACKENDS == config.REFERENCE_ATTENTION_BACKENDS | {"hip"}
    assert config.normalize_attention_backend("HIP") == "hip"
    for bad in ("sdpa", 3, None):
        with pytest.raises(ValueError, match="unknown attention_backend"):
            config.normalize_attention_backend(bad)


def test_layer_pattern_matches_oracle_restatement():
    assert [config.layer_attention_window(i, 8, 512, 4) for i in range(8)] == [512, 512, 512, None, 512, 512, 512, None]
    assert [config.layer_attention_window(i, 3, 512, 4) for i in range(3)] == [512, 512, None]
    for n in range(1, 20):
        for w in (None, 64, 512):
            for every in (None, 1, 3, 4):
                assert [config.layer_attention_window(i, n, w, every) for i in range(n)] == [
                    oracle.layer_attention_window(i, n, w, every) for i in range(n)
                ]
    assert config.normalize_attention_window(0) is None and config.normalize_attention_window(512) == 512
    assert config.normalize_attention_full_every(0) is None and config.normalize_attention_full_every(4) == 4
    for T in (1, 7, 8, 9):
        assert config.attention_window_size(8, T) == oracle.window_size_at(8, T)


def test_resolution_follows_the_reference_rules(monkeypatch):
    """kernels.py:177-181 and :221-228: raise when the fast backend is
    unusable, or fall back to the host's torch backend when allowed."""
    monkeypatch.setattr(kernels, "hip_attention_available", lambda: False)
    with pytest.raises(RuntimeError, match="attention_backend=hip"):
        kernels.resolve_attention_backend("hip")
    assert kernels.resolve_attention_backend("hip", allow_torch_backend=True) == "torch"
    assert kernels.resolve_attention_backend("flash_attn_2") == "flash_attn_2"
    monkeypatch.setattr(kernels, "hip_attention_available", lambda: True)
    assert kernels.resolve_attention_backend("HIP") == "hip"
    with pytest.raises(ValueError):
        kernels.resolve_attention_backend("sdpa")


class _FakePycall:
    """Stands in for the CPython binding: records the forward's arguments."""

    def __init__(self):
        self.calls = []

    def fwd(self, *args):
        self.calls.append(args)
        return 0


@pytest.mark.parametrize("how", ["env", "import"])
def test_forward_falls_back_to_the_c_abi_without_the_torch_extension(monkeypatch, how):
    """The torch extension is an optional host fast path: when it is disabled
    (HLM_ATTN_TORCH_EXT=0) or its import fails (missing, or built against
    another torch), torch_fwd() is None, the failure is cached, and
    attn_fwd_impl launches through the CPython binding of the C ABI with the
    same arguments."""
    import sys

    monkeypatch.setattr(_lib, "_torch_fwd", None)
    if how == "env":
        monkeypatch.setenv("HLM_ATTN_TORCH_EXT", "0")
    else:
        monkeypatch.delenv("HLM_ATTN_TORCH_EXT", raising=False)
        monkeypatch.setitem(sys.modules, "hlm_attn._torch_fwd", None)  # the import raises ImportError
        monkeypatch.delattr(hlm_attn, "_torch_fwd", raising=False)  # (an earlier import left the attribute)
    assert _lib.torch_fwd() is None
    assert _lib._torch_fwd is False  # remembered: no second import attempt
    with pytest.raises(_lib.HipAttentionUnavailable, match="torch extension"):
        _lib.load_torch_fwd()

    pc = _FakePycall()
    monkeypatch.setattr(_lib, "_pycall", pc)
    monkeypatch.setattr(ops, "_check_inputs", lambda q, k, v: None)
    monkeypatch.setattr(ops, "_on_index", lambda i: __import__("contextlib").nullcontext())
    monkeypatch.setattr(ops, "_raw_stream_of", lambda i: 1234)
    B, T, H, D = 2, 64, 4, 64
    q = torch.zeros(B, T, H, D, dtype=torch.bfloat16)
    k = torch.zeros(B, T, 2, D, dtype=torch.bfloat16)
    o, lse = ops.attn_fwd_impl(q, k, k, 16, 0.125)
    assert o.shape == (B, T, H, D) and o.dtype == torch.bfloat16
    assert lse.shape == (B, H, T) and lse.dtype == torch.float32
    assert len(pc.calls) == 1
    args = pc.calls[0]
    assert args[:5] == (q.data_ptr(), k.data_ptr(), k.data_ptr(), o.data_ptr(), lse.data_ptr())
    assert args[6:12] == (1, B, T, H, 2, D)  # nsplit, shape
    assert args[-3:] == (16, 0.125, 1234)  # window, scale, stream


def test_hip_availability_requires_every_module_the_forward_needs(monkeypatch):
    """hip_attention_available() loads the library and its CPython binding
    (both needed by every call); a missing binding makes the backend
    unavailable (so resolve_attention_backend can fall back) instead of
    failing at the first forward.  The torch extension is not required."""
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.version, "hip", "7.0")
    monkeypatch.setattr(_lib, "_torch_fwd", False)
    assert kernels.hip_attention_available()

    def missing():
        raise _lib.HipAttentionUnavailable("no binding")

    monkeypatch.setattr(_lib, "load_pycall", missing)
    assert not kernels.hip_attention_available()
    assert kernels.resolve_attention_backend("hip", allow_torch_backend=True) == "torch"


def test_flop_model_matches_bench():
    import bench

    for T, W in [(2048, 512), (2048, None), (4096, 1024), (16384, 2048), (1024, 256)]:
        assert bench.pairs(T, W) == oracle.causal_window_pairs(T, W)
    f = bench.effective_flops(bench.CONFIGS["cfg2_local"])
    assert round(f["fwd"] / 1e9, 3) == 22.555 and round(f["bwd"] / 1e9, 3) == 45.110
    assert f["bwd_dq"] + f["bwd_dkdv"] == f["bwd"]
    assert math.isclose(bench.PEAK_BF16_TFLOPS, 256 * 4096 * 2.4e9 / 1e12, rel_tol=1e-4)


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}), ([], {"WORLD_SIZE": "2"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    """`bench.py --gpus N` (or a launcher's WORLD_SIZE) with N > 1 exits with a
    message before touching a device: this build measures one GPU."""
    import os
    import subprocess
    import sys

    root = Path(__file__).resolve().parent.parent
    proc = subprocess.run([sys.executable, str(root / "bench.py"), *argv], capture_output=True, text=True,
                          env={**os.environ, **env}, timeout=120, cwd=root)
    assert proc.returncode == 2
    assert "measures one GPU" in proc.stderr
    assert proc.stdout == ""


def test_bench_config_synthesis():
    """cfg5's inputs: bench's fp32 RoPE equals the oracle's rotate-half
    restatement (model.py:105-114 at base 10000, fraction 1.0) on the same
    values; the cfg4 stack takes the reference's layer pattern, and its
    effective work matches the 18-layer total of 6.611 TFLOP."""
    import bench
    from oracle import qk_norm_rope as rope_oracle

    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 300, 3, 128, generator=g)
    cos, sin = rope_oracle.rotary_tables(300, 128, theta=10000.0, fraction=1.0)
    want = rope_oracle.apply_partial_rope(x, cos[None, :, None, :], sin[None, :, None, :])
    assert torch.allclose(bench.rope_rotate(x), want, atol=2e-5, rtol=1e-5)
    assert torch.equal(bench.rope_rotate(x)[:, 0], x[:, 0])  # position 0 is not rotated
    from hlm_attn.config import layer_attention_window

    n, w, every = (bench.CFG4_LAYERS[k] for k in ("n_layer", "window", "full_every"))
    full = [l for l in range(n) if layer_attention_window(l, n, w, every) is None]
    assert full == [3, 7, 11, 15, 17]
    base = bench.CONFIGS["cfg4_local"]
    total = 0
    for l in range(n):
        f = bench.effective_flops(dict(base, W=layer_attention_window(l, n, w, every)))
        total += f["fwd"] + f["bwd"]
    assert round(total / 1e12, 3) == 6.611


# --- q/k RMSNorm + partial RoPE producer --------------------------------------------

def _qk(lib, backward=False, ptr=0x1000, B=1, T=16, H=2, Hkv=2, D=64, rot=16, strides=(2048, 128, 64), eps=1e-6,
        table=0x3000, table_dtype=_lib.TABLE_BF16):
    s = _strides(*strides)
    p = ctypes.c_void_p(ptr) if ptr else None
    t = ctypes.c_void_p(table) if table else None
    out = ctypes.c_void_p(0x2000)
    if backward:
        return lib.hlm_qk_norm_rope_bwd(p, p, out, out, t, t, table_dtype, out, out, B, T, H, Hkv, D, rot, s, s, eps,
                                        None)
    return lib.hlm_qk_norm_rope_fwd(p, p, t, t, table_dtype, out, out, B, T, H, Hkv, D, rot, s, s, eps, None)


@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize(
    "kwargs,code,msg",
    [
        (dict(D=32), -2, "head_dim 32"),
        (dict(rot=8), -2, "rotary_dim 8"),
        (dict(rot=80), -2, "rotary_dim 80"),
        (dict(rot=-16), -2, "rotary_dim -16"),
        (dict(H=0), -1, "bad shape"),
        (dict(eps=0.0), -1, "eps"),
        (dict(eps=float("inf")), -1, "eps"),
        (dict(ptr=None), -1, "null pointer"),
        (dict(ptr=0x1008), -1, "16-byte aligned"),
        (dict(strides=(2048, 100, 64)), -1, "multiple of 8"),
        (dict(table=None), -1, "cos / sin"),
        (dict(table=0x3004), -1, "cos / sin"),
        (dict(table_dtype=2), -1, "table_dtype 2"),
    ],
)
def test_qk_norm_rope_rejects_bad_arguments_before_touching_the_device(backward, kwargs, code, msg):
    lib = _lib.load()
    assert _qk(lib, backward, **kwargs) == code
    assert msg in lib.hlm_attn_last_error().decode()


def test_qk_norm_rope_empty_problems_are_no_ops():
    lib = _lib.load()
    for backward in (False, True):
        assert _qk(lib, backward, B=0) == 0
        assert _qk(lib, backward, T=0) == 0
        assert lib.hlm_attn_last_error() == b""
    # R = 0 needs no tables (plain RMSNorm): validation passes without them
    assert _qk(lib, B=0, rot=0, table=None) == 0


def test_qk_norm_rope_refuses_cpu_tensors_and_describes_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    q = torch.randn(1, 8, 2, 64).bfloat16()
    cos = torch.zeros(8, 16)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        hlm_attn.qk_norm_rope_hip(q, q, cos, cos, 1e-6)
    with FakeTensorMode():
        q = torch.empty(2, 40, 8, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 40, 2, 64, dtype=torch.bfloat16)
        c = torch.empty(1, 40, 1, 16)
        qo_, ko_ = ops.hip_qk_norm_rope(q, k, c, c, 1e-6)
        assert qo_.shape == q.shape and ko_.shape == k.shape and qo_.dtype == torch.bfloat16
        dq, dk = ops.hip_qk_norm_rope_backward(q, k, q, k, c, c, 1e-6)
        assert dq.shape == q.shape and dk.shape == k.shape


def test_rope_table_accepts_the_reference_layouts():
    t = torch.arange(12.0).reshape(3, 4)
    for view in (t, t[None, :, None, :], t[None, None], t[None, None].transpose(1, 2)):
        got, code = ops._rope_table(view, 3)
        assert got.shape == (3, 4) and got.is_contiguous() and torch.equal(got, t) and code == _lib.TABLE_F32
    # bf16 tables (the model's) are passed as they are; other types become fp32
    got, code = ops._rope_table(t.bfloat16()[None, None], 3)
    assert got.dtype == torch.bfloat16 and code == _lib.TABLE_BF16
    got, code = ops._rope_table(t.half(), 3)
    assert got.dtype == torch.float32 and code == _lib.TABLE_F32
    # a prefix of a longer cached table (RotaryEmbedding slices its cache)
    cache = torch.arange(40.0).reshape(1, 1, 10, 4)
    got, _ = ops._rope_table(cache[:, :, :3].transpose(1, 2), 3)
    assert torch.equal(got, cache[0, 0, :3])
    with pytest.raises(RuntimeError, match="does not hold"):
        ops._rope_table(t, 4)


def test_rotary_embedding_matches_the_oracle_tables():
    from oracle import qk_norm_rope as qo

    for dim, fraction in ((64, 0.25), (128, 0.25), (64, 1.0), (10, 0.25)):
        rope = model.RotaryEmbedding(dim, fraction=fraction)
        cos, sin = rope(33, torch.device("cpu"), torch.float32)
        rc, rs = qo.rotary_tables(33, dim, fraction=fraction)
        assert cos.shape == (1, 1, 33, rope.rotary_dim)
        assert torch.equal(cos[0, 0], rc) and torch.equal(sin[0, 0], rs)
    # cached for the longest length seen; shorter calls slice it
    c5, _ = rope(5, torch.device("cpu"), torch.bfloat16)
    assert c5.dtype == torch.bfloat16 and torch.equal(c5[0, 0], qo.rotary_tables(5, 10)[0].bfloat16())


def test_qkv_projection_dispatches_on_qkv_backend():
    cfg = model.AttentionConfig(n_layer=1, n_head=2, n_kv_head=1, n_embd=32, head_dim=64)
    proj = model.QKVProjection(cfg, 0)
    assert proj.qkv_proj.weight.shape == ((2 + 2) * 64, 32)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        proj.to(torch.bfloat16)(torch.randn(1, 4, 32).bfloat16())
    for backend, exc, match in (("triton", RuntimeError, "does not support backend"),
                                ("cuda", ValueError, "unknown qkv_backend")):
        cfg_b = model.AttentionConfig(n_layer=1, n_head=2, n_kv_head=1, n_embd=32, head_dim=64, qkv_backend=backend)
        with pytest.raises(exc, match=match):
            model.QKVProjection(cfg_b, 0)(torch.randn(1, 4, 32))
    assert config.MODULE_BACKENDS == {"torch", "triton", "hip"}
    assert config.normalize_module_backend("qkv_backend", "HIP") == "hip"


# --- LM head: cross-entropy rows -------------------------------------------------

def test_ce_rows_validates_before_touching_the_device():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)

    def ce(dtype=_lib.DTYPE_BF16, stride=64, rows=4, cols=64, n_tokens=4, logits=p, targets=p, loss=p):
        return lib.hlm_ce_rows(logits, dtype, stride, targets, loss, rows, cols, n_tokens, -100, None)

    for kwargs, msg in ((dict(dtype=3), b"logits_dtype"), (dict(stride=32), b"row_stride"),
                        (dict(cols=0), b"bad shape"), (dict(n_tokens=0), b"n_tokens"),
                        (dict(logits=None), b"null"), (dict(loss=None), b"null")):
        assert ce(**kwargs) == -1, kwargs
        assert msg in lib.hlm_attn_last_error(), kwargs
    assert ce(rows=0, logits=None) == 0


def test_linear_ce_chunk_size_follows_the_reference_rule():
    """kernels.py:893-903: a requested size is raised to 2048 and capped at
    n_tokens; otherwise next_pow2(ceil(n_tokens / ceil(V / hidden))), at least 2048."""
    size = kernels.linear_ce_chunk_size
    assert size(16384, 768, 32768, None) == 2048  # ceil(32768/768) = 43 -> next_pow2(382) = 512 -> raised to 2048
    assert size(1 << 20, 768, 32768, None) == 32768  # next_pow2(ceil(2^20 / 43)) = 32768
    assert size(1000, 768, 32768, None) == 1000
    assert size(16384, 768, 32768, 4096) == 4096 and size(16384, 768, 32768, 100) == 2048
    assert size(3000, 768, 32768, 4096) == 3000 and size(100, 64, 33, 0) == 100
    with pytest.raises(RuntimeError, match="nonnegative"):
        size(100, 64, 33, -1)


def test_fused_linear_ce_refuses_cpu_tensors_and_other_backends():
    h = torch.randn(4, 8)
    w = torch.randn(5, 8)
    t = torch.randint(0, 5, (4,))
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        kernels.fused_linear_cross_entropy_with_weight(h, w, None, t, backend="hip")
    with pytest.raises(RuntimeError, match="unsupported fused linear cross entropy backend"):
        kernels.fused_linear_cross_entropy_with_weight(h, w, None, t, backend="triton")
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        ops.hip_linear_ce(torch.randn(2, 8), torch.tensor([0, 1]), 2)
    cfg = model.AttentionConfig(n_layer=1, n_head=1, n_kv_head=1, n_embd=8, vocab_size=5, lm_head_backend="torch")
    with pytest.raises(RuntimeError, match="does not support backend"):
        model.LMHeadProjection(cfg)(h[None], t[None])


# --- residual add + RMSNorm -------------------------------------------------------

def test_residual_rms_norm_validates_before_touching_the_device():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    fwd = lib.hlm_residual_rms_norm_fwd
    bwd = lib.hlm_residual_rms_norm_bwd
    for n, code in ((12, -2), (8200, -2), (0, -1)):
        assert fwd(p, p, p, p, 4, n, 1e-6, None) == code
    assert fwd(p, p, p, p, 4, 64, 0.0, None) == -1 and b"eps" in lib.hlm_attn_last_error()
    assert fwd(p, ctypes.c_void_p(0x1008), p, p, 4, 64, 1e-6, None) == -1
    assert bwd(p, p, None, p, 4, 64, 1e-6, None) == -1
    assert fwd(p, p, p, p, 0, 64, 1e-6, None) == 0 and bwd(None, None, None, None, 0, 64, 1e-6, None) == 0


def test_residual_rms_norm_refuses_cpu_and_dispatches_on_backend_fields():
    x = torch.randn(1, 4, 64)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        hlm_attn.residual_rms_norm_hip(x, x, 1e-6)
    cfg = model.AttentionConfig(n_layer=1, n_head=1, n_kv_head=1, n_embd=64, head_dim=64, mlp_hidden=128,
                                output_backend="torch", down_backend="triton")
    with pytest.raises(RuntimeError, match="does not support backend"):
        model.OutputProjection(cfg)(torch.randn(1, 4, 1, 64), x)
    with pytest.raises(RuntimeError, match="does not support backend"):
        model.DownProjection(cfg)(torch.randn(1, 4, 128), x)
    with FakeTensorModeCtx():
        r = torch.empty(2, 5, 64, dtype=torch.bfloat16)
        out, normed = ops.hip_residual_rms_norm(r, r, 1e-6)
        assert out.shape == r.shape and normed.dtype == torch.bfloat16
        assert ops.hip_residual_rms_norm_backward(r, r, r, 1e-6).shape == r.shape


def FakeTensorModeCtx():
    from torch._subclasses.fake_tensor import FakeTensorMode

    return FakeTensorMode()


def test_other_head_dims_run_zero_padded(fake_op):
    """Dv != Dqk (the reference test's Dqk = 7, Dv = 9, tests/test_kernels.py:103-105)
    and head dims other than 64 / 128 reach the kernels zero-padded to 64 or
    128, with the scale of the true Dqk and the output sliced back to Dv."""
    q = torch.randn(1, 5, 2, 7)
    v = torch.randn(1, 5, 2, 9)
    out = kernels.attention(q, q, v)
    _, _, _, qs, ks, _, scale = fake_op.calls[-1]
    assert qs[-1] == 64 and ks[-1] == 64 and math.isclose(scale, 7 ** -0.5)
    assert out.shape == (1, 5, 2, 9)
    # the fake op echoes q, so the output columns are q's: padding kept q's
    # first 7 columns, zeros after
    assert torch.equal(out[..., :7], q.bfloat16()) and torch.count_nonzero(out[..., 7:]) == 0
    kernels.attention(torch.randn(1, 5, 2, 96), torch.randn(1, 5, 2, 96), torch.randn(1, 5, 2, 80))
    assert fake_op.calls[-1][3][-1] == 128
    assert kernels.padded_head_dim(64, 64) == 64 and kernels.padded_head_dim(65, 8) == 128
    with pytest.raises(RuntimeError, match="at most 128"):
        kernels.attention(torch.randn(1, 5, 2, 192), torch.randn(1, 5, 2, 192), torch.randn(1, 5, 2, 192))
    with pytest.raises(RuntimeError, match="differ"):
        kernels.attention(torch.randn(1, 5, 2, 64), torch.randn(1, 5, 2, 32), torch.randn(1, 5, 2, 64))


# --- host-side arithmetic shared with the kernels ----------------------------

def test_fast_division_matches_integer_division(tmp_path):
    """The producer splits its row index into (batch, time, head) by
    multiply-high division (attn_common.h: FastDiv); fastdiv_check.cpp runs
    that same code on the host against the compiler's integer division over
    184 M (dividend, divisor) pairs, range ends included."""
    import shutil
    import subprocess

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "fastdiv_check"
    src = REPO / "tests" / "fastdiv_check.cpp"
    subprocess.run([hipcc, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950", str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
