#!/usr/bin/env python3
"""Benchmark of the HIP causal sliding-window attention backend on one MI355X.

One "step" is one attention layer's forward + backward through the C ABI
(hlm_attn_fwd, then hlm_attn_bwd on the forward's o and lse) at the BASELINE
workload cfg2: B=8, H=12, T=2048, D=64, window=512, causal, bf16, synthetic
N(0,1) inputs from one seed, resident in HBM before timing starts.  Warm
cache: steps run back to back, as in training.

Prints ONE JSON line: value = effective fwd+bwd TFLOP/s, where effective FLOPs
count only unmasked (query, key) pairs P(T, W): fwd 4*D*P, bwd 8*D*P per
(batch, head).  Also reports ms per layer (fwd, bwd, fwd+bwd), the fraction of
MI355X's dense bf16 MFMA peak, a roofline object for the dominant kernel
(HIP-event timed on the launch stream) and the CPU baseline: the reference's
`torch` backend restated on the host CPU (configs[0] shape, fp32, forward).
A "producer" object times the q/k RMSNorm + partial RoPE kernels that feed
attention (forward and backward) at cfg2's q/k shape against the HBM roofline;
an "eval" object times the evaluation harness's no-grad forwards at batch 1
and ragged T; an "lm_head" object times the LM head's cross-entropy rows
and a "residual_norm" object the residual add + RMSNorm, both against the
HBM roofline.

Steps are eager launches by default (they run ahead of the GPU); --graph times
HIP-graph replays of one captured step instead (the way a training step runs
under torch.compile's CUDA-graph mode).  The default warmup (300 steps) lets
the GPU reach its steady clock before timing starts.

  python bench.py [--steps K] [--warmup W] [--config NAME] [--sweep] [--no-cpu-baseline] [--graph]
                  [--no-producer] [--no-eval] [--no-lm-head]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "hackable-lm_amd"))

METRIC = "attention fwd+bwd effective TFLOPS & % bf16 MFMA peak; ms/layer at T=2048"
# MI355X dense bf16 MFMA peak: 256 CU x 4096 FLOP/clk x 2.4 GHz.
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    "cfg2_local": dict(B=8, T=2048, H=12, D=64, W=512),
    "cfg3_full": dict(B=8, T=2048, H=12, D=64, W=None),
    "cfg4_local": dict(B=4, T=4096, H=12, D=128, W=1024),
    "cfg4_full": dict(B=4, T=4096, H=12, D=128, W=None),
    "cfg5_long": dict(B=1, T=16384, H=16, D=128, W=2048),
}
CPU_CONFIG = dict(B=2, T=1024, H=6, D=64, W=256)
KERNEL_NAMES = {"fwd": "attn_fwd_kernel", "bwd_dq": "attn_bwd_dq_kernel", "bwd_dkdv": "attn_bwd_dkdv_kernel"}


def pairs(T: int, W: int | None) -> int:
    """Unmasked (query, key) pairs per (batch, head): W(W+1)/2 + (T-W)W, or T(T+1)/2."""
    if W is None or W >= T:
        return T * (T + 1) // 2
    return W * (W + 1) // 2 + (T - W) * W


def effective_flops(cfg: dict) -> dict:
    p = pairs(cfg["T"], cfg["W"]) * cfg["B"] * cfg["H"]
    d = cfg["D"]
    return {"fwd": 4 * d * p, "bwd": 8 * d * p, "bwd_dq": 2 * d * p, "bwd_dkdv": 6 * d * p}


def algorithmic_bytes(cfg: dict) -> dict:
    """Compulsory HBM bytes per launch (bf16 tensors, fp32 lse/delta)."""
    n = cfg["B"] * cfg["H"] * cfg["T"]
    d = cfg["D"]
    return {
        "fwd": 8 * n * d + 4 * n,               # q, k, v read; o written; lse written
        "bwd_dq": 12 * n * d + 12 * n,          # q, k, v, o, dO read; dq written; lse read; -lse*log2(e), -delta written
        "bwd_dkdv": 12 * n * d + 8 * n,         # q, k, v, dO read; dk, dv written; -lse*log2(e), -delta read
    }


class Problem:
    """Device buffers and C-ABI launches for one configuration."""

    def __init__(self, cfg: dict, seed: int, device):
        import torch
        from hlm_attn import _lib

        self.torch = torch
        self.lib = _lib.load()
        self.cfg = cfg
        B, T, H, D = cfg["B"], cfg["T"], cfg["H"], cfg["D"]
        g = torch.Generator(device="cpu").manual_seed(seed)
        mk = lambda: torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(device)  # noqa: E731
        self.q, self.k, self.v, self.do = mk(), mk(), mk(), mk()
        self.o = torch.empty_like(self.q)
        self.dq, self.dk, self.dv = (torch.empty_like(self.q) for _ in range(3))
        self.lse = torch.empty(B, H, T, dtype=torch.float32, device=device)
        self.delta = torch.empty(2, B, H, T, dtype=torch.float32, device=device)  # -lse*log2(e), -delta
        st = _lib.strides3
        self.s = {n: st(getattr(self, n)) for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv")}
        self.window = 0 if cfg["W"] is None else cfg["W"]
        self.scale = 1.0 / math.sqrt(D)
        self.device = device
        self.dims = (B, T, H, H, D)

    @property
    def stream(self):
        # torch's current stream at call time (a capture stream inside graph capture)
        return ctypes.c_void_p(self.torch.cuda.current_stream(self.device).cuda_stream)

    def fwd(self):
        rc = self.lib.hlm_attn_fwd(
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.o.data_ptr(), self.lse.data_ptr(),
            *self.dims, self.s["q"], self.s["k"], self.s["v"], self.s["o"], self.window, self.scale, self.stream,
        )
        assert rc == 0, self.lib.hlm_attn_last_error()

    def _bwd(self, fn):
        rc = fn(
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.o.data_ptr(), self.do.data_ptr(),
            self.lse.data_ptr(), self.dq.data_ptr(), self.dk.data_ptr(), self.dv.data_ptr(), self.delta.data_ptr(),
            *self.dims, self.s["q"], self.s["k"], self.s["v"], self.s["o"], self.s["do"], self.s["dq"],
            self.s["dk"], self.s["dv"], self.window, self.scale, self.stream,
        )
        assert rc == 0, self.lib.hlm_attn_last_error()

    def bwd(self):
        self._bwd(self.lib.hlm_attn_bwd)

    def bwd_dq(self):
        self._bwd(self.lib.hlm_attn_bwd_dq)

    def bwd_dkdv(self):
        self._bwd(self.lib.hlm_attn_bwd_dkdv)

    def step(self):
        self.fwd()
        self.bwd()


PRODUCER_CONFIG = dict(B=8, T=2048, H=12, Hkv=12, D=64, R=16)  # cfg2's q/k, model.py's R = D / 4
PRODUCER_SETS = 4  # buffer sets rotated per launch: 4 x 176 MB exceeds the 256 MB last-level cache


def producer_bytes(cfg: dict) -> dict:
    """Compulsory HBM bytes per launch of the q/k RMSNorm + RoPE producer:
    forward reads q, k and the bf16 cos / sin tables and writes q, k (bf16);
    backward also reads the two incoming gradients."""
    n = cfg["B"] * cfg["T"] * (cfg["H"] + cfg["Hkv"]) * cfg["D"] * 2  # one bf16 pass over q and k
    tables = 2 * cfg["T"] * cfg["R"] * 2
    return {"fwd": 2 * n + tables, "bwd": 3 * n + tables}


class ProducerProblem:
    """q / k as strided views of fused (B, T, (H + 2 Hkv) D) projections, as
    model.py:92-99 makes them, fp32 (T, R) tables, and preallocated outputs;
    PRODUCER_SETS independent sets so that consecutive launches touch
    different memory."""

    def __init__(self, cfg: dict, seed: int, device, sets: int = PRODUCER_SETS):
        import torch
        from hlm_attn import _lib

        self.torch, self.lib, self.cfg, self.device = torch, _lib.load(), cfg, device
        B, T, H, Hkv, D, R = (cfg[k] for k in ("B", "T", "H", "Hkv", "D", "R"))
        g = torch.Generator(device="cpu").manual_seed(seed)
        # bf16 tables, as RotaryEmbedding hands them to the producer (model.py:62-70)
        ang = torch.rand(T, R // 2, generator=g) * 6.0
        self.cos = torch.cat((ang.cos(), ang.cos()), -1).to(torch.bfloat16).to(device)
        self.sin = torch.cat((ang.sin(), ang.sin()), -1).to(torch.bfloat16).to(device)
        self.table_dtype = _lib.TABLE_BF16
        self.sets = []
        for _ in range(sets):
            qkv = torch.randn(B, T, (H + 2 * Hkv) * D, generator=g).to(torch.bfloat16).to(device)
            q = qkv[..., : H * D].view(B, T, H, D)
            k = qkv[..., H * D : (H + Hkv) * D].view(B, T, Hkv, D)
            gq = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(device)
            gk = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16).to(device)
            out = (torch.empty_like(gq), torch.empty_like(gk))
            self.sets.append((qkv, q, k, gq, gk, out, _lib.strides3(q), _lib.strides3(k)))
        self.i = 0
        self.dims = (B, T, H, Hkv, D, R)

    def _next(self):
        st = self.sets[self.i]
        self.i = (self.i + 1) % len(self.sets)
        return st

    def fwd(self):
        _, q, k, _, _, (oq, ok), sq, sk = self._next()
        stream = ctypes.c_void_p(self.torch.cuda.current_stream(self.device).cuda_stream)
        rc = self.lib.hlm_qk_norm_rope_fwd(
            q.data_ptr(), k.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(), self.table_dtype,
            oq.data_ptr(), ok.data_ptr(),
            *self.dims, sq, sk, 1e-6, stream,
        )
        assert rc == 0, self.lib.hlm_attn_last_error()

    def bwd(self):
        _, q, k, gq, gk, (dq, dk), sq, sk = self._next()
        stream = ctypes.c_void_p(self.torch.cuda.current_stream(self.device).cuda_stream)
        rc = self.lib.hlm_qk_norm_rope_bwd(
            q.data_ptr(), k.data_ptr(), gq.data_ptr(), gk.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
            self.table_dtype, dq.data_ptr(), dk.data_ptr(), *self.dims, sq, sk, 1e-6, stream,
        )
        assert rc == 0, self.lib.hlm_attn_last_error()


def measure_producer(reps: int, warmup: int, device) -> dict:
    """HIP-event launch times of the producer's forward and backward kernels,
    against the HBM roofline.  Launches rotate over buffer sets larger than the
    last-level cache, so each launch's inputs were last touched three launches
    earlier and come from HBM."""
    import torch

    cfg = PRODUCER_CONFIG
    prob = ProducerProblem(cfg, seed=0, device=device)
    by = producer_bytes(cfg)
    out = {
        "op": "q/k RMSNorm + partial RoPE producer (kernels.py:441-658, model.py:101-126)",
        "workload": f"B={cfg['B']} T={cfg['T']} H=Hkv={cfg['H']} D={cfg['D']} R={cfg['R']}, q/k strided views "
        f"of a fused projection, bf16, bf16 tables",
        "bound": "hbm",
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
    }
    for name, fn in (("fwd", prob.fwd), ("bwd", prob.bwd)):
        for _ in range(warmup):
            fn()
        cold = event_time_ms(torch, fn, reps)
        achieved = by[name] / (cold * 1e-3) / 1e9
        kernel = f"qk_norm_rope_kernel<{cfg['D']}, {'true' if name == 'bwd' else 'false'}, bf16 tables>"
        out[name] = {
            "kernel": kernel,
            "launch_us": round(cold * 1e3, 2),
            "algorithmic_bytes_per_launch": by[name],
            "achieved": round(achieved, 1),
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": read_traffic("producer_cfg2", f"qk_norm_rope_{name}"),
        }
    return out


LM_HEAD_CONFIG = dict(rows=4096, V=32768)  # loss_chunk_size 4096 (config.py:49), the Triton kernel's largest V


def measure_lm_head(reps: int, warmup: int, device) -> dict:
    """HIP-event launch time of the LM head's cross-entropy rows (hlm_ce_rows)
    on one chunk of bf16 logits, against the HBM roofline: 2 * rows * V * 2
    bytes (each logit read once, its gradient written once) plus the targets
    and losses.  Launches alternate between two chunks (537 MB together,
    beyond the 256 MB last-level cache), so the logits come from HBM."""
    import torch

    from hlm_attn import _lib

    lib = _lib.load()
    rows, V = LM_HEAD_CONFIG["rows"], LM_HEAD_CONFIG["V"]
    g = torch.Generator(device="cpu").manual_seed(0)
    bufs = [(torch.randn(rows, V, generator=g) * 3).to(torch.bfloat16).to(device) for _ in range(2)]
    targets = torch.randint(0, V, (rows,), generator=g).to(device)
    loss = torch.empty(rows, dtype=torch.float32, device=device)
    it = [0]

    def launch():
        buf = bufs[it[0]]
        it[0] ^= 1
        rc = lib.hlm_ce_rows(buf.data_ptr(), _lib.DTYPE_BF16, V, targets.data_ptr(), loss.data_ptr(), rows, V,
                             rows, -100, ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
        assert rc == 0, lib.hlm_attn_last_error()

    for _ in range(warmup):
        launch()
    ms = event_time_ms(torch, launch, reps)
    nbytes = 2 * rows * V * 2 + rows * 12
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {
        "op": "LM-head cross-entropy rows, in place (kernels.py:286-336 inside :878-959)",
        "workload": f"rows={rows} V={V} bf16 logits (one loss chunk), random targets",
        "kernel": "ce_rows_vec_kernel<bf16, 16>",
        "bound": "hbm",
        "launch_us": round(ms * 1e3, 2),
        "algorithmic_bytes_per_launch": nbytes,
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": read_traffic("lm_head_ce", "ce_rows_vec_kernel"),
    }


RESNORM_CONFIG = dict(rows=8 * 2048, n=768)  # cfg2's tokens at n_embd = 12 heads x 64


def measure_residual_norm(reps: int, warmup: int, device) -> dict:
    """HIP-event launch times of the residual add + RMSNorm forward and
    backward (hlm_residual_rms_norm_fwd/_bwd) at cfg2's token count, against
    the HBM roofline: forward reads residual and branch and writes out and
    normed, backward reads out, grad_out and grad_normed and writes grad_in,
    each 2 * rows * n bytes.  Launches rotate over 4 buffer sets (800 MB)."""
    import torch

    from hlm_attn import _lib

    lib = _lib.load()
    rows, n = RESNORM_CONFIG["rows"], RESNORM_CONFIG["n"]
    g = torch.Generator(device="cpu").manual_seed(0)
    sets = [[torch.randn(rows, n, generator=g).to(torch.bfloat16).to(device) for _ in range(4)] for _ in range(4)]
    it = [0]

    def nxt():
        st = sets[it[0]]
        it[0] = (it[0] + 1) % len(sets)
        return st

    def stream():
        return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)

    def fwd():
        a, b, c, d = nxt()
        assert lib.hlm_residual_rms_norm_fwd(a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), rows, n,
                                             1e-6, stream()) == 0

    def bwd():
        a, b, c, d = nxt()
        assert lib.hlm_residual_rms_norm_bwd(a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), rows, n,
                                             1e-6, stream()) == 0

    out = {
        "op": "residual add + RMSNorm (model.py:73-75 in OutputProjection / DownProjection)",
        "workload": f"rows={rows} n={n} bf16",
        "bound": "hbm",
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
    }
    nbytes = 4 * rows * n * 2
    for name, fn in (("fwd", fwd), ("bwd", bwd)):
        for _ in range(warmup):
            fn()
        ms = event_time_ms(torch, fn, reps)
        achieved = nbytes / (ms * 1e-3) / 1e9
        out[name] = {
            "launch_us": round(ms * 1e3, 2),
            "algorithmic_bytes_per_launch": nbytes,
            "achieved": round(achieved, 1),
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": read_traffic("residual_norm", f"residual_rms_norm_{name}"),
        }
    return out


EVAL_SHAPES = ((1, 128), (1, 512), (1, 1024), (1, 2048), (8, 2048))  # (B, T) at H=12, D=64


def measure_eval(reps: int, device) -> dict:
    """The evaluation harness's calls (lm_eval_hackable_lm.py:134-160,185-207):
    no-grad forwards at batch 1 and ragged T, without a KV cache, through
    hlm_attn.attention (which skips the op dispatcher when nothing needs
    autograd).  Per shape and window: `call_us`, HIP-event time per call over
    back-to-back calls (host and GPU overlapped, what an evaluation loop
    sees); `kernel_us`, the same through the C ABI alone (GPU-bound); the
    split count the library chose."""
    import torch

    import hlm_attn

    lib = None
    out = {"workload": "no-grad forwards, H=12 D=64, windows 512 and causal; synthetic N(0,1) bf16", "shapes": []}
    for B, T in EVAL_SHAPES:
        for W in (512, None):
            cfg = dict(B=B, T=T, H=12, D=64, W=W)
            prob = Problem(cfg, seed=0, device=device)
            lib = prob.lib
            call = lambda: hlm_attn.attention(prob.q, prob.k, prob.v, window_size=W)  # noqa: E731
            with torch.no_grad():
                for _ in range(20):
                    call()
                call_ms = event_time_ms(torch, call, reps)
            for _ in range(20):
                prob.fwd()
            kern_ms = event_time_ms(torch, prob.fwd, reps)
            fl = 4 * cfg["D"] * pairs(T, W) * B * cfg["H"]
            out["shapes"].append({
                "B": B, "T": T, "window": W,
                "nsplit": lib.hlm_attn_fwd_split_count(B, T, 12, 64, 0 if W is None else W),
                "call_us": round(call_ms * 1e3, 2),
                "kernel_us": round(kern_ms * 1e3, 2),
                "tflops": round(fl / (call_ms * 1e-3) / 1e12, 1),
            })
    return out


def event_time_ms(torch, fn, reps: int) -> float:
    """Average duration of fn's launches, by HIP events on the launch stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def event_times_ms(torch, fn, reps: int, before=None) -> list[float]:
    """Per-launch durations of fn by a HIP-event pair around each launch on
    the launch stream; `before` (e.g. a cache flush) runs ahead of each start
    event, outside the timed pair."""
    pairs_ = []
    for _ in range(reps):
        if before is not None:
            before()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        pairs_.append((start, end))
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in pairs_]


FLUSH_MB = 512  # cold-cache policy: this many MB are written between timed launches (the MALL is 256 MB)


def measure(name: str, steps: int, warmup: int, device, graph: bool = False) -> dict:
    """Times `steps` fwd+bwd steps after `warmup` untimed ones.  By default the
    steps are eager launches from Python (the launches run ahead of the GPU,
    so this is GPU time); with graph=True one step (its three kernel launches)
    is captured once in a HIP graph and replayed per step, as a training step
    under torch.compile's CUDA-graph mode runs it."""
    import torch

    cfg = CONFIGS[name]
    prob = Problem(cfg, seed=0, device=device)

    def eager_wall(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            prob.step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    for _ in range(warmup):
        prob.step()
    eager_ms = eager_wall(steps)
    run_step = prob.step
    if graph:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            prob.step()  # one eager step on the capture stream before capture
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            prob.step()
        run_step = g.replay
        for _ in range(warmup):
            run_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run_step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps

    reps = max(steps, 20)
    kern = {
        "fwd": event_time_ms(torch, prob.fwd, reps),
        "bwd_dq": event_time_ms(torch, prob.bwd_dq, reps),
        "bwd_dkdv": event_time_ms(torch, prob.bwd_dkdv, reps),
    }
    bwd_ms = event_time_ms(torch, prob.bwd, reps)
    step_ms = event_time_ms(torch, run_step, reps)
    # Per-launch medians, warm (back to back) and cold (a 512 MB buffer
    # written before each launch evicts the last-level cache).
    flush_buf = torch.empty(FLUSH_MB * (1 << 20) // 4, dtype=torch.float32, device=device)
    flush = lambda: flush_buf.fill_(1.0)  # noqa: E731
    med = {}
    cold = {}
    for k, fn in (("fwd", prob.fwd), ("bwd_dq", prob.bwd_dq), ("bwd_dkdv", prob.bwd_dkdv), ("bwd", prob.bwd),
                  ("fwd_bwd", prob.step)):
        med[k] = statistics.median(event_times_ms(torch, fn, max(reps, 100)))
        cold[k] = statistics.median(event_times_ms(torch, fn, 50, before=flush))
    del flush_buf
    fl = effective_flops(cfg)
    by = algorithmic_bytes(cfg)
    total = fl["fwd"] + fl["bwd"]
    dominant = max(kern, key=kern.get)
    kernel_name = KERNEL_NAMES[dominant]
    achieved = fl[dominant] / (kern[dominant] * 1e-3) / 1e12
    return {
        "cfg": cfg,
        "wall_ms_per_step": wall_ms,
        "event_ms_per_step": step_ms,
        "eager_wall_ms_per_step": eager_ms,
        "graph": graph,
        "fwd_ms": kern["fwd"],
        "bwd_ms": bwd_ms,
        "kernel_us": {k: round(v * 1e3, 2) for k, v in kern.items()},
        "median_us": {k: round(v * 1e3, 2) for k, v in med.items()},
        "cold_us": {k: round(v * 1e3, 2) for k, v in cold.items()},
        "tflops": {
            "fwd": fl["fwd"] / (kern["fwd"] * 1e-3) / 1e12,
            "bwd": fl["bwd"] / (bwd_ms * 1e-3) / 1e12,
            "fwd_bwd": total / (wall_ms * 1e-3) / 1e12,
            # FlashAttention convention: bwd counted as 2.5x fwd (includes the recompute).
            "fwd_bwd_fa_convention": 3.5 * fl["fwd"] / (wall_ms * 1e-3) / 1e12,
        },
        "dominant": dominant,
        "roofline": {
            "bound": "mfma",
            "kernel": kernel_name,
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "algorithmic_flops_per_launch": fl[dominant],
            "algorithmic_bytes_per_launch": by[dominant],
            "launch_us": round(kern[dominant] * 1e3, 2),
            "traffic": read_traffic(name, kernel_name),
            # The same launch against the HBM roofline (algorithmic bytes / launch time).
            "hbm": {
                "achieved_GBs": round(by[dominant] / (kern[dominant] * 1e-3) / 1e9, 1),
                "peak_GBs": PEAK_HBM_GBS,
                "frac": round(by[dominant] / (kern[dominant] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            },
        },
    }


def read_traffic(config: str, kernel: str):
    """HBM bytes per launch of `kernel` at `config`, from the committed rocprofv3
    PMC summary (profiles/hbm_traffic.md, lines 'traffic <config> <kernel> <bytes>')."""
    path = REPO / "profiles" / "hbm_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.strip().strip("`").split()
        if len(parts) == 4 and parts[0] == "traffic" and parts[1] == config and parts[2] == kernel:
            return int(parts[3])
    return None


def cpu_baseline(budget_s: float = 10.0) -> dict:
    """The reference's `torch` backend (restated in oracle/, kernels.py:785-800)
    on the host CPU: BASELINE configs[0], forward only, fp32."""
    import torch

    from oracle import attention as oracle

    cfg = CPU_CONFIG
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(cfg["B"], cfg["T"], cfg["H"], cfg["D"], generator=g) for _ in range(3))
    run = lambda: oracle.attention_core_torch(q, k, v, cfg["W"])  # noqa: E731
    for _ in range(3):
        run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 10 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    eff = 4 * cfg["D"] * pairs(cfg["T"], cfg["W"]) * cfg["B"] * cfg["H"]
    cpu_model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(eff / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"torch-backend restatement, fp32 forward, B=2 H=6 T=1024 D=64 W=256, "
            f"median of {len(times)} runs after 3 warmups ({sum(times):.1f} s)"
        ),
        "ms": round(med * 1e3, 3),
        "effective_gflop": round(eff / 1e9, 4),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": cpu_model,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # The GPU needs ~20 ms of work after idling before it runs at full speed
    # (the first 100 steps run ~12% slower); 300 steps is ~50 ms.
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--config", default="cfg2_local", choices=sorted(CONFIGS))
    ap.add_argument("--sweep", action="store_true", help="also time every config (printed to stderr)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true", help="time HIP-graph replays of the step instead of eager launches")
    ap.add_argument("--no-producer", action="store_true", help="skip the q/k RMSNorm + RoPE producer's timing")
    ap.add_argument("--no-eval", action="store_true", help="skip the evaluation-path (no-grad, batch 1) timings")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the LM-head cross-entropy timing")
    ap.add_argument(
        "--copy-mib", type=int, default=0,
        help="after timing, run one device-to-device copy of this many MiB: a kernel of known "
        "traffic that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters",
    )
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU: the attention kernel runs on one MI355X's share "
            "(every (batch, head) slice is independent); multi-GPU runs are not part of this build.",
            file=sys.stderr,
        )
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda", 0)

    if args.sweep:
        for name in CONFIGS:
            r = measure(name, max(10, args.steps // 2), args.warmup, device, graph=args.graph)
            print(
                f"{name}: fwd {r['fwd_ms']*1e3:.1f} us ({r['tflops']['fwd']:.0f} TF) | "
                f"bwd {r['bwd_ms']*1e3:.1f} us ({r['tflops']['bwd']:.0f} TF) | "
                f"fwd+bwd {r['wall_ms_per_step']*1e3:.1f} us ({r['tflops']['fwd_bwd']:.0f} TF, "
                f"{100*r['tflops']['fwd_bwd']/PEAK_BF16_TFLOPS:.1f}% peak) | kernels {r['kernel_us']}",
                file=sys.stderr,
                flush=True,
            )

    r = measure(args.config, args.steps, args.warmup, device, graph=args.graph)
    cfg = r["cfg"]
    w = "causal" if cfg["W"] is None else f"window={cfg['W']}"
    line = {
        "metric": METRIC,
        "value": round(r["tflops"]["fwd_bwd"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: one attention layer fwd+bwd, B={cfg['B']} H={cfg['H']} T={cfg['T']} "
            f"D={cfg['D']} {w}, causal, inputs N(0,1) seed 0 resident in HBM, warm cache",
            "B": cfg["B"],
            "H": cfg["H"],
            "T": cfg["T"],
            "head_dim": cfg["D"],
            "window": cfg["W"],
            "parallelism": "single GPU",
        },
        "pct_of_bf16_peak": round(100 * r["tflops"]["fwd_bwd"] / PEAK_BF16_TFLOPS, 2),
        "ms_per_layer": {
            "fwd": round(r["fwd_ms"], 5),
            "bwd": round(r["bwd_ms"], 5),
            "fwd_bwd": round(r["wall_ms_per_step"], 5),
        },
        "tflops": {k: round(v, 2) for k, v in r["tflops"].items()},
        "kernel_us": r["kernel_us"],
        "timing": {
            "step": "HIP-graph replay of one fwd+bwd step" if r["graph"] else "eager launches from Python",
            "eager_wall_ms_per_step": round(r["eager_wall_ms_per_step"], 5),
            "event_ms_per_step": round(r["event_ms_per_step"], 5),
            "cache_policy": "value and kernel_us: warm (steps back to back, means); median_us: per-launch "
            f"medians, warm; cold_us: per-launch medians with {FLUSH_MB} MB written before each launch",
            "median_us": r["median_us"],
            "cold_us": r["cold_us"],
            "cold_tflops_fwd_bwd": round(
                (effective_flops(cfg)["fwd"] + effective_flops(cfg)["bwd"]) / (r["cold_us"]["fwd_bwd"] * 1e-6) / 1e12, 2
            ),
        },
        "roofline": r["roofline"],
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(),
    }
    if not args.no_producer:
        line["producer"] = measure_producer(max(args.steps, 50), 20, device)
    if not args.no_eval:
        line["eval"] = measure_eval(max(args.steps // 2, 50), device)
    if not args.no_lm_head:
        line["lm_head"] = measure_lm_head(max(args.steps // 4, 20), 5, device)
        line["residual_norm"] = measure_residual_norm(max(args.steps // 2, 50), 10, device)
    print(json.dumps(line), flush=True)
    if args.copy_mib:
        n = args.copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy calibration: {args.copy_mib} MiB read, {args.copy_mib} MiB written", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
