#!/usr/bin/env python3
"""Benchmark of the HIP causal sliding-window attention backend on one MI355X.

One "step" is one attention layer's forward + backward through the C ABI
(hlm_attn_fwd, then hlm_attn_bwd on the forward's o and lse) at the BASELINE
workload cfg2: B=8, H=12, T=2048, D=64, window=512, causal, bf16, synthetic
N(0,1) inputs from one seed, resident in HBM before timing starts.  Warm
cache: steps run back to back, as in training.

Timing.  A time-based pre-warm runs steps until the GPU has done >= 200 ms of
work and the last 10 step times agree within 2% (the clock ramps for the first
~100 steps after idling), independent of --warmup; then --warmup untimed
steps; then exactly --steps steps between two HIP events on the launch stream
(torch's current stream, which the C ABI launches on), synchronised before and
after.  value = effective fwd+bwd TFLOP/s of those steps, where effective
FLOPs count only unmasked (query, key) pairs P(T, W): fwd 4*D*P, bwd 8*D*P per
(batch, head).  Wall-clock time of the same steps is a side field.

Prints ONE JSON line with, besides the contract fields: ms per layer (fwd,
bwd, fwd+bwd), the fraction of MI355X's dense bf16 MFMA peak, per-kernel
launch times, a roofline object for the dominant kernel (HIP-event mean over
back-to-back launches), the CPU baseline (the reference's `torch` backend
restated, configs[0] shape, fp32 forward, on the host's cores), and a
"configs" object with every other BASELINE GPU config measured in the same
run: cfg3 (one full-causal layer), cfg4 (the 18-layer stack, per layer and in
total) and cfg5 (q and k RoPE-rotated before the bf16 cast).  "producer",
"eval", "lm_head" and "residual_norm" objects time the neighbouring kernels
(q/k RMSNorm + RoPE, no-grad batch-1 forwards, LM-head cross-entropy rows,
residual add + RMSNorm) against their rooflines.

Steps are eager launches by default (they run ahead of the GPU); --graph times
HIP-graph replays of one captured step instead (the way a training step runs
under torch.compile's CUDA-graph mode).

  python bench.py [--steps K] [--warmup W] [--config NAME] [--kernel-reps N] [--no-configs] [--cold]
                  [--no-cpu-baseline] [--graph] [--no-producer] [--no-eval] [--no-lm-head] [--copy-mib M]
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

    def __init__(self, cfg: dict, seed: int, device, tensors=None):
        """q, k, v, dO ~ N(0,1) from a CPU generator seeded with `seed`,
        rounded to bf16 and copied to the device; or `tensors` = (q, k, v, dO),
        bf16 device tensors of this shape prepared by the caller."""
        import torch
        from hlm_attn import _lib

        self.torch = torch
        self.lib = _lib.load()
        self.cfg = cfg
        B, T, H, D = cfg["B"], cfg["T"], cfg["H"], cfg["D"]
        if tensors is None:
            g = torch.Generator(device="cpu").manual_seed(seed)
            mk = lambda: torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(device)  # noqa: E731
            self.q, self.k, self.v, self.do = mk(), mk(), mk(), mk()
        else:
            self.q, self.k, self.v, self.do = tensors
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

    def bwd_fused(self, part, nbytes: int):
        """The single-pass backward (hlm_attn_bwd_fused, D = 64) into the same
        outputs, with `part` (nbytes) as its partial workspace."""
        rc = self.lib.hlm_attn_bwd_fused(
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.o.data_ptr(), self.do.data_ptr(),
            self.lse.data_ptr(), self.dq.data_ptr(), self.dk.data_ptr(), self.dv.data_ptr(), self.delta.data_ptr(),
            part.data_ptr(), nbytes,
            *self.dims, self.s["q"], self.s["k"], self.s["v"], self.s["o"], self.s["do"], self.s["dq"],
            self.s["dk"], self.s["dv"], self.window, self.scale, self.stream,
        )
        assert rc == 0, self.lib.hlm_attn_last_error()

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
    sees); `kernel_us`, the same launches (split-key when the library splits)
    through the C ABI alone (GPU-bound); the split count the library chose."""
    import torch

    import hlm_attn

    def warm(fn, min_ms=30.0):
        # Back-to-back calls until the GPU has run min_ms of them (the clock
        # ramps up under load; a fixed count of short calls does not get there).
        done = 0.0
        while done < min_ms:
            done += event_time_ms(torch, fn, 10) * 10

    lib = None
    out = {"workload": "no-grad forwards, H=12 D=64, windows 512 and causal; synthetic N(0,1) bf16",
           "timing": "each path warmed for >= 30 ms of GPU time, then HIP events around `reps` back-to-back calls",
           "shapes": []}
    for B, T in EVAL_SHAPES:
        for W in (512, None):
            cfg = dict(B=B, T=T, H=12, D=64, W=W)
            prob = Problem(cfg, seed=0, device=device)
            lib = prob.lib
            nsplit = lib.hlm_attn_fwd_split_count(B, T, 12, 64, 0 if W is None else W)
            call = lambda: hlm_attn.attention(prob.q, prob.k, prob.v, window_size=W)  # noqa: E731
            with torch.no_grad():
                warm(call)
                call_ms = event_time_ms(torch, call, reps)
            kernel = prob.fwd
            if nsplit > 1:  # the same split-key launches the call path makes
                ws = torch.empty(nsplit * B * 12 * T * (64 + 2), dtype=torch.float32, device=device)

                def kernel():
                    rc = lib.hlm_attn_fwd_split(
                        prob.q.data_ptr(), prob.k.data_ptr(), prob.v.data_ptr(), prob.o.data_ptr(), prob.lse.data_ptr(),
                        ws.data_ptr(), nsplit, *prob.dims, prob.s["q"], prob.s["k"], prob.s["v"], prob.s["o"],
                        prob.window, prob.scale, prob.stream)
                    assert rc == 0, lib.hlm_attn_last_error()
            warm(kernel)
            kern_ms = event_time_ms(torch, kernel, reps)
            fl = 4 * cfg["D"] * pairs(T, W) * B * cfg["H"]
            out["shapes"].append({
                "B": B, "T": T, "window": W,
                "nsplit": nsplit,
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


FLUSH_MB = 512  # cold-cache policy (--cold): this many MB are written between timed launches (the MALL is 256 MB)


def prewarm(torch, step, min_ms: float = 200.0, max_s: float = 2.0, block: int = 10, tol: float = 0.02) -> dict:
    """Runs blocks of `block` steps, each timed by one pair of HIP events on
    the launch stream, until the GPU has done at least `min_ms` of work AND
    the last three blocks agree within `tol` of their median, or `max_s`
    seconds have passed.  The MI355X runs its first ~100 cfg2 steps after
    idling ~12% slower while its clock ramps; this loop is independent of
    --warmup, so the timed steps see the steady state however few warmup
    steps the caller asks for."""
    blocks: list[float] = []
    t_end = time.perf_counter() + max_s
    while True:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(block):
            step()
        b.record()
        b.synchronize()
        blocks.append(a.elapsed_time(b))
        last = blocks[-3:]
        spread = (max(last) - min(last)) / statistics.median(last) if len(last) == 3 else float("inf")
        converged = sum(blocks) >= min_ms and spread <= tol
        if converged or time.perf_counter() > t_end:
            return {
                "prewarm_ms": round(sum(blocks), 2),
                "prewarm_steps": block * len(blocks),
                "prewarm_converged": converged,
                "prewarm_last_blocks_spread": round(spread, 4),
                "prewarm_rule": f">= {min_ms:.0f} ms of GPU work and the last 3 blocks of {block} steps within "
                f"{100 * tol:.0f}% of their median (cap {max_s:.0f} s)",
            }


def timed_steps(torch, step, steps: int) -> tuple[float, float]:
    """(event ms per step, wall ms per step) over exactly `steps` steps,
    bracketed by torch.cuda.synchronize() on both sides; the events are
    recorded on the launch stream (torch's current stream, which the C ABI
    launches on)."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


def measure(name: str, steps: int, warmup: int, device, graph: bool = False, kernel_reps: int = 500,
            cold: bool = False) -> dict:
    """cfg `name`: a time-based pre-warm, `warmup` untimed steps, then exactly
    `steps` fwd+bwd steps timed with HIP events (value / ms_per_step), and
    each kernel alone over `kernel_reps` back-to-back launches (kernel_us,
    the roofline).  Steps are eager launches from Python (they run ahead of
    the GPU); with graph=True one step (its three kernel launches) is
    captured once in a HIP graph and replayed per step, as a training step
    under torch.compile's CUDA-graph mode runs it."""
    import torch

    cfg = CONFIGS[name]
    prob = Problem(cfg, seed=0, device=device)
    warm = prewarm(torch, prob.step)
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
    step_ms, wall_ms = timed_steps(torch, run_step, steps)

    kern = {
        "fwd": event_time_ms(torch, prob.fwd, kernel_reps),
        "bwd_dq": event_time_ms(torch, prob.bwd_dq, kernel_reps),
        "bwd_dkdv": event_time_ms(torch, prob.bwd_dkdv, kernel_reps),
    }
    bwd_ms = event_time_ms(torch, prob.bwd, kernel_reps)
    out_cold = None
    if cold:
        # Per-launch medians with a 512 MB buffer written before each launch
        # (evicts the last-level cache), beside the warm per-launch medians.
        flush_buf = torch.empty(FLUSH_MB * (1 << 20) // 4, dtype=torch.float32, device=device)
        flush = lambda: flush_buf.fill_(1.0)  # noqa: E731
        out_cold = {"warm_median_us": {}, "cold_median_us": {}}
        for k, fn in (("fwd", prob.fwd), ("bwd_dq", prob.bwd_dq), ("bwd_dkdv", prob.bwd_dkdv), ("bwd", prob.bwd),
                      ("fwd_bwd", prob.step)):
            out_cold["warm_median_us"][k] = round(statistics.median(event_times_ms(torch, fn, 100)) * 1e3, 2)
            out_cold["cold_median_us"][k] = round(statistics.median(event_times_ms(torch, fn, 50, before=flush)) * 1e3, 2)
        del flush_buf
    fl = effective_flops(cfg)
    by = algorithmic_bytes(cfg)
    total = fl["fwd"] + fl["bwd"]
    dominant = max(kern, key=kern.get)
    kernel_name = KERNEL_NAMES[dominant]
    achieved = fl[dominant] / (kern[dominant] * 1e-3) / 1e12
    return {
        "cfg": cfg,
        "step_ms": step_ms,
        "wall_ms_per_step": wall_ms,
        "prewarm": warm,
        "graph": graph,
        "fwd_ms": kern["fwd"],
        "bwd_ms": bwd_ms,
        "kernel_us": {k: round(v * 1e3, 2) for k, v in kern.items()},
        "kernel_reps": kernel_reps,
        "cold": out_cold,
        "tflops": {
            "fwd": fl["fwd"] / (kern["fwd"] * 1e-3) / 1e12,
            "bwd": fl["bwd"] / (bwd_ms * 1e-3) / 1e12,
            "fwd_bwd": total / (step_ms * 1e-3) / 1e12,
            # FlashAttention convention: bwd counted as 2.5x fwd (includes the recompute).
            "fwd_bwd_fa_convention": 3.5 * fl["fwd"] / (step_ms * 1e-3) / 1e12,
        },
        "dominant": dominant,
        "roofline": {
            "bound": "mfma",
            "kernel": kernel_name,
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": read_traffic(name, kernel_name),
            "algorithmic_flops_per_launch": fl[dominant],
            "algorithmic_bytes_per_launch": by[dominant],
            "launch_us": round(kern[dominant] * 1e3, 2),
            "launches_averaged": kernel_reps,
            # The same launch against the HBM roofline (algorithmic bytes / launch time).
            "hbm": {
                "achieved_GBs": round(by[dominant] / (kern[dominant] * 1e-3) / 1e9, 1),
                "peak_GBs": PEAK_HBM_GBS,
                "frac": round(by[dominant] / (kern[dominant] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            },
        },
    }


def measure_bwd_fused(names, reps: int, device, rounds: int = 5) -> dict:
    """The single-pass backward (hlm_attn_bwd_fused: delta rows, one
    key-stationary pass writing dK, dV and bf16 dQ partials, a reduce of the
    partials) beside the two-kernel backward (hlm_attn_bwd), on the same
    inputs and forward outputs, for the D = 64 configs `names`.  Each path:
    `reps` back-to-back launches timed by HIP events, `rounds` alternating
    rounds, the minimum reported; the results of the two paths compared."""
    import torch

    out = {"timing": f"min over {rounds} alternating rounds of HIP events around {reps} back-to-back launches",
           "configs": {}}
    for name in names:
        cfg = CONFIGS[name]
        prob = Problem(cfg, seed=0, device=device)
        prob.fwd()
        B, T, H, _, D = prob.dims
        nbytes = prob.lib.hlm_attn_bwd_fused_workspace_bytes(B, T, H, D, prob.window)
        assert nbytes > 0, prob.lib.hlm_attn_last_error()
        part = torch.empty(nbytes, dtype=torch.uint8, device=device)
        fused = lambda: prob.bwd_fused(part, nbytes)  # noqa: E731
        prob.bwd()
        two = [t.clone() for t in (prob.dq, prob.dk, prob.dv)]
        fused()
        torch.cuda.synchronize()
        dq_rel = ((prob.dq.float() - two[0].float()).norm() / two[0].float().norm()).item()
        same_dk_dv = bool(torch.equal(prob.dk, two[1]) and torch.equal(prob.dv, two[2]))
        prewarm(torch, prob.bwd, min_ms=50.0)
        times = {"two_kernel": [], "single_pass": []}
        for _ in range(rounds):
            times["two_kernel"].append(event_time_ms(torch, prob.bwd, reps))
            times["single_pass"].append(event_time_ms(torch, fused, reps))
        best = {k: min(v) * 1e3 for k, v in times.items()}
        fl = effective_flops(cfg)["bwd"]
        out["configs"][name] = {
            "bwd_us": {k: round(v, 2) for k, v in best.items()},
            "bwd_tflops": {k: round(fl / (v * 1e-6) / 1e12, 1) for k, v in best.items()},
            "single_pass_over_two_kernel": round(best["single_pass"] / best["two_kernel"], 3),
            "partial_workspace_MB": round(nbytes / 1e6, 1),
            "dk_dv_bit_identical": same_dk_dv,
            "dq_norm_rel_vs_two_kernel": float(f"{dq_rel:.3e}"),
        }
        del prob, part, two
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# The other BASELINE configs, measured in the same run ("configs" object).
# ---------------------------------------------------------------------------

CFG4_LAYERS = dict(n_layer=18, window=1024, full_every=4)
ROPE_BASE = 10000.0  # RoPE base 10000 over positions 0..T-1, whole head


def rope_rotate(x, base: float = ROPE_BASE):
    """Rotate-half RoPE over the whole head dim (model.py:105-114 with
    fraction 1.0, theta = base) of a (B, T, H, D) fp32 tensor, positions
    0..T-1, computed in fp32: the input synthesis of BASELINE configs[4]."""
    import torch

    T, D = x.shape[1], x.shape[3]
    inv_freq = 1.0 / (base ** (torch.arange(0, D, 2, device=x.device, dtype=torch.float32) / D))
    freqs = torch.outer(torch.arange(T, device=x.device, dtype=torch.float32), inv_freq)
    cos, sin = freqs.cos()[None, :, None, :], freqs.sin()[None, :, None, :]
    x1, x2 = x[..., : D // 2], x[..., D // 2 :]
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)


def device_inputs(cfg: dict, seed: int, device, rope: bool = False):
    """q, k, v, dO ~ N(0,1) drawn in that order from a device generator seeded
    with `seed` (fp32, then rounded to bf16); with rope=True, q and k are
    rotated (rope_rotate) in fp32 before the rounding."""
    import torch

    B, T, H, D = cfg["B"], cfg["T"], cfg["H"], cfg["D"]
    g = torch.Generator(device=device).manual_seed(seed)
    out = []
    for i in range(4):
        x = torch.randn(B, T, H, D, generator=g, device=device, dtype=torch.float32)
        if rope and i < 2:
            x = rope_rotate(x)
        out.append(x.to(torch.bfloat16))
        del x
    return out


def _layer_entry(cfg: dict, fwd_ms: float, bwd_ms: float, step_ms: float) -> dict:
    fl = effective_flops(cfg)
    tot = fl["fwd"] + fl["bwd"]
    return {
        "ms_per_layer": {"fwd": round(fwd_ms, 5), "bwd": round(bwd_ms, 5), "fwd_bwd": round(step_ms, 5)},
        "tflops": {
            "fwd": round(fl["fwd"] / (fwd_ms * 1e-3) / 1e12, 2),
            "bwd": round(fl["bwd"] / (bwd_ms * 1e-3) / 1e12, 2),
            "fwd_bwd": round(tot / (step_ms * 1e-3) / 1e12, 2),
        },
        "pct_of_bf16_peak": round(100 * tot / (step_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "effective_gflop_fwd_bwd": round(tot / 1e9, 3),
    }


def measure_single_layer(name: str, reps: int, device, rope: bool = False, prewarm_ms: float = 20.0) -> dict:
    """One layer of config `name`: fwd alone, bwd alone and fwd+bwd steps,
    each the HIP-event mean over `reps` back-to-back launches, after a short
    pre-warm (the GPU is already at its steady clock from the headline
    measurement just before)."""
    import torch

    cfg = CONFIGS[name]
    prob = Problem(cfg, seed=0, device=device, tensors=device_inputs(cfg, 0, device, rope=rope))
    warm = prewarm(torch, prob.step, min_ms=prewarm_ms)
    step_ms = event_time_ms(torch, prob.step, reps)
    fwd_ms = event_time_ms(torch, prob.fwd, reps)
    bwd_ms = event_time_ms(torch, prob.bwd, reps)
    w = "causal" if cfg["W"] is None else f"window={cfg['W']}"
    entry = {
        "workload": f"B={cfg['B']} H={cfg['H']} T={cfg['T']} D={cfg['D']} {w}; q, k, v, dO ~ N(0,1) seed 0"
        + (f", q and k RoPE-rotated (base {ROPE_BASE:g}, positions 0..T-1, whole head) in fp32 before the bf16 cast"
           if rope else ""),
        "reps": reps,
        "prewarm_ms": warm["prewarm_ms"],
        "prewarm_converged": warm["prewarm_converged"],
    }
    entry.update(_layer_entry(cfg, fwd_ms, bwd_ms, step_ms))
    del prob
    torch.cuda.empty_cache()
    return entry


def measure_layer_stack(passes: int, device, seed: int = 0) -> dict:
    """18 attention layers (B=4, H=12, T=4096, D=128),
    layer l's window from the reference's pattern (layer_attention_window(l,
    18, 1024, 4): layers 3, 7, 11, 15 and 17 full causal) and its q, k, v, dO
    from seed + l.  One pass = the forwards of layers 0..17, then the
    backwards of layers 17..0, launched back to back on one stream with a HIP
    event between launches; per-layer times are medians over `passes`
    passes, the totals are the medians of the pass sums and of the whole
    pass."""
    import torch

    from hlm_attn.config import layer_attention_window

    n = CFG4_LAYERS["n_layer"]
    base = CONFIGS["cfg4_local"]
    layers = []
    for l in range(n):
        w = layer_attention_window(l, n, CFG4_LAYERS["window"], CFG4_LAYERS["full_every"])
        cfg = dict(base, W=w)
        layers.append((cfg, Problem(cfg, seed=seed + l, device=device, tensors=device_inputs(cfg, seed + l, device))))

    def one_pass():
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * n + 1)]
        ev[0].record()
        for l in range(n):
            layers[l][1].fwd()
            ev[l + 1].record()
        for l in reversed(range(n)):
            layers[l][1].bwd()
            ev[2 * n - l].record()
        return ev

    warm = prewarm(torch, one_pass, min_ms=20.0, block=2, tol=0.03)
    runs = []
    for _ in range(passes):
        ev = one_pass()
        torch.cuda.synchronize()
        fwd = [ev[l].elapsed_time(ev[l + 1]) for l in range(n)]
        bwd = [ev[2 * n - l - 1].elapsed_time(ev[2 * n - l]) for l in range(n)]
        runs.append((fwd, bwd, ev[0].elapsed_time(ev[2 * n])))
    per_layer = []
    for l in range(n):
        f = statistics.median(r[0][l] for r in runs)
        b = statistics.median(r[1][l] for r in runs)
        e = {"layer": l, "window": layers[l][0]["W"]}
        e.update(_layer_entry(layers[l][0], f, b, f + b))
        per_layer.append(e)
    tot_f = statistics.median(sum(r[0]) for r in runs)
    tot_b = statistics.median(sum(r[1]) for r in runs)
    tot = statistics.median(r[2] for r in runs)
    flops = sum(effective_flops(c)["fwd"] + effective_flops(c)["bwd"] for c, _ in layers)
    flops_f = sum(effective_flops(c)["fwd"] for c, _ in layers)
    del layers
    torch.cuda.empty_cache()
    return {
        "workload": f"{n} layers B={base['B']} H={base['H']} T={base['T']} D={base['D']}, window "
        f"{CFG4_LAYERS['window']} except the full-causal layers of layer_attention_window(l, {n}, "
        f"{CFG4_LAYERS['window']}, {CFG4_LAYERS['full_every']}) (3, 7, 11, 15, 17); layer l's q, k, v, dO ~ N(0,1) "
        "from seed + l; forwards 0..17 then backwards 17..0, back to back",
        "passes": passes,
        "prewarm_ms": warm["prewarm_ms"],
        "prewarm_converged": warm["prewarm_converged"],
        "layers": per_layer,
        "total": {
            "ms": {"fwd": round(tot_f, 4), "bwd": round(tot_b, 4), "fwd_bwd": round(tot, 4)},
            "tflops_fwd_bwd": round(flops / (tot * 1e-3) / 1e12, 2),
            "tflops_fwd": round(flops_f / (tot_f * 1e-3) / 1e12, 2),
            "pct_of_bf16_peak": round(100 * flops / (tot * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
            "effective_tflop": round(flops / 1e12, 4),
        },
    }


def measure_configs(device) -> dict:
    """Every BASELINE GPU config besides the headline one, in this run."""
    return {
        "data": "q, k, v, dO ~ N(0,1) from a seeded device generator (torch.Generator on the GPU), rounded to bf16; "
        "HIP-event means on the launch stream, warm cache",
        # cfg3 runs the headline's kernels (same names and grids) at twice their time; few
        # launches keep the per-kernel averages of a rocprofv3 trace of this run on the headline
        "cfg3_full": measure_single_layer("cfg3_full", 10, device, prewarm_ms=10.0),
        "cfg4_stack": measure_layer_stack(3, device),
        "cfg5_long_rope": measure_single_layer("cfg5_long", 10, device, rope=True),
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
    # As many threads as this process may run on (BASELINE.md's rule).
    threads_before = torch.get_num_threads()
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
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
    torch.set_num_threads(threads_before)
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
        "cores": cores,
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
    # Untimed steps after the time-based pre-warm (which alone brings the GPU
    # to its steady clock, whatever this is).
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2_local", choices=sorted(CONFIGS))
    ap.add_argument("--kernel-reps", type=int, default=500, help="back-to-back launches per kernel timing")
    ap.add_argument("--no-configs", action="store_true", help="skip the other BASELINE configs (cfg3, cfg4, cfg5)")
    ap.add_argument("--cold", action="store_true", help="also time per-launch medians with the cache flushed")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true", help="time HIP-graph replays of the step instead of eager launches")
    ap.add_argument("--no-producer", action="store_true", help="skip the q/k RMSNorm + RoPE producer's timing")
    ap.add_argument("--no-eval", action="store_true", help="skip the evaluation-path (no-grad, batch 1) timings")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the LM-head cross-entropy timing")
    ap.add_argument("--bwd-fused", nargs="?", const="cfg2_local,cfg3_full", default=None, metavar="CONFIGS",
                    help="also time the single-pass backward (hlm_attn_bwd_fused) against the two-kernel one at "
                    "these comma-separated D = 64 configs (default cfg2_local,cfg3_full; object bwd_fused)")
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

    r = measure(args.config, args.steps, args.warmup, device, graph=args.graph, kernel_reps=args.kernel_reps,
                cold=args.cold)
    cfg = r["cfg"]
    w = "causal" if cfg["W"] is None else f"window={cfg['W']}"
    line = {
        "metric": METRIC,
        "value": round(r["tflops"]["fwd_bwd"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_ms"], 5),
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
            "fwd_bwd": round(r["step_ms"], 5),
        },
        "tflops": {k: round(v, 2) for k, v in r["tflops"].items()},
        "kernel_us": r["kernel_us"],
        "timing": {
            "value": f"HIP events on the launch stream around exactly {args.steps} steps (synchronised before and "
            "after); fwd / bwd / kernel_us: HIP-event means over "
            f"{r['kernel_reps']} back-to-back launches",
            "step": "HIP-graph replay of one fwd+bwd step" if r["graph"] else "eager launches from Python",
            "wall_ms_per_step": round(r["wall_ms_per_step"], 5),
            **r["prewarm"],
            "cache_policy": "warm: steps and launches back to back",
        },
        "roofline": r["roofline"],
        "cpu_baseline": None,
    }
    if r["cold"] is not None:
        line["timing"]["cold"] = r["cold"]
    if not args.no_configs:
        line["configs"] = measure_configs(device)
    if not args.no_producer:
        line["producer"] = measure_producer(max(args.steps, 50), 20, device)
    if not args.no_eval:
        line["eval"] = measure_eval(max(args.steps // 2, 50), device)
    if not args.no_lm_head:
        line["lm_head"] = measure_lm_head(max(args.steps // 4, 20), 5, device)
        line["residual_norm"] = measure_residual_norm(max(args.steps // 2, 50), 10, device)
    if args.bwd_fused:
        names = [n for n in args.bwd_fused.split(",") if n]
        bad = [n for n in names if n not in CONFIGS or CONFIGS[n]["D"] != 64]
        if bad:
            print(f"--bwd-fused takes D = 64 configs only, not {bad}", file=sys.stderr)
            return 2
        line["bwd_fused"] = measure_bwd_fused(names, max(args.steps, 50), device)
    if not args.no_cpu_baseline:
        # last: ~10 s of host work, after which the GPU has idled and would need a new pre-warm
        line["cpu_baseline"] = cpu_baseline()
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
