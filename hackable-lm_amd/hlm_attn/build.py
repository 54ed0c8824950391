"""Builds libhlm_attn.so (the HIP kernels + C ABI) for gfx950 with hipcc.

The library is built in-tree next to this file, so it travels with the source
tree to the GPU host.  Usage:  python -m hlm_attn.build  (or build()).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libhlm_attn.so"
SOURCES = ("attn_fwd.hip", "attn_bwd.hip", "qk_norm_rope.hip", "linear_ce.hip", "residual_norm.hip", "capi.hip")
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in device code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",  # MFMA accumulators in VGPRs: no AGPR copies around the softmax
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the HIP attention library needs ROCm's hipcc to build")
    return found


def build(verbose: bool = False, out: Path | None = None, defines: tuple[str, ...] = ()) -> Path:
    """Compiles every kernel source into LIB_PATH (always recompiles).  `out`
    and `defines` (-D flags) build a variant elsewhere, for experiments."""
    target = Path(out) if out is not None else LIB_PATH
    tmp = target.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), *(str(CSRC / s) for s in SOURCES), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only feature flag; drop that line.
    noise = "not a recognized feature for this target"
    log = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{log}")
    if verbose and log.strip():
        print(log, file=sys.stderr)
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(verbose=True))
