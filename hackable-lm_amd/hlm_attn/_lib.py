"""ctypes binding of libhlm_attn.so (the C ABI declared in include/hlm_attn.h).

No torch types cross this boundary: tensors are passed as device pointers plus
int64 strides, the stream as a raw hipStream_t handle.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libhlm_attn.so")
ABI_VERSION = 8

# Every symbol include/hlm_attn.h declares, with its (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.POINTER(ctypes.c_int64)
SIGNATURES = {
    "hlm_attn_abi_version": (_I, []),
    "hlm_attn_last_error": (ctypes.c_char_p, []),
    "hlm_attn_fwd": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _S, _S, _S, _S, _I, _F, _P]),
}
_BWD_ARGTYPES = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _S, _S, _S, _S, _S, _S, _S, _S, _I, _F, _P]
for _name in ("hlm_attn_bwd", "hlm_attn_bwd_dq", "hlm_attn_bwd_dkdv"):
    SIGNATURES[_name] = (_I, _BWD_ARGTYPES)
SIGNATURES["hlm_attn_bwd_noalloc"] = (_I, _BWD_ARGTYPES[:9] + _BWD_ARGTYPES[10:])  # no delta_ws
# the single-pass backward: + partial workspace (pointer, bytes) after delta_ws
SIGNATURES["hlm_attn_bwd_fused"] = (_I, _BWD_ARGTYPES[:10] + [_P, ctypes.c_int64] + _BWD_ARGTYPES[10:])
SIGNATURES["hlm_attn_bwd_fused_workspace_bytes"] = (ctypes.c_int64, [_I, _I, _I, _I, _I])
SIGNATURES["hlm_attn_fwd_split"] = (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _S, _S, _S, _S, _I, _F, _P])
SIGNATURES["hlm_attn_fwd_split_count"] = (_I, [_I, _I, _I, _I, _I])
SIGNATURES["hlm_qk_norm_rope_fwd"] = (_I, [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _S, _S, _F, _P])
SIGNATURES["hlm_qk_norm_rope_bwd"] = (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _S, _S, _F, _P])
TABLE_F32, TABLE_BF16 = 0, 1  # HLM_TABLE_F32 / HLM_TABLE_BF16
DTYPE_F32, DTYPE_BF16 = 0, 1  # HLM_DTYPE_F32 / HLM_DTYPE_BF16
_I64 = ctypes.c_int64
SIGNATURES["hlm_ce_rows"] = (_I, [_P, _I, _I64, _P, _P, _I, _I, _I64, _I, _P])
SIGNATURES["hlm_residual_rms_norm_fwd"] = (_I, [_P, _P, _P, _P, _I64, _I, _F, _P])
SIGNATURES["hlm_residual_rms_norm_bwd"] = (_I, [_P, _P, _P, _P, _I64, _I, _F, _P])

_lib: ctypes.CDLL | None = None


class HipAttentionUnavailable(RuntimeError):
    """The compiled HIP attention library is missing or unusable."""


def load(path: Path | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the library; raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = Path(path) if path is not None else LIB_PATH
    if not target.exists():
        raise HipAttentionUnavailable(
            f"{target} is missing: build it with `python -m hlm_attn.build` "
            "(hipcc --offload-arch=gfx950) before using attention_backend='hip'"
        )
    lib = ctypes.CDLL(str(target))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.hlm_attn_abi_version() != ABI_VERSION:
        raise HipAttentionUnavailable(
            f"{target} has ABI {lib.hlm_attn_abi_version()}, this binding expects {ABI_VERSION}"
        )
    if path is None:
        _lib = lib
    return lib


_pycall = None


def load_pycall():
    """The CPython binding of the forward entry points (_pycall, built with the
    library by hlm_attn.build and linked against it); raises if it is missing."""
    global _pycall
    if _pycall is None:
        load()  # the library first: a missing or stale build raises here
        try:
            from . import _pycall as mod
        except ImportError as e:
            raise HipAttentionUnavailable(
                f"the CPython binding next to {LIB_PATH} is missing ({e}): build it with `python -m hlm_attn.build`"
            ) from e
        _pycall = mod
    return _pycall


_torch_fwd = None  # the extension module once loaded; False once a load failed or it is disabled
_torch_fwd_error = ""


def load_torch_fwd():
    """The torch C++ extension of the no-grad forward (_torch_fwd: checks,
    allocation and launch in one C++ call), built with the library; raises if
    it is missing or unusable.  The forward does not need it: see torch_fwd()."""
    ext = torch_fwd()
    if ext is None:
        raise HipAttentionUnavailable(
            f"the torch extension next to {LIB_PATH} is unavailable ({_torch_fwd_error}): "
            "build it with `python -m hlm_attn.build`"
        )
    return ext


def torch_fwd():
    """The optional torch C++ extension of the forward, or None.

    It only saves host time per call (a few microseconds at batch 1); every
    forward also runs through the C ABI without it.  None when it is missing,
    when it was built against another torch (its import then fails), or when
    HLM_ATTN_TORCH_EXT=0 disables it.  The first failure is remembered, so the
    import is attempted once per process."""
    global _torch_fwd, _torch_fwd_error
    if _torch_fwd is None:
        import os

        if os.environ.get("HLM_ATTN_TORCH_EXT", "1") == "0":
            _torch_fwd, _torch_fwd_error = False, "disabled by HLM_ATTN_TORCH_EXT=0"
        else:
            try:
                load()
                from . import _torch_fwd as mod
            except (ImportError, OSError, HipAttentionUnavailable) as e:
                _torch_fwd, _torch_fwd_error = False, f"{type(e).__name__}: {e}"
            else:
                _torch_fwd = mod
    return _torch_fwd or None


_Strides = ctypes.c_int64 * 3
_strides_cache: dict = {}


def strides3(t) -> ctypes.Array:
    """(batch, time, head) strides of a (B, T, H, D) tensor as an int64[3]
    (shared per distinct stride triple; the library only reads it)."""
    s = t.stride()[:3]
    arr = _strides_cache.get(s)
    if arr is None:
        if len(_strides_cache) > 4096:
            _strides_cache.clear()
        arr = _strides_cache[s] = _Strides(*s)
    return arr


def check(rc: int, lib: ctypes.CDLL) -> None:
    if rc != 0:
        msg = lib.hlm_attn_last_error().decode(errors="replace")
        raise RuntimeError(f"hip attention failed (code {rc}): {msg}")
