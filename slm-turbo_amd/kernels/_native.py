"""ctypes binding of libslmturbo_hip.so (C ABI declared in include/slmturbo.h).

Replaces the reference's JIT ``load_inline`` extension
(kernels/kv_dequant.py:47-86): the library is built ahead of time for gfx950
(``slm-turbo_amd/build_lib.py``) and loaded here once.  Like the reference
loader, a load failure is cached and re-raised on every later call; there is no
CPU fallback.  ``SLMT_LIB`` overrides the library path.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

ABI_VERSION = 3
LIB_NAME = "libslmturbo_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
OUT_F32, OUT_F16 = 0, 1

_lib = None
_lib_error: Exception | None = None
_lock = threading.Lock()

_vp, _i64, _i32, _p_i64, _p_i32, _p_f32 = (
    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)

# name -> (restype, argtypes); mirrors include/slmturbo.h
SIGNATURES = {
    "slmt_last_error": (ctypes.c_char_p, []),
    "slmt_abi_version": (_i32, []),
    "slmt_attention_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "slmt_quantize_store": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _p_i64, _i64, _i32, _i32, _vp]),
    "slmt_quantize_per_channel": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "slmt_quantize_with_rulers": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _vp]),
    "slmt_decode_paged": (_i32, [_vp, _vp, _i64, _i32, _p_i64, _i32, _i32, _i32, _i32, _p_f32, _vp, _i64,
                                 _vp]),
    "slmt_decode_paged_batched": (_i32, [_vp, _i64, _i64, _vp, _i64, _i32, _vp, _i32, _i64, _p_i32, _i32,
                                         _i32, _i32, _i32, _i32, _vp, _i32, _i64, _i64, _vp, _i64, _vp]),
    "slmt_decode_paged_batched_noalloc": (_i32, [_vp, _i64, _i64, _vp, _i64, _i32, _vp, _i32, _i64, _p_i32,
                                                 _i32, _i32, _i32, _i32, _i32, _vp, _i32, _i64, _i64, _vp]),
    "slmt_decode_per_token": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                     _i32, _p_f32, _vp, _i64, _vp]),
    "slmt_decode_per_channel": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                       _i32, _i32, _p_f32, _vp, _i64, _vp]),
    "slmt_prefill_per_channel": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                        _i32, _i32, _i32, _i32, _i32, _p_f32, _vp, _i64, _vp]),
    "slmt_kernel_timing": (_i32, [_i32]),
    "slmt_kernel_timing_read": (_i32, [_p_f32, _i32]),
    "slmt_kernel_timing_kernel": (ctypes.c_char_p, []),
}


def library_path() -> Path:
    return Path(os.environ.get("SLMT_LIB") or str(LIB_PATH))


def load():
    """Load (once) and return the ctypes library; re-raise a cached failure."""
    global _lib, _lib_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if _lib_error is not None:
            raise _lib_error
        try:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"slm-turbo HIP library not found at {path}; build it with "
                    f"`python slm-turbo_amd/build_lib.py` (hipcc, gfx950)")
            lib = ctypes.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.slmt_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{path}: ABI version {lib.slmt_abi_version()} != {ABI_VERSION}")
        except Exception as e:  # cached like the reference's _ext_error
            _lib_error = e
            raise
        _lib = lib
        return lib


_fast = None
_fast_tried = False


def fast():
    """The CPython METH_FASTCALL binding (kernels/_slmt_fast, built from
    csrc/pyfast.c) bound to the loaded library's slmt_quantize_store and
    slmt_decode_paged_batched, or None when it was not built.  It calls the
    same entry points as the ctypes functions, with less per-call overhead."""
    global _fast, _fast_tried
    if _fast_tried:
        return _fast
    lib = load()
    with _lock:
        if not _fast_tried:
            try:
                from . import _slmt_fast as mod
            except ImportError:
                mod = None
            if mod is not None:
                mod.bind(ctypes.cast(lib.slmt_quantize_store, ctypes.c_void_p).value,
                         ctypes.cast(lib.slmt_decode_paged_batched, ctypes.c_void_p).value)
            _fast = mod
            _fast_tried = True
    return _fast


def last_error(lib) -> str:
    msg = lib.slmt_last_error()
    return msg.decode() if msg else ""


def check(lib, rc: int) -> None:
    """Map a non-zero status to RuntimeError carrying the library's message."""
    if rc != OK:
        raise RuntimeError(last_error(lib) or f"slm-turbo HIP call failed with status {rc}")
