"""Quantizers of the reference, restated on the CPU.  TEST INFRASTRUCTURE ONLY.

* Per-channel asymmetric 4-bit quantizer of the standalone path:
  ``compute_scale_zero`` / ``quantize_tensor`` / ``quantize_kv`` in
  kernels/benchmark/benchmark.py:26-74.  Restated with numpy float16 ufuncs:
  numpy evaluates each float16 operation in float32 and rounds the result to
  float16 (nearest-even), which equals the correctly rounded float16 result
  (float32 has >= 2*11+2 significand bits, so the double rounding is
  innocuous) -- the same per-operation rounding torch applies to fp16 tensors.
* Per-token min/step quantize-on-write store: kv_quantize_store_kernel,
  kernels/kv_dequant_kernels.cuh:816-919, restated in C (oracle/store_ref.c)
  and called here through ctypes.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_lib = None


def build_c_oracle() -> Path:
    """Compile oracle/store_ref.c with oracle/Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _clib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build_c_oracle()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.oracle_quantize_store.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64]
        lib.oracle_quantize_store.restype = None
        lib.oracle_quantize_row.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
        lib.oracle_quantize_row.restype = None
        lib.oracle_float_to_half.argtypes = [ctypes.c_float]
        lib.oracle_float_to_half.restype = ctypes.c_uint16
        lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        lib.oracle_half_to_float.restype = ctypes.c_float
        _lib = lib
    return _lib


# ---------------------------------------------------------------------------
# Per-channel quantizer (kernels/benchmark/benchmark.py:26-74)
# ---------------------------------------------------------------------------
def compute_scale_zero(x: np.ndarray, bits: int = 4):
    """Per-(kv, channel) scale/zero over the sequence axis (axis 1).

    Follows kernels/benchmark/benchmark.py:26-42: ``scale = (max-min)/15``,
    ``zero = 0 - round(min/scale)`` (ties to even, pre-guard scale), constant
    channels -> (1, 0), ``zero`` clamped to [0, 15]; every op in fp16.
    x: float16 [KV, S, D] -> (scale, zero) float16 [KV, D].
    """
    x = np.asarray(x, dtype=np.float16)
    q_min, q_max = 0, (1 << bits) - 1
    x_min = x.min(axis=1)
    x_max = x.max(axis=1)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        scale = (x_max - x_min) / np.float16(q_max - q_min)
        zero = np.float16(q_min) - np.round(x_min / scale)
    is_const = x_max == x_min
    scale = np.where(is_const, np.float16(1), scale).astype(np.float16)
    zero = np.where(is_const, np.float16(0), zero).astype(np.float16)
    zero = np.clip(zero, np.float16(q_min), np.float16(q_max)).astype(np.float16)
    return scale, zero


def _to_u8_codes(q: np.ndarray) -> np.ndarray:
    """fp16 codes already clamped to [0, 15] -> uint8.  NaN (only possible when
    a channel's scale underflows to 0) maps to 0."""
    q = np.where(np.isnan(q), np.float16(0), q)
    return q.astype(np.uint8)


def quantize_tensor(x: np.ndarray, scale: np.ndarray, zero: np.ndarray, bits: int = 4):
    """Quantize + pack 2 nibbles per byte (kernels/benchmark/benchmark.py:45-56).

    ``q = clamp(round(x/scale) + zero, 0, 15)`` in fp16; byte j holds dim 2j in
    the low nibble and dim 2j+1 in the high nibble.
    x float16 [KV, S, D] -> uint8 [KV, S, D/2].
    """
    x = np.asarray(x, dtype=np.float16)
    q_max = (1 << bits) - 1
    s = scale[:, None, :]
    z = zero[:, None, :]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = np.round(x / s) + z
    q = np.clip(q, np.float16(0), np.float16(q_max))
    q = _to_u8_codes(q)
    KV, S, D = x.shape
    q = q.reshape(KV, S, D // 2, 2)
    return (q[..., 0] | (q[..., 1] << 4)).astype(np.uint8)


def quantize_kv(k: np.ndarray, v: np.ndarray):
    """(k_packed, k_scale, k_zero, v_packed, v_scale, v_zero)
    (kernels/benchmark/benchmark.py:69-74)."""
    ks, kz = compute_scale_zero(k)
    kp = quantize_tensor(k, ks, kz)
    vs, vz = compute_scale_zero(v)
    vp = quantize_tensor(v, vs, vz)
    return kp, ks, kz, vp, vs, vz


# ---------------------------------------------------------------------------
# Per-token quantize-on-write store (kernels/kv_dequant_kernels.cuh:816-919)
# ---------------------------------------------------------------------------
def quantize_store(key: np.ndarray, value: np.ndarray, kv_cache: np.ndarray,
                   slot_mapping: np.ndarray, block_size: int) -> None:
    """In place: pack key/value [N, KV, D] fp16 into kv_cache
    [num_blocks, block_size, KV, D+8] uint8 at slot_mapping [N] int64."""
    key = np.ascontiguousarray(key, dtype=np.float16)
    value = np.ascontiguousarray(value, dtype=np.float16)
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    assert kv_cache.dtype == np.uint8 and kv_cache.flags.c_contiguous
    N, KV, D = key.shape
    assert kv_cache.shape[2] == KV and kv_cache.shape[3] == D + 8
    num_slots = kv_cache.shape[0] * kv_cache.shape[1]
    _clib().oracle_quantize_store(
        key.ctypes.data, value.ctypes.data, kv_cache.ctypes.data, slots.ctypes.data,
        N, KV, D, int(block_size), num_slots)


def quantize_row(row: np.ndarray):
    """One row of D fp16 values -> (packed uint8 [D/2], fp32 min, fp32 step)."""
    row = np.ascontiguousarray(row, dtype=np.float16)
    D = row.shape[0]
    out = np.zeros(D // 2, dtype=np.uint8)
    mn, st = ctypes.c_float(), ctypes.c_float()
    _clib().oracle_quantize_row(row.ctypes.data, D, out.ctypes.data,
                                ctypes.byref(mn), ctypes.byref(st))
    return out, np.float32(mn.value), np.float32(st.value)


def float_to_half_bits(x: float) -> int:
    """The C oracle's fp32 -> fp16 (nearest-even) conversion, as raw bits."""
    return int(_clib().oracle_float_to_half(ctypes.c_float(x)))


def split_slot(slot_bytes: np.ndarray, D: int):
    """Decode a [..., D+8] packed slot into (k_codes, v_codes, rulers).

    k/v codes: uint8 [..., D] (dim 2j low nibble, 2j+1 high nibble);
    rulers float16 [..., 4] = (k_min, k_step, v_min, v_step) from the
    little-endian bytes at D..D+8 (kernels/kv_dequant_kernels.cuh:511-518).
    """
    kb = slot_bytes[..., : D // 2]
    vb = slot_bytes[..., D // 2: D]
    rul = np.ascontiguousarray(slot_bytes[..., D: D + 8]).view(np.float16)
    return unpack_nibbles(kb), unpack_nibbles(vb), rul


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """uint8 [..., D/2] -> uint8 codes [..., D]; even dim = low nibble
    (kernels/kv_dequant_kernels.cuh:14-17)."""
    lo = packed & 0x0F
    hi = packed >> 4
    return np.stack([lo, hi], axis=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
