# =============================================================================
#  kernels/kv_dequant.py  (MI355X / gfx950)
#
#  Fused 4-bit KV-quantized attention kernels -- HIP, hand-written for CDNA4.
#
#  Python API, signature-compatible with the reference's kernels/kv_dequant.py:
#
#      kv_dequant_decode_attention(...)                 -> [H, 1, D] fp32
#      kv_dequant_prefill_attention(...)                -> [H, M, D] fp32
#      kv_dequant_decode_per_token_attention(...)       -> [H, 1, D] fp32
#      kv_dequant_decode_per_token_paged_attention(...) -> [H, 1, D] fp32
#      kv_quantize_store(...)                           -> None (writes cache)
#
#  plus the batched paged decode the vLLM backend uses (one launch per layer
#  for the whole batch) and the per-channel quantizer on the GPU:
#
#      kv_dequant_decode_paged_batched(...)             -> [B, H, D]
#      quantize_per_channel(x) / quantize_kv(k, v)
#
#  The device code is libslmturbo_hip.so (slm-turbo_amd/csrc), reached through
#  its C ABI (include/slmturbo.h) with ctypes; launches go to the current torch
#  stream.  There is no CPU path: like the reference, calls raise when the
#  native library or a GPU is unavailable.
# =============================================================================
from __future__ import annotations

import contextlib
import math
import threading

import torch

from . import _native

__all__ = [
    "kv_dequant_decode_attention",
    "kv_dequant_prefill_attention",
    "kv_dequant_decode_per_token_attention",
    "kv_quantize_store",
    "kv_dequant_decode_per_token_paged_attention",
    "kv_dequant_decode_paged_batched",
    "quantize_per_channel",
    "quantize_kv",
]

_SUPPORTED_D = (64, 80, 128)


def _load_native_extension():
    """Load (once) the HIP library; a failure is cached and re-raised
    (reference kernels/kv_dequant.py:47-86)."""
    return _native.load()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_fast_mod = None
_fast_checked = False


def _fastcall():
    """The METH_FASTCALL binding of the store and batched decode (None when it
    was not built: the ctypes functions of the same library are used then)."""
    global _fast_mod, _fast_checked
    if not _fast_checked:
        _fast_mod = _native.fast()
        _fast_checked = True
    return _fast_mod
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _stream(device: torch.device) -> int:
    """The current torch stream of ``device`` as a raw hipStream_t."""
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device() if device.index is None else device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


# Workspace per (device, stream): zero-filled once; the kernels leave their
# arrival counters at zero, so calls ordered on one stream can share it.
_ws_lock = threading.Lock()
_ws_cache: dict = {}


# Workspace bytes per (device, B, H, KV, D): the plan depends only on these.
_need_cache: dict = {}


def _workspace(lib, device: torch.device, B: int, H: int, KV: int, D: int,
               stream: int | None = None) -> tuple[int, int]:
    nkey = (device.index, B, H, KV, D)
    need = _need_cache.get(nkey)
    if need is None:
        need = int(lib.slmt_attention_workspace_bytes(B, H, KV, D))
        if need < 0:
            raise RuntimeError(_native.last_error(lib))
        _need_cache[nkey] = need
    key = (device.index, _stream(device) if stream is None else stream)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < need:
        with _ws_lock:
            buf = _ws_cache.get(key)
            if buf is None or buf.numel() < need:
                buf = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=device)
                _ws_cache[key] = buf
    return buf.data_ptr(), buf.numel()


def _on_device(dev: torch.device):
    """Make ``dev`` current for the call (no switch when it already is)."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_common(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero, phase, num_kv_heads):
    """Native-side validation (reference kernels/kv_dequant_cuda.cu:53-76)."""
    _require(q.is_cuda, f"{phase}: q must be a CUDA tensor")
    _require(q.dtype == torch.float16, f"{phase}: q must be fp16")
    _require(k_packed.is_cuda and v_packed.is_cuda, f"{phase}: packed KV must be CUDA tensors")
    _require(k_packed.dtype == torch.uint8 and v_packed.dtype == torch.uint8, f"{phase}: packed KV must be uint8")
    for t in (k_scale, k_zero, v_scale, v_zero):
        _require(t.is_cuda and t.dtype == torch.float16, f"{phase}: scale/zero tensors must be fp16 CUDA")
    D, D2 = q.size(2), k_packed.size(2)
    _require(D == 2 * D2, f"{phase}: D ({D}) must be 2 * D2 ({D2})")
    H = q.size(0)
    _require(num_kv_heads > 0 and H % num_kv_heads == 0,
             f"{phase}: num_kv_heads {num_kv_heads} must divide query heads {H}")


# =============================================================================
#  DECODE attention (per-channel)
# =============================================================================
def kv_dequant_decode_attention(
    q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero,
    BLOCK_N=64, use_quant=True, num_kv_heads=None,
):
    """Fused 4-bit per-channel decode.  Returns [H, 1, D] fp32.

    Same arguments and checks as the reference (kernels/kv_dequant.py:92-123):
        q [H, 1, D] fp16; k/v_packed [KV, S, D//2] uint8; k/v_scale, k/v_zero
        [KV, D] fp16; BLOCK_N in (32, 64); use_quant False attends over raw
        nibbles; num_kv_heads defaults to k_packed.shape[0].
    """
    H, _, D = q.shape
    KV, S, D2 = k_packed.shape
    assert D == D2 * 2, f"D {D} != 2*D2 {D2}"
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    assert BLOCK_N in (32, 64), f"BLOCK_N must be 32 or 64, got {BLOCK_N}"
    num_kv_heads = KV if num_kv_heads is None else num_kv_heads
    assert H % num_kv_heads == 0, f"H {H} not divisible by num_kv_heads {num_kv_heads}"
    assert q.shape == (H, 1, D), f"q {q.shape} != {(H, 1, D)}"

    lib = _load_native_extension()
    phase = "kv_dequant_decode"
    _check_common(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero, phase, num_kv_heads)
    _require(num_kv_heads <= KV, f"{phase}: num_kv_heads {num_kv_heads} exceeds the packed KV heads {KV}")
    dev = q.device
    with _on_device(dev):
        out = torch.empty((H, 1, D), dtype=torch.float32, device=dev)
        if S == 0:  # the reference divides 0 by 0
            return out.fill_(math.nan)
        q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero = (
            t.contiguous() for t in (q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero))
        ws, ws_bytes = _workspace(lib, dev, 1, H, num_kv_heads, D)
        rc = lib.slmt_decode_per_channel(
            _ptr(q), _ptr(k_packed), _ptr(k_scale), _ptr(k_zero), _ptr(v_packed), _ptr(v_scale),
            _ptr(v_zero), H, KV, num_kv_heads, S, D, BLOCK_N, int(bool(use_quant)), _ptr(out),
            ws, ws_bytes, _stream(dev))
        _native.check(lib, rc)
    return out


# =============================================================================
#  PREFILL attention (per-channel)
# =============================================================================
def kv_dequant_prefill_attention(
    q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero,
    BLOCK_M=None, BLOCK_N=None, causal=True, use_quant=True, num_kv_heads=None,
):
    """Fused 4-bit per-channel prefill.  Returns [H, M, D] fp32.

    Same arguments, defaults and tile checks as the reference
    (kernels/kv_dequant.py:129-177).  BLOCK_M/BLOCK_N are validated for API
    compatibility; they do not change the result.  With causal=True query m
    sees keys n <= m (both indexed from 0).
    """
    H, M, D = q.shape
    KV, S, D2 = k_packed.shape
    assert D == D2 * 2, f"D {D} != 2*D2 {D2}"
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    assert q.device == k_packed.device
    num_kv_heads = KV if num_kv_heads is None else num_kv_heads
    assert H % num_kv_heads == 0, f"H {H} not divisible by num_kv_heads {num_kv_heads}"
    if BLOCK_M is None:
        BLOCK_M = 16
    if BLOCK_N is None:
        BLOCK_N = 64 if D == 64 else 32
    assert BLOCK_M in (16, 32), f"BLOCK_M must be 16 or 32, got {BLOCK_M}"
    assert BLOCK_N in (32, 64), f"BLOCK_N must be 32 or 64, got {BLOCK_N}"
    if D != 64:
        assert (BLOCK_M, BLOCK_N) == (16, 32), (
            f"head_dim {D}: only (BLOCK_M=16, BLOCK_N=32) fits the "
            f"48 KB shared budget; got ({BLOCK_M}, {BLOCK_N})"
        )

    lib = _load_native_extension()
    phase = "kv_dequant_prefill"
    _check_common(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero, phase, num_kv_heads)
    _require(q.dim() == 3, f"{phase}: q must be [H, M, D], got {list(q.shape)}")
    _require(num_kv_heads <= KV, f"{phase}: num_kv_heads {num_kv_heads} exceeds the packed KV heads {KV}")
    dev = q.device
    with _on_device(dev):
        out = torch.empty((H, M, D), dtype=torch.float32, device=dev)
        if M == 0:
            return out
        if S == 0:
            return out.fill_(math.nan)
        q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero = (
            t.contiguous() for t in (q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero))
        ws, ws_bytes = _workspace(lib, dev, M, H, num_kv_heads, D)
        rc = lib.slmt_prefill_per_channel(
            _ptr(q), _ptr(k_packed), _ptr(k_scale), _ptr(k_zero), _ptr(v_packed), _ptr(v_scale),
            _ptr(v_zero), H, KV, num_kv_heads, M, S, D, BLOCK_M, BLOCK_N, int(bool(causal)),
            int(bool(use_quant)), _ptr(out), ws, ws_bytes, _stream(dev))
        _native.check(lib, rc)
    return out


# =============================================================================
#  PER-TOKEN DECODE attention  (contiguous per-token buffers)
# =============================================================================
def kv_dequant_decode_per_token_attention(
    q, k_packed, k_min, k_step, v_packed, v_min, v_step,
    BLOCK_N=64, num_kv_heads=None,
):
    """Per-token (min, step) decode over contiguous buffers.  Returns [H, 1, D]
    fp32 (reference kernels/kv_dequant.py:189-217).

        q [H, 1, D] fp16; k/v_packed [KV, S, D//2] uint8;
        k/v_min, k/v_step [KV, S] fp16; value = nibble * step + min.
    """
    H, _, D = q.shape
    KV, S, D2 = k_packed.shape
    assert D == D2 * 2, f"D {D} != 2*D2 {D2}"
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    assert BLOCK_N in (32, 64), f"BLOCK_N must be 32 or 64, got {BLOCK_N}"
    num_kv_heads = KV if num_kv_heads is None else num_kv_heads
    assert H % num_kv_heads == 0, f"H {H} not divisible by num_kv_heads {num_kv_heads}"

    lib = _load_native_extension()
    phase = "per-token decode"
    _require(q.is_cuda and q.dtype == torch.float16, f"{phase}: q must be fp16 CUDA")
    _require(q.dim() == 3 and q.size(1) == 1, f"{phase}: q must be [H, 1, D], got {list(q.shape)}")
    _require(k_packed.is_cuda and v_packed.is_cuda and k_packed.dtype == torch.uint8
             and v_packed.dtype == torch.uint8, f"{phase}: packed KV must be uint8 CUDA tensors")
    for t in (k_min, k_step, v_min, v_step):
        _require(t.is_cuda and t.dtype == torch.float16 and tuple(t.shape) == (KV, S),
                 f"{phase}: min/step tensors must be fp16 CUDA [KV, S]")
    _require(num_kv_heads <= KV, f"{phase}: num_kv_heads {num_kv_heads} exceeds the packed KV heads {KV}")
    dev = q.device
    with _on_device(dev):
        out = torch.empty((H, 1, D), dtype=torch.float32, device=dev)
        if S == 0:
            return out.fill_(math.nan)
        q, k_packed, k_min, k_step, v_packed, v_min, v_step = (
            t.contiguous() for t in (q, k_packed, k_min, k_step, v_packed, v_min, v_step))
        ws, ws_bytes = _workspace(lib, dev, 1, H, num_kv_heads, D)
        rc = lib.slmt_decode_per_token(
            _ptr(q), _ptr(k_packed), _ptr(k_min), _ptr(k_step), _ptr(v_packed), _ptr(v_min),
            _ptr(v_step), H, KV, num_kv_heads, S, D, BLOCK_N, _ptr(out), ws, ws_bytes, _stream(dev))
        _native.check(lib, rc)
    return out


# =============================================================================
#  QUANTIZE-ON-WRITE store into the packed paged cache
# =============================================================================
def kv_quantize_store(key, value, kv_cache, slot_mapping, block_size):
    """Quantize-on-write: pack fp16 K/V rows into the 4-bit cache slots
    (reference kernels/kv_dequant.py:220-233).

        key, value:   [N, KV, D] fp16 (rows may be strided over tokens)
        kv_cache:     [num_blocks, block_size, KV, D+8] uint8, contiguous
        slot_mapping: [N] int64; slot < 0 is skipped
        block_size:   the cache's block size
    """
    assert key.dim() == 3, f"key must be [N, KV, D], got {key.shape}"
    assert kv_cache.is_contiguous(), "kv_cache must be contiguous"
    lib = _load_native_extension()
    # Called once per layer and step: every check reads each attribute once and
    # formats its message only when it fails.
    if not (key.is_cuda and value.is_cuda and key.dtype is torch.float16 and value.dtype is torch.float16):
        raise RuntimeError("store: key/value must be fp16 CUDA")
    if kv_cache.dtype is not torch.uint8:
        raise RuntimeError("store: kv_cache must be uint8")
    kshape = key.shape
    N, KV, D = kshape
    if D not in _SUPPORTED_D:
        raise RuntimeError(f"store: head_dim must be 64/80/128, got {D}")
    SLOT = D + 8
    cshape = kv_cache.shape
    if cshape[-1] != SLOT:
        raise RuntimeError(f"store: cache slot size {cshape[-1]} != expected {SLOT}")
    if slot_mapping.dtype is not torch.int64 or slot_mapping.numel() != N:
        raise RuntimeError("store: slot_mapping must be int64 of length N")
    if value.shape != kshape:
        raise RuntimeError(f"store: value must be [N, KV, D] like key, got {list(value.shape)}")
    if len(cshape) != 4 or cshape[2] != KV or cshape[1] != block_size:
        raise RuntimeError(f"store: kv_cache must be [num_blocks, {block_size}, {KV}, {SLOT}], got {list(cshape)}")
    # token-strided rows are read in place; anything else is made contiguous
    ks, vs = key.stride(), value.stride()
    if not (ks[2] == 1 and ks[1] == D and ks[0] % 2 == 0):
        key, ks = key.contiguous(), (KV * D,)
    if not (vs[2] == 1 and vs[1] == D and vs[0] % 2 == 0):
        value, vs = value.contiguous(), (KV * D,)
    if not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.contiguous()
    di = key.get_device()
    args = (key.data_ptr(), ks[0], value.data_ptr(), vs[0], kv_cache.data_ptr(), cshape[0], int(block_size),
            slot_mapping.data_ptr(), N, KV, D)
    fast = _fastcall()
    if _raw_stream is not None and di == _current_device():
        stream = _raw_stream(di)
        rc = fast.quantize_store(*args, stream) if fast else lib.slmt_quantize_store(*args, stream)
    else:
        with torch.cuda.device(di):
            rc = lib.slmt_quantize_store(*args, _stream(key.device))
    if rc:
        _native.check(lib, rc)


# =============================================================================
#  PAGED PER-TOKEN DECODE (one request, reference API)
# =============================================================================
def kv_dequant_decode_per_token_paged_attention(
    q, kv_cache, block_table, seq_len, block_size, num_kv_heads,
):
    """Paged per-token decode for one request, reading the packed cache through
    its block table.  Returns [H, 1, D] fp32
    (reference kernels/kv_dequant.py:236-257).

        q [H, 1, D] fp16; kv_cache [num_blocks, block_size, KV, D+8] uint8;
        block_table [max_blocks] int64 (int32 accepted); seq_len, block_size,
        num_kv_heads ints.
    """
    H, _, D = q.shape
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    assert H % num_kv_heads == 0, f"H {H} not divisible by num_kv_heads {num_kv_heads}"
    assert kv_cache.size(-1) == D + 8, f"cache slot must be D+8, got {kv_cache.size(-1)}"
    lib = _load_native_extension()
    _require(q.is_cuda and q.dtype == torch.float16, "paged decode: q must be fp16 CUDA")
    _require(q.dim() == 3 and q.size(1) == 1, f"paged decode: q must be [H, 1, D], got {list(q.shape)}")
    _require(kv_cache.dtype == torch.uint8, "paged decode: kv_cache must be uint8")
    _require(kv_cache.size(-1) == D + 8, "paged decode: cache slot size must be D+8")
    _require(kv_cache.dim() == 4 and kv_cache.size(2) == num_kv_heads,
             f"paged decode: kv_cache must be [num_blocks, block_size, {num_kv_heads}, {D + 8}]")
    _require(block_table.dtype in (torch.int64, torch.int32), "paged decode: block_table must be int64 or int32")
    seq_len = int(seq_len)
    dev = q.device
    with _on_device(dev):
        out = torch.empty((H, 1, D), dtype=torch.float32, device=dev)
        if seq_len <= 0:
            return out.fill_(math.nan)
        _require(block_table.numel() * int(block_size) >= seq_len,
                 f"paged decode: block_table holds {block_table.numel()} blocks, fewer than seq_len {seq_len} needs")
        q = q.contiguous()
        kv_cache = kv_cache.contiguous()
        block_table = block_table.to(device=dev, dtype=torch.int64).contiguous()
        ws, ws_bytes = _workspace(lib, dev, 1, H, num_kv_heads, D)
        rc = lib.slmt_decode_paged(
            _ptr(q), _ptr(kv_cache), kv_cache.size(0), int(block_size), _ptr(block_table), seq_len,
            H, num_kv_heads, D, _ptr(out), ws, ws_bytes, _stream(dev))
        _native.check(lib, rc)
    return out


# =============================================================================
#  BATCHED PAGED DECODE (one launch for a whole decode batch)
# =============================================================================
def kv_dequant_decode_paged_batched(
    q, kv_cache, block_tables, seq_lens, block_size, num_kv_heads, out=None, out_dtype=None,
):
    """Paged per-token decode for a batch in ONE launch.  Returns [B, H, D].

    The batched form of ``kv_dequant_decode_per_token_paged_attention`` that the
    vLLM backend calls once per layer instead of once per request
    (reference adapters/vllm_adapter.py:271-279):
        q            [B, H, D] fp16 (strides: any, with unit stride over D)
        kv_cache     [num_blocks, block_size, KV, D+8] uint8
        block_tables [B, max_blocks] int32 or int64 (device)
        seq_lens     [B] int32 (device; read by the kernel, no host sync)
        out          optional [B, H, D] fp32/fp16 tensor written in place
        out_dtype    fp32 (default) or fp16 when ``out`` is not given
    Sequences of length 0 produce zeros.
    """
    assert q.dim() == 3, f"q must be [B, H, D], got {tuple(q.shape)}"
    B, H, D = q.shape
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    assert H % num_kv_heads == 0, f"H {H} not divisible by num_kv_heads {num_kv_heads}"
    cshape = kv_cache.shape
    assert cshape[-1] == D + 8, f"cache slot must be D+8, got {cshape[-1]}"
    lib = _load_native_extension()
    # Called once per layer and step: every check reads each attribute once and
    # formats its message only when it fails.
    if not (q.is_cuda and q.dtype is torch.float16):
        raise RuntimeError("paged decode: q must be fp16 CUDA")
    if not (kv_cache.is_cuda and kv_cache.dtype is torch.uint8 and kv_cache.is_contiguous()):
        raise RuntimeError("paged decode: kv_cache must be a contiguous uint8 CUDA tensor")
    if not (len(cshape) == 4 and cshape[1] == block_size and cshape[2] == num_kv_heads):
        raise RuntimeError(f"paged decode: kv_cache must be [num_blocks, {block_size}, {num_kv_heads}, {D + 8}]")
    bt_dtype = block_tables.dtype
    bt_stride = block_tables.stride()
    if not (block_tables.dim() == 2 and block_tables.size(0) == B and bt_stride[1] == 1
            and (bt_dtype is torch.int32 or bt_dtype is torch.int64) and block_tables.is_cuda):
        raise RuntimeError("paged decode: block_tables must be an int32/int64 CUDA tensor [B, max_blocks]")
    if not (seq_lens.is_cuda and seq_lens.dtype is torch.int32 and seq_lens.numel() == B):
        raise RuntimeError("paged decode: seq_lens must be an int32 CUDA tensor [B]")
    dev = q.device
    with _on_device(dev):
        if out is None:
            out = torch.empty((B, H, D), dtype=out_dtype or torch.float32, device=dev)
        out_dtype = out.dtype
        out_stride = out.stride()
        if not ((out_dtype is torch.float32 or out_dtype is torch.float16) and out.shape == (B, H, D)
                and out_stride[2] == 1):
            raise RuntimeError("paged decode: out must be fp32/fp16 [B, H, D] with unit stride over D")
        if B == 0:
            return out
        qs = q.stride()
        if qs[2] != 1 or qs[1] % 8 or qs[0] % 8 or q.data_ptr() % 16:
            q = q.contiguous()
            qs = q.stride()
        seq_lens = seq_lens.contiguous()
        stream = _stream(dev)
        ws, ws_bytes = _workspace(lib, dev, B, H, num_kv_heads, D, stream)
        fast = _fastcall()
        rc = (fast.decode_paged_batched if fast else lib.slmt_decode_paged_batched)(
            q.data_ptr(), qs[0], qs[1], kv_cache.data_ptr(), cshape[0], int(block_size),
            block_tables.data_ptr(), 64 if bt_dtype is torch.int64 else 32, bt_stride[0],
            seq_lens.data_ptr(), 0, B, H, num_kv_heads, D, out.data_ptr(),
            _native.OUT_F16 if out_dtype is torch.float16 else _native.OUT_F32,
            out_stride[0], out_stride[1], ws, ws_bytes, stream)
        if rc:
            _native.check(lib, rc)
    return out


# =============================================================================
#  PER-CHANNEL QUANTIZER on the GPU
# =============================================================================
def quantize_per_channel(x):
    """Per-channel asymmetric 4-bit quantizer of the standalone path, on the GPU.

    Bit-exact with the reference's host torch code
    (kernels/benchmark/benchmark.py:26-56):  x [KV, S, D] fp16 ->
    (packed [KV, S, D//2] uint8, scale [KV, D] fp16, zero [KV, D] fp16).
    """
    assert x.dim() == 3, f"x must be [KV, S, D], got {tuple(x.shape)}"
    KV, S, D = x.shape
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    lib = _load_native_extension()
    _require(x.is_cuda and x.dtype == torch.float16, "quantize: x must be fp16 CUDA")
    _require(S >= 1, "quantize: the sequence axis must not be empty")
    dev = x.device
    with _on_device(dev):
        x = x.contiguous()
        packed = torch.empty((KV, S, D // 2), dtype=torch.uint8, device=dev)
        scale = torch.empty((KV, D), dtype=torch.float16, device=dev)
        zero = torch.empty((KV, D), dtype=torch.float16, device=dev)
        rc = lib.slmt_quantize_per_channel(_ptr(x), KV, S, D, _ptr(packed), _ptr(scale), _ptr(zero),
                                           _stream(dev))
        _native.check(lib, rc)
    return packed, scale, zero


def quantize_tensor(x, scale, zero_point, bits=4, out=None):
    """Quantize + pack with given (fixed) rulers, on the GPU: the reference's
    quantize_tensor (kernels/benchmark/benchmark.py:45-56), which its model
    harness uses to append new tokens with the rulers frozen at the first
    decode (:213-216).

        x:           [KV, S, D] fp16 (unit stride over D)
        scale, zero_point: [KV, D] fp16, e.g. from quantize_per_channel
        out:         optional uint8 [KV, S, D//2] (unit stride over the last
                     dim), e.g. ``cache[:, prev:n]``, written in place
    Returns the packed codes; bit-exact with the reference's fp16 torch code.
    """
    assert bits == 4, "only 4-bit packing is supported"
    assert x.dim() == 3, f"x must be [KV, S, D], got {tuple(x.shape)}"
    KV, S, D = x.shape
    assert D in (64, 80, 128), f"head_dim must be 64/80/128, got {D}"
    lib = _load_native_extension()
    if not (x.is_cuda and x.dtype is torch.float16):
        raise RuntimeError("quantize_tensor: x must be fp16 CUDA")
    for t in (scale, zero_point):
        if not (t.is_cuda and t.dtype is torch.float16 and tuple(t.shape) == (KV, D)):
            raise RuntimeError(f"quantize_tensor: scale/zero_point must be fp16 CUDA [{KV}, {D}]")
    dev = x.device
    with _on_device(dev):
        if out is None:
            out = torch.empty((KV, S, D // 2), dtype=torch.uint8, device=dev)
        if not (out.is_cuda and out.dtype is torch.uint8 and tuple(out.shape) == (KV, S, D // 2)
                and (S == 0 or out.stride(2) == 1)):
            raise RuntimeError(f"quantize_tensor: out must be uint8 [{KV}, {S}, {D // 2}] with unit stride over the last dim")
        xs = x.stride()
        if xs[2] != 1 or xs[1] % 2 or xs[0] % 2 or x.data_ptr() % 4:
            x = x.contiguous()
            xs = x.stride()
        scale, zero_point = scale.contiguous(), zero_point.contiguous()
        os_ = out.stride()
        rc = lib.slmt_quantize_with_rulers(x.data_ptr(), xs[0], xs[1], KV, S, D, scale.data_ptr(),
                                           zero_point.data_ptr(), out.data_ptr(), os_[0], os_[1], _stream(dev))
        if rc:
            _native.check(lib, rc)
    return out


def quantize_kv(k, v):
    """(k_packed, k_scale, k_zero, v_packed, v_scale, v_zero), like the
    reference's quantize_kv (kernels/benchmark/benchmark.py:69-74)."""
    kp, ks, kz = quantize_per_channel(k)
    vp, vs, vz = quantize_per_channel(v)
    return kp, ks, kz, vp, vs, vz
