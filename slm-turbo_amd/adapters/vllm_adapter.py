"""vLLM attention backend for the packed 4-bit KV cache, on MI355X kernels.

Mirrors the backend surface of the reference's adapters/vllm_adapter.py:
* ``QuantizedKVAttentionImpl`` (reference :159-284): quantize-on-write
  (``do_kv_cache_update``), prefill with SDPA on the current chunk's fp16
  K/V, paged 4-bit decode;
* ``QuantizedKVAttentionBackend`` (:286-319): ``get_name() == "CUSTOM"``,
  ``get_impl_cls``, ``get_kv_cache_shape`` -> (num_blocks, block_size,
  num_kv_heads, head_size + 8) uint8, identity stride order;
* ``_patch_attention_layer_spec`` (:102-138): makes vLLM size each layer's
  cache pages at the packed slot;
* ``register_plugin`` (:329-336): the ``vllm.general_plugins`` entry point,
  idempotent.

Differences from the reference, on purpose:
* decode is ONE batched kernel launch per layer that reads vLLM's device
  ``seq_lens`` and ``block_table`` directly (int32 tables are read as they
  are): no per-request loop, no ``.tolist()`` host sync, no int64 copies;
  the result is written straight into vLLM's output buffer;
* a prefill chunk that continues cached context (the reference supports the
  first chunk only) attends over the packed cache: every query token is one
  sequence of the same batched launch (also one launch, no host sync);
* the vLLM-independent logic lives in ``PackedKVAttentionMixin`` so it runs
  without vLLM (tests drive it with a fake ``attn_metadata`` carrying
  ``seq_lens``, ``block_table``, ``num_actual_tokens``, ``max_query_len`` --
  the fields the reference reads at :214, :218, :262, :264);
* a missing kernel library raises instead of silently skipping the cache
  write (the cache is packed: no stock kernel can read it).

When vLLM is not importable the module still imports (degraded mode):
``VLLM_AVAILABLE`` is False, ``register_plugin()`` returns without
registering, and the two classes are defined on top of the mixin alone.
"""
from __future__ import annotations

import logging
from typing import Any, Optional

import torch

logger = logging.getLogger("slm_turbo.vllm_adapter")

VLLM_AVAILABLE = False
VLLM_IMPORT_ERROR: Optional[str] = None
try:  # optional heavy dependency
    import vllm  # noqa: F401

    if getattr(vllm, "__file__", None) is None:
        raise ImportError("vllm resolves to an empty namespace package")
    VLLM_AVAILABLE = True
except Exception as e:  # pragma: no cover - depends on the environment
    VLLM_IMPORT_ERROR = f"{type(e).__name__}: {e}"

SUPPORTED_HEAD_SIZES = (64, 80, 128)
# Decode attention served by the kernel in this process (diagnostics): query
# rows, one per request of a decode step, as the reference counts its
# per-request calls (adapters/vllm_adapter.py:63,279), and batched launches.
_KERNEL_CALLS = 0
_KERNEL_LAUNCHES = 0


def packed_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int) -> tuple:
    """Packed cache layout (reference adapters/vllm_adapter.py:300-308): per
    (block, position, KV head) a slot of head_size + 8 bytes -- K nibbles
    [0, D/2), V nibbles [D/2, D), fp16 k_min, k_step, v_min, v_step."""
    return (num_blocks, block_size, num_kv_heads, head_size + 8)


def packed_slot_bytes(head_size: int) -> int:
    return head_size + 8


class PackedKVAttentionMixin:
    """vLLM-independent part of the attention impl.

    Needs ``num_heads``, ``head_size``, ``num_kv_heads`` and ``scale`` on the
    instance (vLLM's impl base class sets them; the standalone class below
    takes them as arguments).
    """

    _slm_ops: Any = None

    def _slm_kernels(self):
        """The kernel entry points; raises if the HIP library is unusable."""
        if self._slm_ops is None:
            from kernels import kv_dequant
            from kernels import _native

            _native.load()                     # raises with the build hint if missing
            self._slm_ops = kv_dequant
        return self._slm_ops

    # ---- quantize-on-write: once per token batch, before forward ----------
    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        """Quantize fp16 K/V [N, KV, D] per token and store the packed slots
        at ``slot_mapping`` (reference :183-201).  Padding slots (< 0) are
        skipped by the kernel."""
        if kv_cache is None or kv_cache.numel() == 0:
            return
        kd = self._slm_kernels()
        kd.kv_quantize_store(key, value, kv_cache, slot_mapping, kv_cache.shape[1])

    # ---- forward ------------------------------------------------------------
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        """Attention for the step's tokens (reference :204-228): prefill when
        any request has more than one query token, else paged decode."""
        num_tokens = query.shape[0]
        if output is None:
            output = torch.zeros(num_tokens, self.num_heads * self.head_size, dtype=query.dtype,
                                 device=query.device)
        if attn_metadata is None:
            return output.fill_(0)
        N = int(attn_metadata.num_actual_tokens)
        if N <= 0:
            return output.fill_(0)
        q = query[:N]
        if int(attn_metadata.max_query_len) > 1:
            if self._one_first_chunk(attn_metadata):
                attn_out = self._prefill_attention(q, key[:N], value[:N], kv_cache, attn_metadata)
                self._store_output(output, attn_out, N)
            else:
                self._chunked_attention(q, kv_cache, attn_metadata, output, N)
        else:
            self._decode_attention(q, kv_cache, attn_metadata, output, N)
        return output

    @staticmethod
    def _store_output(output, attn_out, N):
        if output.ndim == 3:
            output[:N] = attn_out.to(output.dtype)
        else:
            output[:N] = attn_out.reshape(N, -1).to(output.dtype)

    # ---- prefill: SDPA on the chunk's fp16 K/V (first chunk) ----------------
    def _prefill_attention(self, query, key, value, kv_cache, attn_metadata):
        """Causal SDPA over the current chunk's raw K/V (reference :231-245),
        for steps whose requests have no earlier context; a continuation
        goes through _chunked_attention."""
        Hq, Hk = query.shape[1], key.shape[1]
        q_t = query.transpose(0, 1).unsqueeze(0)
        k_t = key.transpose(0, 1).unsqueeze(0)
        v_t = value.transpose(0, 1).unsqueeze(0)
        out = torch.nn.functional.scaled_dot_product_attention(
            q_t, k_t, v_t, is_causal=True, scale=self.scale, enable_gqa=Hk < Hq)
        return out[0].transpose(0, 1)

    # ---- chunked prefill continuing cached context -------------------------
    @staticmethod
    def _one_first_chunk(attn_metadata) -> bool:
        """True when a multi-token step is exactly one request's first chunk:
        one request (``query_start_loc`` has two entries) whose sequence is
        all query (host-side ``max_seq_len == max_query_len``).  Only then is
        one causal SDPA over all the step's tokens per-request attention; the
        reference applies it to every multi-token step (:216-220), where with
        two requests the later one attends to the earlier one's tokens and a
        continuation loses its cached context.  Both facts are host-side
        (a tensor shape and two ints): no device sync.  Metadata without
        ``query_start_loc``/``max_seq_len`` (the fields the reference reads,
        :214-218) is taken as one first chunk, as the reference takes it."""
        qsl = getattr(attn_metadata, "query_start_loc", None)
        max_seq_len = getattr(attn_metadata, "max_seq_len", None)
        if qsl is None or max_seq_len is None:
            return True
        return qsl.shape[0] - 1 == 1 and int(max_seq_len) == int(attn_metadata.max_query_len)

    def _chunked_attention(self, query, kv_cache, attn_metadata, output, N):
        """Every multi-token step other than one request's first chunk: first
        chunks of several requests, chunks that continue cached context and
        the decode tokens of the same step, over the packed cache (the
        reference leaves chunked continuation unsupported,
        adapters/vllm_adapter.py:238-239).  Query
        token i of request r sits at absolute position p = seq_len[r] -
        query_len[r] + (i - query_start[r]) and attends to tokens [0, p] of r,
        all of which this step's do_kv_cache_update has already written.  Each
        query token becomes one sequence of length p + 1 with r's block-table
        row: one batched launch, index arithmetic on the device, no host sync."""
        qsl = attn_metadata.query_start_loc.to(torch.int64)       # [R+1]
        R = qsl.numel() - 1
        tok = torch.arange(N, device=query.device, dtype=torch.int64)
        req = torch.searchsorted(qsl[1:].contiguous(), tok, right=True)   # request of each token
        qlen = (qsl[1:] - qsl[:-1])[req]
        seq = attn_metadata.seq_lens[:R].to(torch.int64)[req]
        pos = seq - qlen + (tok - qsl[:-1][req])
        tables = attn_metadata.block_table[:R][req]
        self._paged_attention(query, kv_cache, (pos + 1).to(torch.int32), tables, output, N)

    # ---- decode: one batched launch over every request ----------------------
    def _decode_attention(self, query, kv_cache, attn_metadata, output, N):
        """query [N, H, D] (one token per request), kv_cache [nb, bs, KV, D+8]
        uint8; reads attn_metadata.seq_lens [N] and .block_table [N, max]
        on the device.  Writes output[:N]."""
        self._paged_attention(query, kv_cache, attn_metadata.seq_lens[:N], attn_metadata.block_table[:N],
                              output, N)

    def _paged_attention(self, query, kv_cache, seq_lens, block_table, output, N):
        """One batched paged decode launch: query row n attends to the first
        seq_lens[n] tokens of block-table row n.  Writes output[:N] (in place
        when the output buffer allows)."""
        global _KERNEL_CALLS, _KERNEL_LAUNCHES
        kd = self._slm_kernels()
        block_size, num_kv_heads = kv_cache.shape[1], kv_cache.shape[2]
        if seq_lens.dtype != torch.int32:
            seq_lens = seq_lens.to(torch.int32)
        H, D = self.num_heads, self.head_size
        out3 = None
        if output.dtype in (torch.float16, torch.float32) and output.is_contiguous():
            out3 = output[:N].view(N, H, D)        # written in place
        res = kd.kv_dequant_decode_paged_batched(query, kv_cache, block_table, seq_lens, block_size,
                                                 num_kv_heads, out=out3,
                                                 out_dtype=None if out3 is not None else torch.float32)
        if out3 is None:
            self._store_output(output, res, N)
        _KERNEL_CALLS += N
        _KERNEL_LAUNCHES += 1
        if not getattr(self, "_slm_logged", False):       # once per layer implementation, as the reference
            self._slm_logged = True
            logger.info("slm-turbo 4-bit decode kernel serving inside vLLM (head_size=%d)", self.head_size)


# ---------------------------------------------------------------------------
# vLLM registration (only where vLLM is importable)
# ---------------------------------------------------------------------------
_BACKEND_REGISTERED = False
_SPEC_PATCHED = False


def _patch_attention_layer_spec() -> bool:
    """Make vLLM allocate each CUSTOM-backend layer's cache at the packed
    slot size (reference :102-138): wrap ``Attention.get_kv_cache_spec`` to
    return a spec whose page holds head_size + 8 bytes per (position, KV
    head) in uint8.  Idempotent; False when the vLLM API is not there."""
    global _SPEC_PATCHED
    if _SPEC_PATCHED:
        return True
    try:
        from vllm.model_executor.layers.attention.attention import Attention
        from vllm.v1.kv_cache_interface import TQFullAttentionSpec
    except Exception as e:
        logger.warning("packed-cache spec patch unavailable (%s)", e)
        return False
    original = Attention.get_kv_cache_spec

    def get_kv_cache_spec(self, vllm_config):
        spec = original(self, vllm_config)
        backend = getattr(self, "attn_backend", None)
        if backend is not None and backend.get_name() == "CUSTOM":
            return TQFullAttentionSpec(
                block_size=spec.block_size, num_kv_heads=self.num_kv_heads, head_size=self.head_size,
                head_size_v=self.head_size_v, dtype=torch.uint8, kv_quant_mode=spec.kv_quant_mode,
                tq_slot_size=packed_slot_bytes(self.head_size))
        return spec

    Attention.get_kv_cache_spec = get_kv_cache_spec
    _SPEC_PATCHED = True
    return True


def _define_vllm_classes():
    """Impl and backend on top of vLLM's Triton backend (metadata builder,
    paged bookkeeping); None on interface drift."""
    try:
        from vllm.v1.attention.backends.triton_attn import TritonAttentionBackend, TritonAttentionImpl
    except Exception as e:
        logger.warning("vLLM attention API not found (%s); CUSTOM backend disabled", e)
        return None

    class _Impl(PackedKVAttentionMixin, TritonAttentionImpl):
        """Packed 4-bit KV cache: quantize-on-write + batched paged decode."""

        def __init__(self, *args, **kwargs):
            super().__init__(*args, **kwargs)
            self._slm_kernels()                # fail at construction, not mid-step

    class _Backend(TritonAttentionBackend):
        @staticmethod
        def get_name() -> str:
            return "CUSTOM"

        @staticmethod
        def get_impl_cls() -> type:
            return _Impl

        @staticmethod
        def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                               cache_dtype_str: str = "auto") -> tuple:
            return packed_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size)

        @staticmethod
        def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple:
            raise NotImplementedError   # physical layout == logical layout

        @classmethod
        def supports_batch_invariance(cls) -> bool:
            return True

    _Impl.__name__ = _Impl.__qualname__ = "QuantizedKVAttentionImpl"
    _Backend.__name__ = _Backend.__qualname__ = "QuantizedKVAttentionBackend"
    return _Impl, _Backend


class _StandaloneImpl(PackedKVAttentionMixin):
    """The impl without vLLM: the attributes vLLM's base class would set."""

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: Optional[int] = None,
                 **_: Any):
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads or num_heads


class _StandaloneBackend:
    """The backend's static surface without vLLM."""

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls() -> type:
        return QuantizedKVAttentionImpl

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple:
        return packed_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size)

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple:
        raise NotImplementedError

    @classmethod
    def supports_batch_invariance(cls) -> bool:
        return True


_classes = _define_vllm_classes() if VLLM_AVAILABLE else None
if _classes is not None:
    QuantizedKVAttentionImpl, QuantizedKVAttentionBackend = _classes
else:
    QuantizedKVAttentionImpl = _StandaloneImpl
    QuantizedKVAttentionImpl.__name__ = QuantizedKVAttentionImpl.__qualname__ = "QuantizedKVAttentionImpl"
    QuantizedKVAttentionBackend = _StandaloneBackend
    QuantizedKVAttentionBackend.__name__ = QuantizedKVAttentionBackend.__qualname__ = "QuantizedKVAttentionBackend"


def _register_custom_backend() -> bool:
    """Register QuantizedKVAttentionBackend as vLLM's CUSTOM backend
    (reference :140-327).  False without vLLM or on interface drift."""
    global _BACKEND_REGISTERED
    if _BACKEND_REGISTERED:
        return True
    if not VLLM_AVAILABLE or _classes is None:
        return False
    try:
        from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend
    except Exception as e:  # interface drift
        logger.warning("vLLM backend registry not found (%s)", e)
        return False
    _patch_attention_layer_spec()
    register_backend(AttentionBackendEnum.CUSTOM, f"{__name__}.QuantizedKVAttentionBackend")
    _BACKEND_REGISTERED = True
    logger.info("slm-turbo packed 4-bit KV backend registered as --attention-backend CUSTOM")
    return True


def register_plugin() -> None:
    """``vllm.general_plugins`` entry point (reference :329-336): runs in
    every vLLM process; idempotent; a no-op in degraded mode."""
    if not _register_custom_backend() and not VLLM_AVAILABLE:
        logger.info("vLLM not importable (%s): CUSTOM backend not registered", VLLM_IMPORT_ERROR)


def backend_status() -> dict:
    """What this process can do: vLLM present, backend registered, kernel
    library loadable (with the error if not)."""
    status = {"vllm_available": VLLM_AVAILABLE, "vllm_error": VLLM_IMPORT_ERROR,
              "backend_registered": _BACKEND_REGISTERED, "kernel_calls": _KERNEL_CALLS,
              "kernel_launches": _KERNEL_LAUNCHES}
    try:
        from kernels import _native

        _native.load()
        status["kernels"] = True
    except Exception as e:
        status["kernels"] = False
        status["kernels_error"] = f"{type(e).__name__}: {e}"
    return status
