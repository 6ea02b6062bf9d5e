"""vLLM backend surface (reference adapters/vllm_adapter.py:102-336) without vLLM.

CPU tests drive the backend with a fake ``attn_metadata`` (the fields the
reference reads: seq_lens, block_table, num_actual_tokens, max_query_len)
and a recording stand-in for the kernel module, to check the static surface,
degraded mode and the dispatch (one batched decode launch per layer, the
store's arguments, prefill routing).  GPU tests run the real kernels through
the backend against the oracle.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from adapters import vllm_adapter as va
from common import assert_close, make_paged_case, paged_reference
from oracle import quant as oq


class _RecordingKernels:
    """Stand-in for kernels.kv_dequant that records calls."""

    def __init__(self):
        self.decode_calls = []
        self.store_calls = []

    def kv_dequant_decode_paged_batched(self, q, kv_cache, block_tables, seq_lens, block_size, num_kv_heads,
                                        out=None, out_dtype=None):
        self.decode_calls.append(dict(q=q, kv_cache=kv_cache, block_tables=block_tables, seq_lens=seq_lens,
                                      block_size=block_size, num_kv_heads=num_kv_heads, out=out))
        res = torch.full(q.shape, 0.5, dtype=out.dtype if out is not None else (out_dtype or torch.float32))
        if out is not None:
            out.copy_(res)
            return out
        return res

    def kv_quantize_store(self, key, value, kv_cache, slot_mapping, block_size):
        self.store_calls.append(dict(key=key, value=value, kv_cache=kv_cache, slot_mapping=slot_mapping,
                                     block_size=block_size))


def _impl(H=8, D=64, KV=2, kernels=None):
    impl = va.QuantizedKVAttentionImpl(num_heads=H, head_size=D, scale=D ** -0.5, num_kv_heads=KV)
    if kernels is not None:
        impl._slm_ops = kernels
    return impl


def _meta(seq_lens, block_table, max_query_len=1, n=None):
    seq_lens = torch.as_tensor(seq_lens, dtype=torch.int32)
    return SimpleNamespace(seq_lens=seq_lens, block_table=torch.as_tensor(block_table, dtype=torch.int32),
                           num_actual_tokens=len(seq_lens) if n is None else n, max_query_len=max_query_len)


# ---------------------------------------------------------------- static surface
def test_backend_static_surface():
    B = va.QuantizedKVAttentionBackend
    assert B.get_name() == "CUSTOM"
    assert B.get_impl_cls() is va.QuantizedKVAttentionImpl
    assert B.get_kv_cache_shape(100, 16, 8, 128) == (100, 16, 8, 136)
    assert B.get_kv_cache_shape(7, 32, 2, 64, "auto") == (7, 32, 2, 72)
    assert B.supports_batch_invariance() is True
    with pytest.raises(NotImplementedError):
        B.get_kv_cache_stride_order()
    assert va.packed_slot_bytes(80) == 88
    assert va.SUPPORTED_HEAD_SIZES == (64, 80, 128)


def test_degraded_mode_without_vllm():
    assert not va.VLLM_AVAILABLE and va.VLLM_IMPORT_ERROR
    assert va.register_plugin() is None        # no vLLM: nothing registered, no exception
    assert va.register_plugin() is None        # idempotent
    assert va._register_custom_backend() is False
    assert va._patch_attention_layer_spec() is False
    st = va.backend_status()
    assert st["vllm_available"] is False and st["backend_registered"] is False
    assert {"kernels", "kernel_calls"} <= set(st)


def test_impl_needs_the_kernel_library(monkeypatch):
    from kernels import _native

    def broken():
        raise RuntimeError("slm-turbo HIP library not found at /nowhere")
    monkeypatch.setattr(_native, "load", broken)
    impl = _impl()
    with pytest.raises(RuntimeError, match="library not found"):
        impl.do_kv_cache_update(None, torch.zeros(1, 2, 64), torch.zeros(1, 2, 64),
                                torch.zeros(1, 16, 2, 72, dtype=torch.uint8), torch.zeros(1, dtype=torch.int64))


# ---------------------------------------------------------------- dispatch
def test_decode_is_one_batched_launch_per_layer():
    k = _RecordingKernels()
    impl = _impl(H=8, D=64, KV=2, kernels=k)
    N = 5
    q = torch.randn(N, 8, 64).half()
    cache = torch.zeros(9, 16, 2, 72, dtype=torch.uint8)
    tables = torch.arange(N * 3, dtype=torch.int32).reshape(N, 3) % 9
    meta = _meta([3, 40, 0, 17, 33], tables)
    out = torch.zeros(N, 8 * 64, dtype=torch.float16)
    res = impl.forward(None, q, q, q, cache, meta, out)
    assert res is out
    assert len(k.decode_calls) == 1                 # not one per request
    c = k.decode_calls[0]
    assert c["q"].shape == (N, 8, 64) and c["block_size"] == 16 and c["num_kv_heads"] == 2
    assert c["seq_lens"].dtype == torch.int32 and torch.equal(c["seq_lens"], meta.seq_lens)
    assert c["block_tables"].dtype == torch.int32   # vLLM's int32 table, not copied to int64
    assert torch.equal(c["block_tables"], tables)
    assert c["out"] is not None and c["out"].data_ptr() == out.data_ptr()   # written in place
    assert torch.all(out == 0.5)


def test_decode_counts_requests_and_logs_once(caplog):
    """The reference's diagnostics (adapters/vllm_adapter.py:63,279-283): a
    counter of decode requests served and one "serving inside vLLM" log line
    per layer implementation; launches are counted beside it."""
    import logging

    k = _RecordingKernels()
    impl = _impl(H=8, D=64, KV=2, kernels=k)
    N = 4
    q = torch.randn(N, 8, 64).half()
    cache = torch.zeros(9, 16, 2, 72, dtype=torch.uint8)
    meta = _meta([3, 40, 5, 17], torch.zeros((N, 3), dtype=torch.int32))
    before = va.backend_status()
    with caplog.at_level(logging.INFO, logger="slm_turbo.vllm_adapter"):
        for _ in range(3):
            impl.forward(None, q, q, q, cache, meta, torch.zeros(N, 8 * 64, dtype=torch.float16))
    after = va.backend_status()
    assert after["kernel_calls"] - before["kernel_calls"] == 3 * N
    assert after["kernel_launches"] - before["kernel_launches"] == 3
    lines = [r.getMessage() for r in caplog.records if "serving inside vLLM" in r.getMessage()]
    assert lines == ["slm-turbo 4-bit decode kernel serving inside vLLM (head_size=64)"]


def test_decode_only_the_actual_tokens():
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    q = torch.randn(6, 8, 64).half()
    meta = _meta([5, 6, 7, 8], torch.zeros(4, 2, dtype=torch.int32), n=3)
    out = torch.full((6, 512), -1.0, dtype=torch.float16)
    impl.forward(None, q, q, q, torch.zeros(2, 16, 2, 72, dtype=torch.uint8), meta, out)
    c = k.decode_calls[0]
    assert c["q"].shape[0] == 3 and c["seq_lens"].numel() == 3 and c["block_tables"].shape[0] == 3
    assert torch.all(out[:3] == 0.5) and torch.all(out[3:] == -1.0)


def test_decode_into_non_contiguous_output_copies():
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    q = torch.randn(2, 8, 64).half()
    big = torch.zeros(2, 1024, dtype=torch.float16)
    out = big[:, :512]                                  # non-contiguous view
    impl.forward(None, q, q, q, torch.zeros(2, 16, 2, 72, dtype=torch.uint8),
                 _meta([4, 4], torch.zeros(2, 1, dtype=torch.int32)), out)
    assert k.decode_calls[0]["out"] is None
    assert torch.all(big[:, :512] == 0.5) and torch.all(big[:, 512:] == 0)


def test_empty_or_missing_metadata_gives_zeros():
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    q = torch.randn(3, 8, 64).half()
    cache = torch.zeros(2, 16, 2, 72, dtype=torch.uint8)
    out = torch.ones(3, 512, dtype=torch.float16)
    assert torch.all(impl.forward(None, q, q, q, cache, None, out) == 0)
    out.fill_(1)
    meta = _meta([1, 1, 1], torch.zeros(3, 1, dtype=torch.int32), n=0)
    assert torch.all(impl.forward(None, q, q, q, cache, meta, out) == 0)
    assert torch.all(impl.forward(None, q, q, q, cache, meta, None) == 0)   # allocates the output
    assert not k.decode_calls


def test_store_arguments():
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    key = torch.randn(4, 2, 64).half()
    cache = torch.zeros(3, 32, 2, 72, dtype=torch.uint8)
    slots = torch.tensor([0, 5, -1, 70])
    impl.do_kv_cache_update(None, key, key, cache, slots)
    assert len(k.store_calls) == 1 and k.store_calls[0]["block_size"] == 32
    assert k.store_calls[0]["slot_mapping"] is slots
    impl.do_kv_cache_update(None, key, key, torch.zeros(0, 32, 2, 72, dtype=torch.uint8), slots)
    impl.do_kv_cache_update(None, key, key, None, slots)
    assert len(k.store_calls) == 1                     # empty / missing cache: nothing stored


def test_prefill_routes_to_causal_sdpa_over_the_chunk():
    """max_query_len > 1: causal attention over the chunk's raw K/V with the
    layer's scale and GQA (reference :231-245); checked on the CPU against
    an explicit float64 causal softmax."""
    k = _RecordingKernels()
    H, KV, D, N = 8, 2, 64, 6
    impl = _impl(H=H, D=D, KV=KV, kernels=k)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(N, H, D, generator=g)
    key = torch.randn(N, KV, D, generator=g)
    val = torch.randn(N, KV, D, generator=g)
    out = torch.zeros(N, H * D)
    impl.forward(None, q, key, val, torch.zeros(1, 16, KV, D + 8, dtype=torch.uint8),
                 _meta([N], torch.zeros(1, 1), max_query_len=N, n=N), out)
    assert not k.decode_calls
    qd, kd, vd = q.double(), key.double(), val.double()
    ref = torch.zeros(N, H, D, dtype=torch.float64)
    for h in range(H):
        kv = h // (H // KV)
        s = (qd[:, h] @ kd[:, kv].T) * D ** -0.5
        s = s.masked_fill(torch.triu(torch.ones(N, N, dtype=torch.bool), 1), float("-inf"))
        ref[:, h] = torch.softmax(s, -1) @ vd[:, kv]
    assert_close(out.reshape(N, H, D).numpy(), ref.numpy(), atol=1e-5, rtol=1e-5)


def _chunk_meta(seq_lens, query_lens, block_table):
    """A mixed step: request r has query_lens[r] new tokens and seq_lens[r]
    tokens in total (the new ones included)."""
    qsl = torch.zeros(len(query_lens) + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(torch.as_tensor(query_lens, dtype=torch.int32), 0)
    return SimpleNamespace(seq_lens=torch.as_tensor(seq_lens, dtype=torch.int32),
                           block_table=torch.as_tensor(block_table, dtype=torch.int32),
                           query_start_loc=qsl, num_actual_tokens=int(qsl[-1]),
                           max_query_len=max(query_lens), max_seq_len=max(seq_lens))


def test_chunked_prefill_continuation_is_one_launch():
    """A chunk continuing 20 cached tokens, a first chunk of 3 and a decode
    token in one step: every query token becomes one sequence of the batched
    launch, with its absolute position + 1 as length and its request's row."""
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    tables = torch.tensor([[4, 5], [6, 0], [7, 8]], dtype=torch.int32)
    meta = _chunk_meta(seq_lens=[25, 3, 40], query_lens=[5, 3, 1], block_table=tables)
    q = torch.randn(9, 8, 64).half()
    out = torch.zeros(9, 512, dtype=torch.float16)
    impl.forward(None, q, q, q, torch.zeros(9, 16, 2, 72, dtype=torch.uint8), meta, out)
    assert len(k.decode_calls) == 1
    c = k.decode_calls[0]
    assert c["seq_lens"].tolist() == [21, 22, 23, 24, 25, 1, 2, 3, 40]
    assert c["block_tables"].tolist() == [[4, 5]] * 5 + [[6, 0]] * 3 + [[7, 8]]
    assert torch.all(out == 0.5)


def test_one_first_chunk_keeps_the_reference_prefill():
    """One request with no earlier context keeps the reference's SDPA
    prefill over the chunk's raw K/V."""
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    meta = _chunk_meta(seq_lens=[4], query_lens=[4], block_table=torch.zeros(1, 1, dtype=torch.int32))
    q = torch.randn(4, 8, 64)
    out = torch.zeros(4, 512)
    impl.forward(None, q, q[:, :2], q[:, :2], torch.zeros(2, 16, 2, 72, dtype=torch.uint8), meta, out)
    assert k.decode_calls == []
    assert torch.all(torch.isfinite(out)) and not torch.all(out == 0)


def test_several_first_chunks_attend_per_request():
    """Two first chunks in one step: one causal SDPA over all 7 tokens would
    let request 1 attend to request 0's tokens, so the step goes through the
    packed cache, each token over its own request's prefix."""
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    tables = torch.tensor([[3], [5]], dtype=torch.int32)
    meta = _chunk_meta(seq_lens=[4, 3], query_lens=[4, 3], block_table=tables)
    q = torch.randn(7, 8, 64).half()
    out = torch.zeros(7, 512, dtype=torch.float16)
    impl.forward(None, q, q, q, torch.zeros(6, 16, 2, 72, dtype=torch.uint8), meta, out)
    assert len(k.decode_calls) == 1
    c = k.decode_calls[0]
    assert c["seq_lens"].tolist() == [1, 2, 3, 4, 1, 2, 3]
    assert c["block_tables"].tolist() == [[3]] * 4 + [[5]] * 3


def test_short_continuation_beside_a_longer_first_chunk():
    """A 10-token first chunk and a request with 6 cached + 2 new tokens:
    max_seq_len == max_query_len == 10, yet the second request has context.
    It must attend to its own 6 cached tokens, not to the other request."""
    k = _RecordingKernels()
    impl = _impl(kernels=k)
    tables = torch.tensor([[1], [2]], dtype=torch.int32)
    meta = _chunk_meta(seq_lens=[10, 8], query_lens=[10, 2], block_table=tables)
    assert meta.max_seq_len == meta.max_query_len
    q = torch.randn(12, 8, 64).half()
    out = torch.zeros(12, 512, dtype=torch.float16)
    impl.forward(None, q, q, q, torch.zeros(3, 16, 2, 72, dtype=torch.uint8), meta, out)
    c = k.decode_calls[0]
    assert c["seq_lens"].tolist() == list(range(1, 11)) + [7, 8]
    assert c["block_tables"].tolist() == [[1]] * 10 + [[2]] * 2


# ---------------------------------------------------------------- on the GPU
@pytest.mark.gpu
def test_backend_decode_matches_oracle_with_vllm_metadata():
    """Real kernels through the backend: int32 block table and int32 device
    seq_lens as vLLM passes them, fp16 output written in place."""
    H, KV, D = 32, 8, 128
    case = make_paged_case(seed=77, B=6, H=H, KV=KV, D=D, lens=[1, 900, 0, 2500, 33, 4096])
    ref = paged_reference(case)
    impl = _impl(H=H, D=D, KV=KV)
    dev = "cuda:0"
    q = case.q.to(dev)
    cache = torch.from_numpy(case.kv_cache).to(dev)
    meta = _meta(case.seq_lens, case.block_tables)
    meta.seq_lens, meta.block_table = meta.seq_lens.to(dev), meta.block_table.to(dev)
    out = torch.zeros(6, H * D, dtype=torch.float16, device=dev)
    impl.forward(None, q, q, q, cache, meta, out)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy().reshape(6, H, D), ref, what="backend decode")


@pytest.mark.gpu
def test_backend_store_is_bit_exact():
    H, KV, D, bs = 8, 2, 80, 16
    g = torch.Generator().manual_seed(5)
    key = torch.randn(11, KV, D, generator=g).half()
    val = torch.randn(11, KV, D, generator=g).half()
    slots = torch.tensor([3, 4, 5, -1, 17, 18, 40, 41, 63, 0, 1], dtype=torch.int64)
    ref = np.zeros((4, bs, KV, D + 8), dtype=np.uint8)
    oq.quantize_store(key.numpy(), val.numpy(), ref, slots.numpy(), bs)
    impl = _impl(H=H, D=D, KV=KV)
    cache = torch.zeros(ref.shape, dtype=torch.uint8, device="cuda:0")
    impl.do_kv_cache_update(None, key.cuda(), val.cuda(), cache, slots.cuda())
    torch.cuda.synchronize()
    assert np.array_equal(cache.cpu().numpy(), ref)


def _mixed_step_matches_oracle(lens, qlens, seed):
    """Real kernels: request r has lens[r] tokens in the packed cache, the
    last qlens[r] of them new in this step; every query token is checked
    against the oracle over its own request's prefix of the packed cache."""
    H, KV, D = 32, 8, 128
    case = make_paged_case(seed=seed, B=len(lens), H=H, KV=KV, D=D, lens=lens)
    N = sum(qlens)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(N, H, D, generator=g).half()
    # the oracle case: one sequence per query token
    rows, vlens = [], []
    for r, (L, n) in enumerate(zip(lens, qlens)):
        for i in range(n):
            rows.append(case.block_tables[r])
            vlens.append(L - n + i + 1)
    vcase = type(case)(q=q, kv_cache=case.kv_cache, block_tables=torch.stack(rows),
                       seq_lens=torch.tensor(vlens, dtype=torch.int32), block_size=case.block_size,
                       num_kv_heads=KV)
    ref = paged_reference(vcase)
    impl = _impl(H=H, D=D, KV=KV)
    dev = "cuda:0"
    meta = _chunk_meta(lens, qlens, case.block_tables)
    for f in ("seq_lens", "block_table", "query_start_loc"):
        setattr(meta, f, getattr(meta, f).to(dev))
    out = torch.zeros(N, H * D, dtype=torch.float16, device=dev)
    impl.forward(None, q.to(dev), q.to(dev), q.to(dev), torch.from_numpy(case.kv_cache).to(dev), meta, out)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy().reshape(N, H, D), ref, what="mixed step")


@pytest.mark.gpu
def test_backend_chunked_prefill_matches_oracle():
    """Chunks of 7 and 12 tokens continuing 300 and 1000 cached tokens, and
    one decode token, in one step."""
    _mixed_step_matches_oracle([307, 1012, 90], [7, 12, 1], seed=91)


@pytest.mark.gpu
def test_backend_first_chunks_and_short_continuation_match_oracle():
    """Two first chunks (10 and 5 tokens) and a continuation of 6 cached
    tokens by 2 new ones in one step: each request attends to its own tokens
    only."""
    _mixed_step_matches_oracle([10, 8, 5], [10, 2, 5], seed=93)
