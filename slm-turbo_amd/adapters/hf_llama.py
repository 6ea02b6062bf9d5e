"""transformers attention hook over the packed 4-bit paged KV cache, and the
full-model greedy decode harness of a Llama-style model
(reference kernels/benchmark/benchmark.py:187-269).

The reference registers ``slm_kernel`` in transformers' attention registry
(benchmark.py:196-237): for batch 1 and one query token it quantizes the
layer's K/V per channel (rulers fixed at the first decode step), appends the
new token's codes and calls the per-channel decode kernel; everything else,
and the fp16 K/V themselves, stay with transformers' own cache and eager
attention.  ``_run_model`` (:240-269) then times greedy decode steps of a
``LlamaForCausalLM``.

Here the hook serves a whole decode batch from the packed per-token paged
cache that the vLLM backend uses (the layout of the batch-64 paged decode):

* ``PackedKVCache`` holds, per layer, a pool of ``[num_blocks, block_size,
  num_kv_heads, head_dim + 8]`` uint8 blocks (4-bit K and V codes, fp16
  k_min, k_step, v_min, v_step per token and KV head) and one block table per
  sequence, a random permutation of the pool as a paged allocator leaves it.
  transformers keeps no cache of its own in this mode (``use_cache=False``):
  the packed slots are the only copy of K/V.
* ``packed_kv_attention`` (registered as ``ATTN_PACKED``) quantizes the step's
  new K/V into their slots with one store launch per layer.  A decode step
  (one query token per sequence) is then ONE batched paged decode launch for
  all sequences.  The first prefill chunk attends causally over its own fp16
  K/V, as the reference's prefill does; a later chunk that continues cached
  context attends over the packed cache, each query token being one sequence
  of the same batched launch.
* ``fp16_attention`` (registered as ``ATTN_FP16``) is the baseline: fp16 K/V in
  transformers' ``DynamicCache`` and, for decode, the arithmetic of
  transformers' ``eager_attention_forward`` (K/V heads repeated to the query
  heads, fp16 scores, softmax in fp32, fp16 probabilities times V), with each
  batched product taking contiguous operands.
* ``per_channel_attention`` (registered as ``ATTN_PER_CHANNEL``) is the
  reference's own harness restated for the per-channel kernels: batch 1, one
  query token, the layer's fp16 K/V from transformers' cache quantized per
  channel and attended by the per-channel decode, with the rulers either fixed
  at the first decode step (new tokens appended against them) or refreshed
  every step (``PerChannelKV``); every other call is the fp16 baseline.
* ``greedy_decode`` runs prefill plus N greedy decode steps in any mode,
  ``run_decode_benchmark`` times the decode steps of the batched modes and
  ``run_per_channel_benchmark`` the reference's batch-1 per-channel modes
  (tokens/s).

The model is a random-init ``LlamaForCausalLM`` built locally from a
``LlamaConfig`` (``llama_1b_config``: 22 layers, hidden 2048, 32 query / 4 KV
heads, head_dim 64, SwiGLU MLP 5632, RMSNorm, RoPE theta 1e4, vocab 32000);
nothing is downloaded.

All sequences of a batch have the same length (equal-length prompts, as in
the full-model workload: batch 32, prompt 4096, 128 new tokens).  The decode
kernel applies softmax scale 1/sqrt(head_dim), Llama's own scaling; any other
scale is refused.
"""
from __future__ import annotations

import math
import time
from typing import Any, Optional

import torch

ATTN_PACKED = "slm_packed_kv"
ATTN_FP16 = "slm_fp16_eager"
ATTN_PER_CHANNEL = "slm_per_channel"

# Stand-in for the kernel module (tests replace it); None -> kernels.kv_dequant
_kernel_module: Any = None


def _kd():
    """The kernel entry points; raises if the HIP library is unusable."""
    global _kernel_module
    if _kernel_module is None:
        from kernels import _native
        from kernels import kv_dequant

        _native.load()                          # raises with the build hint if missing
        _kernel_module = kv_dequant
    return _kernel_module


def llama_1b_config(**overrides):
    """The 1.1B Llama-style configuration of the full-model workload (the
    TinyLlama-1.1B shape the reference benchmarks, benchmark.py:180)."""
    from transformers import LlamaConfig

    kw = dict(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=22,
              num_attention_heads=32, num_key_value_heads=4, head_dim=64, hidden_act="silu",
              rms_norm_eps=1e-5, max_position_embeddings=8192,
              rope_parameters={"rope_type": "default", "rope_theta": 10000.0},
              tie_word_embeddings=False, attention_bias=False, mlp_bias=False)
    kw.update(overrides)
    return LlamaConfig(**kw)


def build_model(config, device="cuda:0", dtype=torch.float16, seed: int = 0):
    """A random-init ``LlamaForCausalLM`` of ``config`` on ``device`` in
    ``dtype`` (weights initialised where they live, then cast)."""
    from transformers import LlamaForCausalLM

    torch.manual_seed(seed)
    with torch.device(device):
        model = LlamaForCausalLM(config)
    return model.to(dtype).eval()


def register_attention() -> None:
    """Register both attention functions with transformers (idempotent)."""
    from transformers import AttentionInterface

    AttentionInterface.register(ATTN_PACKED, packed_kv_attention)
    AttentionInterface.register(ATTN_FP16, fp16_attention)
    AttentionInterface.register(ATTN_PER_CHANNEL, per_channel_attention)


def set_attention(model, name: str) -> None:
    """Route every attention layer of ``model`` to the registered ``name``."""
    register_attention()
    model.config._attn_implementation = name
    for layer in model.model.layers:
        layer.self_attn.config._attn_implementation = name


# =============================================================================
#  packed per-token paged cache
# =============================================================================
class PackedKVCache:
    """Per-layer packed 4-bit paged caches for a batch of equal-length sequences.

    ``advance(n)`` is called once before each forward that adds ``n`` tokens
    to every sequence: it sets the slot of each new token (``slots``, int64,
    sequence-major like the K/V rows the store reads), the sequence lengths
    after the step (``seq_lens``, int32, read by the decode kernel on the
    device) and the tokens' positions (``position_ids``, for RoPE).
    """

    def __init__(self, num_layers: int, batch: int, max_len: int, num_kv_heads: int, head_dim: int,
                 block_size: int = 16, device="cuda:0", seed: int = 0):
        if head_dim not in (64, 80, 128):
            raise ValueError(f"packed cache: head_dim must be 64/80/128, got {head_dim}")
        self.num_layers, self.batch, self.max_len = num_layers, batch, max_len
        self.num_kv_heads, self.head_dim, self.block_size = num_kv_heads, head_dim, block_size
        self.device = torch.device(device)
        blocks_per_seq = -(-max_len // block_size)
        g = torch.Generator().manual_seed(seed)
        perm = torch.randperm(batch * blocks_per_seq, generator=g).to(torch.int32)
        self.block_tables = perm.view(batch, blocks_per_seq).to(self.device)
        shape = (batch * blocks_per_seq, block_size, num_kv_heads, head_dim + 8)
        self.layers = [torch.zeros(shape, dtype=torch.uint8, device=self.device) for _ in range(num_layers)]
        self.length = 0
        self.step_tokens = 0
        # a decode step's metadata lives in fixed buffers, rewritten in place,
        # so that a captured decode step reads the current step's values
        self._slots1 = torch.zeros(batch, dtype=torch.int64, device=self.device)
        self._pos1 = torch.zeros((batch, 1), dtype=torch.int64, device=self.device)
        self.seq_lens = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self.slots: Optional[torch.Tensor] = None
        self.position_ids: Optional[torch.Tensor] = None

    def nbytes(self) -> int:
        """Bytes of packed cache held, over all layers."""
        return sum(t.numel() for t in self.layers)

    def advance(self, n: int) -> None:
        if n <= 0:
            raise ValueError("advance: n must be positive")
        if self.length + n > self.max_len:
            raise ValueError(f"packed cache full: {self.length} + {n} tokens > capacity {self.max_len}")
        bs, L = self.block_size, self.length
        if n == 1:                                  # in place: no allocation, no host-to-device copy
            self._slots1.copy_(self.block_tables[:, L // bs]).mul_(bs).add_(L % bs)
            self._pos1.fill_(L)
            self.slots, self.position_ids = self._slots1, self._pos1
        else:
            pos = torch.arange(L, L + n, device=self.device)
            blocks = self.block_tables[:, pos // bs].long()                           # [B, n]
            self.slots = (blocks * bs + pos % bs).reshape(-1)                         # [B * n]
            self.position_ids = pos.unsqueeze(0).expand(self.batch, n)
        self.length += n
        self.step_tokens = n
        self.seq_lens.fill_(self.length)


def _check_scale(scaling, D: int) -> None:
    if scaling is not None and abs(float(scaling) * math.sqrt(D) - 1.0) > 1e-6:
        raise ValueError(f"packed KV attention applies 1/sqrt(head_dim); got scaling {scaling} for head_dim {D}")


def causal_prefill(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling) -> torch.Tensor:
    """Causal attention of a first prefill chunk over its own fp16 K/V:
    query [B, H, T, D], key/value [B, KV, T, D] -> [B, H, T, D].  On the GPU
    only the flash / memory-efficient SDPA kernels are allowed."""
    G = query.shape[1] // key.shape[1]
    if G > 1:
        key = key.repeat_interleave(G, dim=1)
        value = value.repeat_interleave(G, dim=1)
    sdpa = torch.nn.functional.scaled_dot_product_attention
    if query.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return sdpa(query, key, value, is_causal=True, scale=scaling)
    return sdpa(query, key, value, is_causal=True, scale=scaling)


def packed_kv_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                        packed_kv_cache: Optional[PackedKVCache] = None, **kwargs):
    """transformers attention function over ``PackedKVCache`` (pass the cache
    as the forward's ``packed_kv_cache=`` keyword).  query [B, H, T, D],
    key/value [B, KV, T, D] (this step's tokens) -> ([B, T, H, D], None)."""
    cache = packed_kv_cache
    if cache is None:
        raise ValueError(f"attention '{ATTN_PACKED}' needs the forward's packed_kv_cache= argument")
    B, H, T, D = query.shape
    KV = key.shape[1]
    if (B, KV, D) != (cache.batch, cache.num_kv_heads, cache.head_dim) or T != cache.step_tokens:
        raise ValueError(f"packed KV attention: step of [B={B}, KV={KV}, T={T}, D={D}] does not match the "
                         f"cache [B={cache.batch}, KV={cache.num_kv_heads}, T={cache.step_tokens}, "
                         f"D={cache.head_dim}]")
    _check_scale(scaling, D)
    kd = _kd()
    layer = cache.layers[module.layer_idx]
    bs = cache.block_size
    rows = lambda t: t.transpose(1, 2).reshape(B * T, KV, D)       # [B*T, KV, D], sequence-major
    kd.kv_quantize_store(rows(key), rows(value), layer, cache.slots, bs)
    out_dtype = torch.float16 if query.dtype == torch.float16 else torch.float32
    if T == 1:
        out = kd.kv_dequant_decode_paged_batched(query[:, :, 0], layer, cache.block_tables, cache.seq_lens,
                                                 bs, KV, out_dtype=out_dtype)
        return out.to(query.dtype).unsqueeze(1), None
    if cache.length == T:
        return causal_prefill(query, key, value, scaling).transpose(1, 2), None
    # continuation chunk: query token t of a sequence attends over its own prefix
    q = query.transpose(1, 2).reshape(B * T, H, D)
    tables = cache.block_tables.repeat_interleave(T, dim=0)
    first = cache.length - T
    lens = torch.arange(first + 1, cache.length + 1, dtype=torch.int32, device=query.device).repeat(B)
    out = kd.kv_dequant_decode_paged_batched(q, layer, tables, lens, bs, KV, out_dtype=out_dtype)
    return out.to(query.dtype).view(B, T, H, D), None


def fp16_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """fp16 baseline over transformers' cache.  query [B, H, T, D], key/value
    [B, KV, S, D] (all cached tokens) -> ([B, T, H, D], None).  A first prefill
    chunk (S == T) is causal; a decode step (T == 1) follows transformers'
    eager_attention_forward (repeat_kv, fp16 scores, fp32 softmax)."""
    B, H, T, D = query.shape
    KV, S = key.shape[1], key.shape[2]
    if scaling is None:
        scaling = D ** -0.5
    if T > 1:
        if S != T:
            raise NotImplementedError("fp16 baseline: prefill must start from an empty cache")
        return causal_prefill(query, key, value, scaling).transpose(1, 2), None
    G = H // KV
    kx = key[:, :, None].expand(B, KV, G, S, D).reshape(B, H, S, D)       # copies, as repeat_kv does
    vx = value[:, :, None].expand(B, KV, G, S, D).reshape(B, H, S, D)
    scores = torch.matmul(kx, query.transpose(2, 3).contiguous()) * scaling   # [B, H, S, 1]
    probs = torch.softmax(scores, dim=2, dtype=torch.float32).to(query.dtype)
    out = torch.matmul(probs.transpose(2, 3).contiguous(), vx)            # [B, H, 1, D]
    return out.transpose(1, 2), None


# =============================================================================
#  per-channel hook (the reference's batch-1 harness)
# =============================================================================
class PerChannelKV:
    """State of the per-channel hook for one generation (reference
    kernels/benchmark/benchmark.py:196-237; pass it as the forward's
    ``per_channel_kv=`` keyword).

    ``mode="fixed"``: at a layer's first decode step its whole K/V is
    quantized per channel (``quantize_kv``) into a code buffer with
    ``headroom`` free tokens; later steps quantize only the new tokens against
    those frozen rulers (``quantize_tensor``) into the buffer, which grows by
    ``headroom`` when full.  ``mode="refresh"``: every step re-quantizes the
    layer's whole K/V (rulers always fit the data, O(S) work per step).
    ``layers[i]`` holds layer i's codes, rulers and token count; ``calls``
    counts the decode kernel calls.
    """

    def __init__(self, mode: str = "fixed", headroom: int = 256):
        if mode not in ("fixed", "refresh"):
            raise ValueError(f"per-channel mode must be 'fixed' or 'refresh', got {mode!r}")
        self.mode, self.headroom = mode, headroom
        self.layers: dict = {}
        self.calls = 0

    def packed(self, layer_idx: int, kf: torch.Tensor, vf: torch.Tensor):
        """(k_packed, k_scale, k_zero, v_packed, v_scale, v_zero) of layer
        ``layer_idx`` for the K/V ``kf``/``vf`` [KV, S, D] fp16 of all its
        tokens so far."""
        kd = _kd()
        S = kf.shape[1]
        if self.mode == "refresh":
            return kd.quantize_kv(kf, vf)
        st = self.layers.get(layer_idx)
        if st is None or S < st["n"]:
            kp, ks, kz, vp, vs, vz = kd.quantize_kv(kf, vf)
            KV, _, half = kp.shape
            kb = torch.zeros((KV, S + self.headroom, half), dtype=torch.uint8, device=kp.device)
            vb = torch.zeros_like(kb)
            kb[:, :S] = kp
            vb[:, :S] = vp
            st = self.layers[layer_idx] = dict(kb=kb, vb=vb, ks=ks, kz=kz, vs=vs, vz=vz, n=S)
        elif S > st["n"]:
            prev = st["n"]
            if S > st["kb"].shape[1]:
                grow = lambda b: torch.cat([b, b.new_zeros((b.shape[0], S - b.shape[1] + self.headroom,
                                                            b.shape[2]))], dim=1)
                st["kb"], st["vb"] = grow(st["kb"]), grow(st["vb"])
            kd.quantize_tensor(kf[:, prev:], st["ks"], st["kz"], out=st["kb"][:, prev:S])
            kd.quantize_tensor(vf[:, prev:], st["vs"], st["vz"], out=st["vb"][:, prev:S])
            st["n"] = S
        n = st["n"]
        return st["kb"][:, :n], st["ks"], st["kz"], st["vb"][:, :n], st["vs"], st["vz"]


def per_channel_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                          per_channel_kv: Optional[PerChannelKV] = None, **kwargs):
    """The reference's ``slm_kernel`` attention (benchmark.py:196-237) over the
    per-channel kernels: for batch 1, one query token and more than one cached
    token, the layer's K/V (transformers' cache, [1, KV, S, D]) are quantized
    per channel as ``per_channel_kv`` says and attended by
    ``kv_dequant_decode_attention``; anything else is the fp16 baseline.
    query [B, H, T, D] -> ([B, T, H, D], None)."""
    B, H, T, D = query.shape
    KV, S = key.shape[1], key.shape[2]
    if per_channel_kv is None or not (B == 1 and T == 1 and S > 1):
        return fp16_attention(module, query, key, value, attention_mask, scaling, dropout, **kwargs)
    _check_scale(scaling, D)
    kd = _kd()
    kf = key[0].to(torch.float16).contiguous()
    vf = value[0].to(torch.float16).contiguous()
    kp, ks, kz, vp, vs, vz = per_channel_kv.packed(module.layer_idx, kf, vf)
    out = kd.kv_dequant_decode_attention(query[0].to(torch.float16), kp, ks, kz, vp, vs, vz, num_kv_heads=KV)
    per_channel_kv.calls += 1
    return out.to(query.dtype).transpose(0, 1).unsqueeze(0), None     # [1, 1, H, D]


# =============================================================================
#  greedy decode and timing
# =============================================================================
class DecodeRunner:
    """One model forward per call in either mode, holding that mode's cache.

    ``graph=True`` (packed mode on the GPU) captures the decode step (one
    token per sequence, all layers: projections, store, batched paged decode,
    MLP, head) once in a HIP graph and replays it for every later step.  The
    step's inputs sit in fixed buffers (token ids, positions, slots, sequence
    lengths) that the host rewrites in place before each replay; the first
    decode step runs eagerly on the capture stream (it allocates the kernels'
    workspace and the libraries' handles for that stream) and is captured
    right after.  Prefill chunks always run eagerly.
    """

    def __init__(self, model, mode: str, batch: int, max_len: int, block_size: int = 16, seed: int = 0,
                 graph: bool = False):
        cfg = model.config
        self.model, self.mode = model, mode
        self.graph = None
        self.per_channel: Optional[PerChannelKV] = None
        self._use_graph = bool(graph)
        if graph and mode != "packed":
            raise ValueError("graph capture serves the packed mode only")
        if mode == "packed":
            set_attention(model, ATTN_PACKED)
            head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
            dev = next(model.parameters()).device
            self.cache = PackedKVCache(cfg.num_hidden_layers, batch, max_len, cfg.num_key_value_heads, head_dim,
                                       block_size, dev, seed)
        elif mode == "fp16" or mode.startswith("per_channel_"):
            from transformers import DynamicCache

            if mode == "fp16":
                set_attention(model, ATTN_FP16)
            else:
                if batch != 1:
                    raise ValueError("the per-channel modes serve batch 1 (the reference's harness)")
                self.per_channel = PerChannelKV(mode[len("per_channel_"):])
                set_attention(model, ATTN_PER_CHANNEL)
            self.cache = DynamicCache(config=cfg)
            self.length = 0
        else:
            raise ValueError(f"mode must be 'packed', 'fp16', 'per_channel_fixed' or 'per_channel_refresh', "
                             f"got {mode!r}")

    @torch.no_grad()
    def __call__(self, ids: torch.Tensor) -> torch.Tensor:
        """Logits of the last position, [B, vocab]."""
        n = ids.shape[1]
        if self.mode == "packed":
            self.cache.advance(n)
            if self._use_graph and n == 1:
                return self._graph_step(ids)
            out = self._forward(ids)
        else:
            pos = torch.arange(self.length, self.length + n, device=ids.device).unsqueeze(0).expand(ids.shape[0], n)
            self.length += n
            extra = {} if self.per_channel is None else {"per_channel_kv": self.per_channel}
            out = self.model(ids, position_ids=pos, past_key_values=self.cache, use_cache=True, logits_to_keep=1,
                             **extra)
        return out.logits[:, -1]

    def _forward(self, ids):
        return self.model(ids, position_ids=self.cache.position_ids, use_cache=False, logits_to_keep=1,
                          packed_kv_cache=self.cache)

    def _graph_step(self, ids: torch.Tensor) -> torch.Tensor:
        if self.graph is not None:
            self._ids.copy_(ids)
            self.graph.replay()
            return self._logits[:, -1].clone()
        self._ids = ids.clone()
        stream = self._stream = torch.cuda.Stream(self._ids.device)   # default priority; kept alive
        stream.wait_stream(torch.cuda.current_stream(self._ids.device))
        with torch.cuda.stream(stream):
            logits = self._forward(self._ids).logits[:, -1].clone()
        torch.cuda.current_stream(self._ids.device).wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(self.graph, stream=stream):
            self._logits = self._forward(self._ids).logits
        return logits


def graph_node_types(graph) -> dict:
    """Node counts by type of a captured graph (kept with ``keep_graph=True``):
    {"kernel": n, "memset": n, ...}, read through the HIP runtime the process
    has loaded."""
    import ctypes

    names = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty", 6: "wait_event",
             7: "event_record", 10: "mem_alloc", 11: "mem_free"}
    path = next((ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln), "libamdhip64.so")
    hip = ctypes.CDLL(path)
    g = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(g, None, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    nodes = (ctypes.c_void_p * n.value)()
    if hip.hipGraphGetNodes(g, nodes, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    counts: dict = {}
    t = ctypes.c_int(0)
    for i in range(n.value):
        if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t)) != 0:
            raise RuntimeError("hipGraphNodeGetType failed")
        key = names.get(t.value, f"type{t.value}")
        counts[key] = counts.get(key, 0) + 1
    return counts


@torch.no_grad()
def greedy_decode(model, input_ids: torch.Tensor, new_tokens: int, mode: str, block_size: int = 16,
                  seed: int = 0, forced: Optional[torch.Tensor] = None, graph: bool = False):
    """Prefill ``input_ids`` [B, P], then ``new_tokens`` greedy decode steps.

    Returns (tokens [B, new_tokens], logits [new_tokens + 1, B, vocab] of the
    prefill and every step, decode seconds, prefill seconds).  ``forced``
    [B, new_tokens] feeds given tokens instead of the greedy ones (so two
    modes can be compared step by step on the same inputs).  ``graph``
    replays the packed decode step from a HIP graph (``DecodeRunner``).
    """
    B, P = input_ids.shape
    run = DecodeRunner(model, mode, B, P + new_tokens, block_size, seed, graph=graph)
    sync = torch.cuda.synchronize if input_ids.is_cuda else (lambda: None)
    sync()
    t0 = time.perf_counter()
    logits = [run(input_ids)]
    sync()
    t1 = time.perf_counter()
    toks = []
    nxt = logits[0].argmax(-1, keepdim=True)
    for i in range(new_tokens):
        if forced is not None:
            nxt = forced[:, i:i + 1]
        toks.append(nxt)
        logits.append(run(nxt))
        nxt = logits[-1].argmax(-1, keepdim=True)
    sync()
    t2 = time.perf_counter()
    return torch.cat(toks, dim=1), torch.stack(logits), t2 - t1, t1 - t0


def run_decode_benchmark(batch: int = 32, prompt: int = 4096, new_tokens: int = 128, device="cuda:0",
                         seed: int = 0, repeats: int = 2, config=None) -> dict:
    """Tokens/s of greedy decode for the packed 4-bit path (eager, and with
    the decode step replayed from a HIP graph) and the fp16 eager baseline on
    one random-init model and one random prompt batch.

    Each mode runs ``repeats`` full generations (the first warms kernels and
    allocator); the last one's decode steps are timed, synchronised only at
    both ends.  tokens/s = batch x new_tokens / decode seconds.
    """
    config = config or llama_1b_config()
    model = build_model(config, device, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    ids = torch.randint(0, config.vocab_size, (batch, prompt), generator=g).to(device)
    res: dict = {"batch": batch, "prompt": prompt, "new_tokens": new_tokens,
                 "layers": config.num_hidden_layers, "hidden": config.hidden_size,
                 "heads": config.num_attention_heads, "kv_heads": config.num_key_value_heads,
                 "head_dim": config.head_dim, "params": sum(p.numel() for p in model.parameters())}
    kept = {}
    for key, mode, graph in (("fp16", "fp16", False), ("packed", "packed", False),
                             ("packed_graph", "packed", True)):
        for _ in range(repeats):
            toks, logits, dec_s, pre_s = greedy_decode(model, ids, new_tokens, mode, seed=seed, graph=graph)
            kept[key] = (toks, logits[0].float(), logits[1].float())
            del logits
            torch.cuda.empty_cache()
        res[key] = {"tokens_per_s": batch * new_tokens / dec_s, "ms_per_step": dec_s / new_tokens * 1e3,
                     "prefill_s": pre_s}
    res["speedup"] = res["packed"]["tokens_per_s"] / res["fp16"]["tokens_per_s"]
    res["speedup_graph"] = res["packed_graph"]["tokens_per_s"] / res["fp16"]["tokens_per_s"]
    per_token = config.num_hidden_layers * config.num_key_value_heads
    res["kv_cache_bytes"] = {"packed": per_token * batch * (prompt + new_tokens) * (config.head_dim + 8),
                             "fp16": per_token * batch * (prompt + new_tokens) * config.head_dim * 4}
    # agreement of the two modes: the prefill is the same computation; the
    # first decode step differs by the 4-bit K/V; greedy tokens then diverge
    # where the random model's logits are nearly tied
    a, b = kept["fp16"], kept["packed"]
    res["prefill_logits_max_abs_diff"] = float((a[1] - b[1]).abs().max())
    res["first_decode_logits_cosine_min"] = float(torch.nn.functional.cosine_similarity(a[2], b[2], dim=-1).min())
    res["greedy_token_agreement"] = float((a[0] == b[0]).float().mean())
    res["graph_tokens_equal_eager"] = bool(torch.equal(kept["packed"][0], kept["packed_graph"][0]))
    return res


def run_per_channel_benchmark(prompt: int = 512, new_tokens: int = 64, device="cuda:0", seed: int = 0,
                              repeats: int = 2, warm: int = 6, config=None) -> dict:
    """The reference's model-level table (benchmark.py:240-269, 316-331) on the
    1.1B model: batch-1 greedy decode with the fp16 baseline and the two
    per-channel modes (rulers fixed at the first decode step, or refreshed
    every step), steady-state tokens/s over the steps after the first
    ``warm``, each mode ``repeats`` times (the last is kept)."""
    config = config or llama_1b_config()
    model = build_model(config, device, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    ids = torch.randint(0, config.vocab_size, (1, prompt), generator=g).to(device)
    res: dict = {"batch": 1, "prompt": prompt, "new_tokens": new_tokens, "warm": warm,
                 "layers": config.num_hidden_layers, "heads": config.num_attention_heads,
                 "kv_heads": config.num_key_value_heads, "head_dim": config.head_dim}
    kept = {}
    for mode in ("fp16", "per_channel_fixed", "per_channel_refresh"):
        for _ in range(repeats):
            run = DecodeRunner(model, mode, 1, prompt + new_tokens, seed=seed)
            with torch.no_grad():
                logits = [run(ids)]
                nxt = logits[0].argmax(-1, keepdim=True)
                times, toks = [], []
                for _i in range(new_tokens):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    logits.append(run(nxt))
                    nxt = logits[-1].argmax(-1, keepdim=True)
                    torch.cuda.synchronize()
                    times.append(time.perf_counter() - t0)
                    toks.append(nxt)
            steady = times[warm:]
            kept[mode] = (torch.cat(toks, dim=1), logits[1].float())
            res[mode] = {"tokens_per_s": len(steady) / sum(steady), "ms_per_step": sum(steady) / len(steady) * 1e3}
            if run.per_channel is not None:
                res[mode]["kernel_calls"] = run.per_channel.calls
            del run, logits
            torch.cuda.empty_cache()
    for mode in ("per_channel_fixed", "per_channel_refresh"):
        res[mode]["speedup_vs_fp16"] = res[mode]["tokens_per_s"] / res["fp16"]["tokens_per_s"]
        res[mode]["first_decode_logits_cosine"] = float(torch.nn.functional.cosine_similarity(
            kept["fp16"][1], kept[mode][1], dim=-1).min())
        res[mode]["greedy_token_agreement"] = float((kept["fp16"][0] == kept[mode][0]).float().mean())
    return res
