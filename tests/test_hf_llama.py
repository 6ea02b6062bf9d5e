"""transformers attention hook and full-model decode harness
(reference kernels/benchmark/benchmark.py:187-269).

CPU tests replace the kernel module with the oracle (its quantize-on-write
store and float64 paged decode) to check the hook's host logic: the slot of
every token through a permuted block table, sequence lengths, the first
prefill chunk, decode steps, continuation chunks, layer indexing and the
errors.  The expected outputs are built without the block tables: every
sequence's tokens are quantized into a cache of its own in logical order.
GPU tests run the same sequence of steps through the HIP kernels (within
max-abs 2e-3 / rel 1e-2 plus fp16 output rounding) and a small random-init
Llama end to end.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from adapters import hf_llama as hl
from common import assert_close
from oracle import attention as oa
from oracle import quant as oq


class _OracleKernels:
    """CPU stand-in for kernels.kv_dequant: the oracle's store and decode."""

    def __init__(self):
        self.decode_calls = 0
        self.store_calls = 0

    def kv_quantize_store(self, key, value, kv_cache, slot_mapping, block_size):
        self.store_calls += 1
        arr = kv_cache.numpy()                     # shares memory with the CPU tensor
        oq.quantize_store(key.half().numpy(), value.half().numpy(), arr, slot_mapping.numpy(), block_size)

    def kv_dequant_decode_paged_batched(self, q, kv_cache, block_tables, seq_lens, block_size, num_kv_heads,
                                        out=None, out_dtype=None):
        self.decode_calls += 1
        assert block_size == kv_cache.shape[1] and num_kv_heads == kv_cache.shape[2]
        r = oa.decode_paged_batched(q.half().numpy(), kv_cache.numpy(), block_tables.numpy(), seq_lens.numpy())
        return torch.from_numpy(r).to(out_dtype or torch.float32)


@pytest.fixture
def oracle_kernels(monkeypatch):
    k = _OracleKernels()
    monkeypatch.setattr(hl, "_kernel_module", k)
    return k


# ---------------------------------------------------------------- expected values
class _LogicalCache:
    """Each sequence's tokens quantized in logical order (no block table)."""

    def __init__(self, B, cap, KV, D):
        self.c = np.zeros((B, cap, 1, KV, D + 8), dtype=np.uint8)
        self.n = 0

    def append(self, k, v):                        # k, v [B, KV, T, D]
        T = k.shape[2]
        slots = np.arange(self.n, self.n + T, dtype=np.int64)
        for b in range(k.shape[0]):
            oq.quantize_store(k[b].transpose(0, 1).contiguous().cpu().half().numpy(),
                              v[b].transpose(0, 1).contiguous().cpu().half().numpy(), self.c[b], slots, 1)
        self.n += T

    def decode(self, b, q, L):                     # q [H, D] -> [H, D], over the first L tokens
        return oa.decode_paged(q.cpu().half().numpy(), self.c[b], np.arange(L), L)


def _expected(logical, q, k, v, first):
    """[B, T, H, D] float64 for one step whose tokens start at ``first``."""
    B, H, T, D = q.shape
    logical.append(k, v)
    out = np.zeros((B, T, H, D))
    for b in range(B):
        if first == 0 and T > 1:                   # first chunk: causal over its raw fp16 K/V
            K = k[b].cpu().half().numpy().astype(np.float64)
            V = v[b].cpu().half().numpy().astype(np.float64)
            out[b] = oa.attend_causal(q[b].cpu().half().numpy(), K, V).transpose(1, 0, 2)
        else:
            for t in range(T):
                out[b, t] = logical.decode(b, q[b, :, t], first + t + 1)
    return out


def _steps(dev, dtype, B=3, H=8, KV=2, D=64, plan=(21, 1, 1, 3, 1), seed=0):
    """Random q/k/v for each step of ``plan`` (tokens per step), fp16 values."""
    g = torch.Generator().manual_seed(seed)
    for T in plan:
        mk = lambda *s: torch.randn(s, generator=g).half().to(dtype).to(dev)
        yield T, mk(B, H, T, D), mk(B, KV, T, D), mk(B, KV, T, D) * 2


def _drive(dev, dtype, B=3, H=8, KV=2, D=64, bs=8, plan=(21, 1, 1, 3, 1), layers=2, check_layer=1):
    """Run ``plan`` through packed_kv_attention for ``layers`` layers; yield
    (got, expected) of ``check_layer`` per step."""
    cap = sum(plan) + 2
    cache = hl.PackedKVCache(layers, B, cap, KV, D, block_size=bs, device=dev, seed=5)
    logical = _LogicalCache(B, cap, KV, D)
    steps = list(_steps(dev, dtype, B, H, KV, D, plan))
    other = list(_steps(dev, dtype, B, H, KV, D, plan, seed=99))
    first = 0
    for (T, q, k, v), (_, q2, k2, v2) in zip(steps, other):
        cache.advance(T)
        got = None
        for layer in range(layers):
            args = (q, k, v) if layer == check_layer else (q2, k2, v2)
            o, w = hl.packed_kv_attention(SimpleNamespace(layer_idx=layer), *args, None, scaling=D ** -0.5,
                                          packed_kv_cache=cache)
            assert w is None and o.shape == (B, T, H, D) and o.dtype == dtype
            if layer == check_layer:
                got = o
        yield T, got.float().cpu().numpy(), _expected(logical, q, k, v, first)
        first += T


# ---------------------------------------------------------------- CPU: host logic
def test_hook_steps_match_logical_order(oracle_kernels):
    """Prefill 21 tokens, decode, decode, a 3-token continuation, decode; block
    size 8 over a permuted pool, two layers."""
    n = 0
    for T, got, ref in _drive("cpu", torch.float32):
        assert_close(got, ref, atol=1e-5, rtol=1e-5, what=f"step of {T} tokens")
        n += 1
    assert n == 5
    # one store per layer and step; decodes: 3 decode steps + 1 continuation, per layer
    assert oracle_kernels.store_calls == 10 and oracle_kernels.decode_calls == 8


def test_cache_slots_follow_block_tables(oracle_kernels):
    """Token t of sequence b sits in block table[b, t // bs], row t % bs."""
    B, KV, D, bs = 2, 2, 64, 4
    cache = hl.PackedKVCache(1, B, 11, KV, D, block_size=bs, device="cpu", seed=3)
    g = torch.Generator().manual_seed(0)
    k = torch.randn((B, KV, 11, D), generator=g).half().float()
    v = torch.randn((B, KV, 11, D), generator=g).half().float()
    q = torch.randn((B, 4, 11, D), generator=g).half().float()
    cache.advance(11)
    hl.packed_kv_attention(SimpleNamespace(layer_idx=0), q, k, v, None, packed_kv_cache=cache)
    assert cache.seq_lens.tolist() == [11, 11] and cache.position_ids.tolist() == [list(range(11))] * 2
    tables = cache.block_tables.numpy()
    for b in range(B):
        for t in range(11):
            ref = np.zeros((1, 1, KV, D + 8), dtype=np.uint8)
            oq.quantize_store(k[b, :, t:t + 1].transpose(0, 1).half().numpy(),
                              v[b, :, t:t + 1].transpose(0, 1).half().numpy(), ref, np.zeros(1, np.int64), 1)
            assert np.array_equal(cache.layers[0][tables[b, t // bs], t % bs].numpy(), ref[0, 0])
    # the pool holds every block exactly once
    assert sorted(tables.reshape(-1).tolist()) == list(range(B * 3))


def test_hook_errors(oracle_kernels):
    cache = hl.PackedKVCache(1, 2, 4, 2, 64, device="cpu")
    q, kv = torch.zeros((2, 4, 1, 64)), torch.zeros((2, 2, 1, 64))
    mod = SimpleNamespace(layer_idx=0)
    with pytest.raises(ValueError, match="packed_kv_cache"):
        hl.packed_kv_attention(mod, q, kv, kv, None)
    cache.advance(1)
    with pytest.raises(ValueError, match="1/sqrt"):
        hl.packed_kv_attention(mod, q, kv, kv, None, scaling=0.5, packed_kv_cache=cache)
    with pytest.raises(ValueError, match="does not match"):
        hl.packed_kv_attention(mod, q, kv[:, :1], kv[:, :1], None, packed_kv_cache=cache)
    cache.advance(3)
    with pytest.raises(ValueError, match="full"):
        cache.advance(1)
    with pytest.raises(ValueError, match="head_dim"):
        hl.PackedKVCache(1, 1, 4, 1, 96, device="cpu")


def _tiny_config(**kw):
    base = dict(vocab_size=97, hidden_size=256, intermediate_size=384, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=256)
    base.update(kw)
    return hl.llama_1b_config(**base)


def _compare_modes(dev, dtype, B=3, P=37, N=6, bs=8):
    model = hl.build_model(_tiny_config(), dev, dtype=dtype, seed=1)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, 97, (B, P), generator=g).to(dev)
    forced = torch.randint(0, 97, (B, N), generator=g).to(dev)
    ref_run = hl.DecodeRunner(model, "fp16", B, P + N)
    ref = [ref_run(ids)] + [ref_run(forced[:, i:i + 1]) for i in range(N)]
    run = hl.DecodeRunner(model, "packed", B, P + N, block_size=bs, seed=4)
    got = [run(ids)] + [run(forced[:, i:i + 1]) for i in range(N)]
    # the prompt's K/V are computed identically in both modes: the packed slots
    # hold exactly the oracle's quantization of transformers' fp16 cache
    tables = run.cache.block_tables.cpu().numpy()
    for layer in range(2):
        kc = ref_run.cache.layers[layer].keys[:, :, :P]           # [B, KV, P, D]
        vc = ref_run.cache.layers[layer].values[:, :, :P]
        packed = run.cache.layers[layer].cpu().numpy()
        for b in range(B):
            want = np.zeros((P, 1, 2, 72), dtype=np.uint8)
            oq.quantize_store(kc[b].transpose(0, 1).cpu().half().numpy(), vc[b].transpose(0, 1).cpu().half().numpy(),
                              want, np.arange(P, dtype=np.int64), 1)
            t = np.arange(P)
            assert np.array_equal(packed[tables[b, t // bs], t % bs], want[:, 0]), f"layer {layer} seq {b}"
    return ref, got


# 4-bit per-token K/V carry ~10% relative noise (step / sqrt(12) against a
# spread of ~6 sigma over 15 steps), so the logits of the two modes agree in
# direction, not to the bit: the exact checks are the cache bytes above and the
# hook-level tests.
COSINE_MIN = 0.99


def test_tiny_model_modes_agree(oracle_kernels):
    ref, got = _compare_modes("cpu", torch.float32)
    assert torch.equal(ref[0], got[0])                             # same prefill computation
    for i in range(1, len(ref)):
        cos = torch.nn.functional.cosine_similarity(ref[i].double(), got[i].double(), dim=-1)
        assert float(cos.min()) > COSINE_MIN, f"step {i}: cosine {float(cos.min())}"
    assert oracle_kernels.decode_calls == 2 * (len(ref) - 1)       # one batched decode per layer and step


def test_greedy_decode_shapes(oracle_kernels):
    model = hl.build_model(_tiny_config(), "cpu", dtype=torch.float32)
    ids = torch.randint(0, 97, (2, 9), generator=torch.Generator().manual_seed(0))
    toks, logits, dec_s, pre_s = hl.greedy_decode(model, ids, 4, "packed")
    assert toks.shape == (2, 4) and logits.shape == (5, 2, 97) and dec_s >= 0 and pre_s >= 0
    assert torch.equal(toks[:, 0], logits[0].argmax(-1))
    assert torch.equal(toks[:, 1:], logits[1:4].argmax(-1).T)
    with pytest.raises(ValueError, match="mode"):
        hl.greedy_decode(model, ids, 1, "int8")


def test_full_model_configuration():
    cfg = hl.llama_1b_config()
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads,
            cfg.head_dim, cfg.intermediate_size, cfg.vocab_size) == (22, 2048, 32, 4, 64, 5632, 32000)
    assert cfg.rope_parameters["rope_theta"] == 10000.0 and cfg.hidden_act == "silu"
    with torch.device("meta"):
        from transformers import LlamaForCausalLM
        n = sum(p.numel() for p in LlamaForCausalLM(cfg).parameters())
    assert 1.09e9 < n < 1.11e9


# ---------------------------------------------------------------- GPU: HIP kernels
@pytest.mark.gpu
@pytest.mark.parametrize("H,KV,D,bs", [(8, 2, 64, 8), (32, 4, 64, 16), (32, 8, 128, 16)])
def test_hook_steps_on_the_gpu(H, KV, D, bs):
    for T, got, ref in _drive("cuda:0", torch.float16, H=H, KV=KV, D=D, bs=bs):
        assert_close(got, ref, what=f"H={H} KV={KV} D={D} step of {T} tokens")


@pytest.mark.gpu
def test_tiny_model_modes_agree_on_the_gpu():
    ref, got = _compare_modes("cuda:0", torch.float16)
    assert torch.equal(ref[0], got[0])
    for i in range(1, len(ref)):
        cos = torch.nn.functional.cosine_similarity(ref[i].double(), got[i].double(), dim=-1)
        assert float(cos.min()) > COSINE_MIN, f"step {i}: cosine {float(cos.min())}"


@pytest.mark.gpu
def test_graph_replays_match_eager_decode():
    """Two layers of the 1.1B shape, batch 32: every replay of the captured
    decode step (eager steps of another runner and a synchronisation between
    replays) gives the eager step's logits and cache bytes bit for bit, and the
    captured graph holds kernels only (no memset node)."""
    cfg = hl.llama_1b_config(num_hidden_layers=2)
    model = hl.build_model(cfg, "cuda:0", seed=3)
    B, P, N = 32, 100, 6
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, cfg.vocab_size, (B, P), generator=g).to("cuda:0")
    forced = torch.randint(0, cfg.vocab_size, (B, N), generator=g).to("cuda:0")
    eager = hl.DecodeRunner(model, "packed", B, P + N, seed=4)
    graphed = hl.DecodeRunner(model, "packed", B, P + N, seed=4, graph=True)
    assert torch.equal(eager(ids), graphed(ids))
    for i in range(N):
        tok = forced[:, i:i + 1]
        want = eager(tok)
        got = graphed(tok)
        torch.cuda.synchronize()
        assert torch.equal(want, got), f"decode step {i}: max diff {float((want - got).abs().max())}"
    for layer in range(2):
        assert torch.equal(eager.cache.layers[layer], graphed.cache.layers[layer])
    counts = hl.graph_node_types(graphed.graph)
    print("captured decode step:", counts)
    assert counts.get("kernel", 0) > 0 and counts.get("memset", 0) == 0, counts


class _TorchDecode:
    """The HIP store, with the decode done by torch fp32 dequant-then-attend."""

    def __init__(self):
        from kernels import kv_dequant
        self.kd = kv_dequant

    def kv_quantize_store(self, *a):
        self.kd.kv_quantize_store(*a)

    def kv_dequant_decode_paged_batched(self, q, kv_cache, block_tables, seq_lens, block_size, num_kv_heads,
                                        out=None, out_dtype=None):
        from test_gpu_fullsize import BS, reference
        assert block_size == BS
        return reference(q, kv_cache, block_tables, seq_lens.cpu(), num_kv_heads).to(out_dtype or torch.float32)


@pytest.mark.gpu
def test_full_depth_decode_kernel_matches_torch_decode(monkeypatch):
    """22 layers of the 1.1B shape, batch 4, prompt 600: logits with the HIP
    decode and with a torch fp32 decode of the same packed cache agree to
    within the kernel tolerance carried through the depth; the difference to
    the fp16 path is the 4-bit K/V alone."""
    cfg = hl.llama_1b_config()
    model = hl.build_model(cfg, "cuda:0", seed=5)
    B, P, N = 4, 600, 3
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, cfg.vocab_size, (B, P), generator=g).to("cuda:0")
    forced = torch.randint(0, cfg.vocab_size, (B, N), generator=g).to("cuda:0")

    def run(mode):
        r = hl.DecodeRunner(model, mode, B, P + N, seed=2)
        return [r(ids)] + [r(forced[:, i:i + 1]) for i in range(N)]

    hip = run("packed")
    monkeypatch.setattr(hl, "_kernel_module", _TorchDecode())
    ref = run("packed")
    cos = lambda a, b: float(torch.nn.functional.cosine_similarity(a.double(), b.double(), dim=-1).min())
    for i in range(1, N + 1):
        c = cos(hip[i], ref[i])
        print(f"step {i}: cosine HIP vs torch decode {c:.6f}")
        assert c > 0.999, f"step {i}: cosine {c}"


# ---------------------------------------------------------------- per-channel hook (batch 1)
class _OraclePerChannel:
    """CPU stand-in for the per-channel entry points: the oracle's quantizer
    (fp16 round-after-every-op, benchmark.py:26-74) and float64 decode."""

    def __init__(self):
        self.decode_calls = 0

    def quantize_kv(self, k, v):
        return tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in oq.quantize_kv(k.numpy(), v.numpy()))

    def quantize_tensor(self, x, scale, zero_point, bits=4, out=None):
        r = torch.from_numpy(oq.quantize_tensor(x.numpy(), scale.numpy(), zero_point.numpy()))
        if out is None:
            return r
        out.copy_(r)
        return out

    def kv_dequant_decode_attention(self, q, kp, ks, kz, vp, vs, vz, num_kv_heads=None):
        self.decode_calls += 1
        r = oa.decode_per_channel(q.numpy(), kp.numpy(), ks.numpy(), kz.numpy(), vp.numpy(), vs.numpy(),
                                  vz.numpy())
        return torch.from_numpy(r).float()


def _per_channel_steps(dev, mode, H=8, KV=2, D=64, S0=20, steps=4, headroom=2, seed=3):
    """Drive per_channel_attention for decode steps over a growing fp16 K/V
    (S0, S0 + 1, ...): yields (S, got [1,1,H,D], k [KV,S,D], v, q [H,1,D], state)."""
    g = torch.Generator().manual_seed(seed)
    st = hl.PerChannelKV(mode, headroom=headroom)
    K = (torch.randn((1, KV, S0 + steps, D), generator=g) * 1.5).half()
    V = torch.randn((1, KV, S0 + steps, D), generator=g).half()
    for i in range(steps):
        S = S0 + i
        q = torch.randn((1, H, 1, D), generator=g).half()
        o, w = hl.per_channel_attention(SimpleNamespace(layer_idx=0), q.to(dev), K[:, :, :S].to(dev),
                                        V[:, :, :S].to(dev), None, scaling=D ** -0.5, per_channel_kv=st)
        assert w is None and o.shape == (1, 1, H, D)
        yield S, o.float().cpu(), K[0, :, :S], V[0, :, :S], q[0], st


def _check_per_channel(dev, mode, **kw):
    first = None
    for S, got, k, v, q, st in _per_channel_steps(dev, mode, **kw):
        kn, vn = k.numpy(), v.numpy()
        if mode == "refresh" or first is None:
            ks, kz = oq.compute_scale_zero(kn)
            vs, vz = oq.compute_scale_zero(vn)
            first = first or (ks, kz, vs, vz)
        else:
            ks, kz, vs, vz = first                  # rulers frozen at the first decode step
        kp, vp = oq.quantize_tensor(kn, ks, kz), oq.quantize_tensor(vn, vs, vz)
        if mode == "fixed":
            lay = st.layers[0]
            assert lay["n"] == S
            assert np.array_equal(lay["kb"][:, :S].cpu().numpy(), kp), f"K codes, {S} tokens"
            assert np.array_equal(lay["vb"][:, :S].cpu().numpy(), vp), f"V codes, {S} tokens"
            assert np.array_equal(lay["ks"].cpu().numpy(), ks) and np.array_equal(lay["vz"].cpu().numpy(), vz)
        ref = oa.decode_per_channel(q.numpy(), kp, ks, kz, vp, vs, vz)          # [H, 1, D]
        # the hook returns the model's dtype (fp16): its rounding is inside rel 1e-2
        assert_close(got[0, 0].numpy(), ref[:, 0], what=f"per-channel {mode}, {S} tokens")
    assert st.calls == kw.get("steps", 4)


@pytest.mark.parametrize("mode", ["fixed", "refresh"])
def test_per_channel_hook_matches_reference_harness(mode, monkeypatch):
    """Rulers frozen at the first decode step with each new token quantized
    against them (the buffer growing past its headroom), or re-derived every
    step: codes bit-exact with the reference quantizer, outputs within the bar."""
    monkeypatch.setattr(hl, "_kernel_module", _OraclePerChannel())
    _check_per_channel("cpu", mode)


def test_per_channel_hook_routes_other_calls_to_fp16(monkeypatch):
    k = _OraclePerChannel()
    monkeypatch.setattr(hl, "_kernel_module", k)
    st = hl.PerChannelKV("fixed")
    g = torch.Generator().manual_seed(0)
    q, kk, vv = (torch.randn(s, generator=g) for s in ((2, 4, 1, 64), (2, 2, 9, 64), (2, 2, 9, 64)))
    hl.per_channel_attention(SimpleNamespace(layer_idx=0), q, kk, vv, None, per_channel_kv=st)   # batch 2
    hl.per_channel_attention(SimpleNamespace(layer_idx=0), q[:1].expand(1, 4, 9, 64).contiguous(),
                             kk[:1], vv[:1], None, per_channel_kv=st)                         # prefill
    assert k.decode_calls == 0 and st.calls == 0
    with pytest.raises(ValueError, match="mode"):
        hl.PerChannelKV("int8")


def test_tiny_model_per_channel_modes(monkeypatch):
    """Batch-1 greedy decode of a tiny model in both per-channel modes: one
    decode call per layer and step, logits close to the fp16 path."""
    k = _OraclePerChannel()
    monkeypatch.setattr(hl, "_kernel_module", k)
    model = hl.build_model(_tiny_config(), "cpu", dtype=torch.float32, seed=1)
    ids = torch.randint(0, 97, (1, 30), generator=torch.Generator().manual_seed(2))
    _, ref, _, _ = hl.greedy_decode(model, ids, 5, "fp16")
    for mode in ("per_channel_fixed", "per_channel_refresh"):
        before = k.decode_calls
        toks, logits, _, _ = hl.greedy_decode(model, ids, 5, mode)
        assert toks.shape == (1, 5) and torch.equal(logits[0], ref[0])
        assert k.decode_calls - before == 2 * 5
        cos = torch.nn.functional.cosine_similarity(ref[1].double(), logits[1].double(), dim=-1)
        assert float(cos.min()) > 0.95, (mode, float(cos.min()))
    with pytest.raises(ValueError, match="batch 1"):
        hl.DecodeRunner(model, "per_channel_fixed", 2, 40)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fixed", "refresh"])
@pytest.mark.parametrize("H,KV,D", [(32, 4, 64), (12, 2, 128)])
def test_per_channel_hook_on_the_gpu(mode, H, KV, D):
    """The same steps through the HIP quantizers and per-channel decode."""
    _check_per_channel("cuda:0", mode, H=H, KV=KV, D=D, S0=300, steps=4, headroom=2)


@pytest.mark.gpu
def test_per_channel_model_modes_on_the_gpu():
    """Two layers of the 1.1B shape at batch 1: both per-channel modes decode
    through the HIP kernels, one decode call per layer and step, and their
    first-step logits match the fp16 path's in direction."""
    cfg = hl.llama_1b_config(num_hidden_layers=2)
    model = hl.build_model(cfg, "cuda:0", seed=3)
    ids = torch.randint(0, cfg.vocab_size, (1, 200), generator=torch.Generator().manual_seed(4)).to("cuda:0")
    _, ref, _, _ = hl.greedy_decode(model, ids, 4, "fp16")
    for mode in ("per_channel_fixed", "per_channel_refresh"):
        run = hl.DecodeRunner(model, mode, 1, 204)
        logits = [run(ids)]
        nxt = logits[0].argmax(-1, keepdim=True)
        for _ in range(4):
            logits.append(run(nxt))
            nxt = logits[-1].argmax(-1, keepdim=True)
        assert run.per_channel.calls == 2 * 4
        assert torch.equal(logits[0], ref[0])
        cos = float(torch.nn.functional.cosine_similarity(ref[1].double(), logits[1].double(), dim=-1).min())
        print(f"{mode}: first decode step cosine vs fp16 {cos:.5f}")
        assert cos > 0.95
