"""The CPU baseline's torch composition (oracle/cpu_path.py) against the float64
oracle (oracle/attention.py).

cpu_path restates the reference's CPU check path (kernels/benchmark/benchmark.py:
59-66,112-117): dequantize in fp32, round to fp16, repeat_interleave the KV heads,
fp32 SDPA.  bench.py times it as the CPU baseline and compares it with the GPU
output, so it is pinned here on its own:

* paged_decode against decode_paged_batched on caches written by the oracle's
  store: several block sizes and head groupings, lengths 0, 1, 15, 16, 17 and a
  few hundred, scrambled block tables.  The only difference between the two is
  cpu_path's fp16 rounding of the dequantized K/V (relative 2^-11), so they
  agree far inside the 2e-3 bar;
* decode_per_channel against the oracle's per-channel decode with the same fp16
  rounding (round_fp16=True): agreement to fp32 precision;
* planted mistakes in a copy of the composition (min and step swapped, the GQA
  map h % KV instead of h // G, high and low nibbles swapped) each fail the
  same comparison, so the comparison can see them.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from common import assert_close, make_paged_case
from oracle import attention as oatt
from oracle import cpu_path
from oracle import quant as oq


@pytest.mark.parametrize("B,H,KV,D,bs,lens", [
    (5, 8, 2, 64, 16, [0, 1, 15, 16, 17]),
    (3, 32, 8, 128, 16, [300, 1, 129]),
    (3, 6, 3, 80, 8, [33, 0, 90]),
    (2, 4, 4, 128, 32, [64, 200]),
])
def test_paged_decode_matches_float64_oracle(B, H, KV, D, bs, lens):
    case = make_paged_case(7 + D, B, H, KV, D, block_size=bs, lens=lens)
    ref = oatt.decode_paged_batched(case.q.numpy(), case.kv_cache, case.block_tables.numpy(),
                                    case.seq_lens.numpy())
    got = cpu_path.paged_decode(case.q, torch.from_numpy(case.kv_cache), case.block_tables,
                                case.seq_lens, bs, KV)
    assert_close(got.numpy(), ref, atol=2e-3, rtol=1e-2, what="cpu_path.paged_decode")
    # the two differ only by the fp16 rounding of K/V: tighter than the bar
    assert np.abs(got.numpy() - ref).max() < 1e-3


def test_paged_decode_subset_of_sequences():
    case = make_paged_case(3, 4, 8, 2, 64, lens=[20, 40, 60, 80])
    full = cpu_path.paged_decode(case.q, torch.from_numpy(case.kv_cache), case.block_tables,
                                 case.seq_lens, 16, 2)
    part = cpu_path.paged_decode(case.q, torch.from_numpy(case.kv_cache), case.block_tables,
                                 case.seq_lens, 16, 2, seqs=[1, 3])
    assert torch.equal(part[1], full[1]) and torch.equal(part[3], full[3])
    assert not part[0].any() and not part[2].any()


def _per_channel_case(seed, H, KV, S, D):
    g = np.random.default_rng(seed)
    k = g.standard_normal((KV, S, D)).astype(np.float16)
    v = g.standard_normal((KV, S, D)).astype(np.float16)
    kp, ks, kz, vp, vs, vz = oq.quantize_kv(k, v)
    q = g.standard_normal((H, 1, D)).astype(np.float16)
    return q, kp, ks, kz, vp, vs, vz


@pytest.mark.parametrize("H,KV,S,D", [(32, 4, 512, 64), (32, 8, 1024, 128), (8, 8, 33, 128)])
def test_decode_per_channel_matches_float64_oracle(H, KV, S, D):
    q, kp, ks, kz, vp, vs, vz = _per_channel_case(H + S, H, KV, S, D)
    ref = oatt.decode_per_channel(q, kp, ks, kz, vp, vs, vz, round_fp16=True)
    t = torch.from_numpy
    got = cpu_path.decode_per_channel(t(q), t(kp), t(ks), t(kz), t(vp), t(vs), t(vz))
    assert_close(got.numpy(), ref, atol=1e-5, rtol=1e-5, what="cpu_path.decode_per_channel")


# ---------------------------------------------------------------- planted mistakes
def _paged_variant(q, kv_cache, tables, lens, bs, KV, mistake):
    """cpu_path.paged_decode's composition with one planted mistake."""
    B, H, D = q.shape
    G = H // KV
    out = torch.zeros((B, H, D), dtype=torch.float32)
    for b in range(B):
        L = int(lens[b])
        n = torch.arange(L)
        slots = kv_cache[tables[b].long()[n // bs], n % bs]
        rul = slots[..., D:].contiguous().view(torch.float16).float()
        kb, vb = slots[..., : D // 2], slots[..., D // 2: D]

        def unpack(x):
            lo, hi = x & 0x0F, x >> 4
            if mistake == "nibbles":
                lo, hi = hi, lo
            return torch.stack([lo, hi], dim=-1).flatten(-2).float()

        if mistake == "ruler_order":
            k = unpack(kb) * rul[..., 0:1] + rul[..., 1:2]
        else:
            k = unpack(kb) * rul[..., 1:2] + rul[..., 0:1]
        v = unpack(vb) * rul[..., 3:4] + rul[..., 2:3]
        k = k.half().float().permute(1, 0, 2)
        v = v.half().float().permute(1, 0, 2)
        idx = torch.arange(H) % KV if mistake == "gqa_map" else torch.arange(H) // G
        out[b] = F.scaled_dot_product_attention(q[b].float()[:, None, :], k[idx], v[idx])[:, 0]
    return out


@pytest.mark.parametrize("mistake", ["ruler_order", "gqa_map", "nibbles"])
def test_planted_mistakes_are_seen(mistake):
    case = make_paged_case(11, 3, 8, 2, 64, lens=[40, 70, 100])
    ref = oatt.decode_paged_batched(case.q.numpy(), case.kv_cache, case.block_tables.numpy(),
                                    case.seq_lens.numpy())
    args = (case.q, torch.from_numpy(case.kv_cache), case.block_tables, case.seq_lens, 16, 2)
    good = _paged_variant(*args, mistake=None)
    assert_close(good.numpy(), ref, atol=2e-3, rtol=1e-2, what="unplanted variant")
    bad = _paged_variant(*args, mistake=mistake)
    with pytest.raises(AssertionError):
        assert_close(bad.numpy(), ref, atol=2e-3, rtol=1e-2, what=mistake)
