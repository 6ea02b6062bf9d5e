"""Pins the dequant-then-attend oracle (oracle/attention.py) by properties the
mathematics fixes, each chosen so that a plausible mistake fails it:

* torch's float64 SDPA over repeat_interleave'd KV heads (a library routine
  written independently of the oracle) -- catches a wrong scale, GQA map or
  softmax axis;
* S = 1 gives the dequantized V row; q = 0 gives the mean of V;
* permuting physical blocks together with the block table changes nothing;
* per-token rulers with step = scale and min = -zero * scale reproduce the
  per-channel path (when every row has the same rulers);
* causal prefill row m equals decode over keys 0..m;
* paged gather addresses cache[block_row[n // bs], n % bs, kv];
* the batched paged oracle equals per-request decode and gives zeros for
  empty sequences.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import quant as oq


def _rand_packed(rng, KV, S, D):
    return rng.integers(0, 256, (KV, S, D // 2), dtype=np.uint8)


def _sdpa_reference(q, K, V):
    """q [H, M, D], K/V [KV, S, D] float64 through torch SDPA with GQA expanded."""
    H, KV = q.shape[0], K.shape[0]
    Kt = torch.from_numpy(K).repeat_interleave(H // KV, dim=0)
    Vt = torch.from_numpy(V).repeat_interleave(H // KV, dim=0)
    return F.scaled_dot_product_attention(torch.from_numpy(q), Kt, Vt).numpy()


@pytest.mark.parametrize("H,KV,D,S", [(4, 4, 64, 37), (12, 2, 128, 50), (8, 1, 80, 9)])
def test_attend_matches_torch_sdpa(H, KV, D, S):
    rng = np.random.default_rng(H * 100 + S)
    q = rng.standard_normal((H, 3, D))
    K = rng.standard_normal((KV, S, D))
    V = rng.standard_normal((KV, S, D))
    np.testing.assert_allclose(oa.attend(q, K, V), _sdpa_reference(q, K, V), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(oa.attend(q[:, 0], K, V), _sdpa_reference(q[:, :1], K, V)[:, 0], rtol=1e-10)


def test_single_token_returns_its_value_row():
    rng = np.random.default_rng(1)
    H, KV, D = 8, 2, 64
    kp, vp = _rand_packed(rng, KV, 1, D), _rand_packed(rng, KV, 1, D)
    mins = rng.standard_normal((KV, 1)).astype(np.float16)
    steps = (rng.random((KV, 1)) + 0.1).astype(np.float16)
    q = rng.standard_normal((H, 1, D)).astype(np.float16)
    out = oa.decode_per_token(q, kp, mins, steps, vp, mins, steps)
    V = oq.unpack_nibbles(vp).astype(np.float64) * steps.astype(np.float64)[..., None] + \
        mins.astype(np.float64)[..., None]
    for h in range(H):
        np.testing.assert_allclose(out[h, 0], V[h // (H // KV), 0], rtol=0, atol=1e-12)


def test_zero_query_averages_values():
    rng = np.random.default_rng(2)
    KV, S, D = 2, 33, 64
    kp, vp = _rand_packed(rng, KV, S, D), _rand_packed(rng, KV, S, D)
    scale = (rng.random((KV, D)) + 0.05).astype(np.float16)
    zero = rng.integers(0, 16, (KV, D)).astype(np.float16)
    out = oa.decode_per_channel(np.zeros((4, 1, D), np.float16), kp, scale, zero, vp, scale, zero)
    V = oa.dequant_per_channel(vp, scale, zero)
    np.testing.assert_allclose(out[:, 0], np.repeat(V.mean(axis=1), 2, axis=0), rtol=1e-12, atol=1e-12)


def test_raw_nibbles_when_quantization_is_off():
    rng = np.random.default_rng(3)
    kp = _rand_packed(rng, 1, 5, 64)
    got = oa.dequant_per_channel(kp, np.full((1, 64), 7, np.float16), np.full((1, 64), 3, np.float16),
                                 use_quant=False)
    assert np.array_equal(got, oq.unpack_nibbles(kp).astype(np.float64))


def test_per_token_equals_per_channel_with_equal_rulers():
    """min = -zero*scale, step = scale for every token -> same dequant."""
    rng = np.random.default_rng(4)
    H, KV, S, D = 6, 3, 20, 64
    kp, vp = _rand_packed(rng, KV, S, D), _rand_packed(rng, KV, S, D)
    s, z = np.float16(0.125), np.float16(5)
    scale = np.full((KV, D), s, np.float16)
    zero = np.full((KV, D), z, np.float16)
    mins = np.full((KV, S), -z * s, np.float16)
    steps = np.full((KV, S), s, np.float16)
    q = rng.standard_normal((H, 1, D)).astype(np.float16)
    a = oa.decode_per_channel(q, kp, scale, zero, vp, scale, zero)
    b = oa.decode_per_token(q, kp, mins, steps, vp, mins, steps)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_causal_prefill_rows_are_prefix_decodes():
    rng = np.random.default_rng(5)
    H, KV, M, D = 4, 2, 7, 64
    q = rng.standard_normal((H, M, D))
    K = rng.standard_normal((KV, M, D))
    V = rng.standard_normal((KV, M, D))
    out = oa.attend_causal(q, K, V, causal=True)
    for m in range(M):
        np.testing.assert_allclose(out[:, m], oa.attend(q[:, m], K[:, : m + 1], V[:, : m + 1]), rtol=1e-12)
    np.testing.assert_allclose(oa.attend_causal(q, K, V, causal=False), oa.attend(q, K, V), rtol=1e-12)


def test_empty_sequence_is_nan_like_the_reference():
    out = oa.attend(np.ones((2, 64)), np.zeros((1, 0, 64)), np.zeros((1, 0, 64)))
    assert np.isnan(out).all()


def _paged(rng, B, KV, D, bs, lens):
    nblk = [(L + bs - 1) // bs for L in lens]
    total = sum(nblk)
    cache = rng.integers(0, 256, (total, bs, KV, D + 8), dtype=np.uint8)
    # sane rulers (finite fp16 min/step) in every slot
    rul = np.stack([rng.standard_normal((total, bs, KV)), rng.random((total, bs, KV)) + 0.01,
                    rng.standard_normal((total, bs, KV)), rng.random((total, bs, KV)) + 0.01], -1)
    cache[..., D:] = rul.astype(np.float16).view(np.uint8).reshape(total, bs, KV, 8)
    perm = rng.permutation(total)
    tables = np.zeros((B, max(nblk)), dtype=np.int64)
    off = 0
    for b in range(B):
        tables[b, : nblk[b]] = perm[off: off + nblk[b]]
        off += nblk[b]
    return cache, tables


def test_gather_paged_addresses_block_then_position():
    rng = np.random.default_rng(6)
    KV, D, bs = 2, 64, 4
    cache, tables = _paged(rng, 1, KV, D, bs, [10])
    kp, vp, rul = oa.gather_paged(cache, tables[0], 10)
    for n in range(10):
        slot = cache[tables[0, n // bs], n % bs]
        for kv in range(KV):
            assert np.array_equal(kp[kv, n], slot[kv, : D // 2])
            assert np.array_equal(vp[kv, n], slot[kv, D // 2: D])
            assert np.array_equal(rul[kv, n].view(np.uint8), slot[kv, D:])


def test_block_permutation_invariance():
    rng = np.random.default_rng(7)
    H, KV, D, bs = 8, 2, 64, 4
    cache, tables = _paged(rng, 1, KV, D, bs, [23])
    q = rng.standard_normal((H, D)).astype(np.float16)
    ref = oa.decode_paged(q, cache, tables[0], 23)
    perm = rng.permutation(cache.shape[0])
    inv = np.argsort(perm)
    cache2 = cache[perm]                      # block i moves to position inv[i]
    np.testing.assert_allclose(oa.decode_paged(q, cache2, inv[tables[0]], 23), ref, rtol=1e-12)


def test_batched_paged_equals_per_request_and_zero_for_empty():
    rng = np.random.default_rng(8)
    B, H, KV, D, bs = 4, 4, 2, 64, 8
    lens = [5, 0, 17, 8]
    cache, tables = _paged(rng, B, KV, D, bs, [max(1, L) for L in lens])
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    out = oa.decode_paged_batched(q, cache, tables, lens)
    assert np.all(out[1] == 0)
    for b in (0, 2, 3):
        np.testing.assert_allclose(out[b], oa.decode_paged(q[b], cache, tables[b], lens[b]), rtol=0)
