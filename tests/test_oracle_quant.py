"""Pins the oracle's quantizers (CPU only).

Per-channel quantizer (reference kernels/benchmark/benchmark.py:26-66):
  * bit-exact against golden vectors written by tests/golden/make_golden_quant.py
    from the reference's own torch functions;
  * known answers computed by hand (constant channel, [-1, 1] channel, clamps,
    ties-to-even) so a wrong rounding mode or a dropped op fails.
Per-token store (reference kernels/kv_dequant_kernels.cuh:816-919):
  * known answers (constant row, exact lattice rows, NaN guard, skipped slots);
  * exact-arithmetic properties: the step is the correctly rounded fp32
    (max-min)/15 and every code is the round-half-up nearest lattice point,
    up to fp32 rounding of the quotient;
  * the fp32 -> fp16 ruler conversion matches numpy's nearest-even cast.
"""
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import quant as oq
from oracle.attention import dequant_per_channel

GOLDEN = Path(__file__).resolve().parent / "golden" / "per_channel_quant.npz"


def _cases():
    z = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in z.files})
    return z, names


@pytest.mark.parametrize("name", _cases()[1])
def test_per_channel_matches_reference_golden(name):
    z, _ = _cases()
    x = z[f"{name}__x"].view(np.float16)
    scale, zero = oq.compute_scale_zero(x)
    packed = oq.quantize_tensor(x, scale, zero)
    assert np.array_equal(scale.view(np.uint16), z[f"{name}__scale"])
    assert np.array_equal(zero.view(np.uint16), z[f"{name}__zero"])
    assert np.array_equal(packed, z[f"{name}__packed"])
    deq = dequant_per_channel(packed, scale, zero).astype(np.float32)
    ref = z[f"{name}__deq"]
    same = (deq == ref) | (np.isnan(deq) & np.isnan(ref))
    assert same.all()


def test_per_channel_known_answers():
    """Hand-computed answers (fp16 arithmetic worked out on paper)."""
    S = 16
    x = np.zeros((1, S, 64), dtype=np.float16)
    x[0, :, 0] = 0.75                                    # constant
    x[0, :, 1] = np.linspace(-1, 1, S)                   # [-1, 1]
    x[0, :, 2] = np.linspace(0.5, 3.0, S)                # all positive
    x[0, :, 3] = np.linspace(-3.0, -0.5, S)              # all negative
    x[0, :, 4] = np.float16(-6.5)                        # [-6.5, 6.5]
    x[0, 0, 4] = np.float16(6.5)
    scale, zero = oq.compute_scale_zero(x)
    codes = oq.unpack_nibbles(oq.quantize_tensor(x, scale, zero))[0]
    # constant channel: scale 1, zero 0, code = clamp(round(0.75), 0, 15) = 1
    assert (float(scale[0, 0]), float(zero[0, 0])) == (1.0, 0.0)
    assert (codes[:, 0] == 1).all()
    # [-1, 1]: 2/15 -> fp16 0.13330078125 (= 273 * 2^-11); -1/that = -7.5018 -> fp16 -7.5;
    # round half to even -> -8; zero = 8; codes 0 at -1 and clamp(8 + 8) = 15 at +1
    assert float(scale[0, 1]) == 273 * 2.0 ** -11
    assert float(zero[0, 1]) == 8.0
    assert codes[0, 1] == 0 and codes[-1, 1] == 15
    # all positive: zero = -round(0.5 / 0.16663) = -3 -> clamps to 0
    assert float(zero[0, 2]) == 0.0
    # all negative: 2.5/15 -> fp16 0.1666259765625; -3/that = -18.004 -> zero 18 -> clamps to 15
    assert float(scale[0, 3]) == 0.1666259765625
    assert float(zero[0, 3]) == 15.0
    # [-6.5, 6.5]: 13/15 -> fp16 0.86669921875 (1775 * 2^-11); -6.5/that = -7.49972 -> fp16 -7.5
    # -> round half to even -8 -> zero 8 (round-half-away would give the same; -8.5 below tests that)
    assert float(scale[0, 4]) == 1775 * 2.0 ** -11
    assert float(zero[0, 4]) == 8.0
    # round(-6.5) = -6 (even), not -7: x = -6.5 with scale 1 (constant channel) and zero 0 -> code 0
    y = np.full((1, 4, 64), np.float16(2.5))
    s2, z2 = oq.compute_scale_zero(y)
    assert (oq.unpack_nibbles(oq.quantize_tensor(y, s2, z2)) == 2).all()   # round(2.5) = 2


def test_nibble_order():
    """Even dim in the low nibble, odd dim in the high nibble."""
    x = np.zeros((1, 2, 64), dtype=np.float16)
    x[0, 1, 0] = 1.0   # dim 0 high code in token 1 -> low nibble
    x[0, 1, 1] = 0.0
    x[0, 0, 1] = 1.0   # dim 1 high code in token 0 -> high nibble
    scale, zero = oq.compute_scale_zero(x)
    p = oq.quantize_tensor(x, scale, zero)
    assert p[0, 1, 0] & 0x0F == 15 and p[0, 1, 0] >> 4 == 0
    assert p[0, 0, 0] & 0x0F == 0 and p[0, 0, 0] >> 4 == 15


# ---------------------------------------------------------------------- store
def _store_one(row, KV=1, D=None, slot=0, bs=16):
    row = np.asarray(row, dtype=np.float16)
    D = row.shape[0]
    key = np.tile(row, (1, KV, 1)).reshape(1, KV, D)
    cache = np.full((2, bs, KV, D + 8), 0xAB, dtype=np.uint8)
    oq.quantize_store(key, key, cache, np.array([slot], dtype=np.int64), bs)
    return cache


def test_store_constant_row():
    c = _store_one(np.full(128, 0.75))
    k, v, r = oq.split_slot(c[0, 0, 0], 128)
    assert (k == 0).all() and (v == 0).all()
    assert r[0] == np.float16(0.75) and r[1] == np.float16(1.0)


def test_store_lattice_row():
    codes = np.arange(128) % 16
    row = (-1.0 + codes * 0.125).astype(np.float16)      # min -1, max 0.875, step 0.125
    c = _store_one(row)
    k, _, r = oq.split_slot(c[0, 0, 0], 128)
    assert np.array_equal(k, codes)
    assert r[0] == np.float16(-1.0) and r[1] == np.float16(0.125)


def test_store_nan_rows_and_guard():
    # all-NaN row, D = 128: min/max are NaN, !(step > 0) -> step 1, codes 0
    c = _store_one(np.full(128, np.nan))
    k, _, r = oq.split_slot(c[0, 0, 0], 128)
    assert (k == 0).all()
    assert np.isnan(r[0]) and r[1] == np.float16(1.0)
    # all-NaN row, D = 64: the reference's +inf/-inf padding threads win
    c = _store_one(np.full(64, np.nan))
    k, _, r = oq.split_slot(c[0, 0, 0], 64)
    assert (k == 0).all()
    assert r[0] == np.float16(np.inf) and r[1] == np.float16(1.0)
    row = np.linspace(-1, 1, 64); row[5] = np.nan         # NaN ignored by min/max
    c = _store_one(row)
    k, _, r = oq.split_slot(c[0, 0, 0], 64)
    assert r[0] == np.float16(-1.0) and k[5] == 0 and k[-1] == 15


def test_store_skips_negative_and_out_of_range_slots():
    key = np.ones((3, 2, 64), dtype=np.float16)
    cache = np.full((2, 16, 2, 72), 0x5A, dtype=np.uint8)
    oq.quantize_store(key, key, cache, np.array([-1, 32, 99], dtype=np.int64), 16)
    assert (cache == 0x5A).all()


def test_store_slot_addressing():
    """slot = block * bs + pos; KV heads interleave inside the token row."""
    g = np.random.default_rng(0)
    KV, D, bs = 3, 80, 8
    key = g.standard_normal((4, KV, D)).astype(np.float16)
    val = g.standard_normal((4, KV, D)).astype(np.float16)
    slots = np.array([0, 9, 23, 7], dtype=np.int64)
    cache = np.zeros((4, bs, KV, D + 8), dtype=np.uint8)
    oq.quantize_store(key, val, cache, slots, bs)
    for t, s in enumerate(slots):
        for h in range(KV):
            pk, mn, st = oq.quantize_row(key[t, h])
            pv, _, _ = oq.quantize_row(val[t, h])
            slot = cache[s // bs, s % bs, h]
            assert np.array_equal(slot[: D // 2], pk) and np.array_equal(slot[D // 2: D], pv)
            assert slot[D:D + 2].view(np.float16)[0] == np.float16(mn)


def _f32_round(fr: Fraction) -> np.float32:
    """Correctly rounded fp32 (nearest, ties to even) of an exact rational."""
    x = np.float32(float(fr))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - fr)
        if best is None or d < best[0] or (d == best[0] and int(c.view(np.uint32)) % 2 == 0):
            best = (d, c)
    return best[1]


@pytest.mark.parametrize("seed", range(6))
def test_store_exact_arithmetic_properties(seed):
    g = np.random.default_rng(seed)
    scale = [1.0, 1e-3, 300.0, 8.0, 1.0, 0.02][seed]
    row = (g.standard_t(3, 128) * scale).astype(np.float16)
    packed, mn, step = oq.quantize_row(row)
    xs = [Fraction(float(v)) for v in row.astype(np.float64)]
    fmin, fmax = min(xs), max(xs)
    assert Fraction(float(mn)) == fmin
    diff32 = _f32_round(fmax - fmin)                       # IEEE fp32 subtraction
    assert step == _f32_round(Fraction(float(diff32)) / 15)  # IEEE fp32 division by 15
    codes = oq.unpack_nibbles(packed)
    for x, c in zip(xs, codes):
        t = (x - fmin) / Fraction(float(step))            # exact quotient
        exact = min(15, int(t + Fraction(1, 2)))          # round half up, clamp
        if abs((t + Fraction(1, 2)) - round(t + Fraction(1, 2))) > Fraction(1, 1 << 18):
            assert c == exact, (float(x), float(t), c, exact)
        else:
            assert c in (exact - 1, exact)                 # quotient within fp32 rounding of a tie


def test_float_to_half_matches_numpy():
    g = np.random.default_rng(0)
    vals = np.concatenate([
        g.standard_normal(4000).astype(np.float32) * 10.0 ** g.integers(-9, 6, 4000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e30, -1e30, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf], dtype=np.float32),
        np.arange(0, 65536, dtype=np.uint16).view(np.float16)[:0x7C00].astype(np.float32) * np.float32(1.0009765625),
    ])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oq.float_to_half_bits(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref), vals[got != ref][:5]
    assert oq.float_to_half_bits(float("nan")) & 0x7C00 == 0x7C00
