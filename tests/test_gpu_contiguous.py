"""GPU parity of the standalone (contiguous) entry points against the oracle:
per-channel decode and prefill (reference kernels/kv_dequant_kernels.cuh:113-502),
per-token decode (:528-655) and the per-channel quantizer on the GPU
(reference host code kernels/benchmark/benchmark.py:26-56, bit-exact)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from common import assert_close, kv_values
from oracle import attention as oa
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = Path(__file__).resolve().parent / "golden" / "per_channel_quant.npz"


def _kd():
    from kernels import kv_dequant
    return kv_dequant


def _outliers(x: torch.Tensor, gen, frac=0.01, factor=8.0):
    KV, S, D = x.shape
    n = max(1, int(np.ceil(frac * KV * D)))
    for c in torch.randperm(KV * D, generator=gen)[:n].tolist():
        x[c // D, :, c % D] *= factor
    return x


# ------------------------------------------------------------------ quantizer
def _same_fp16(got, ref):
    """Bit-exact fp16, except that any NaN matches any NaN (the sign and
    payload of a NaN produced by 0/0 differ between x86 and the GPU)."""
    same = (got.view(np.uint16) == ref.view(np.uint16)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), f"{int((~same).sum())} values differ, first at {np.argwhere(~same)[:3].tolist()}"


@pytest.mark.parametrize("name", sorted({k.split("__")[0] for k in np.load(GOLDEN).files}))
def test_quantize_per_channel_matches_reference_golden(name):
    z = np.load(GOLDEN)
    x = torch.from_numpy(z[f"{name}__x"].view(np.float16).copy())
    packed, scale, zero = _kd().quantize_per_channel(x.to(DEV))
    torch.cuda.synchronize()
    _same_fp16(scale.cpu().numpy(), z[f"{name}__scale"].view(np.float16))
    _same_fp16(zero.cpu().numpy(), z[f"{name}__zero"].view(np.float16))
    assert np.array_equal(packed.cpu().numpy(), z[f"{name}__packed"])


@pytest.mark.parametrize("name", sorted({k.split("__")[0] for k in np.load(GOLDEN).files}))
def test_quantize_tensor_with_rulers_matches_reference_golden(name):
    """The fixed-ruler append packs the reference quantizer's own (x, scale,
    zero) into exactly the reference's bytes."""
    z = np.load(GOLDEN)
    x = torch.from_numpy(z[f"{name}__x"].view(np.float16).copy()).to(DEV)
    scale = torch.from_numpy(z[f"{name}__scale"].view(np.float16).copy()).to(DEV)
    zero = torch.from_numpy(z[f"{name}__zero"].view(np.float16).copy()).to(DEV)
    packed = _kd().quantize_tensor(x, scale, zero)
    torch.cuda.synchronize()
    assert np.array_equal(packed.cpu().numpy(), z[f"{name}__packed"])


@pytest.mark.parametrize("KV,S0,S1,D", [(2, 64, 1, 128), (4, 512, 37, 64), (2, 100, 300, 80), (1, 16, 8, 128)])
def test_quantize_tensor_appends_with_frozen_rulers(KV, S0, S1, D):
    """The reference's model-harness append (kernels/benchmark/benchmark.py:
    205-216): rulers from the first S0 tokens, new tokens (some outside the
    rulers' range, so the clamp acts) packed into a slice of a preallocated
    [KV, capacity, D/2] cache; bytes outside the slice stay as they were."""
    g = torch.Generator().manual_seed(S0 + S1 + D)
    x0 = _outliers(torch.randn(KV, S0, D, generator=g), g).half()
    x1 = (3.0 * torch.randn(KV, S1, D, generator=g)).half()
    _, scale, zero = _kd().quantize_per_channel(x0.to(DEV))
    cap = S0 + S1 + 9
    cache = torch.full((KV, cap, D // 2), 0xA5, dtype=torch.uint8, device=DEV)
    # a token-strided source, as a slice of a longer [KV, L, D] tensor
    src = torch.cat([x0, x1], dim=1).to(DEV)[:, S0:, :]
    _kd().quantize_tensor(src, scale, zero, out=cache[:, S0:S0 + S1])
    torch.cuda.synchronize()
    ref = oq.quantize_tensor(x1.numpy(), scale.cpu().numpy(), zero.cpu().numpy())
    got = cache.cpu().numpy()
    assert np.array_equal(got[:, S0:S0 + S1], ref)
    assert (got[:, :S0] == 0xA5).all() and (got[:, S0 + S1:] == 0xA5).all()
    codes = np.stack([ref & 15, ref >> 4], axis=-1)
    assert (codes == 0).any() and (codes == 15).any()      # both clamps were exercised


def test_quantize_tensor_special_values():
    """NaN, +-inf, +-0, +-65504 and subnormal inputs against tiny, unit and
    huge rulers, bit-exact with the oracle (NaN codes become 0 on both)."""
    D, KV = 64, 2
    vals = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 65504.0, -65504.0, 6e-8, -6e-8, 1.0, -1.0,
                     0.5, 1.5, 2.5, 7.49, 7.51], dtype=np.float16)
    x = np.resize(vals, (KV, 8, D)).astype(np.float16)
    scale = np.resize(np.array([6e-8, 1.0, 4096.0, 0.0133], dtype=np.float16), (KV, D)).astype(np.float16)
    zero = np.resize(np.array([0.0, 8.0, 15.0, 3.0], dtype=np.float16), (KV, D)).astype(np.float16)
    got = _kd().quantize_tensor(torch.from_numpy(x).to(DEV), torch.from_numpy(scale).to(DEV),
                                torch.from_numpy(zero).to(DEV))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oq.quantize_tensor(x, scale, zero))


@pytest.mark.parametrize("KV,S,D", [(4, 512, 64), (2, 2048, 128), (2, 333, 80), (8, 1, 128)])
def test_quantize_per_channel_matches_oracle(KV, S, D):
    g = torch.Generator().manual_seed(S + D)
    x = _outliers(torch.randn(KV, S, D, generator=g), g).half()
    packed, scale, zero = _kd().quantize_per_channel(x.to(DEV))
    torch.cuda.synchronize()
    s_ref, z_ref = oq.compute_scale_zero(x.numpy())
    p_ref = oq.quantize_tensor(x.numpy(), s_ref, z_ref)
    _same_fp16(scale.cpu().numpy(), s_ref)
    _same_fp16(zero.cpu().numpy(), z_ref)
    assert np.array_equal(packed.cpu().numpy(), p_ref)


# ------------------------------------------------------------------ per-channel decode
def _pc_inputs(seed, H, KV, S, D, outliers=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, 1, D, generator=g).half()
    k = torch.randn(KV, S, D, generator=g)
    v = torch.randn(KV, S, D, generator=g)
    if outliers:
        k, v = _outliers(k, g), _outliers(v, g)
    kp, ks, kz, vp, vs, vz = oq.quantize_kv(k.half().numpy(), v.half().numpy())
    return q, [torch.from_numpy(a) for a in (kp, ks, kz, vp, vs, vz)]


@pytest.mark.parametrize("H,KV,D,S,outl", [(4, 4, 64, 512, False),            # config 1
                                           (12, 2, 128, 512, True),            # config 2
                                           (12, 2, 128, 1024, True),
                                           (12, 2, 128, 2048, True),
                                           (32, 4, 64, 1024, False), (32, 8, 128, 700, False),
                                           (14, 2, 64, 333, False), (8, 8, 80, 97, False)])
def test_decode_per_channel(H, KV, D, S, outl):
    q, t = _pc_inputs(H * 7 + S, H, KV, S, D, outl)
    out = _kd().kv_dequant_decode_attention(q.to(DEV), *[x.to(DEV) for x in t], num_kv_heads=KV)
    torch.cuda.synchronize()
    assert out.shape == (H, 1, D) and out.dtype == torch.float32
    ref = oa.decode_per_channel(q.numpy(), *[x.numpy() for x in t])
    assert_close(out.cpu().numpy(), ref, what="per-channel decode")
    # The reference benchmark's own check rounds the dequantized KV to fp16
    # before attending (kernels/benchmark/benchmark.py:112).  Against that
    # oracle the bar widens by the two oracles' own difference.
    ref16 = oa.decode_per_channel(q.numpy(), *[x.numpy() for x in t], round_fp16=True)
    gap = np.abs(ref16 - ref).max()
    assert_close(out.cpu().numpy(), ref16, atol=2e-3 + gap, what="vs fp16-rounded dequant")


def test_decode_per_channel_raw_nibbles_and_block_n():
    q, t = _pc_inputs(5, 8, 2, 300, 128)
    kd = _kd()
    raw = kd.kv_dequant_decode_attention(q.to(DEV), *[x.to(DEV) for x in t], BLOCK_N=32,
                                         use_quant=False, num_kv_heads=2)
    torch.cuda.synchronize()
    ref = oa.decode_per_channel(q.numpy(), *[x.numpy() for x in t], use_quant=False)
    assert_close(raw.cpu().numpy(), ref, what="use_quant=False")


def test_decode_per_channel_fewer_kv_heads_than_tensor():
    """num_kv_heads < k_packed.shape[0]: only the first heads are attended."""
    q, t = _pc_inputs(6, 8, 4, 200, 64)
    out = _kd().kv_dequant_decode_attention(q.to(DEV), *[x.to(DEV) for x in t], num_kv_heads=2)
    torch.cuda.synchronize()
    kp, ks, kz, vp, vs, vz = [x.numpy() for x in t]
    ref = oa.decode_per_channel(q.numpy(), kp[:2], ks[:2], kz[:2], vp[:2], vs[:2], vz[:2])
    assert_close(out.cpu().numpy(), ref)


# ------------------------------------------------------------------ prefill
@pytest.mark.parametrize("H,KV,D,M,S,causal", [(32, 4, 64, 256, 256, True), (14, 2, 64, 100, 100, True),
                                               (8, 2, 128, 64, 64, True), (8, 8, 80, 50, 50, False),
                                               (4, 4, 64, 40, 70, True), (4, 2, 64, 70, 40, True)])
def test_prefill_per_channel(H, KV, D, M, S, causal):
    g = torch.Generator().manual_seed(M * 3 + S)
    q = torch.randn(H, M, D, generator=g).half()
    k = torch.randn(KV, S, D, generator=g).half()
    v = torch.randn(KV, S, D, generator=g).half()
    kp, ks, kz, vp, vs, vz = [torch.from_numpy(a) for a in oq.quantize_kv(k.numpy(), v.numpy())]
    kw = {} if D == 64 else {"BLOCK_M": 16, "BLOCK_N": 32}
    out = _kd().kv_dequant_prefill_attention(q.to(DEV), kp.to(DEV), ks.to(DEV), kz.to(DEV), vp.to(DEV),
                                             vs.to(DEV), vz.to(DEV), causal=causal, num_kv_heads=KV, **kw)
    torch.cuda.synchronize()
    ref = oa.prefill_per_channel(q.numpy(), kp.numpy(), ks.numpy(), kz.numpy(), vp.numpy(), vs.numpy(),
                                 vz.numpy(), causal=causal)
    assert out.shape == (H, M, D)
    assert_close(out.cpu().numpy(), ref, what="prefill")


def _pf_inputs(seed, H, KV, M, S, D, outliers=False, t3=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, M, D, generator=g).half()
    if t3:
        k, v = kv_values(g, (KV, S, D), "t3"), kv_values(g, (KV, S, D), "t3")
    else:
        k, v = torch.randn(KV, S, D, generator=g), torch.randn(KV, S, D, generator=g)
    if outliers:
        k, v = _outliers(k, g), _outliers(v, g)
    kp, ks, kz, vp, vs, vz = oq.quantize_kv(k.half().numpy(), v.half().numpy())
    return q, [torch.from_numpy(a) for a in (kp, ks, kz, vp, vs, vz)]


def _prefill(q, t, **kw):
    out = _kd().kv_dequant_prefill_attention(q.to(DEV), *[x.to(DEV) for x in t], **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# head_dim 64 and 128 run on the matrix-core kernel: query blocks of 64 rows,
# key tiles of 64, so these cover partial blocks and tiles, M > S and M < S
@pytest.mark.parametrize("H,KV,D,M,S,causal,outl,t3", [
    (32, 4, 64, 512, 512, True, False, False),     # the reference's op-level prefill shapes
    (14, 2, 64, 1024, 1024, True, False, False),
    (12, 2, 128, 300, 300, True, True, False),      # config-2 heads, 1 % outlier channels x8
    (8, 2, 128, 129, 1000, False, False, True),     # Student-t K/V, non-causal
    (8, 8, 64, 65, 63, True, True, False),          # M > S
    (4, 1, 128, 1, 777, True, False, False),        # a single row
    (16, 2, 64, 200, 1500, True, False, True)])     # M < S
def test_prefill_matrix_cores(H, KV, D, M, S, causal, outl, t3):
    q, t = _pf_inputs(H + M + S, H, KV, M, S, D, outl, t3)
    out = _prefill(q, t, causal=causal, num_kv_heads=KV)
    ref = oa.prefill_per_channel(q.numpy(), *[x.numpy() for x in t], causal=causal)
    assert_close(out, ref, what=f"prefill H={H} KV={KV} D={D} M={M} S={S}")


# Long causal prefills (up to 32 query blocks): one and two query heads per
# workgroup, both head dims, outliers and Student-t K/V, and S > M with a partial
# last block; a second call gives the same bits.
@pytest.mark.parametrize("H,KV,D,M,S,outl,t3", [
    (4, 2, 128, 2048, 2048, False, False),
    (8, 2, 64, 2048, 2048, True, False),
    (24, 2, 128, 1536, 1536, False, True),
    (32, 4, 64, 1536, 1536, False, False),
    (8, 4, 64, 1000, 1300, False, False)])
def test_prefill_matrix_cores_long(H, KV, D, M, S, outl, t3):
    q, t = _pf_inputs(H * 7 + M, H, KV, M, S, D, outl, t3)
    out = _prefill(q, t, causal=True, num_kv_heads=KV)
    ref = oa.prefill_per_channel(q.numpy(), *[x.numpy() for x in t], causal=True)
    assert_close(out, ref, what=f"long prefill H={H} KV={KV} D={D} M={M} S={S}")
    assert np.array_equal(out, _prefill(q, t, causal=True, num_kv_heads=KV))


# The two 4096-query causal prefills that bench.py --op-level times (two query
# heads per workgroup, every query block from 1 to 64 key tiles): heads spread
# over every KV head checked against the oracle head by head, and a second call
# gives the same bits.
@pytest.mark.parametrize("H,KV,D,heads", [
    (32, 4, 64, (0, 9, 18, 31)),
    (12, 2, 128, (0, 5, 6, 11))])
def test_prefill_matrix_cores_bench_shapes(H, KV, D, heads):
    S = 4096
    q, t = _pf_inputs(H + D, H, KV, S, S, D)
    out = _prefill(q, t, causal=True, num_kv_heads=KV)
    G = H // KV
    for h in heads:
        kv = h // G
        kvt = [x[kv:kv + 1].numpy() for x in t]
        ref = oa.prefill_per_channel(q[h:h + 1].numpy(), *kvt, causal=True)
        assert_close(out[h:h + 1], ref, what=f"bench-shape prefill H={H} KV={KV} D={D} head {h}")
    assert np.array_equal(out, _prefill(q, t, causal=True, num_kv_heads=KV))


def test_prefill_matrix_cores_unaligned_rulers():
    """V scale / zero point views that start 2 bytes into their storage (the
    epilogue's 8-byte ruler loads then take the 2-byte path)."""
    q, t = _pf_inputs(12, 8, 2, 200, 400, 64)
    qd = q.to(DEV)
    dev_t = [x.to(DEV) for x in t]
    for i in (4, 5):                                 # v_scale, v_zero
        big = torch.empty((t[i].numel() + 1,), dtype=t[i].dtype, device=DEV)
        big[1:] = dev_t[i].reshape(-1)
        dev_t[i] = big[1:].view(t[i].shape)
        assert dev_t[i].data_ptr() % 8 != 0
    out = _kd().kv_dequant_prefill_attention(qd, *dev_t, causal=True, num_kv_heads=2)
    torch.cuda.synchronize()
    ref = oa.prefill_per_channel(q.numpy(), *[x.numpy() for x in t], causal=True)
    assert_close(out.cpu().numpy(), ref, what="unaligned V rulers")


def test_prefill_matrix_cores_raw_nibbles_and_tensor_heads():
    """use_quant=False (raw codes), and num_kv_heads < k_packed.shape[0]."""
    q, t = _pf_inputs(9, 8, 4, 100, 300, 64)
    out = _prefill(q, t, causal=True, use_quant=False, num_kv_heads=4)
    ref = oa.prefill_per_channel(q.numpy(), *[x.numpy() for x in t], causal=True, use_quant=False)
    assert_close(out, ref, what="use_quant=False")
    out = _prefill(q, t, causal=True, num_kv_heads=2)
    kp, ks, kz, vp, vs, vz = [x.numpy() for x in t]
    ref = oa.prefill_per_channel(q.numpy(), kp[:2], ks[:2], kz[:2], vp[:2], vs[:2], vz[:2], causal=True)
    assert_close(out, ref, what="num_kv_heads=2 of 4")


def test_prefill_matrix_cores_fractional_zero_points():
    """Zero points need not be integers: the kernel takes the integer part into
    the operand and the rest in fp32."""
    q, t = _pf_inputs(10, 8, 2, 130, 200, 128)
    g = torch.Generator().manual_seed(3)
    t[2] = (t[2].float() + torch.rand(t[2].shape, generator=g) * 3 - 1.5).half()   # k_zero
    t[5] = (t[5].float() + torch.rand(t[5].shape, generator=g) * 3 - 1.5).half()   # v_zero
    out = _prefill(q, t, causal=True, num_kv_heads=2)
    ref = oa.prefill_per_channel(q.numpy(), *[x.numpy() for x in t], causal=True)
    assert_close(out, ref, what="fractional zero points")


# ------------------------------------------------------------------ per-token contiguous decode
@pytest.mark.parametrize("H,KV,D,S", [(32, 8, 128, 1000), (4, 4, 64, 17), (12, 2, 80, 333)])
def test_decode_per_token_contiguous(H, KV, D, S):
    g = torch.Generator().manual_seed(S)
    q = torch.randn(H, 1, D, generator=g).half()
    k = kv_values(g, (S, KV, D))
    v = kv_values(g, (S, KV, D))
    # quantize rows with the oracle store into a scratch cache, then unpack to the contiguous layout
    cache = np.zeros((S, 1, KV, D + 8), dtype=np.uint8)
    oq.quantize_store(k.numpy(), v.numpy(), cache, np.arange(S, dtype=np.int64), 1)
    slots = cache[:, 0].transpose(1, 0, 2)                              # [KV, S, D+8]
    kp, vp = slots[..., : D // 2].copy(), slots[..., D // 2: D].copy()
    rul = np.ascontiguousarray(slots[..., D:]).view(np.float16)         # [KV, S, 4]
    kmin, kstep, vmin, vstep = (np.ascontiguousarray(rul[..., i]) for i in range(4))
    tens = [torch.from_numpy(a).to(DEV) for a in (kp, kmin, kstep, vp, vmin, vstep)]
    out = _kd().kv_dequant_decode_per_token_attention(q.to(DEV), *tens, num_kv_heads=KV)
    torch.cuda.synchronize()
    ref = oa.decode_per_token(q.numpy(), kp, kmin, kstep, vp, vmin, vstep)
    assert_close(out.cpu().numpy(), ref, what="per-token decode")


# One sequence, head_dim 64 / 128, up to 8 query heads per KV head and 16384
# keys: the split (KV head, key chunk) kernel; 20000 keys take the general path.
@pytest.mark.parametrize("H,KV,D,S,outl", [(8, 8, 64, 1, False), (6, 2, 128, 17, True), (24, 8, 64, 5000, False),
                                           (16, 2, 128, 9000, True), (4, 4, 128, 20000, False),
                                           (8, 1, 64, 3333, False)])
def test_decode_per_channel_split_chunks(H, KV, D, S, outl):
    q, t = _pc_inputs(H + S, H, KV, S, D, outl)
    kd = _kd()
    for _ in range(2):                        # the arrival counters must be left at zero
        out = kd.kv_dequant_decode_attention(q.to(DEV), *[x.to(DEV) for x in t], num_kv_heads=KV)
        torch.cuda.synchronize()
        ref = oa.decode_per_channel(q.numpy(), *[x.numpy() for x in t])
        assert_close(out.cpu().numpy(), ref, what=f"H={H} KV={KV} D={D} S={S}")
