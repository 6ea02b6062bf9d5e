"""GPU parity on wide-dynamic-range inputs: the decode's number formats.

The reference scores in fp32 from the fp16 query and fp32-dequantized keys
(kernels/kv_dequant_kernels.cuh:752-756) and accumulates P.V in fp32
(:780-790).  These cases stress exactly where a narrower query or weight
format would show, all against the float64 dequant-then-attend oracle at
max-abs 2e-3 / rel 1e-2:

* queries with 1 % of their channels scaled x8 and x64 (outlier channels);
* Student-t(3) queries;
* queries scaled so that the scores span tens of logits (a peaked softmax);
* K/V rows whose ranges are 2^-20 wide or reach +-60000;
* stale cache slots past a sequence's end filled with 0xFF bytes (NaN rulers),
  as a reused paged block may hold.

Each case runs through the batched paged decode (whole-row kernel shapes and
the per-wave fallback), the per-token contiguous decode and the per-channel
decode.
"""
import numpy as np
import pytest
import torch

from common import PagedCase, assert_close, kv_values, make_paged_case, paged_reference, student_t3
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
QMODES = ["outlier8", "outlier64", "t3", "peak6", "peak13", "peak25"]


def _kd():
    from kernels import kv_dequant
    return kv_dequant


def _shape_q(q: torch.Tensor, mode: str, seed: int) -> torch.Tensor:
    """q [..., D] fp16 -> the wide-range variant `mode` (fp16)."""
    g = torch.Generator().manual_seed(seed)
    D = q.shape[-1]
    x = q.float()
    if mode.startswith("outlier"):
        nch = max(1, int(np.ceil(0.01 * D)))
        ch = torch.randperm(D, generator=g)[:nch]
        x[..., ch] *= float(mode[len("outlier"):])
    elif mode == "t3":
        x = student_t3(g, tuple(x.shape))
    elif mode.startswith("peak"):
        x = x * float(mode[len("peak"):])
    return x.half()


def _run_paged(case: PagedCase, out_dtype=torch.float32):
    kd = _kd()
    out = kd.kv_dequant_decode_paged_batched(
        case.q.to(DEV), torch.from_numpy(case.kv_cache).to(DEV), case.block_tables.to(DEV),
        case.seq_lens.to(DEV), case.block_size, case.num_kv_heads, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("dist", ["normal", "t3"])
@pytest.mark.parametrize("qmode", QMODES)
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (32, 4, 64), (64, 8, 128), (32, 8, 64), (8, 8, 80),
                                    (12, 3, 128)])
def test_paged_wide_range_queries(H, KV, D, qmode, dist, paged_kernel):
    case = make_paged_case(seed=3 * H + D, B=3, H=H, KV=KV, D=D, len_range=(200, 1500), dist=dist)
    case.q = _shape_q(case.q, qmode, seed=D + H)
    assert_close(_run_paged(case), paged_reference(case), what=f"H={H} KV={KV} D={D} q={qmode} kv={dist} {paged_kernel}")


def _extreme_kv(g, L, KV, D):
    """K/V rows of every kind: normal, 2^-20-wide, +-60000 and Student-t."""
    rows = kv_values(g, (L, KV, D)).float()
    kind = torch.randint(0, 4, (L, KV), generator=g)
    tiny = 0.5 + torch.rand((L, KV, D), generator=g) * 2.0 ** -20
    huge = (torch.rand((L, KV, D), generator=g) * 2 - 1) * 60000.0
    t3 = student_t3(g, (L, KV, D))
    rows = torch.where((kind == 1)[..., None], tiny, rows)
    rows = torch.where((kind == 2)[..., None], huge, rows)
    rows = torch.where((kind == 3)[..., None], t3, rows)
    return rows.half()


@pytest.mark.parametrize("qmode", ["normal", "peak13"])
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (32, 4, 64), (8, 8, 80)])
def test_paged_extreme_rulers(H, KV, D, qmode, paged_kernel):
    """Rows whose steps are near fp16's smallest subnormal or its largest normal."""
    g = torch.Generator().manual_seed(17 + D)
    lens = [300, 1100, 57]
    case = make_paged_case(seed=5, B=3, H=H, KV=KV, D=D, lens=lens)
    tables = case.block_tables
    for b, L in enumerate(lens):
        k, v = _extreme_kv(g, L, KV, D), _extreme_kv(g, L, KV, D)
        pos = torch.arange(L)
        slots = tables[b, pos // case.block_size].to(torch.int64) * case.block_size + pos % case.block_size
        oq.quantize_store(k.numpy(), v.numpy(), case.kv_cache, slots.numpy(), case.block_size)
    if qmode != "normal":
        case.q = _shape_q(case.q, qmode, seed=D)
    ref = paged_reference(case)
    assert np.isfinite(ref).all()
    assert_close(_run_paged(case), ref, what=f"extreme rulers H={H} KV={KV} D={D} q={qmode} {paged_kernel}")


@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (32, 4, 64), (64, 8, 128), (8, 8, 80)])
def test_paged_stale_slots_past_the_end(H, KV, D, paged_kernel):
    """Slots a sequence does not own hold 0xFF bytes (NaN rulers): no effect on the output."""
    lens = [1, 15, 17, 63, 65, 700]
    case = make_paged_case(seed=23, B=len(lens), H=H, KV=KV, D=D, lens=lens)
    ref = paged_reference(case)
    clean = case.kv_cache
    dirty = np.full_like(clean, 0xFF)
    tables = case.block_tables.numpy()
    for b, L in enumerate(lens):
        n = np.arange(L)
        blk = tables[b, n // case.block_size]
        dirty[blk, n % case.block_size] = clean[blk, n % case.block_size]
    case.kv_cache = dirty
    got = _run_paged(case)
    assert np.isfinite(got).all(), "stale slots leaked into the output"
    assert_close(got, ref, what=f"stale slots H={H} KV={KV} D={D} {paged_kernel}")


@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (32, 4, 64)])
def test_paged_fp16_output_at_the_bar(H, KV, D, paged_kernel):
    """fp16 output within the same 2e-3 / 1e-2 bar (its rounding is inside rel 1e-2)."""
    case = make_paged_case(seed=29, B=4, H=H, KV=KV, D=D, len_range=(1, 2500), dist="t3")
    case.q = _shape_q(case.q, "peak13", seed=3)
    assert_close(_run_paged(case, out_dtype=torch.float16), paged_reference(case),
                 what=f"fp16 out H={H} KV={KV} D={D} {paged_kernel}")


# ------------------------------------------------------------------ contiguous layouts
def _contig_per_token(g, H, KV, D, S, dist):
    k = kv_values(g, (S, KV, D), dist)
    v = kv_values(g, (S, KV, D), dist)
    bs = 16
    nb = (S + bs - 1) // bs
    cache = np.zeros((nb, bs, KV, D + 8), dtype=np.uint8)
    oq.quantize_store(k.numpy(), v.numpy(), cache, np.arange(S, dtype=np.int64), bs)
    slots = cache.reshape(nb * bs, KV, D + 8)[:S].transpose(1, 0, 2)    # [KV, S, D+8]
    kp = np.ascontiguousarray(slots[..., : D // 2])
    vp = np.ascontiguousarray(slots[..., D // 2: D])
    rul = np.ascontiguousarray(slots[..., D:]).view(np.float16)        # [KV, S, 4]
    return kp, vp, rul


@pytest.mark.parametrize("qmode", QMODES)
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (16, 2, 64), (8, 4, 80)])
def test_per_token_contiguous_wide_range_queries(H, KV, D, qmode):
    kd = _kd()
    g = torch.Generator().manual_seed(7 * D + H)
    S = 1200
    kp, vp, rul = _contig_per_token(g, H, KV, D, S, "t3")
    q = _shape_q(torch.randn((H, 1, D), generator=g).half(), qmode, seed=H)
    K = oatt.dequant_per_token(kp, rul[..., 0], rul[..., 1])
    V = oatt.dequant_per_token(vp, rul[..., 2], rul[..., 3])
    ref = oatt.attend(q[:, 0].numpy(), K, V)
    r = [torch.from_numpy(np.ascontiguousarray(rul[..., i])).to(DEV) for i in range(4)]
    out = kd.kv_dequant_decode_per_token_attention(
        q.to(DEV), torch.from_numpy(kp).to(DEV), r[0], r[1], torch.from_numpy(vp).to(DEV), r[2], r[3],
        num_kv_heads=KV)
    torch.cuda.synchronize()
    assert_close(out[:, 0].cpu().numpy(), ref, what=f"per-token H={H} KV={KV} D={D} q={qmode}")


@pytest.mark.parametrize("qmode", QMODES)
@pytest.mark.parametrize("H,KV,D,S", [(12, 2, 128, 2048), (32, 4, 64, 512), (8, 8, 80, 700),
                                      (12, 2, 128, 20000)])
def test_per_channel_decode_wide_range_queries(H, KV, D, S, qmode):
    kd = _kd()
    g = torch.Generator().manual_seed(11 * D + S)
    x = student_t3(g, (2, KV, S, D)).half().numpy()
    kp, ks, kz, vp, vs, vz = oq.quantize_kv(x[0], x[1])
    packed, scale, zero = (kp, vp), (ks, vs), (kz, vz)
    q = _shape_q(torch.randn((H, 1, D), generator=g).half(), qmode, seed=S)
    K = oatt.dequant_per_channel(packed[0], scale[0], zero[0])
    V = oatt.dequant_per_channel(packed[1], scale[1], zero[1])
    ref = oatt.attend(q[:, 0].numpy(), K, V)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    out = kd.kv_dequant_decode_attention(q.to(DEV), t(packed[0]), t(scale[0]), t(zero[0]), t(packed[1]),
                                         t(scale[1]), t(zero[1]), num_kv_heads=KV)
    torch.cuda.synchronize()
    assert_close(out[:, 0].cpu().numpy(), ref, what=f"per-channel H={H} KV={KV} D={D} S={S} q={qmode}")


# ------------------------------------------------------------------ long context, dominant token
SINK_GAPS = (9.0, 12.0, 15.0, 16.5)          # nats by which the sink leads, per query head (h % 4)
_SINK_CASES: dict = {}                # built once per module run: ~180 MB of cache per shape


def _sink_case(H: int, KV: int, D: int, lens=(131071, 32770), seed: int = 41):
    """Position 0 of every sequence is an attention sink whose score leads the
    others by SINK_GAPS[h % 4] nats for query head h; the other scores lie
    within about +-0.3 nats of each other.  The sink's V row is near zero and
    the tail's V rows carry a per-dimension offset (N(1, 1)), so the output is
    the tail's weight (L - 1) e^-gap (0.9 % of the softmax mass at 131071
    tokens and 16.5 nats) times the offset: a decode that drops or
    mis-weights the tail's small weights misses it.  Built once per shape and
    shared by the kernels under test, with its float64 reference."""
    key = (H, KV, D, tuple(lens), seed)
    if key in _SINK_CASES:
        return _SINK_CASES[key]
    g = torch.Generator().manual_seed(seed)
    bs = 16
    lens_t = torch.as_tensor(lens, dtype=torch.int64)
    nblk = (lens_t + bs - 1) // bs
    total = int(nblk.sum())
    perm = torch.randperm(total, generator=g)
    tables = torch.zeros((len(lens), int(nblk.max())), dtype=torch.int32)
    off = 0
    for b in range(len(lens)):
        n = int(nblk[b])
        tables[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    top = max(SINK_GAPS)
    t = top / np.sqrt(D)                      # sink K row: score c * t * sqrt(D) = gap for q = c * ones
    c = torch.tensor([SINK_GAPS[h % 4] / top for h in range(H)])
    q = (c[None, :, None] * torch.ones((len(lens), H, D))).half()
    cache = np.zeros((total, bs, KV, D + 8), dtype=np.uint8)
    for b, L in enumerate(lens):
        k = torch.randn((L, KV, D), generator=g) * 0.1
        k[0] = t
        v = torch.randn((L, KV, D), generator=g) + 1.0
        v[0] = torch.randn((KV, D), generator=g) * 0.01
        pos = torch.arange(L)
        slots = tables[b, pos // bs].to(torch.int64) * bs + pos % bs
        oq.quantize_store(k.half().numpy(), v.half().numpy(), cache, slots.numpy(), bs)
        del k, v
    case = PagedCase(q, cache, tables, lens_t.to(torch.int32), bs, KV)
    ref = paged_reference(case)
    _SINK_CASES[key] = (case, ref)
    return case, ref


@pytest.mark.parametrize("H,KV,D", [(64, 8, 128), (32, 8, 128)])
def test_paged_long_context_sink(H, KV, D, paged_kernel):
    """131071 and 32770 tokens behind a sink 9 to 16.5 nats ahead, through
    both whole-row kernels, against the float64 oracle at the 2e-3 / 1e-2 bar."""
    case, ref = _sink_case(H, KV, D)
    # the tail carries a visible share of the output in every head
    assert (np.abs(ref[0]).mean(axis=-1) > 5e-3).all()
    assert_close(_run_paged(case), ref, what=f"sink H={H} KV={KV} D={D} kernel={paged_kernel}")


def test_paged_long_context_sink_per_wave_kernel():
    """The same through the per-wave kernel (three KV heads: no whole-row shape)."""
    case, ref = _sink_case(24, 3, 128)
    assert_close(_run_paged(case), ref, what="sink H=24 KV=3 D=128 per-wave")


@pytest.mark.parametrize("qmode", ["peak13", "peak25"])
def test_paged_long_context_peaked_query(qmode, paged_kernel):
    """A peaked softmax (q x 13, x 25) over 120000 N(0,1) tokens."""
    key = ("peaked", qmode)
    if key not in _SINK_CASES:
        case = make_paged_case(seed=43, B=1, H=32, KV=8, D=128, lens=[120000])
        case.q = _shape_q(case.q, qmode, seed=43)
        _SINK_CASES[key] = (case, paged_reference(case))
    case, ref = _SINK_CASES[key]
    assert_close(_run_paged(case), ref, what=f"long peaked q={qmode} kernel={paged_kernel}")
