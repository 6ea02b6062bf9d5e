"""GPU parity: quantize-on-write store and paged decode against the oracle.

Store: packed bytes and fp16 rulers bit-exact with the oracle's restatement of
kv_quantize_store_kernel (reference kernels/kv_dequant_kernels.cuh:816-919).
Decode: within max-abs 2e-3 / rel 1e-2 of float64 dequant-then-attend.
"""
import numpy as np
import pytest
import torch

from common import PagedCase, assert_close, kv_values, make_paged_case, paged_reference
from oracle import quant as oq

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _kd():
    from kernels import kv_dequant
    return kv_dequant


# ------------------------------------------------------------------ store
@pytest.mark.parametrize("D", [64, 80, 128])
@pytest.mark.parametrize("dist", ["normal", "t3"])
def test_store_bit_exact(D, dist):
    kd = _kd()
    g = torch.Generator().manual_seed(D + (7 if dist == "t3" else 0))
    N, KV, bs, nb = 37, 4, 16, 8
    key = kv_values(g, (N, KV, D), dist)
    value = kv_values(g, (N, KV, D), dist) * 3
    slots = torch.randperm(nb * bs, generator=g)[:N].to(torch.int64)
    slots[5] = -1                                      # padding token: skipped
    ref = np.random.default_rng(1).integers(0, 256, (nb, bs, KV, D + 8), dtype=np.uint8)
    gpu_cache = torch.from_numpy(ref.copy()).to(DEV)
    oq.quantize_store(key.numpy(), value.numpy(), ref, slots.numpy(), bs)
    kd.kv_quantize_store(key.to(DEV), value.to(DEV), gpu_cache, slots.to(DEV), bs)
    torch.cuda.synchronize()
    got = gpu_cache.cpu().numpy()
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} bytes differ"


def test_store_edge_rows():
    """Constant rows, lattice rows, signed zeros, NaN/inf rows, huge ranges."""
    kd = _kd()
    D, KV, bs = 128, 2, 16
    rows = []
    rows.append(np.full(D, 0.75))                                  # constant -> step 1, codes 0
    rows.append(-1.0 + np.arange(D) % 16 * 0.125)                  # exact lattice points
    rows.append(np.where(np.arange(D) % 2 == 0, -0.0, 0.0))        # signed zeros only
    r = np.linspace(-2, 2, D); r[3] = np.nan; rows.append(r)       # NaN ignored by min/max
    r = np.linspace(-2, 2, D); r[7] = np.inf; rows.append(r)       # inf range
    rows.append(np.linspace(-60000, 60000, D))                     # max-min overflows fp16 range
    rows.append(np.linspace(0, 2.0 ** -20, D))                     # tiny step
    rows.append(np.full(D, np.nan))                                # all NaN -> step guard
    x = np.stack(rows).astype(np.float16)
    N = x.shape[0]
    key = np.repeat(x[:, None, :], KV, axis=1)
    value = key[::-1].copy()
    slots = np.arange(N, dtype=np.int64) * 3
    nb = (slots.max() + bs) // bs + 1
    ref = np.zeros((nb, bs, KV, D + 8), dtype=np.uint8)
    gpu_cache = torch.zeros(ref.shape, dtype=torch.uint8, device=DEV)
    oq.quantize_store(key, value, ref, slots, bs)
    kd.kv_quantize_store(torch.from_numpy(key).to(DEV), torch.from_numpy(value).to(DEV), gpu_cache,
                         torch.from_numpy(slots).to(DEV), bs)
    torch.cuda.synchronize()
    got = gpu_cache.cpu().numpy()
    kb, vb, rg = oq.split_slot(got, D)
    kr, vr, rr = oq.split_slot(ref, D)
    assert np.array_equal(kb, kr) and np.array_equal(vb, vr), "codes differ"
    # rulers bit-exact except NaN payloads (any NaN matches any NaN)
    gb, rb = rg.view(np.uint16), rr.view(np.uint16)
    same = (gb == rb) | (np.isnan(rg) & np.isnan(rr))
    assert same.all(), f"rulers differ at {np.argwhere(~same)[:5]}"


def test_store_strided_tokens():
    """Key/value as views into a fused qkv buffer (token stride > KV*D)."""
    kd = _kd()
    g = torch.Generator().manual_seed(3)
    N, H, KV, D, bs = 9, 8, 2, 128, 16
    qkv = torch.randn((N, (H + 2 * KV) * D), generator=g).half()
    key = qkv[:, H * D:(H + KV) * D].view(N, KV, D)
    value = qkv[:, (H + KV) * D:].view(N, KV, D)
    slots = torch.arange(N, dtype=torch.int64) + 5
    ref = np.zeros((2, bs, KV, D + 8), dtype=np.uint8)
    oq.quantize_store(key.contiguous().numpy(), value.contiguous().numpy(), ref, slots.numpy(), bs)
    qkv_d = qkv.to(DEV)
    kd_key = qkv_d[:, H * D:(H + KV) * D].view(N, KV, D)
    kd_val = qkv_d[:, (H + KV) * D:].view(N, KV, D)
    cache = torch.zeros(ref.shape, dtype=torch.uint8, device=DEV)
    kd.kv_quantize_store(kd_key, kd_val, cache, slots.to(DEV), bs)
    torch.cuda.synchronize()
    assert np.array_equal(cache.cpu().numpy(), ref)


# ------------------------------------------------------------------ paged decode
def _run_batched(case: PagedCase, out_dtype=torch.float32, bt_dtype=torch.int32):
    kd = _kd()
    out = kd.kv_dequant_decode_paged_batched(
        case.q.to(DEV), torch.from_numpy(case.kv_cache).to(DEV), case.block_tables.to(bt_dtype).to(DEV),
        case.seq_lens.to(DEV), case.block_size, case.num_kv_heads, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (4, 4, 64), (12, 2, 128), (14, 2, 64), (8, 8, 80),
                                    (16, 8, 64), (64, 8, 128), (32, 4, 128),
                                    # whole-row kernel: 4 KV heads x 1 wave, 2 KV heads x 2 waves,
                                    # several head groups per launch; odd KV falls back
                                    (16, 4, 128), (16, 2, 128), (24, 6, 128), (48, 6, 128), (64, 16, 128),
                                    (12, 3, 128),
                                    # the same whole-row shapes at head_dim 64
                                    (32, 4, 64), (32, 8, 64), (16, 4, 64), (16, 2, 64), (8, 2, 64),
                                    (24, 6, 64), (64, 16, 64), (48, 6, 64)])
def test_paged_batched_matches_oracle(H, KV, D, paged_kernel):
    case = make_paged_case(seed=H * 131 + D, B=5, H=H, KV=KV, D=D, len_range=(1, 700))
    assert_close(_run_batched(case), paged_reference(case), what=f"H={H} KV={KV} D={D}")


@pytest.mark.parametrize("bs", [1, 8, 16, 32, 48])
@pytest.mark.parametrize("D", [64, 128])
def test_paged_block_sizes(bs, D, paged_kernel):
    case = make_paged_case(seed=bs, B=4, H=8, KV=2, D=D, block_size=bs, len_range=(1, 300))
    assert_close(_run_batched(case), paged_reference(case), what=f"bs={bs} D={D}")


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (64, 8, 128), (16, 2, 128), (32, 4, 64)])
def test_paged_block_sizes_whole_row_shapes(H, KV, D, bs, paged_kernel):
    """Blocks of 32-128 tokens at the shapes the whole-row kernels take
    (8 KV heads x 1 wave, 4 x 2 with the token split, 2 x 2 at head_dim 128,
    2 x 2 at 64): a wave's staged rows then span several rows of one block,
    and a 64-token tile covers part of a block instead of four of them."""
    case = make_paged_case(seed=bs + H, B=4, H=H, KV=KV, D=D, block_size=bs, len_range=(1, 1500))
    assert_close(_run_batched(case), paged_reference(case), what=f"bs={bs} H={H} KV={KV} D={D}")


@pytest.mark.parametrize("D", [64, 128])
def test_paged_edge_lengths_and_formats(D, paged_kernel):
    """Lengths 0, 1, 15, 16, 17 and a long one; int64 tables; fp16 output."""
    case = make_paged_case(seed=11, B=7, H=32, KV=8, D=D, lens=[0, 1, 15, 16, 17, 3000, 0])
    ref = paged_reference(case)
    assert_close(_run_batched(case), ref, what="int32/fp32")
    assert_close(_run_batched(case, bt_dtype=torch.int64), ref, what="int64 tables")
    assert_close(_run_batched(case, out_dtype=torch.float16), ref, what="fp16 out")
    assert np.all(_run_batched(case)[[0, 6]] == 0.0)


@pytest.mark.parametrize("H,KV,D", [(64, 8, 128), (32, 4, 64), (16, 2, 128)])
def test_paged_edge_lengths_eight_heads_per_kv(H, KV, D, paged_kernel):
    """8 query heads per KV head around the 32-token halves of a tile (the two
    waves of a KV head split a tile's tokens at head_dim 128): a sequence with
    no token in the second half, exactly one half, one token past it, and the
    tile boundaries, mixed with long ones so sequences share workgroups."""
    lens = [0, 1, 15, 31, 32, 33, 63, 64, 65, 95, 97, 2000, 5000, 0, 2]
    case = make_paged_case(seed=H + D, B=len(lens), H=H, KV=KV, D=D, lens=lens)
    ref = paged_reference(case)
    got = _run_batched(case)
    assert_close(got, ref, what=f"G=8 edge lengths H={H} D={D}")
    assert_close(_run_batched(case, out_dtype=torch.float16), ref, what="fp16 out")
    assert np.all(got[[0, 13]] == 0.0)


_LONG_CASES = {}


@pytest.mark.parametrize("H,KV,D,L", [(32, 4, 64, 120000), (16, 2, 128, 100000)])
def test_paged_one_sequence_over_hundreds_of_workgroups(H, KV, D, L, paged_kernel):
    """One long sequence beside two short ones: the stream-K split spreads it
    over every workgroup of the launch (hundreds of partial pieces), so the
    merge combines it in many batches of pieces, each rescaled to the running
    maximum of the ones before."""
    key = (H, KV, D, L)
    if key not in _LONG_CASES:   # the case and its float64 reference, shared by both kernels
        case = make_paged_case(seed=L + D, B=3, H=H, KV=KV, D=D, lens=[L, 7, 0])
        _LONG_CASES[key] = (case, paged_reference(case))
    case, ref = _LONG_CASES[key]
    got = _run_batched(case)
    assert_close(got, ref, what=f"one sequence of {L} tokens, H={H} D={D}")
    assert np.all(got[2] == 0.0)


def test_paged_student_t_long_context():
    """Config-4 shaped heads (64 q / 8 kv, D=128) with heavy-tailed K/V."""
    case = make_paged_case(seed=4, B=2, H=64, KV=8, D=128, len_range=(4000, 9000), dist="t3")
    assert_close(_run_batched(case), paged_reference(case), what="t3")


def test_single_request_api_matches_batched():
    kd = _kd()
    case = make_paged_case(seed=21, B=3, H=32, KV=8, D=128, len_range=(100, 900))
    ref = paged_reference(case)
    cache = torch.from_numpy(case.kv_cache).to(DEV)
    for b in range(3):
        o = kd.kv_dequant_decode_per_token_paged_attention(
            case.q[b][:, None, :].to(DEV), cache, case.block_tables[b].to(torch.int64).to(DEV),
            int(case.seq_lens[b]), case.block_size, case.num_kv_heads)
        torch.cuda.synchronize()
        assert o.shape == (32, 1, 128) and o.dtype == torch.float32
        assert_close(o[:, 0].cpu().numpy(), ref[b], what=f"request {b}")


def test_repeated_calls_reuse_workspace():
    """Arrival counters are self-cleaning: back-to-back calls agree."""
    case = make_paged_case(seed=5, B=16, H=32, KV=8, D=128, len_range=(200, 3000))
    a = _run_batched(case)
    b = _run_batched(case)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("D", [64, 128])
def test_split_sequences_alternating_inputs(D):
    """Sequences split over many workgroups, alternating two different inputs
    through the same workspace: each call must merge its own partials."""
    a = make_paged_case(seed=31, B=2, H=32, KV=8, D=D, len_range=(6000, 9000))
    b = make_paged_case(seed=32, B=3, H=32, KV=8, D=D, len_range=(3000, 9000))
    ra, rb = paged_reference(a), paged_reference(b)
    for i in range(3):
        assert_close(_run_batched(a), ra, what=f"a[{i}]")
        assert_close(_run_batched(b), rb, what=f"b[{i}]")


def test_mixed_shapes_share_workspace():
    """Calls of different shapes on one stream share the cached workspace:
    their partial results must never land on another shape's counters."""
    cases = [make_paged_case(seed=41, B=5, H=14, KV=2, D=64, len_range=(100, 700)),
             make_paged_case(seed=42, B=2, H=32, KV=8, D=128, len_range=(3000, 6000)),
             make_paged_case(seed=43, B=9, H=12, KV=2, D=80, len_range=(1, 900))]
    refs = [paged_reference(c) for c in cases]
    for i in (0, 1, 2, 0, 2, 1, 0):
        assert_close(_run_batched(cases[i]), refs[i], what=f"case {i}")


@pytest.mark.parametrize("D", [64, 128])
def test_batch_beyond_the_length_stash(D, paged_kernel):
    """300 sequences: the whole-row kernel keeps the first 256 lengths in LDS
    and reads the rest from memory; lengths 0..40 include empty sequences."""
    g = torch.Generator().manual_seed(D)
    lens = torch.randint(0, 41, (300,), generator=g).tolist()
    case = make_paged_case(seed=D + 1, B=300, H=32, KV=8, D=D, lens=lens)
    got = _run_batched(case)
    assert_close(got, paged_reference(case), what=f"B=300 D={D}")
    assert np.all(got[np.asarray(lens) == 0] == 0.0)


@pytest.mark.parametrize("bs,D", [(64, 128), (128, 64), (64, 64)])
def test_large_block_sizes_whole_row(bs, D, paged_kernel):
    case = make_paged_case(seed=bs + D, B=6, H=32, KV=8, D=D, block_size=bs, len_range=(1, 900))
    assert_close(_run_batched(case), paged_reference(case), what=f"bs={bs} D={D}")


@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (32, 4, 64)])
def test_one_long_sequence_over_every_workgroup(H, KV, D, paged_kernel):
    """A single 40K-token sequence: every workgroup holds a piece of it and the
    merge combines all of them."""
    case = make_paged_case(seed=H + D, B=1, H=H, KV=KV, D=D, lens=[40000], dist="t3")
    assert_close(_run_batched(case), paged_reference(case), what=f"one 40K sequence H={H} D={D}")
