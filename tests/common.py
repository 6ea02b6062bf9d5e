"""Shared synthetic workloads and checks for the tests, the smoke test and the
benchmark's CPU baseline.  Inputs are generated on the CPU from a seeded
torch.Generator, so the GPU, the oracle and the CPU baseline see identical
tensors."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import attention as oatt
from oracle import quant as oq

# Parity bar for attention outputs (max-abs 2e-3 and rel 1e-2, fp32 accumulation).
ATOL, RTOL = 2e-3, 1e-2


# Every assert_close records (what, max abs error, share of the bar used) here;
# tests/conftest.py writes the list out when SLMT_ENVELOPE_OUT names a file.
ENVELOPE: list = []


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what="output"):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    both_nan = np.isnan(got) & np.isnan(ref)
    err = np.abs(got - ref)
    if got.size:
        e = np.where(both_nan, 0.0, err)
        ENVELOPE.append({"what": what, "max_abs_err": float(np.nanmax(e)),
                         "bar_used": float(np.nanmax(e / (atol + rtol * np.abs(np.nan_to_num(ref))))),
                         "atol": atol, "rtol": rtol})
    bad = ~both_nan & ~(err <= atol + rtol * np.abs(ref))
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err, -1)), got.shape)
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.size} elements outside "
                             f"atol={atol} rtol={rtol}; worst at {i}: got {got[i]!r} ref {ref[i]!r} "
                             f"(max abs err {np.nanmax(np.where(both_nan, 0, err)):.3e})")


def student_t3(gen: torch.Generator, shape) -> torch.Tensor:
    """Student-t with nu=3 from normals: z / sqrt(chi2_3 / 3)."""
    z = torch.randn(shape, generator=gen)
    chi2 = (torch.randn((3, *shape), generator=gen) ** 2).sum(0)
    return z / torch.sqrt(chi2 / 3.0)


def kv_values(gen, shape, dist="normal"):
    if dist == "normal":
        x = torch.randn(shape, generator=gen)
    elif dist == "t3":
        x = student_t3(gen, shape)
    else:
        raise ValueError(dist)
    return x.half()


@dataclass
class PagedCase:
    q: torch.Tensor              # [B, H, D] fp16
    kv_cache: np.ndarray         # [num_blocks, bs, KV, D+8] uint8 (written by the oracle store)
    block_tables: torch.Tensor   # [B, max_blocks] int32
    seq_lens: torch.Tensor       # [B] int32
    block_size: int
    num_kv_heads: int

    @property
    def algorithmic_bytes(self) -> int:
        B, H, D = self.q.shape
        L = self.seq_lens.numpy().astype(np.int64)
        blocks = (L + self.block_size - 1) // self.block_size
        return int(L.sum() * self.num_kv_heads * (D + 8) + B * H * D * 2 + B * H * D * 4
                   + blocks.sum() * 4 + B * 4)


def make_paged_case(seed: int, B: int, H: int, KV: int, D: int, block_size: int = 16,
                    lens=None, len_range=(512, 8193), dist: str = "normal",
                    extra_blocks: int = 0) -> PagedCase:
    """Random lengths (or the given ones), K/V ~ dist quantized by the oracle's
    store, block tables a random permutation of exactly the blocks needed."""
    g = torch.Generator().manual_seed(seed)
    if lens is None:
        lens = torch.randint(len_range[0], len_range[1], (B,), generator=g)
    lens = torch.as_tensor(lens, dtype=torch.int64)
    nblk = (lens + block_size - 1) // block_size
    total = int(nblk.sum()) + extra_blocks
    perm = torch.randperm(max(total, 1), generator=g)[:total]
    maxb = max(int(nblk.max()) if B else 0, 1)
    tables = torch.zeros((B, maxb), dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(nblk[b])
        tables[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn((B, H, D), generator=g).half()
    cache = np.zeros((max(total, 1), block_size, KV, D + 8), dtype=np.uint8)
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        k = kv_values(g, (L, KV, D), dist)
        v = kv_values(g, (L, KV, D), dist)
        pos = torch.arange(L)
        slots = tables[b, pos // block_size].to(torch.int64) * block_size + pos % block_size
        oq.quantize_store(k.numpy(), v.numpy(), cache, slots.numpy(), block_size)
    return PagedCase(q, cache, tables, lens.to(torch.int32), block_size, KV)


def paged_reference(case: PagedCase, seqs=None) -> np.ndarray:
    """float64 dequant-then-attend for every (or the listed) sequence(s)."""
    q = case.q.numpy()
    out = np.zeros(q.shape, dtype=np.float64)
    tables = case.block_tables.numpy()
    for b in (range(q.shape[0]) if seqs is None else seqs):
        L = int(case.seq_lens[b])
        if L > 0:
            out[b] = oatt.decode_paged(q[b], case.kv_cache, tables[b], L)
    return out
