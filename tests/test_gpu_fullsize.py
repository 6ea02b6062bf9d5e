"""Full-size paged decode workloads on the GPU.

* The headline configuration: batch 64, lengths U[512, 8192] (seed 0), 32 query
  / 8 KV heads, head_dim 128, block 16, K/V ~ N(0, 1).
* The long-context configuration: batch 8, lengths U[32768, 131072], 64 query /
  8 KV heads, head_dim 128, block 16, K/V ~ Student-t(3).
* The full-model workload's attention: batch 32, lengths U[4096, 4224], 32
  query / 4 KV heads, head_dim 64, block 16.

Caches are filled on the device by the store kernel, block tables are a random
permutation of exactly the blocks needed.  At these sizes the float64 oracle
is too slow for a test, so the decode is checked against a torch fp32
dequant-then-attend of the same cache bytes (per-token nib * step + min,
reference kernels/kv_dequant_kernels.cuh:14-24,666-670,713-722; softmax(q K^T /
sqrt(D)) V) and against a size-independent property: permuting the physical
blocks, with the block table permuted to match, leaves every output bit
unchanged.  Every case runs through both whole-row kernels (the matrix-core
default and the vector-ALU kernel); each workload and its reference are built
once per module run."""
from __future__ import annotations

import math

import pytest
import torch

from common import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BS = 16


def _kd():
    from kernels import kv_dequant as kd
    return kd


def _values(gen, n, KV, D, dist):
    if dist == "normal":
        return torch.randn((n, KV, D), generator=gen, device=DEV)
    # Student-t(3): z / sqrt(chi2_3 / 3)
    z = torch.randn((n, KV, D), generator=gen, device=DEV)
    chi2 = (torch.randn((3, n, KV, D), generator=gen, device=DEV) ** 2).sum(0)
    return z / torch.sqrt(chi2 / 3.0)


def build(seed, B, H, KV, D, lo, hi, dist):
    kd = _kd()
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g)
    nblk = (lens + BS - 1) // BS
    total = int(nblk.sum())
    perm = torch.randperm(total, generator=g)
    tables = torch.zeros((B, int(nblk.max())), dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(nblk[b])
        tables[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn((B, H, D), generator=g).half().to(DEV)
    slots = torch.cat([tables[b, torch.arange(int(lens[b])) // BS].long() * BS + torch.arange(int(lens[b])) % BS
                       for b in range(B)]).to(DEV)
    cache = torch.zeros((total, BS, KV, D + 8), dtype=torch.uint8, device=DEV)
    gg = torch.Generator(device=DEV).manual_seed(seed * 7919 + 1)
    for t0 in range(0, slots.numel(), 1 << 16):
        n = min(1 << 16, slots.numel() - t0)
        k = _values(gg, n, KV, D, dist).half()
        v = _values(gg, n, KV, D, dist).half()
        kd.kv_quantize_store(k, v, cache, slots[t0:t0 + n], BS)
    torch.cuda.synchronize()
    return lens.to(torch.int32), tables, q, cache


def reference(q, cache, tables, lens, KV):
    """torch fp32 dequant-then-attend, one sequence at a time."""
    B, H, D = q.shape
    G = H // KV
    out = torch.empty((B, H, D), dtype=torch.float32, device=DEV)
    for b in range(B):
        L = int(lens[b])
        nb = (L + BS - 1) // BS
        rows = cache[tables[b, :nb].long().to(DEV)].reshape(nb * BS, KV, D + 8)[:L]
        # byte j of a half holds dim 2j (low nibble) and dim 2j+1 (high nibble)
        def unpack(x):
            return torch.stack((x & 15, x >> 4), dim=-1).reshape(L, KV, D).float()
        rul = rows[..., D:D + 8].contiguous().view(torch.float16).float()   # k_min, k_step, v_min, v_step
        K = unpack(rows[..., :D // 2]) * rul[..., 1:2] + rul[..., 0:1]
        V = unpack(rows[..., D // 2:D]) * rul[..., 3:4] + rul[..., 2:3]
        qb = q[b].float().reshape(KV, G, D)
        s = torch.matmul(qb, K.permute(1, 2, 0).contiguous()) / math.sqrt(D)   # [KV, G, L]
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p, V.permute(1, 0, 2).contiguous()).reshape(H, D)
    return out


_BUILT: dict = {}


def workload(name):
    """(lens, tables, q, cache, reference) of a named full-size workload."""
    if name not in _BUILT:
        seed, B, H, KV, D, lo, hi, dist = {
            "headline": (0, 64, 32, 8, 128, 512, 8192, "normal"),
            "long-context": (0, 8, 64, 8, 128, 32768, 131072, "t3"),
            "full-model-attention": (0, 32, 32, 4, 64, 4096, 4224, "normal"),
        }[name]
        lens, tables, q, cache = build(seed, B, H, KV, D, lo, hi, dist)
        _BUILT[name] = (lens, tables, q, cache, reference(q, cache, tables, lens, KV).cpu().numpy())
    return _BUILT[name]


def decode(q, cache, tables, lens, KV):
    kd = _kd()
    out = kd.kv_dequant_decode_paged_batched(q, cache, tables.to(DEV), lens.to(DEV), BS, KV)
    torch.cuda.synchronize()
    return out


def test_headline_configuration_full_size(paged_kernel):
    lens, tables, q, cache, ref = workload("headline")
    got = decode(q, cache, tables, lens, 8)
    assert_close(got.cpu().numpy(), ref, what=f"batch 64, U[512,8192], {paged_kernel}")


def test_long_context_configuration_full_size(paged_kernel):
    B, KV = 8, 8
    lens, tables, q, cache, ref = workload("long-context")
    got = decode(q, cache, tables, lens, KV)
    assert_close(got.cpu().numpy(), ref, what=f"batch 8, U[32768,131072], Student-t, {paged_kernel}")

    # physical block permutation: same logical sequences, every bit unchanged
    nb = cache.shape[0]
    g = torch.Generator().manual_seed(1)
    perm = torch.randperm(nb, generator=g)                 # old block i -> new position perm[i]
    moved = torch.empty_like(cache)
    moved[perm.to(DEV)] = cache
    tables2 = tables.clone()
    used = tables2 >= 0
    tables2[used] = perm[tables2[used].long()].to(torch.int32)
    for b in range(B):                                     # entries past a sequence's blocks stay unused
        n = (int(lens[b]) + BS - 1) // BS
        tables2[b, n:] = 0
    got2 = decode(q, moved, tables2, lens, KV)
    assert torch.equal(got, got2)


def test_full_model_attention_shape(paged_kernel):
    """The full-model workload's decode: batch 32, 32 query / 4 KV heads,
    head_dim 64, lengths U[4096, 4224] (a 4096-token prompt plus up to 128
    generated tokens)."""
    lens, tables, q, cache, ref = workload("full-model-attention")
    got = decode(q, cache, tables, lens, 4)
    assert_close(got.cpu().numpy(), ref, what=f"batch 32, H=32 KV=4 D=64, U[4096,4224], {paged_kernel}")
