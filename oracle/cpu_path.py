"""The reference's CPU torch path, restated.  TEST INFRASTRUCTURE ONLY (and the
timed CPU baseline of bench.py).

The reference checks and benchmarks its kernels against a plain torch
composition (kernels/benchmark/benchmark.py:59-66,112-117): dequantize the
packed codes in fp32, round to fp16, broadcast the KV heads to the query heads
with repeat_interleave and call F.scaled_dot_product_attention.  The reference
has no CPU path for the paged per-token format, so ``paged_decode`` follows the
paged kernel's semantics (kernels/kv_dequant_kernels.cuh:708-747): gather each
token's slot through the block table, dequantize ``nibble * step + min``, then
the same attention.  Attention runs in fp32 on the CPU (fp16 SDPA has no fast
CPU kernel).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def unpack(packed: torch.Tensor) -> torch.Tensor:
    """uint8 [..., D/2] -> uint8 codes [..., D]; even dim = low nibble."""
    lo = packed & 0x0F
    hi = packed >> 4
    return torch.stack([lo, hi], dim=-1).flatten(-2)


def dequant_per_channel(packed, scale, zero):
    """kernels/benchmark/benchmark.py:59-66: (q - zero) * scale in fp32."""
    q = unpack(packed).float()
    return (q - zero.float().unsqueeze(1)) * scale.float().unsqueeze(1)


def decode_per_channel(q, kp, ks, kz, vp, vs, vz):
    """q [H, 1, D] fp16 -> [H, 1, D] fp32 via dequant -> fp16 -> GQA broadcast -> SDPA."""
    H, KV = q.shape[0], kp.shape[0]
    k = dequant_per_channel(kp, ks, kz).half().float().repeat_interleave(H // KV, dim=0)
    v = dequant_per_channel(vp, vs, vz).half().float().repeat_interleave(H // KV, dim=0)
    return F.scaled_dot_product_attention(q.float(), k, v)


def paged_decode(q, kv_cache, block_tables, seq_lens, block_size: int, num_kv_heads: int,
                 seqs=None):
    """q [B, H, D] fp16; kv_cache [nb, bs, KV, D+8] uint8; -> [B, H, D] fp32."""
    B, H, D = q.shape
    G = H // num_kv_heads
    out = torch.zeros((B, H, D), dtype=torch.float32)
    for b in (range(B) if seqs is None else seqs):
        L = int(seq_lens[b])
        if L == 0:
            continue
        n = torch.arange(L)
        blocks = block_tables[b].long()[n // block_size]
        slots = kv_cache[blocks, n % block_size]                   # [L, KV, D+8]
        rul = slots[..., D:].contiguous().view(torch.float16).float()   # [L, KV, 4]
        k = unpack(slots[..., : D // 2]).float() * rul[..., 1:2] + rul[..., 0:1]
        v = unpack(slots[..., D // 2: D]).float() * rul[..., 3:4] + rul[..., 2:3]
        k = k.half().float().permute(1, 0, 2).repeat_interleave(G, dim=0)   # [H, L, D]
        v = v.half().float().permute(1, 0, 2).repeat_interleave(G, dim=0)
        out[b] = F.scaled_dot_product_attention(q[b].float()[:, None, :], k, v)[:, 0]
    return out
