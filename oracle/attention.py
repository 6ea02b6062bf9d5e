"""Dequant-then-attend in float64.  TEST INFRASTRUCTURE ONLY.

Restates the arithmetic every decode/prefill kernel of the reference fuses:
unpack nibbles -> dequantize -> q.K / sqrt(D) -> softmax -> P.V, with exact
(float64) softmax instead of the kernels' chunked online softmax, which is
mathematically the same function.

Reference semantics followed (file:line in the reference repository):
* nibble order: even dim = low nibble, odd dim = high nibble
  (kernels/kv_dequant_kernels.cuh:14-17);
* per-channel dequant ``(nib - z) * s``, raw nibble when use_quant is False
  (kernels/kv_dequant_kernels.cuh:189-194; kernels/benchmark/benchmark.py:59-66);
* per-token dequant ``nib * step + min`` (kernels/kv_dequant_kernels.cuh:591-592,646);
* GQA map ``kv_head = h // (H / KV)`` (kernels/kv_dequant_kernels.cuh:143);
* softmax scale fixed at 1/sqrt(D) (kernels/kv_dequant_kernels.cuh:167,703);
* paged slot ``cache[block_row[n // bs], n % bs, kv_head, :]`` with K bytes at
  [0, D/2), V bytes at [D/2, D), fp16 (k_min, k_step, v_min, v_step) at D..D+8
  (kernels/kv_dequant_kernels.cuh:666-670,713-722,736-747);
* causal prefill mask ``m >= n`` with queries and keys both indexed from 0
  (kernels/kv_dequant_kernels.cuh:396-398).
"""
from __future__ import annotations

import numpy as np

from .quant import unpack_nibbles


def dequant_per_channel(packed, scale, zero, use_quant: bool = True, round_fp16: bool = False):
    """[KV, S, D/2] u8 + [KV, D] fp16 rulers -> float64 [KV, S, D].

    round_fp16=True additionally rounds the dequantized values to fp16 as the
    reference benchmark does before its SDPA check
    (kernels/benchmark/benchmark.py:112)."""
    codes = unpack_nibbles(np.asarray(packed)).astype(np.float64)
    if not use_quant:
        return codes
    s = np.asarray(scale, dtype=np.float16).astype(np.float32)[:, None, :]
    z = np.asarray(zero, dtype=np.float16).astype(np.float32)[:, None, :]
    vals = (codes.astype(np.float32) - z) * s          # fp32, like dequantize_tensor
    if round_fp16:
        vals = vals.astype(np.float16)
    return vals.astype(np.float64)


def dequant_per_token(packed, mins, steps):
    """[KV, S, D/2] u8 + [KV, S] fp16 min/step -> float64 [KV, S, D]."""
    codes = unpack_nibbles(np.asarray(packed)).astype(np.float64)
    # contiguous rulers: broadcasting strided fp16 views is ~10x slower
    mn = np.ascontiguousarray(np.asarray(mins, dtype=np.float16), dtype=np.float64)[..., None]
    st = np.ascontiguousarray(np.asarray(steps, dtype=np.float16), dtype=np.float64)[..., None]
    codes *= st
    codes += mn
    return codes


def gather_paged(kv_cache, block_row, seq_len: int):
    """Read one request's tokens from the packed paged cache.

    kv_cache uint8 [num_blocks, bs, KV, D+8]; block_row int [>= ceil(S/bs)].
    Returns (k_packed [KV,S,D/2], v_packed [KV,S,D/2], rulers fp16 [KV,S,4]).
    """
    kv_cache = np.asarray(kv_cache)
    nb, bs, KV, slot = kv_cache.shape
    D = slot - 8
    n = np.arange(seq_len)
    blocks = np.asarray(block_row, dtype=np.int64)[n // bs]
    slots = kv_cache[blocks, n % bs]                     # [S, KV, D+8]
    slots = np.transpose(slots, (1, 0, 2))               # [KV, S, D+8]
    kp = slots[..., : D // 2]
    vp = slots[..., D // 2: D]
    rul = np.ascontiguousarray(slots[..., D: D + 8]).view(np.float16)
    return kp, vp, rul


def attend(q, K, V):
    """softmax(q K^T / sqrt(D)) V per query head, float64.

    q [H, D] or [H, M, D]; K, V [KV, S, D].  Returns [H, D] / [H, M, D].
    S == 0 gives NaN, as the reference kernels do (0/0)."""
    q = np.asarray(q, dtype=np.float64)
    squeeze = q.ndim == 2
    if squeeze:
        q = q[:, None, :]
    H, M, D = q.shape
    KV, S, _ = K.shape
    G = H // KV
    out = np.empty((H, M, D), dtype=np.float64)
    if S == 0:
        out.fill(np.nan)
        return out[:, 0] if squeeze else out
    for h in range(H):
        kv = h // G
        s = q[h] @ K[kv].T / np.sqrt(D)                  # [M, S]
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[h] = p @ V[kv]
    return out[:, 0] if squeeze else out


def attend_causal(q, K, V, causal: bool = True):
    """Prefill: q [H, M, D], K/V [KV, S, D]; query row m sees keys n <= m when
    causal (kernels/kv_dequant_kernels.cuh:396-398).  Rows with no visible key
    are NaN."""
    q = np.asarray(q, dtype=np.float64)
    H, M, D = q.shape
    KV, S, _ = K.shape
    G = H // KV
    out = np.empty((H, M, D), dtype=np.float64)
    n = np.arange(S)
    for h in range(H):
        kv = h // G
        s = q[h] @ K[kv].T / np.sqrt(D)                  # [M, S]
        if causal:
            mask = n[None, :] > np.arange(M)[:, None]
            s = np.where(mask, -np.inf, s)
        mx = s.max(axis=1, keepdims=True)
        with np.errstate(invalid="ignore"):
            p = np.exp(s - mx)
            p /= p.sum(axis=1, keepdims=True)
        out[h] = p @ V[kv]
    return out


def decode_per_channel(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero,
                       use_quant: bool = True, round_fp16: bool = False):
    """kv_dequant_decode_attention semantics: q [H, 1, D] -> [H, 1, D]."""
    K = dequant_per_channel(k_packed, k_scale, k_zero, use_quant, round_fp16)
    V = dequant_per_channel(v_packed, v_scale, v_zero, use_quant, round_fp16)
    q = np.asarray(q, dtype=np.float16).astype(np.float64)
    return attend(q[:, 0, :], K, V)[:, None, :]


def prefill_per_channel(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero,
                        causal: bool = True, use_quant: bool = True, round_fp16: bool = False):
    """kv_dequant_prefill_attention semantics: q [H, M, D] -> [H, M, D]."""
    K = dequant_per_channel(k_packed, k_scale, k_zero, use_quant, round_fp16)
    V = dequant_per_channel(v_packed, v_scale, v_zero, use_quant, round_fp16)
    q = np.asarray(q, dtype=np.float16).astype(np.float64)
    return attend_causal(q, K, V, causal)


def decode_per_token(q, k_packed, k_min, k_step, v_packed, v_min, v_step):
    """kv_dequant_decode_per_token_attention semantics: q [H,1,D] -> [H,1,D]."""
    K = dequant_per_token(k_packed, k_min, k_step)
    V = dequant_per_token(v_packed, v_min, v_step)
    q = np.asarray(q, dtype=np.float16).astype(np.float64)
    return attend(q[:, 0, :], K, V)[:, None, :]


def decode_paged(q, kv_cache, block_row, seq_len: int):
    """kv_dequant_decode_per_token_paged_attention semantics for one request:
    q [H, D] (or [H, 1, D]) -> [H, D]."""
    q = np.asarray(q, dtype=np.float16).astype(np.float64).reshape(q.shape[0], -1)
    kp, vp, rul = gather_paged(kv_cache, block_row, seq_len)
    K = dequant_per_token(kp, rul[..., 0], rul[..., 1])
    V = dequant_per_token(vp, rul[..., 2], rul[..., 3])
    return attend(q, K, V)


def decode_paged_batched(q, kv_cache, block_tables, seq_lens):
    """The batched decode: q [B, H, D], block_tables [B, max_blocks],
    seq_lens [B] -> [B, H, D].  Sequences of length 0 give zeros (the batched
    API's defined result; the adapter skips them, like the reference's
    adapters/vllm_adapter.py:271-274)."""
    q = np.asarray(q)
    B, H, D = q.shape
    out = np.zeros((B, H, D), dtype=np.float64)
    for b in range(B):
        L = int(seq_lens[b])
        if L > 0:
            out[b] = decode_paged(q[b], kv_cache, block_tables[b], L)
    return out
