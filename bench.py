#!/usr/bin/env python3
"""Benchmark of the batched paged 4-bit GQA decode attention on one MI355X.

Workload (the headline configuration): one decode step of 64 sequences with
lengths drawn uniformly from [512, 8192] (seed 0), 32 query / 8 KV heads,
head_dim 128, block size 16, K/V ~ N(0, 1) quantized into the packed per-token
min/step cache [num_blocks, 16, 8, 136] (uint8), block tables a random
permutation of exactly the blocks needed.  A step is one launch of the fused
dequant + attention over the whole batch; inputs are resident in HBM.  Three
independent caches and queries (~303 MB of KV each, together above the 256 MB
Infinity Cache) are rotated so no step is served from it.

Steady state: a freshly started process needs about 200 back-to-back decode
launches (~20 ms) before the GPU settles (the first ~100 launches run ~20 %
slower).  Before its W warmup steps, the benchmark therefore runs the decode
untimed for --prewarm-ms (default 100 ms); the JSON line reports it.

Printed: one JSON line with the throughput in algorithmic GB/s (packed KV +
rulers, q, fp32 out, block-table entries and lengths actually read) over K
back-to-back steps, the time per step, the roofline object for the decode
kernel (its own duration from a HIP event pair stamped from its dispatch on the
launch stream, slmt_kernel_timing, over K further launches) and
a CPU baseline (the reference's CPU torch path on a bounded sample of the same
workload).

    python bench.py [--gpus 1] [--steps 500] [--warmup 400] [--prewarm-ms 100] [--no-cpu]
                    [--workload headline|long-context|full-model-attention]

--workload picks another decode shape for the same measurement (the default
is the headline configuration above):
* long-context: batch 8, lengths U[32768, 131072], 64 query / 8 KV heads,
  head_dim 128, K/V ~ Student-t(3); also times the quantize-on-write append of
  one new token per sequence;
* full-model-attention: the attention of one layer of the full-model decode
  step below, batch 32, lengths U[4096, 4224], 32 query / 4 KV heads, head_dim 64.

--op-level first prints one line per standalone per-channel decode workload
(batch 1, 4/4 heads, head_dim 64, 512 keys; and 12/2 heads, head_dim 128, 512 /
1024 / 2048 keys with 1 % outlier channels), each with its roofline object and
the reference's CPU torch path timed beside it; then the reference's op-level
tables (one JSON line per case):
per-channel decode (32/4 and 14/2 heads at head_dim 64, 32/8 at 128; S = 512,
1024, 2048) and causal prefill (32/4 and 14/2 at 64; S = 512, 1024), each
against fp16 SDPA over the dequantized K/V broadcast to the query heads
(err_vs_dequantized), the error against fp16 SDPA over the unquantized K/V
(err_vs_fp16, the quantization's cost) and the KV bytes (fp16 broadcast to
the query heads against packed).

--per-channel-model instead prints the reference's model-level comparison:
batch-1 greedy decode of the same random-init 1.1B model, prompt 512, 64 new
tokens, steady-state tokens/s of the fp16 path and of the per-channel hook with
rulers fixed at the first decode step and with rulers refreshed every step.

--full-model instead prints the line of the full-model workload: greedy
decode of a random-init Llama-style 1.1B model (22 layers, hidden 2048, 32 /
4 heads, head_dim 64, MLP 5632), batch 32, prompt 4096 random token ids, 128
new tokens, tokens/s of the packed 4-bit KV path (decode step replayed from a
HIP graph; eager also reported) against the fp16 eager baseline (attention
hook in slm-turbo_amd/adapters/hf_llama.py).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time
from dataclasses import dataclass
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "slm-turbo_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "decode-attn µs/step + HBM GB/s (% of 8 TB/s), D=128 GQA paged 4-bit"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E peak
BS = 16


@dataclass(frozen=True)
class Workload:
    """One decode step's shape: B sequences with lengths U[lo, hi] (seed 0),
    H query / KV heads of head_dim D, K/V drawn from ``dist``; ``sets``
    independent caches and queries are rotated per step."""
    name: str
    B: int
    H: int
    KV: int
    D: int
    lo: int
    hi: int
    dist: str
    sets: int
    text: str

    @property
    def tag(self) -> str:
        return f"paged_decode_b{self.B}_h{self.H}_kv{self.KV}_d{self.D}"

    @property
    def metric(self) -> str:
        if self.name == "headline":
            return METRIC
        return f"decode-attn µs/step + HBM GB/s (% of 8 TB/s), D={self.D} GQA paged 4-bit, {self.name}"


WORKLOADS = {
    "headline": Workload("headline", 64, 32, 8, 128, 512, 8192, "normal", 3,
                         "paged per-token 4-bit decode attention, batch 64, lengths U[512,8192] seed 0, "
                         "32 q / 8 KV heads, head_dim 128, block 16"),
    "long-context": Workload("long-context", 8, 64, 8, 128, 32768, 131072, "t3", 2,
                             "paged per-token 4-bit decode attention, batch 8, lengths U[32768,131072] seed 0, "
                             "64 q / 8 KV heads, head_dim 128, block 16, K/V Student-t(3)"),
    "full-model-attention": Workload("full-model-attention", 32, 32, 4, 64, 4096, 4224, "normal", 3,
                                     "paged per-token 4-bit decode attention of one layer of the 1.1B "
                                     "Llama-style decode step, batch 32, lengths U[4096,4224] seed 0, "
                                     "32 q / 4 KV heads, head_dim 64, block 16"),
}


def traffic_file(w: Workload) -> Path:
    return ROOT / "profiles" / f"{w.tag}_traffic.txt"


COUNTERS_FILE = ROOT / "profiles" / "paged_decode_valu_counters.txt"


def kernel_source_sha() -> str:
    """sha256 (16 hex digits) of the HIP sources the library is built from
    (slm-turbo_amd/csrc, every file, in name order).  The counter summaries under
    profiles/ carry the value of the build they measured, so a bench line can
    say whether its committed counters describe the kernels it ran."""
    import hashlib

    h = hashlib.sha256()
    for f in sorted((ROOT / "slm-turbo_amd" / "csrc").iterdir()):
        if f.is_file():
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def profile_stamp(path: Path):
    """The kernel_source_sha line of a committed profile summary, or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("kernel_source_sha:"):
            return line.split(":", 1)[1].strip()
    return None


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--prewarm-ms", type=float, default=100.0,
                    help="untimed decode launches for at least this long before the warmup steps")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="headline")
    ap.add_argument("--sets", type=int, default=0,
                    help="independent cache/query sets rotated per step (0: the workload's own)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--op-level", action="store_true",
                    help="the reference's op-level per-channel decode/prefill tables instead of the paged decode")
    ap.add_argument("--full-model", action="store_true",
                    help="time full-model greedy decode (1.1B Llama-style) instead of the kernel")
    ap.add_argument("--fm-batch", type=int, default=32)
    ap.add_argument("--fm-prompt", type=int, default=4096)
    ap.add_argument("--fm-new-tokens", type=int, default=128)
    ap.add_argument("--per-channel-model", action="store_true",
                    help="the reference's model-level table instead: batch-1 greedy decode of the 1.1B model, "
                         "fp16 against the per-channel hook with fixed and with refreshed rulers")
    ap.add_argument("--pc-prompt", type=int, default=512)
    ap.add_argument("--pc-new-tokens", type=int, default=64)
    ap.add_argument("--calibrate-copy-mb", type=int, default=0,
                    help="also run a plain device copy of this many MB (counter calibration)")
    return ap.parse_args(argv)


def build_workload(seed: int, sets: int, dev, w: Workload = WORKLOADS["headline"]):
    import torch

    from kernels import kv_dequant as kd

    B, H, KV, D = w.B, w.H, w.KV, w.D
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(w.lo, w.hi + 1, (B,), generator=g)
    nblk = (lens + BS - 1) // BS
    total = int(nblk.sum())
    perm = torch.randperm(total, generator=g)
    maxb = int(nblk.max())
    tables = torch.zeros((B, maxb), dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(nblk[b])
        tables[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    # flat slot of every token of every sequence
    slot_chunks = []
    for b in range(B):
        pos = torch.arange(int(lens[b]))
        slot_chunks.append(tables[b, pos // BS].long() * BS + pos % BS)
    slots = torch.cat(slot_chunks).to(dev)
    N = slots.numel()
    qs, caches = [], []
    for s in range(sets):
        qs.append(torch.randn((B, H, D), generator=g).half().to(dev))
        cache = torch.empty((total, BS, KV, D + 8), dtype=torch.uint8, device=dev)
        gg = torch.Generator(device=dev).manual_seed(seed * 1000 + s)

        def values(n):
            z = torch.randn((n, KV, D), generator=gg, device=dev)
            if w.dist == "t3":                     # Student-t(3): z / sqrt(chi2_3 / 3)
                chi2 = (torch.randn((3, n, KV, D), generator=gg, device=dev) ** 2).sum(0)
                z = z / torch.sqrt(chi2 / 3.0)
            return z.half()

        chunk = 1 << 16
        for t0 in range(0, N, chunk):
            n = min(chunk, N - t0)
            k = values(n)
            v = values(n)
            kd.kv_quantize_store(k, v, cache, slots[t0:t0 + n], BS)
        caches.append(cache)
    torch.cuda.synchronize()
    return lens, tables, qs, caches


def algorithmic_bytes(lens, w: Workload = WORKLOADS["headline"]) -> int:
    """Bytes a perfect kernel must move per step: packed KV + rulers of every
    token, q (fp16), out (fp32), the block-table entries used and the lengths."""
    B, H, KV, D = w.B, w.H, w.KV, w.D
    L = [int(x) for x in lens]
    blocks = sum((x + BS - 1) // BS for x in L)
    return sum(L) * KV * (D + 8) + B * H * D * 2 + B * H * D * 4 + blocks * 4 + B * 4


def read_traffic(w: Workload = WORKLOADS["headline"]):
    """HBM bytes per launch measured with rocprofv3 counters (committed summary)."""
    path = traffic_file(w)
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the platform's machine string."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def read_counter(key: str, w: Workload = WORKLOADS["headline"]):
    """Per-launch instruction count `key` (valu_instructions_per_launch or
    mfma_instructions_per_launch, rocprofv3 SQ_INSTS_VALU / SQ_INSTS_MFMA) from
    the committed counter summary, or None."""
    path = COUNTERS_FILE
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(f"{key}[{w.name}]:"):
            return int(float(line.split(":", 1)[1]))
    return None


# Issue time of a VALU wave instruction on one SIMD (16 lanes x 4 passes) and of
# the 16x16x64 int8 / 16x16x32 fp16 MFMA instructions, at the 2.1 GHz shader
# clock measured under this load, and the SIMDs of an MI355X.
VALU_CYCLES, MFMA_CYCLES, LOAD_CLOCK_GHZ, SIMDS = 4, 16, 2.1, 1024


def cpu_baseline(lens, tables, q, cache_gpu, out_gpu, budget_s: float, w: Workload = WORKLOADS["headline"]):
    """The reference's CPU torch path (oracle/cpu_path.py) on a bounded sample."""
    import torch

    B, H, KV, D = w.B, w.H, w.KV, w.D

    from oracle import cpu_path

    # every CPU of this process's affinity mask
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cache = cache_gpu.cpu()
    qc = q.cpu()
    # grow the sample (sequences in order) until one pass takes ~budget/4
    seqs, t_one = [0], 0.0
    cpu_path.paged_decode(qc, cache, tables, lens, BS, KV, seqs=[0])          # warm-up
    while True:
        t0 = time.perf_counter()
        out = cpu_path.paged_decode(qc, cache, tables, lens, BS, KV, seqs=seqs)
        t_one = time.perf_counter() - t0
        if t_one >= budget_s / 4 or len(seqs) == B:
            break
        seqs = list(range(min(B, len(seqs) * 2)))
    times = [t_one]
    while sum(times) < budget_s * 0.75 and len(times) < 10:
        t0 = time.perf_counter()
        out = cpu_path.paged_decode(qc, cache, tables, lens, BS, KV, seqs=seqs)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    L = [int(lens[b]) for b in seqs]
    nbytes = sum(L) * KV * (D + 8) + len(seqs) * (H * D * 6 + 4) + sum((x + BS - 1) // BS for x in L) * 4
    err = float((out[seqs] - out_gpu.cpu()[seqs]).abs().max())
    return {
        "value": round(nbytes / t / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{len(seqs)} of {B} sequences ({sum(L)} tokens), median of {len(times)} runs, "
                  f"{t * 1e3:.1f} ms/run; fp32 SDPA after fp16-rounded dequant",
        "us_per_sample_step": round(t * 1e6, 1),
        "cpu_model": cpu_model(),
        "max_abs_diff_vs_gpu": err,
    }


def per_channel_configs(kd, dev, timeit, cpu_budget_s) -> None:
    """The two standalone per-channel decode workloads, one JSON line each, with
    `roofline` and `cpu_baseline` objects like the paged line's:
    * batch 1, 4 query / 4 KV heads, head_dim 64, 512 keys, K/V and q ~ N(0,1);
    * batch 1, 12 query / 2 KV heads (Qwen2-1.5B-shaped), head_dim 128, 512 / 1024 /
      2048 keys, K/V ~ N(0,1) with 1 % of the channels scaled x8.
    Bytes per call: packed K and V (KV * S * D), their fp16 scale and zero per
    channel (8 * KV * D), q fp16 (2 * H * D) and the fp32 output (4 * H * D).
    `achieved` divides them by the mean time of back-to-back Python calls (these
    calls are launch-latency bound).  The CPU baseline is the reference's torch
    composition (oracle/cpu_path.decode_per_channel) on the same inputs."""
    import torch

    cases = [("per-channel decode, batch 1, 4 q / 4 KV heads, head_dim 64, 512 keys", 4, 4, 64, 512, False)]
    cases += [(f"per-channel decode, batch 1, 12 q / 2 KV heads, head_dim 128, {S} keys, 1 % outlier channels x8",
               12, 2, 128, S, True) for S in (512, 1024, 2048)]
    for name, H, KV, D, S, outliers in cases:
        g = torch.Generator().manual_seed(S + H)
        k = torch.randn((KV, S, D), generator=g)
        v = torch.randn((KV, S, D), generator=g)
        if outliers:
            for x in (k, v):
                n = max(1, math.ceil(0.01 * KV * D))
                for c in torch.randperm(KV * D, generator=g)[:n].tolist():
                    x[c // D, :, c % D] *= 8.0
        q = torch.randn((H, 1, D), generator=g).half().to(dev)
        kp, ks, kz, vp, vs, vz = kd.quantize_kv(k.half().to(dev), v.half().to(dev))
        args = (q, kp, ks, kz, vp, vs, vz)
        run = lambda: kd.kv_dequant_decode_attention(*args, num_kv_heads=KV)
        out = run()
        us = timeit(run, 2000, warmup=2000)   # the first calls of a process run while the GPU clocks settle
        nbytes = KV * S * D + 8 * KV * D + 2 * H * D + 4 * H * D
        achieved = nbytes / us / 1e3
        line = {
            "metric": "per-channel 4-bit decode µs/call + HBM GB/s (% of 8 TB/s)",
            "value": round(achieved, 3), "unit": "GB/s", "us_per_call": round(us, 2),
            "higher_is_better": True, "dtype": "int4 codes x fp16 query, fp32 accumulate",
            "data": "synthetic", "config": {"workload": name, "H": H, "KV": KV, "D": D, "S": S},
            # a call moves 0.1-0.5 MB (HBM floor below 0.1 µs): its time is the
            # launch and a few dependent memory round trips, so the binding
            # limit is latency; achieved/frac are still priced against HBM
            "roofline": {"bound": "latency", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 6), "traffic": None,
                         "algorithmic_bytes": nbytes, "hbm_floor_us": round(nbytes / HBM_PEAK_GBS / 1e3, 4),
                         "note": "time per back-to-back Python call: launch-latency bound"},
        }
        if cpu_budget_s is not None:
            line["cpu_baseline"] = per_channel_cpu_baseline([t.cpu() for t in args], out.cpu(), nbytes,
                                                            min(cpu_budget_s, 5.0))
        print(json.dumps(line), flush=True)


def per_channel_cpu_baseline(args, out_gpu, nbytes: int, budget_s: float) -> dict:
    """oracle/cpu_path.decode_per_channel timed on the host cores."""
    import torch

    from oracle import cpu_path

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = cpu_path.decode_per_channel(*args)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end and len(times) < 2000:
        t0 = time.perf_counter()
        out = cpu_path.decode_per_channel(*args)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {
        "value": round(nbytes / t / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": f"the whole call, median of {len(times)} runs, {t * 1e6:.1f} µs/run; "
                  "fp32 SDPA after fp16-rounded dequant",
        "us_per_call": round(t * 1e6, 1), "cpu_model": cpu_model(),
        "max_abs_diff_vs_gpu": float((out - out_gpu).abs().max()),
    }


def op_level(args) -> int:
    """The reference's op-level tables (kernels/benchmark/benchmark.py:106-174) on this
    GPU: per-channel decode and causal prefill through the HIP kernels against fp16 SDPA
    over the dequantized K/V broadcast to the query heads.  One JSON line per case."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from kernels import kv_dequant as kd

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    def timeit(fn, iters, warmup=5):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters * 1e3           # µs per call

    def dequant(packed, scale, zero):                    # (codes - zero) * scale, fp32
        codes = torch.stack([packed & 15, packed >> 4], dim=-1).flatten(-2).float()
        return (codes - zero.float()[:, None, :]) * scale.float()[:, None, :]

    def sdpa(q, k, v, causal):
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q[None], k[None], v[None], is_causal=causal)[0]

    per_channel_configs(kd, dev, timeit, None if args.no_cpu else args.cpu_seconds)

    cases = [("decode", H, KV, D, S, 200) for H, KV, D in ((32, 4, 64), (14, 2, 64), (32, 8, 128))
             for S in (512, 1024, 2048)]
    cases += [("prefill", H, KV, D, S, 50) for H, KV, D in ((32, 4, 64), (14, 2, 64)) for S in (512, 1024)]
    # beyond the reference's table: prefills long enough to be compute-bound,
    # timed at steady state (40 warmup calls, best of 3 runs of 20 calls)
    extra = [("prefill", 32, 4, 64, 4096, 20), ("prefill", 12, 2, 128, 4096, 20)]
    for phase, H, KV, D, S, iters in cases + extra:
        longrun = (phase, H, KV, D, S, iters) in extra
        tm = (lambda fn, n: min(timeit(fn, n, warmup=40 if r == 0 else 0) for r in range(3))) if longrun else timeit
        g = torch.Generator(device=dev).manual_seed(0)
        M = 1 if phase == "decode" else S
        q = torch.randn((H, M, D), generator=g, device=dev).half()
        k = torch.randn((KV, S, D), generator=g, device=dev).half()
        v = torch.randn((KV, S, D), generator=g, device=dev).half()
        kp, ks, kz, vp, vs, vz = kd.quantize_kv(k, v)
        kb = dequant(kp, ks, kz).half().repeat_interleave(H // KV, dim=0)
        vb = dequant(vp, vs, vz).half().repeat_interleave(H // KV, dim=0)
        causal = phase == "prefill"
        if causal:
            run = lambda: kd.kv_dequant_prefill_attention(q, kp, ks, kz, vp, vs, vz, causal=True, num_kv_heads=KV)
        else:
            run = lambda: kd.kv_dequant_decode_attention(q, kp, ks, kz, vp, vs, vz, num_kv_heads=KV)
        out = run()
        line = {"metric": f"op-level {phase} µs/call, per-channel 4-bit vs fp16 SDPA", "phase": phase,
                "H": H, "KV": KV, "D": D, "S": S, "kernel_us": round(tm(run, iters), 2)}
        try:
            ref = sdpa(q, kb, vb, causal)
            line["err_vs_dequantized"] = float((out - ref.float()).abs().max())
            # the quantization's own cost: against fp16 SDPA over the unquantized K/V
            G = H // KV
            ref16 = sdpa(q, k.repeat_interleave(G, dim=0), v.repeat_interleave(G, dim=0), causal)
            line["err_vs_fp16"] = float((out - ref16.float()).abs().max())
            line["fp16_sdpa_us"] = round(tm(lambda: sdpa(q, kb, vb, causal), iters), 2)
            line["speedup_vs_fp16_sdpa"] = round(line["fp16_sdpa_us"] / line["kernel_us"], 3)
        except RuntimeError as e:                         # no flash / memory-efficient kernel here
            line["fp16_sdpa_us"] = None
            line["fp16_sdpa_error"] = str(e).splitlines()[0][:160]
        packed_bytes = 2 * KV * S * (D // 2) + 4 * KV * D * 2
        line["kv_bytes"] = {"fp16_broadcast": 2 * H * S * D * 2, "packed": packed_bytes}
        if phase == "decode":
            line["packed_gb_per_s"] = round(packed_bytes / line["kernel_us"] / 1e3, 2)
        else:   # causal: QK and PV over the S (S + 1) / 2 visible pairs, 2 flops per multiply-add
            line["tflops"] = round(4.0 * H * D * S * (S + 1) / 2 / line["kernel_us"] / 1e6, 2)
        if longrun:
            line["extra"] = "beyond the reference's op-level table; steady state, best of 3 x 20 calls"
        print(json.dumps(line), flush=True)
    return 0


def full_model(args) -> int:
    """One JSON line: tokens/s of greedy decode, packed 4-bit KV vs fp16 eager."""
    import torch

    from adapters import hf_llama

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    r = hf_llama.run_decode_benchmark(args.fm_batch, args.fm_prompt, args.fm_new_tokens, "cuda:0", args.seed)
    B, N = r["batch"], r["new_tokens"]
    result = {
        "metric": "full-model greedy decode tokens/s, packed 4-bit KV vs fp16 eager",
        "value": round(r["packed_graph"]["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": N,
        "warmup": 1,
        "ms_per_step": round(r["packed_graph"]["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 weights/activations; int4 KV codes",
        "data": "synthetic: random-init weights (seed 0), random prompt token ids",
        "config": {"workload": f"Llama-style 1.1B greedy decode, batch {B}, prompt {r['prompt']}, {N} new tokens",
                   **{k: r[k] for k in ("batch", "prompt", "new_tokens", "layers", "hidden", "heads",
                                        "kv_heads", "head_dim", "params")}},
        "fp16_eager": {k: round(v, 4) for k, v in r["fp16"].items()},
        "packed_eager": {k: round(v, 4) for k, v in r["packed"].items()},
        "packed_graph": {k: round(v, 4) for k, v in r["packed_graph"].items()},
        "speedup_vs_fp16_eager": round(r["speedup_graph"], 3),
        "speedup_eager_vs_fp16_eager": round(r["speedup"], 3),
        "graph_tokens_equal_eager": r["graph_tokens_equal_eager"],
        "kv_cache_bytes": r["kv_cache_bytes"],
        "prefill_logits_max_abs_diff": r["prefill_logits_max_abs_diff"],
        "first_decode_logits_cosine_min": r["first_decode_logits_cosine_min"],
        "greedy_token_agreement": round(r["greedy_token_agreement"], 4),
    }
    print(json.dumps(result))
    return 0


def per_channel_model(args) -> int:
    """One JSON line: the reference's model-level comparison
    (kernels/benchmark/benchmark.py:240-269, 316-331) on the random-init 1.1B
    model: steady-state batch-1 greedy decode tokens/s of the fp16 path and of
    the per-channel hook with fixed and with refreshed rulers."""
    import torch

    from adapters import hf_llama

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    r = hf_llama.run_per_channel_benchmark(args.pc_prompt, args.pc_new_tokens, "cuda:0", args.seed)
    steady = r["new_tokens"] - r["warm"]
    result = {
        "metric": "batch-1 greedy decode tokens/s, per-channel 4-bit hook vs fp16 eager",
        "value": round(r["per_channel_fixed"]["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steady,
        "warmup": r["warm"],
        "ms_per_step": round(r["per_channel_fixed"]["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 weights/activations; int4 per-channel KV codes",
        "data": "synthetic: random-init weights (seed 0), random prompt token ids",
        "config": {"workload": f"Llama-style 1.1B greedy decode, batch 1, prompt {r['prompt']}, "
                               f"{r['new_tokens']} new tokens (the first {r['warm']} untimed)",
                   **{k: r[k] for k in ("prompt", "new_tokens", "layers", "heads", "kv_heads", "head_dim")}},
        "fp16_eager": {k: round(v, 4) for k, v in r["fp16"].items()},
        "per_channel_fixed": {k: round(v, 4) for k, v in r["per_channel_fixed"].items()},
        "per_channel_refresh": {k: round(v, 4) for k, v in r["per_channel_refresh"].items()},
        "note": "the logits cosine and token agreement against fp16 measure the per-channel 4-bit "
                "quantization of the cache; random-init weights give near-flat logits, so greedy tokens "
                "part at the first step. The hook's kernel output is checked against the float64 oracle "
                "in tests/test_hf_llama.py",
    }
    print(json.dumps(result))
    return 0


def main(argv=None) -> int:
    args = parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (the decode path has no cross-GPU "
              f"exchange); asked for --gpus {args.gpus} / WORLD_SIZE {world}.", file=sys.stderr)
        return 2
    if args.full_model:
        return full_model(args)
    if args.per_channel_model:
        return per_channel_model(args)
    if args.op_level:
        return op_level(args)

    import torch

    from kernels import _native
    from kernels import kv_dequant as kd

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    w = WORKLOADS[args.workload]
    B, H, KV, D = w.B, w.H, w.KV, w.D
    sets = args.sets or w.sets
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lens, tables, qs, caches = build_workload(args.seed, sets, dev, w)
    tables_d = tables.to(dev)
    lens_d = lens.to(torch.int32).to(dev)
    nb = caches[0].shape[0]
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)

    # correctness of the launch path (Python API) before timing
    ref_out = kd.kv_dequant_decode_paged_batched(qs[0], caches[0], tables_d, lens_d, BS, KV)

    lib = _native.load()
    ws, ws_bytes = kd._workspace(lib, dev, B, H, KV, D)
    stream = torch.cuda.current_stream(dev)
    fn = lib.slmt_decode_paged_batched
    argsets = [(q.data_ptr(), H * D, D, c.data_ptr(), nb, BS, tables_d.data_ptr(), 32, tables_d.stride(0),
                lens_d.data_ptr(), 0, B, H, KV, D, out.data_ptr(), _native.OUT_F32, H * D, D, ws, ws_bytes,
                stream.cuda_stream) for q, c in zip(qs, caches)]

    if args.calibrate_copy_mb:
        n = args.calibrate_copy_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"calibration copy: {n} bytes read, {n} bytes written", file=sys.stderr)

    prewarm = 0
    t_pre = time.perf_counter()
    while (time.perf_counter() - t_pre) * 1e3 < args.prewarm_ms:
        for i in range(16):
            _native.check(lib, fn(*argsets[i % sets]))
        torch.cuda.synchronize()
        prewarm += 16
    for i in range(args.warmup):
        _native.check(lib, fn(*argsets[i % sets]))
    torch.cuda.synchronize()

    K = args.steps
    ms_per_step, kernel_us, launch_us, kernel_name = time_steps(lib, fn, argsets, K, stream)
    nbytes = algorithmic_bytes(lens, w)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    mean_launch = statistics.fmean(launch_us)
    # the dominant kernel's own duration (the whole-row decode); calls that
    # take another kernel record none, and then the whole call is used
    mean_kernel = statistics.fmean(kernel_us) if kernel_us else mean_launch
    achieved = nbytes / (mean_kernel * 1e-6) / 1e9
    result = {
        "metric": w.metric,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "prewarm": {"ms": args.prewarm_ms, "launches": prewarm},
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes x fp16 query (QK) and x fp16 weights (PV), fp32 accumulate",
        "data": "synthetic: K,V ~ " + ("Student-t(3)" if w.dist == "t3" else "N(0,1)")
                + " fp16 quantized into the packed cache; q ~ N(0,1)",
        "config": {
            "workload": w.text,
            "batch": B, "num_heads": H, "num_kv_heads": KV, "head_dim": D, "block_size": BS,
            "total_tokens": int(lens.sum()), "algorithmic_bytes": nbytes,
            "rotated_sets": sets, "out_dtype": "fp32",
        },
        "kernel": kernel_name or "per-wave kernel (attention_kernel)",
        "roofline": roofline(nbytes, achieved, w, mean_kernel, ms_per_step * 1e3),
        "kernel_us": ({
            "mean": round(mean_kernel, 2),
            "median": round(statistics.median(kernel_us), 2),
            "p10": round(kernel_us[len(kernel_us) // 10], 2),
            "p90": round(kernel_us[(9 * len(kernel_us)) // 10], 2),
            "note": "decode kernel alone: HIP events stamped from its dispatch (slmt_kernel_timing)",
        } if kernel_us else None),
        "launch_us": {
            "mean": round(mean_launch, 2),
            "median": round(statistics.median(launch_us), 2),
            "p10": round(launch_us[len(launch_us) // 10], 2),
            "p90": round(launch_us[(9 * len(launch_us)) // 10], 2),
            "note": "whole call (decode + merge kernels) inside an event pair",
        },
    }
    if kernel_name.startswith("mfma_kernel"):
        result["vector_alu_kernel"] = time_vector_alu_kernel(lib, fn, argsets, K, stream, nbytes)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(lens, tables, qs[0], caches[0], ref_out, args.cpu_seconds, w)
    else:
        result["cpu_baseline"] = None
    result["append"] = time_append(kd, caches[-1], tables, lens, w, dev)
    print(json.dumps(result))
    return 0


def time_steps(lib, fn, argsets, K: int, stream):
    """K steps back to back with events only at the ends (the whole-job rate),
    then K more with an event pair around every call while the library times the
    decode kernel alone (slmt_kernel_timing: a HIP event pair stamped from the
    kernel's dispatch on the launch stream; its duration, without the merge
    kernel that follows, is the roofline's).  The per-call events add a few µs
    of idle stream time per step, so they stay out of the first measurement.
    Returns (ms per step, sorted kernel µs, sorted per-call µs, kernel name)."""
    import torch

    from kernels import _native

    sets = len(argsets)
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()                     # single process: the barrier is this sync
    t_start.record(stream)
    for i in range(K):
        fn(*argsets[i % sets])
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    _native.check(lib, lib.slmt_kernel_timing(1))
    for i in range(K):
        ev[i][0].record(stream)
        fn(*argsets[i % sets])
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    lib.slmt_kernel_timing(0)
    kbuf = (ctypes.c_float * K)()
    nk = lib.slmt_kernel_timing_read(kbuf, K)
    if nk < 0:
        raise RuntimeError("kernel timing: " + _native.last_error(lib))
    name = (lib.slmt_kernel_timing_kernel() or b"").decode() if nk else ""
    return total_ms / K, sorted(kbuf[:nk]), sorted(a.elapsed_time(b) * 1e3 for a, b in ev), name


def time_vector_alu_kernel(lib, fn, argsets, K: int, stream, nbytes: int) -> dict:
    """The same steps through the vector-ALU whole-row kernel (no matrix cores;
    SLMT_PAGED_DECODE=valu, which the library reads on every call), timed the
    same way in this process after the matrix-core kernel's figures."""
    import torch

    from kernels import _native

    old = os.environ.get("SLMT_PAGED_DECODE")
    os.environ["SLMT_PAGED_DECODE"] = "valu"
    try:
        for i in range(200):
            _native.check(lib, fn(*argsets[i % len(argsets)]))
        torch.cuda.synchronize()
        ms, kus, _, name = time_steps(lib, fn, argsets, K, stream)
    finally:
        if old is None:
            os.environ.pop("SLMT_PAGED_DECODE", None)
        else:
            os.environ["SLMT_PAGED_DECODE"] = old
    mean_k = statistics.fmean(kus) if kus else None
    return {
        "kernel": name,
        "us_per_step": round(ms * 1e3, 2),
        "value": round(nbytes / (ms * 1e-3) / 1e9, 2),
        "pct_of_hbm_peak": round(100.0 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
        "kernel_us_mean": round(mean_k, 2) if mean_k else None,
        "frac": round(nbytes / (mean_k * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if mean_k else None,
        "note": "vector-ALU whole-row kernel (SLMT_PAGED_DECODE=valu), same steps and timing as the main line",
    }


def roofline(nbytes: int, achieved: float, w: Workload, kernel_us: float, step_us: float) -> dict:
    """The roofline object: achieved algorithmic GB/s against the HBM peak, the
    counter-measured HBM bytes, and three floors of a launch: HBM (bytes at
    8 TB/s), VALU issue (SQ_INSTS_VALU wave instructions x 4 cycles over 1024
    SIMDs at 2.1 GHz) and matrix cores (SQ_INSTS_MFMA x 16 cycles over 1024
    SIMDs at 2.1 GHz; both MFMA shapes used are 16-cycle instructions).
    `bound` names the largest floor; achieved/peak/frac stay in HBM GB/s, and
    `frac_of_binding_floor` is that floor over the kernel's time.  The counter
    figures come from the committed summaries; `counters` says whether they
    were measured on the kernel sources this run was built from."""
    hbm_floor = nbytes / (HBM_PEAK_GBS * 1e9) * 1e6
    valu = read_counter("valu_instructions_per_launch", w)
    mfma = read_counter("mfma_instructions_per_launch", w)
    clock = LOAD_CLOCK_GHZ * 1e9
    valu_floor = valu * VALU_CYCLES / SIMDS / clock * 1e6 if valu else None
    mfma_floor = mfma * MFMA_CYCLES / SIMDS / clock * 1e6 if mfma else None
    floors = {"hbm": hbm_floor, "valu": valu_floor or 0.0, "mfma": mfma_floor or 0.0}
    binding = max(floors, key=floors.get)
    sha = kernel_source_sha()
    return {
        "bound": binding,
        "achieved": round(achieved, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "frac_per_step": round(nbytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "frac_of_binding_floor": round(floors[binding] / kernel_us, 4),
        "traffic": read_traffic(w),
        "hbm_floor_us": round(hbm_floor, 2),
        "valu_instructions": valu,
        "valu_floor_us": round(valu_floor, 2) if valu_floor else None,
        "mfma_instructions": mfma,
        "mfma_floor_us": round(mfma_floor, 2) if mfma_floor else None,
        "binding": binding,
        "counters": {
            "kernel_source_sha": sha,
            "traffic_file": traffic_file(w).name,
            "traffic_measured_on_this_source": profile_stamp(traffic_file(w)) == sha,
            "instructions_file": COUNTERS_FILE.name,
            "instructions_measured_on_this_source": profile_stamp(COUNTERS_FILE) == sha,
        },
    }


def time_append(kd, cache, tables, lens, w: Workload, dev, calls: int = 200) -> dict:
    """Quantize-on-write of one new token per sequence (the decode step's
    append), timed over ``calls`` back-to-back launches.  It rewrites each
    sequence's last slot, so it runs after everything that reads the cache."""
    import torch

    g = torch.Generator(device=dev).manual_seed(7)
    k = torch.randn((w.B, w.KV, w.D), generator=g, device=dev).half()
    v = torch.randn((w.B, w.KV, w.D), generator=g, device=dev).half()
    last = (lens - 1).long()
    slots = (tables[torch.arange(w.B), last // BS].long() * BS + last % BS).to(dev)
    for _ in range(20):
        kd.kv_quantize_store(k, v, cache, slots, BS)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(calls):
        kd.kv_quantize_store(k, v, cache, slots, BS)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / calls
    return {"tokens": w.B, "us_per_call": round(us, 2),
            "note": "one new token per sequence, K/V fp16 in, packed slot + rulers out; launch-latency bound"}


if __name__ == "__main__":
    sys.exit(main())
