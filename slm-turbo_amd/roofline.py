"""Roofline classification with architecture-keyed peaks (reference roofline.py:5-32).

``_estimate_peak_compute(device)`` and ``classify_bottleneck(snapshot,
device)`` keep the reference's signatures and units: peak compute in
Gop/s, bandwidth in GB/s, so the ridge point is in ops per byte.

The reference prices every device as ``sm_count * ops_per_sm * 1.5 GHz``
with an NVIDIA-only table, so an AMD part falls through to 128 ops per
clock.  Here AMD Instinct parts are keyed by their gfx number and priced at
their real engine clock:

=========  =====  =========  ==========  ===============  ==================
arch       CUs    clock GHz  HBM GB/s    FP32 vector TF   FP16 MFMA dense TF
=========  =====  =========  ==========  ===============  ==================
gfx950     256    2.4        8000        157.3            2516.6
gfx942     304    2.1        5300        163.4            1307.4
=========  =====  =========  ==========  ===============  ==================

FP32 vector throughput is 256 flops per CU per clock (4 SIMDs x 16 lanes x
FMA x packed pairs); ``_estimate_peak_compute`` reports it, which is the
roof of code that does not use matrix cores (the decode path here).

The 4-bit decode attention path is priced by two more roofs: the VALU
*instruction* rate (16 lanes per SIMD per clock whatever an instruction's
width, ``valu_lane_ops_per_s``) and the matrix-core issue rate (16 cycles per
16x16x64 int8 or 16x16x32 fp16 product).  ``decode_attention_bounds`` prices
both decode kernels with their per-token instruction mix.
"""
from __future__ import annotations

from dataclasses import dataclass

from schema import Bottleneck, DeviceProfile, ProfileSnapshot


@dataclass(frozen=True)
class ArchPeaks:
    """Published dense peaks of one AMD Instinct architecture."""
    arch: str
    compute_units: int
    clock_ghz: float
    hbm_gbps: float
    fp32_flops_per_cu_clk: int         # vector (non-matrix) FP32
    fp16_mfma_flops_per_cu_clk: int    # dense matrix-core FP16/BF16
    lds_bytes_per_cu: int
    sustained_clock_ghz: float         # shader clock measured under a full decode load

    @property
    def fp32_vector_gflops(self) -> float:
        return self.compute_units * self.fp32_flops_per_cu_clk * self.clock_ghz

    @property
    def fp16_mfma_gflops(self) -> float:
        return self.compute_units * self.fp16_mfma_flops_per_cu_clk * self.clock_ghz

    @property
    def valu_lane_ops_per_s(self) -> float:
        """VALU lane-instructions per second: 4 SIMDs x 16 lanes per CU per clock."""
        return self.compute_units * 64 * self.clock_ghz * 1e9


AMD_ARCHS = {
    950: ArchPeaks("gfx950", 256, 2.4, 8000.0, 256, 4096, 160 * 1024, 2.1),
    942: ArchPeaks("gfx942", 304, 2.1, 5300.0, 256, 2048, 64 * 1024, 2.1),
}

# NVIDIA: FP32 ops per SM per clock by compute capability, priced at the
# reference's nominal 1.5 GHz (it has no per-part clock).
_NVIDIA_OPS_PER_SM = {75: 128, 80: 256, 86: 256, 89: 512, 90: 512}
_NVIDIA_CLOCK_GHZ = 1.5
_DEFAULT_OPS_PER_SM = 128


def arch_peaks(device: DeviceProfile) -> ArchPeaks | None:
    """Peaks of an AMD Instinct device (keyed by gfx number), else None."""
    return AMD_ARCHS.get(device.sm_version)


def _estimate_peak_compute(device: DeviceProfile) -> float:
    """Peak non-matrix compute in Gop/s (reference roofline.py:5-17).

    AMD parts: measured CU count of the profile x 256 FP32 flops per CU per
    clock x the architecture's clock.  Others: the reference's table.
    """
    peaks = arch_peaks(device)
    if peaks is not None:
        return device.sm_count * peaks.fp32_flops_per_cu_clk * peaks.clock_ghz
    ops = _NVIDIA_OPS_PER_SM.get(device.sm_version, _DEFAULT_OPS_PER_SM)
    return device.sm_count * ops * _NVIDIA_CLOCK_GHZ


def ridge_point(device: DeviceProfile) -> float:
    """Ops per byte where the memory and compute roofs meet."""
    return _estimate_peak_compute(device) / device.memory_bandwidth_gbps


def classify_bottleneck(snapshot: ProfileSnapshot, device: DeviceProfile) -> Bottleneck:
    """Memory- or compute-bound per phase (reference roofline.py:20-32)."""
    ridge = ridge_point(device)
    prefill_intensity = snapshot.prefill_flops / snapshot.prefill_memory_bytes
    decode_intensity = snapshot.decode_flops / snapshot.decode_memory_bytes
    return Bottleneck(
        prefill="compute_bound" if prefill_intensity > ridge else "memory_bound",
        decode="compute_bound" if decode_intensity > ridge else "memory_bound",
    )


def mi355x_profile(vram_mb: int = 288 * 1024) -> DeviceProfile:
    """DeviceProfile of one MI355X (gfx950) at its published peaks."""
    p = AMD_ARCHS[950]
    return DeviceProfile(name="AMD Instinct MI355X", sm_version=950, memory_bandwidth_gbps=p.hbm_gbps,
                         vram_mb=vram_mb, sm_count=p.compute_units, supports_tensor_cores=True,
                         supports_async_copy=True)


# ----------------------------------------------------------------------------
# 4-bit paged decode attention: both roofs
# ----------------------------------------------------------------------------
def decode_attention_bytes(seq_lens, num_heads: int, num_kv_heads: int, head_dim: int, block_size: int = 16,
                           table_entry_bytes: int = 4, out_bytes: int = 4) -> int:
    """Algorithmic HBM bytes of one batched paged decode step: packed K+V
    and rulers of every token, q (fp16), out, the block-table entries read
    and the lengths."""
    lens = [int(x) for x in seq_lens]
    B = len(lens)
    kv = sum(lens) * num_kv_heads * (head_dim + 8)
    blocks = sum((L + block_size - 1) // block_size for L in lens)
    return kv + B * num_heads * head_dim * (2 + out_bytes) + blocks * table_entry_bytes + B * 4


def decode_attention_flops(seq_lens, num_heads: int, head_dim: int) -> int:
    """QK and PV multiply-adds, 2 flops each: 4 * D * H * sum(L)."""
    return 4 * head_dim * num_heads * sum(int(x) for x in seq_lens)


# Per (token, query head) cost of the two whole-row decode kernels, from their
# compiled main loops and checked against rocprofv3 SQ_INSTS_VALU / SQ_INSTS_MFMA
# (a wave handles 4 query heads of one KV head, 64 tokens per tile, whatever
# the group size):
# * matrix-core kernel (csrc/attention_mfma.hip): per 64-token tile and wave,
#   VALU = 1.125 D (QK nibble unpack 6 per i8 MFMA, PV operand build 24 per 32
#   tokens x 32 V bytes) + 289 (limb combine, softmax and weights, addressing),
#   i.e. 433 wave instructions at D = 128 (measured 433) and 361 at D = 64
#   (measured 378); matrix cores: 4 D/64 v_mfma_i32_16x16x64_i8 for QK and
#   8 D/64 v_mfma_f32_16x16x32_f16 for PV, 16 cycles each;
# * vector-ALU kernel (csrc/attention_rows.hip): QK and PV on v_dot2c_f32_f16
#   (D/2 lane-ops each per (token, head)), nibble unpack 5 D/32 for QK and D/8
#   for PV, ~54 for the score, softmax and weights: 218 lane-ops at D = 128
#   (measured 13.7 wave instructions per (token, KV head)).
MFMA_CYCLES = 16


def decode_valu_ops_per_token_head(head_dim: int, kernel: str = "mfma") -> float:
    """VALU lane-operations per (token, query head) of the decode kernel."""
    if kernel == "mfma":
        return (1.125 * head_dim + 289.0) * 64 / (64 * 4)
    return 1.28125 * head_dim + 54.0


def decode_mfma_cycles_per_token_head(head_dim: int, kernel: str = "mfma") -> float:
    """Matrix-core cycles (on one SIMD) per (token, query head) of the decode."""
    if kernel != "mfma":
        return 0.0
    per_tile = (4 * head_dim // 64 + 8 * head_dim // 64) * MFMA_CYCLES
    return per_tile / (64 * 4)


def decode_attention_bounds(seq_lens, num_heads: int, num_kv_heads: int, head_dim: int,
                            device: DeviceProfile, block_size: int = 16, kernel: str = "mfma") -> dict:
    """Lower bounds on one decode step's time (seconds) from HBM bandwidth,
    the VALU instruction rate and the matrix-core issue rate, and which one
    binds.  AMD parts are priced at their sustained clock under this load
    (2.1 GHz measured on gfx950, below the 2.4 GHz peak clock)."""
    peaks = arch_peaks(device)
    nbytes = decode_attention_bytes(seq_lens, num_heads, num_kv_heads, head_dim, block_size)
    t_hbm = nbytes / (device.memory_bandwidth_gbps * 1e9)
    tokens = sum(int(x) for x in seq_lens)
    lane_ops = tokens * num_heads * decode_valu_ops_per_token_head(head_dim, kernel)
    mfma_cycles = tokens * num_heads * decode_mfma_cycles_per_token_head(head_dim, kernel)
    if peaks is not None:
        clock = peaks.sustained_clock_ghz * 1e9
        rate = device.sm_count * 64 * clock
        t_mfma = mfma_cycles / (device.sm_count * 4) / clock
    else:
        rate = _estimate_peak_compute(device) * 1e9 / 2      # FMA lanes of the reference's table
        t_mfma = 0.0
    t_valu = lane_ops / rate
    times = {"hbm": t_hbm, "valu": t_valu, "mfma": t_mfma}
    bound = max(times, key=times.get)
    return {"bytes": nbytes, "hbm_s": t_hbm, "valu_lane_ops": lane_ops, "valu_s": t_valu,
            "mfma_cycles": mfma_cycles, "mfma_s": t_mfma, "bound": bound,
            "max_hbm_fraction": min(1.0, t_hbm / times[bound]) if times[bound] > 0 else 1.0}
