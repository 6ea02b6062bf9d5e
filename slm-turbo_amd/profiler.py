"""ROCm device probe (reference profiler.py:7-34) and KV-cache capacity figures
for the packed slot (reference schema.py:27-38, adapters/vllm_adapter.py:561-589).

``device_info(device_id)`` fills the reference's ``DeviceProfile`` from the HIP
device properties instead of NVML:

* ``sm_version`` is the gfx number (950 for MI355X, 942 for MI300X), the key of
  the architecture tables in ``roofline``;
* ``sm_count`` is the number of compute units, ``vram_mb`` the HBM size;
* ``memory_bandwidth_gbps`` comes from ``get_bandwidth``: the published peak of
  a known architecture, else 2 x memory clock x bus width from amdsmi, else
  0.0.  The amdsmi figure is a lower bound: on MI355X it gives 4096 GB/s for
  HBM3E that moves 8000 GB/s (more than two transfers per reported clock);
* ``supports_tensor_cores`` means matrix cores (MFMA, gfx908 and later CDNA
  parts) and ``supports_async_copy`` direct global-to-LDS loads (gfx940 and
  later).

``kv_cache_bytes_per_token`` gives the cache bytes one token takes in every
layer: the packed slot (head_dim/2 bytes of K codes, head_dim/2 of V codes and
four fp16 rulers per KV head) or, for comparison, fp16 K and V.
"""
from __future__ import annotations

import re

from roofline import AMD_ARCHS
from schema import DeviceProfile


def gfx_number(arch_name: str) -> int:
    """The numeric part of a gfx target name: 'gfx950:sramecc+:xnack-' -> 950
    (a letter suffix such as gfx90a's is dropped: 90).  0 when there is none."""
    m = re.match(r"\s*gfx(\d+)", arch_name or "")
    return int(m.group(1)) if m else 0


def _amdsmi_bandwidth(device_id: int) -> float:
    """Memory clock x bus width from amdsmi, in GB/s (0.0 when unavailable)."""
    try:
        import amdsmi
    except Exception:
        return 0.0
    try:
        amdsmi.amdsmi_init()
        try:
            handle = amdsmi.amdsmi_get_processor_handles()[device_id]
            vram = amdsmi.amdsmi_get_gpu_vram_info(handle)
            width_bits = float(vram.get("vram_bit_width", 0) or 0)
            clk = amdsmi.amdsmi_get_clk_freq(handle, amdsmi.AmdSmiClkType.MEM)
            freqs = [f for f in clk.get("frequency", []) if f]
            if not width_bits or not freqs:
                return 0.0
            return 2.0 * max(freqs) * (width_bits / 8.0) / 1e9   # Hz x bytes -> GB/s
        finally:
            amdsmi.amdsmi_shut_down()
    except Exception:
        return 0.0


def bandwidth_of(arch_name: str, device_id: int = 0) -> float:
    """Theoretical peak HBM bandwidth in GB/s of a device with this gfx name."""
    peaks = AMD_ARCHS.get(gfx_number(arch_name))
    if peaks is not None:
        return peaks.hbm_gbps
    return _amdsmi_bandwidth(device_id)


def get_bandwidth(device_id: int) -> float:
    """Theoretical peak HBM bandwidth of GPU ``device_id`` in GB/s (reference
    profiler.py:25-34, which reads NVML clocks)."""
    import torch

    props = torch.cuda.get_device_properties(device_id)
    return bandwidth_of(getattr(props, "gcnArchName", ""), device_id)


def device_info(device_id: int = 0) -> DeviceProfile:
    """DeviceProfile of GPU ``device_id`` (reference profiler.py:7-22)."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("No CUDA device available")
    props = torch.cuda.get_device_properties(device_id)
    arch = getattr(props, "gcnArchName", "")
    gfx = gfx_number(arch)
    return DeviceProfile(
        name=props.name,
        sm_version=gfx,
        memory_bandwidth_gbps=bandwidth_of(arch, device_id),
        vram_mb=props.total_memory // 1024 // 1024,
        sm_count=props.multi_processor_count,
        supports_tensor_cores=908 <= gfx < 1000,
        supports_async_copy=940 <= gfx < 1000,
    )


def kv_cache_bytes_per_token(num_kv_heads: int, head_dim: int, num_layers: int, packed: bool = True,
                             dtype_bytes: int = 2) -> int:
    """Cache bytes one token takes over all layers: the packed 4-bit slot
    (head_dim + 8 bytes per KV head: K and V codes plus fp16 k_min, k_step,
    v_min, v_step), or fp16 K and V (reference schema.py:27-38) when not
    packed."""
    if packed:
        return num_layers * num_kv_heads * (head_dim + 8)
    return 2 * num_kv_heads * head_dim * num_layers * dtype_bytes
