"""Data types of the roofline classifier (reference schema.py:41-53, 92-106).

Only the three types the roofline needs are defined here, with the
reference's field names and meanings:

* ``DeviceProfile`` -- one accelerator.  ``sm_version`` is the architecture
  key: the CUDA compute capability for NVIDIA parts (75, 80, 86, 89, 90) and
  the gfx number for AMD Instinct parts (942 = MI300X, 950 = MI355X);
  ``sm_count`` is SMs or compute units.
* ``ProfileSnapshot`` -- flop and byte counts of a model's prefill and
  decode phases.
* ``Bottleneck`` -- the verdict per phase.
"""
from __future__ import annotations

from typing import Literal

from pydantic import BaseModel


class DeviceProfile(BaseModel):
    name: str
    sm_version: int
    memory_bandwidth_gbps: float
    vram_mb: int
    sm_count: int
    supports_tensor_cores: bool
    supports_async_copy: bool

    @property
    def is_small_gpu(self) -> bool:
        """Under 6 GB and without matrix units (reference schema.py:50-53)."""
        return self.vram_mb < 6000 and not self.supports_tensor_cores


class ProfileSnapshot(BaseModel):
    prefill_flops: float
    decode_flops: float                 # per decode token
    prefill_memory_bytes: float
    decode_memory_bytes: float
    model_params: int
    model_size_bytes: float
    kv_cache_bytes_per_token: int


class Bottleneck(BaseModel):
    prefill: Literal["memory_bound", "compute_bound"]
    decode: Literal["memory_bound", "compute_bound"]
