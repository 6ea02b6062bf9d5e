"""Roofline classifier (reference roofline.py:5-32) with MI355X peaks.

Known answers are the published MI355X / MI300X figures; the NVIDIA path is
checked against the reference's own formula (sm_count x ops_per_sm x 1.5).
"""
import math

import pytest
import torch

import roofline as rl
from schema import Bottleneck, DeviceProfile, ProfileSnapshot


def _dev(sm_version, sm_count, bw, tc=True):
    return DeviceProfile(name="x", sm_version=sm_version, memory_bandwidth_gbps=bw, vram_mb=80000,
                         sm_count=sm_count, supports_tensor_cores=tc, supports_async_copy=True)


def test_mi355x_peaks_match_published_figures():
    p = rl.AMD_ARCHS[950]
    assert p.arch == "gfx950" and p.compute_units == 256
    assert math.isclose(p.fp32_vector_gflops / 1e3, 157.3, rel_tol=1e-3)      # 157.3 TFLOP/s FP32 vector
    assert math.isclose(p.fp16_mfma_gflops / 1e6, 2.5, rel_tol=0.01)          # ~2.5 PFLOP/s dense FP16
    assert math.isclose(p.valu_lane_ops_per_s, 256 * 64 * 2.4e9)              # 39.3 T lane-ops/s
    dev = rl.mi355x_profile()
    assert dev.sm_version == 950 and dev.memory_bandwidth_gbps == 8000.0 and not dev.is_small_gpu
    assert math.isclose(rl._estimate_peak_compute(dev), 256 * 256 * 2.4)      # Gop/s
    assert math.isclose(rl.ridge_point(dev), 256 * 256 * 2.4 / 8000.0)        # ~19.7 op/B


def test_mi300x_peaks():
    p = rl.AMD_ARCHS[942]
    assert math.isclose(p.fp32_vector_gflops / 1e3, 163.4, rel_tol=1e-3)
    assert math.isclose(p.fp16_mfma_gflops / 1e6, 1.3074, rel_tol=1e-3)


@pytest.mark.parametrize("smv,ops", [(75, 128), (80, 256), (86, 256), (89, 512), (90, 512), (61, 128)])
def test_nvidia_path_keeps_reference_formula(smv, ops):
    dev = _dev(smv, 40, 500.0)
    assert rl._estimate_peak_compute(dev) == 40 * ops * 1.5
    assert rl.arch_peaks(dev) is None


def test_profile_cu_count_scales_amd_peak():
    """A partitioned part (fewer CUs in its profile) is priced by its CUs."""
    assert math.isclose(rl._estimate_peak_compute(_dev(950, 32, 1000.0)), 32 * 256 * 2.4)


def test_classify_bottleneck_on_mi355x():
    dev = rl.mi355x_profile()
    ridge = rl.ridge_point(dev)
    snap = ProfileSnapshot(prefill_flops=ridge * 10 * 1e6, decode_flops=ridge * 0.5 * 1e6,
                           prefill_memory_bytes=1e6, decode_memory_bytes=1e6, model_params=1,
                           model_size_bytes=1.0, kv_cache_bytes_per_token=1)
    b = rl.classify_bottleneck(snap, dev)
    assert isinstance(b, Bottleneck) and b.prefill == "compute_bound" and b.decode == "memory_bound"
    # exactly at the ridge: not above it -> memory bound (strict inequality, as the reference)
    snap2 = snap.model_copy(update={"prefill_flops": ridge * 1e6})
    assert rl.classify_bottleneck(snap2, dev).prefill == "memory_bound"


def test_gfx950_no_longer_falls_through_to_default():
    """The reference's table would price gfx950 at 128 ops x 1.5 GHz."""
    dev = rl.mi355x_profile()
    fallback = 256 * 128 * 1.5
    assert rl._estimate_peak_compute(dev) == pytest.approx(fallback * 3.2)    # 2x ops/clk, 1.6x clock


def test_decode_bytes_and_flops_closed_form():
    lens = [1, 16, 17, 100]
    H, KV, D, bs = 32, 8, 128, 16
    got = rl.decode_attention_bytes(lens, H, KV, D, bs)
    blocks = 1 + 1 + 2 + 7
    assert got == sum(lens) * KV * (D + 8) + 4 * H * D * 6 + blocks * 4 + 4 * 4
    assert rl.decode_attention_bytes(lens, H, KV, D, bs, table_entry_bytes=8, out_bytes=2) == \
        sum(lens) * KV * (D + 8) + 4 * H * D * 4 + blocks * 8 + 16
    assert rl.decode_attention_flops(lens, H, D) == 4 * D * H * sum(lens)


def test_decode_bytes_match_the_benchmark_formula():
    """roofline's byte count and bench.py's (written separately) agree."""
    import bench

    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 8193, (64,), generator=g)
    assert rl.decode_attention_bytes(lens.tolist(), 32, 8, 128, 16) == bench.algorithmic_bytes(lens)


# Upper bound of measured / algorithmic HBM bytes per decode launch.  The
# batch-32, 4096-key workload at head_dim 64 splits each sequence over ~12 of
# 768 workgroups, and the (m, l, o) partials those write (3.4 MB, read back by
# the merge kernel) are outside the algorithmic bytes; its two KV-head groups
# also share the 64-byte line where a cache row's halves meet.
TRAFFIC_BOUND = {"headline": 1.1, "long-context": 1.1, "full-model-attention": 1.15}


@pytest.mark.parametrize("name", ["headline", "long-context", "full-model-attention"])
def test_benchmark_workloads_have_traffic_summaries(name):
    """Every bench.py workload has a committed counter summary whose HBM bytes
    per launch sit just above the algorithmic bytes of its seeded lengths."""
    import bench

    w = bench.WORKLOADS[name]
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(w.lo, w.hi + 1, (w.B,), generator=g)
    alg = bench.algorithmic_bytes(lens, w)
    assert alg == rl.decode_attention_bytes(lens.tolist(), w.H, w.KV, w.D, bench.BS)
    traffic = bench.read_traffic(w)
    assert traffic is not None and 1.0 <= traffic / alg < TRAFFIC_BOUND[name]


@pytest.mark.parametrize("name", ["headline", "long-context", "full-model-attention"])
def test_benchmark_roofline_bound_is_the_largest_floor(name):
    """bench.py's roofline object names the largest of its three floors as the
    bound and says whether its committed counters match the kernel sources."""
    import bench

    w = bench.WORKLOADS[name]
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(w.lo, w.hi + 1, (w.B,), generator=g)
    alg = bench.algorithmic_bytes(lens, w)
    r = bench.roofline(alg, 5000.0, w, kernel_us=60.0, step_us=64.0)
    floors = {"hbm": r["hbm_floor_us"], "valu": r["valu_floor_us"] or 0.0, "mfma": r["mfma_floor_us"] or 0.0}
    assert r["bound"] == r["binding"] == max(floors, key=floors.get)
    assert r["frac"] == pytest.approx(5000.0 / 8000.0)
    assert r["frac_per_step"] == pytest.approx(alg / 64e-6 / 8e12, rel=1e-3)
    assert r["frac_of_binding_floor"] == pytest.approx(floors[r["bound"]] / 60.0, rel=1e-3)
    sha = r["counters"]["kernel_source_sha"]
    assert len(sha) == 16 and int(sha, 16) >= 0 and sha == bench.kernel_source_sha()
    assert isinstance(r["counters"]["traffic_measured_on_this_source"], bool)


def test_decode_attention_intensity_is_below_the_ridge():
    """4-bit paged decode at G = 4 is memory bound on MI355X by the flop roof
    (~15 flop/B against a ~19.7 flop/B ridge)."""
    lens = [4096] * 64
    flops = rl.decode_attention_flops(lens, 32, 128)
    nbytes = rl.decode_attention_bytes(lens, 32, 8, 128)
    assert 14.0 < flops / nbytes < 16.0 < rl.ridge_point(rl.mi355x_profile())


def test_valu_roof_and_bound_selection():
    dev = rl.mi355x_profile()
    lens = [4096] * 64
    # vector-ALU kernel: priced at 218 lane-ops per (token, head) at D = 128 and
    # the 2.1 GHz sustained clock; at G = 4 it cannot reach the HBM roof
    r = rl.decode_attention_bounds(lens, 32, 8, 128, dev, kernel="valu")
    per = rl.decode_valu_ops_per_token_head(128, "valu")
    assert per == pytest.approx(218.0)
    assert math.isclose(r["valu_lane_ops"], sum(lens) * 32 * per)
    assert math.isclose(r["valu_s"], r["valu_lane_ops"] / (256 * 64 * 2.1e9))
    assert math.isclose(r["hbm_s"], r["bytes"] / 8e12)
    assert r["mfma_s"] == 0.0 and r["bound"] == "valu" and r["max_hbm_fraction"] < 0.8
    # doubling the query heads per KV head doubles VALU work, not bytes (much)
    r8 = rl.decode_attention_bounds(lens, 64, 8, 128, dev, kernel="valu")
    assert r8["valu_s"] == pytest.approx(2 * r["valu_s"])
    assert r8["max_hbm_fraction"] < r["max_hbm_fraction"]


def test_matrix_core_kernel_is_hbm_bound_at_group_4():
    """The matrix-core decode: 433 VALU wave instructions and 24 16-cycle
    products per 64-token tile and wave at D = 128 (the counters' figures)."""
    dev = rl.mi355x_profile()
    lens = [4096] * 64
    assert rl.decode_valu_ops_per_token_head(128) * 4 == pytest.approx(433.0)
    assert rl.decode_mfma_cycles_per_token_head(128) * 64 * 4 == 24 * 16
    r = rl.decode_attention_bounds(lens, 32, 8, 128, dev)
    assert r["bound"] == "hbm" and r["max_hbm_fraction"] == 1.0
    assert r["valu_s"] < r["hbm_s"] and r["mfma_s"] < 0.3 * r["hbm_s"]
    assert math.isclose(r["mfma_s"], r["mfma_cycles"] / 1024 / 2.1e9)


# ---------------------------------------------------------------- device probe
def test_device_probe_helpers():
    import profiler
    assert profiler.gfx_number("gfx950:sramecc+:xnack-") == 950
    assert profiler.gfx_number("gfx942") == 942
    assert profiler.gfx_number("") == 0
    assert profiler.bandwidth_of("gfx950:sramecc+:xnack-") == 8000.0
    assert profiler.bandwidth_of("gfx942") == 5300.0


def test_packed_kv_bytes_per_token():
    """Llama-1.1B-shaped (22 layers, 4 KV heads, head_dim 64): 72-byte packed
    slot per KV head and layer against 2 x 64 x 2 bytes of fp16 K and V."""
    import profiler
    assert profiler.kv_cache_bytes_per_token(4, 64, 22) == 22 * 4 * 72
    assert profiler.kv_cache_bytes_per_token(4, 64, 22, packed=False) == 2 * 4 * 64 * 22 * 2
    assert profiler.kv_cache_bytes_per_token(8, 128, 1) == 8 * 136     # one cache row of the decode


def test_device_info_without_a_gpu_raises():
    import torch
    import profiler
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="No CUDA device available"):
        profiler.device_info(0)


@pytest.mark.gpu
def test_device_info_on_the_gpu():
    import profiler
    d = profiler.device_info(0)
    assert d.sm_version == 950 and d.sm_count >= 256
    assert d.memory_bandwidth_gbps == 8000.0
    assert d.vram_mb > 250 * 1024
    assert d.supports_tensor_cores and d.supports_async_copy
