"""Write golden vectors for the reference's per-channel host quantizer.

Run in the development container only (the reference tree is not present where
the GPU tests run):

    python tests/golden/make_golden_quant.py /root/reference

It imports the reference's pure-torch quantizer functions --
``compute_scale_zero``, ``quantize_tensor`` and ``dequantize_tensor`` from
kernels/benchmark/benchmark.py:26-66 -- evaluates them on CPU tensors of
seeded and hand-built inputs, and stores inputs and outputs as data in
``tests/golden/per_channel_quant.npz``.  These are the only reference functions
whose exact fp16 evaluation (rounding after every torch op) no closed form or
known-answer test fixes completely; every other oracle function is pinned
without running reference code.

Nothing else reads the reference: the fixture file is plain data
(fp16 bit patterns as uint16, uint8 codes, float32 dequantized values).
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "per_channel_quant.npz"


def load_reference_quantizer(ref_root: Path):
    sys.path.insert(0, str(ref_root))
    spec = importlib.util.spec_from_file_location(
        "slm_turbo_reference_benchmark", ref_root / "kernels" / "benchmark" / "benchmark.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def edge_case_tensor() -> torch.Tensor:
    """[1, 16, 64] fp16 with hand-built channels covering the quantizer's edges."""
    g = torch.Generator().manual_seed(123)
    x = torch.randn(1, 16, 64, generator=g).half()
    x[0, :, 0] = 0.75                                  # constant channel -> scale 1, zero 0
    x[0, :, 1] = torch.linspace(-1, 1, 16).half()      # [-1, 1]: scale fp16(2/15), zero 8
    x[0, :, 2] = torch.linspace(0.5, 3.0, 16).half()   # all positive: zero clamps to 0
    x[0, :, 3] = torch.linspace(-3.0, -0.5, 16).half() # all negative: zero clamps to 15
    x[0, :, 4] = torch.arange(16).half() * 0.5 - 3.25  # values on half-steps (rounding ties)
    x[0, :, 5] = torch.tensor([1.0, -2.0 ** -11] * 8).half()  # max-min not exact in fp16
    x[0, :, 6] = torch.tensor([2.0 ** -24, 0.0] * 8).half()   # subnormal range: scale underflows
    x[0, :, 7] = torch.tensor([60000.0, -60000.0] * 8).half() # near fp16 max range (overflow path)
    x[0, :, 8] = torch.tensor([-0.0, 0.0] * 8).half()         # signed zeros only
    x[0, :, 9] = torch.linspace(-6.5, 6.5, 16).half()         # zero = -round(min/scale) tie cases
    x[0, :, 10] = torch.linspace(0.0, 1.0, 16).half()         # min exactly zero
    x[0, :, 11] = torch.tensor([5.0] * 15 + [5.0009765625]).half()  # one-ulp range
    return x


def make_cases(torch_gen_seed: int = 0):
    g = torch.Generator().manual_seed(torch_gen_seed)
    cases = {}
    cases["randn_kv2_s64_d64"] = torch.randn(2, 64, 64, generator=g).half()
    x = torch.randn(2, 48, 128, generator=g)
    ch = torch.randperm(2 * 128, generator=g)[:3]
    for c in ch.tolist():
        x[c // 128, :, c % 128] *= 8.0                 # 1% outlier channels x8
    cases["outlier_kv2_s48_d128"] = x.half()
    cases["randn_kv1_s40_d80"] = (torch.randn(1, 40, 80, generator=g) * 3.0).half()
    z = torch.randn(2, 32, 128, generator=g)
    chi2 = (torch.randn(3, 2, 32, 128, generator=g) ** 2).sum(0)
    cases["studentt3_kv2_s32_d128"] = (z / torch.sqrt(chi2 / 3.0)).half()   # Student-t, nu=3
    cases["edges_kv1_s16_d64"] = edge_case_tensor()
    return cases


def main(argv):
    ref_root = Path(argv[1] if len(argv) > 1 else "/root/reference")
    ref = load_reference_quantizer(ref_root)
    arrays = {}
    for name, x in make_cases().items():
        scale, zero = ref.compute_scale_zero(x)
        packed = ref.quantize_tensor(x, scale, zero)
        deq = ref.dequantize_tensor(packed, scale, zero)
        arrays[f"{name}__x"] = x.view(torch.int16).numpy().view(np.uint16)
        arrays[f"{name}__scale"] = scale.view(torch.int16).numpy().view(np.uint16)
        arrays[f"{name}__zero"] = zero.view(torch.int16).numpy().view(np.uint16)
        arrays[f"{name}__packed"] = packed.numpy().astype(np.uint8)
        arrays[f"{name}__deq"] = deq.numpy().astype(np.float32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main(sys.argv)
