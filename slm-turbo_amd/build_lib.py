"""Build libslmturbo_hip.so for gfx950 (MI355X) from slm-turbo_amd/csrc.

    python slm-turbo_amd/build_lib.py            # build (parallel hipcc)
    python slm-turbo_amd/build_lib.py --verbose  # also print kernel resource usage

Each .hip translation unit is compiled to an object in slm-turbo_amd/_build/
and the objects are linked into slm-turbo_amd/kernels/libslmturbo_hip.so,
which kernels/kv_dequant.py loads through ctypes.  csrc/pyfast.c becomes the
CPython module kernels/_slmt_fast (gcc), a low-overhead binding of the two
per-layer entry points of that same library.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "kernels" / "libslmturbo_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=fast-honor-pragmas",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # keep hipcc from forming packed-fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core accumulators in ordinary VGPRs: the softmax reads and rescales
    # them every tile, which the AGPR form pays for with v_accvgpr copies
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd, verbose):
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "--hip-link" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)
    return out


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    extra = ["-Rpass-analysis=kernel-resource-usage"] if verbose else []

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        _run([cc, *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)], verbose)
        return obj

    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    build_fastcall(verbose)
    return LIB


def build_fastcall(verbose: bool = False) -> Path:
    """kernels/_slmt_fast<ext>: the METH_FASTCALL binding (host C, no device code)."""
    gcc = shutil.which("gcc") or shutil.which("cc")
    if gcc is None:
        raise RuntimeError("gcc not found (needed for the CPython binding kernels/_slmt_fast)")
    out = PKG / "kernels" / ("_slmt_fast" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    _run([gcc, "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{sysconfig.get_paths()['include']}",
          str(CSRC / "pyfast.c"), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    path = build(verbose=args.verbose, jobs=args.jobs)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
