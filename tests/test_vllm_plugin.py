"""vLLM plugin registration against a stub ``vllm`` package (CPU).

vLLM is not installed here, so a minimal stand-in of the five vLLM names the
adapter binds to is written to a temporary directory:
``vllm.model_executor.layers.attention.attention.Attention``,
``vllm.v1.kv_cache_interface.TQFullAttentionSpec``,
``vllm.v1.attention.backends.triton_attn.{TritonAttentionBackend,TritonAttentionImpl}``
and ``vllm.v1.attention.backends.registry.{AttentionBackendEnum,register_backend}``
(the names the reference's adapters/vllm_adapter.py:112-113,151-152 imports).
A child process with that directory on its path then imports the adapter the
way vLLM's plugin loader does (through the ``vllm.general_plugins`` entry point
declared in pyproject.toml, reference pyproject.toml:48-49) and checks what
``register_plugin()`` did.  A child process keeps the stub out of this test
session's ``sys.modules``.
"""
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

STUB_FILES = {
    "vllm/__init__.py": "STUB = True\n",
    "vllm/model_executor/__init__.py": "",
    "vllm/model_executor/layers/__init__.py": "",
    "vllm/model_executor/layers/attention/__init__.py": "",
    "vllm/model_executor/layers/attention/attention.py": '''
        from dataclasses import dataclass

        @dataclass
        class FullAttentionSpec:
            block_size: int
            num_kv_heads: int
            head_size: int
            dtype: object
            kv_quant_mode: str = "none"

        class Attention:
            def __init__(self, backend, num_kv_heads=8, head_size=128, block_size=16):
                self.attn_backend = backend
                self.num_kv_heads = num_kv_heads
                self.head_size = head_size
                self.head_size_v = head_size
                self.block_size = block_size

            def get_kv_cache_spec(self, vllm_config):
                return FullAttentionSpec(block_size=self.block_size, num_kv_heads=self.num_kv_heads,
                                         head_size=self.head_size, dtype="float16")
    ''',
    "vllm/v1/__init__.py": "",
    "vllm/v1/kv_cache_interface.py": '''
        from dataclasses import dataclass

        @dataclass
        class TQFullAttentionSpec:
            block_size: int
            num_kv_heads: int
            head_size: int
            head_size_v: int
            dtype: object
            kv_quant_mode: str
            tq_slot_size: int

            @property
            def page_size_bytes(self):
                return self.block_size * self.num_kv_heads * self.tq_slot_size
    ''',
    "vllm/v1/attention/__init__.py": "",
    "vllm/v1/attention/backends/__init__.py": "",
    "vllm/v1/attention/backends/triton_attn.py": '''
        class TritonAttentionImpl:
            def __init__(self, num_heads, head_size, scale, num_kv_heads=None, *args, **kwargs):
                self.num_heads = num_heads
                self.head_size = head_size
                self.scale = scale
                self.num_kv_heads = num_kv_heads or num_heads

        class TritonAttentionBackend:
            @staticmethod
            def get_name():
                return "TRITON_ATTN"

            @staticmethod
            def get_impl_cls():
                return TritonAttentionImpl
    ''',
    "vllm/v1/attention/backends/registry.py": '''
        import enum

        class AttentionBackendEnum(enum.Enum):
            FLASH_ATTN = "flash"
            TRITON_ATTN = "triton"
            CUSTOM = "custom"

        REGISTERED = []

        def register_backend(enum_member, class_path):
            REGISTERED.append((enum_member, class_path))
    ''',
}

CHILD = r'''
import importlib, sys
import tomli
import torch

# 1. the entry point vLLM's plugin loader would run, from pyproject.toml
with open(sys.argv[1], "rb") as f:
    eps = tomli.load(f)["project"]["entry-points"]["vllm.general_plugins"]
assert list(eps) == ["slm-turbo"], eps
mod_name, fn_name = eps["slm-turbo"].split(":")
assert (mod_name, fn_name) == ("adapters.vllm_adapter", "register_plugin")
plugin = getattr(importlib.import_module(mod_name), fn_name)

import adapters.vllm_adapter as va
assert plugin is va.register_plugin
assert va.VLLM_AVAILABLE, va.VLLM_IMPORT_ERROR
from vllm.v1.attention.backends import registry
from vllm.v1.attention.backends.triton_attn import TritonAttentionBackend, TritonAttentionImpl
from vllm.model_executor.layers.attention.attention import Attention
from vllm.v1.kv_cache_interface import TQFullAttentionSpec

# 2. registration: CUSTOM -> this module's backend class, once
assert registry.REGISTERED == [], registry.REGISTERED
plugin()
plugin()                                            # idempotent
assert len(registry.REGISTERED) == 1, registry.REGISTERED
member, path = registry.REGISTERED[0]
assert member is registry.AttentionBackendEnum.CUSTOM
assert path == "adapters.vllm_adapter.QuantizedKVAttentionBackend", path
m, c = path.rsplit(".", 1)
Backend = getattr(importlib.import_module(m), c)
assert Backend is va.QuantizedKVAttentionBackend
assert issubclass(Backend, TritonAttentionBackend)
assert Backend.get_name() == "CUSTOM" and Backend.__name__ == "QuantizedKVAttentionBackend"
assert Backend.get_kv_cache_shape(10, 16, 8, 128) == (10, 16, 8, 136)
try:
    Backend.get_kv_cache_stride_order()
    raise AssertionError("stride order must raise NotImplementedError")
except NotImplementedError:
    pass
Impl = Backend.get_impl_cls()
assert Impl is va.QuantizedKVAttentionImpl and Impl.__name__ == "QuantizedKVAttentionImpl"
assert issubclass(Impl, TritonAttentionImpl) and issubclass(Impl, va.PackedKVAttentionMixin)
# the mixin's forward and cache update win over the Triton impl's
assert Impl.forward is va.PackedKVAttentionMixin.forward
assert Impl.do_kv_cache_update is va.PackedKVAttentionMixin.do_kv_cache_update

# 3. the cache spec patch: packed uint8 slots for CUSTOM layers only
spec = Attention(Backend, num_kv_heads=8, head_size=128).get_kv_cache_spec(None)
assert isinstance(spec, TQFullAttentionSpec), spec
assert spec.dtype is torch.uint8 and spec.tq_slot_size == 136 and spec.block_size == 16
assert spec.num_kv_heads == 8 and spec.head_size == 128 and spec.head_size_v == 128
assert spec.page_size_bytes == 16 * 8 * 136
spec64 = Attention(Backend, num_kv_heads=4, head_size=64, block_size=32).get_kv_cache_spec(None)
assert spec64.tq_slot_size == 72 and spec64.block_size == 32
other = Attention(TritonAttentionBackend).get_kv_cache_spec(None)
assert not isinstance(other, TQFullAttentionSpec) and other.dtype == "float16"
assert va._patch_attention_layer_spec() is True     # idempotent: not wrapped twice
spec2 = Attention(Backend).get_kv_cache_spec(None)
assert isinstance(spec2, TQFullAttentionSpec)

# 4. the impl fails at construction when the kernel library is missing
try:
    Impl(num_heads=32, head_size=128, scale=128 ** -0.5, num_kv_heads=8)
    raise AssertionError("construction must fail without the HIP library")
except RuntimeError as e:
    assert "not found" in str(e), e
st = va.backend_status()
assert st["vllm_available"] and st["backend_registered"] and st["kernels"] is False
print("PLUGIN_OK")
'''


def _write_stub(root: Path) -> None:
    for rel, text in STUB_FILES.items():
        p = root / rel
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_text(textwrap.dedent(text))


def test_pyproject_maps_the_reference_import_names():
    """The package mapping setuptools builds from: `adapters` and `kernels`
    (and the top-level modules) resolve to slm-turbo_amd/ and ship the HIP
    library (this image's setuptools predates pyproject support, so the
    table is read with tomli and checked against the tree)."""
    import tomli

    with open(ROOT / "pyproject.toml", "rb") as f:
        cfg = tomli.load(f)
    assert cfg["build-system"]["build-backend"] == "setuptools.build_meta"
    st = cfg["tool"]["setuptools"]
    src = ROOT / st["package-dir"][""]
    assert src == ROOT / "slm-turbo_amd"
    for pkg in st["packages"]:
        assert (src / pkg / "__init__.py").is_file(), pkg
    assert set(st["packages"]) == {"adapters", "kernels"}
    for mod in st["py-modules"]:
        assert (src / f"{mod}.py").is_file(), mod
    assert st["package-data"]["kernels"] == ["libslmturbo_hip.so", "_slmt_fast*.so"]
    eps = cfg["project"]["entry-points"]["vllm.general_plugins"]
    assert eps == {"slm-turbo": "adapters.vllm_adapter:register_plugin"}


def test_register_plugin_with_a_stub_vllm(tmp_path):
    _write_stub(tmp_path / "stub")
    env = dict(os.environ)
    # the installed layout: the stub vllm, then the package directory
    env["PYTHONPATH"] = os.pathsep.join([str(tmp_path / "stub"), str(ROOT / "slm-turbo_amd")])
    env["SLMT_LIB"] = str(tmp_path / "missing" / "libslmturbo_hip.so")
    res = subprocess.run([sys.executable, "-c", CHILD, str(ROOT / "pyproject.toml")], env=env,
                         capture_output=True, text=True, timeout=300, cwd=tmp_path)
    assert res.returncode == 0 and "PLUGIN_OK" in res.stdout, res.stdout + res.stderr


if __name__ == "__main__":
    sys.exit(pytest.main([__file__, "-q"]))
