"""C ABI of libslmturbo_hip.so without a GPU: the library loads, exports every
function include/slmturbo.h declares with the ctypes signatures the binding
uses, and argument validation (which runs on the host before any HIP call)
rejects bad requests with the reference's wording.  No compute call is made.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from kernels import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "slmturbo.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(slmt_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _native.library_path().exists():
        pytest.fail(f"{_native.library_path()} is not built: run `python slm-turbo_amd/build_lib.py`")
    return _native.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = _declared()
    assert {"slmt_decode_paged", "slmt_decode_paged_batched"} <= set(names) and len(names) >= 10
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (slmt_[a-z0-9_]+)", out))
    assert set(names) <= exported, f"declared but not exported: {set(names) - exported}"
    assert set(names) == set(_native.SIGNATURES), "ctypes binding and header disagree"
    for n in names:
        assert getattr(lib, n) is not None


def test_argument_counts_match_the_header(lib):
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, args) in _native.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), name


def test_version_and_workspace_sizes(lib):
    import torch

    assert lib.slmt_abi_version() == _native.ABI_VERSION
    assert lib.slmt_attention_workspace_bytes(1, 32, 8, 96) == -1
    assert b"head_dim must be 64/80/128" in lib.slmt_last_error()
    assert lib.slmt_attention_workspace_bytes(1, 32, 6, 128) == -1
    assert b"workspace: invalid sizes" in lib.slmt_last_error()
    if not torch.cuda.is_available():
        # the split-partial region is sized by the device's CU count
        assert lib.slmt_attention_workspace_bytes(64, 32, 8, 128) == -1
        assert b"could not query the device" in lib.slmt_last_error()
        return
    counters = 1 << 20
    a = lib.slmt_attention_workspace_bytes(64, 32, 8, 128)
    b = lib.slmt_attention_workspace_bytes(128, 32, 8, 128)
    assert counters * 4 <= lib.slmt_attention_workspace_bytes(0, 32, 8, 128) <= a <= b


def _paged_args(**kw):
    a = dict(q=16, qs=4096, qh=128, cache=16, nb=4, bs=16, bt=16, bits=32, bts=4, sl=None, fixed=5,
             B=1, H=32, KV=8, D=128, out=16, od=_native.OUT_F32, os_=4096, oh=128, ws=None, wsb=0)
    a.update(kw)
    return [a["q"], a["qs"], a["qh"], a["cache"], a["nb"], a["bs"], a["bt"], a["bits"], a["bts"], a["sl"],
            a["fixed"], a["B"], a["H"], a["KV"], a["D"], a["out"], a["od"], a["os_"], a["oh"], a["ws"],
            a["wsb"], None]


def _paged(lib, **kw):
    return lib.slmt_decode_paged_batched(*_paged_args(**kw))


PAGED_VALIDATION = [
    (dict(D=96), b"head_dim must be 64/80/128"),
    (dict(KV=6), b"H not divisible by num_kv_heads"),
    (dict(bs=0), b"block_size must be positive"),
    (dict(bits=16), b"block table must be int32 or int64"),
    (dict(od=7), b"out dtype must be fp32 or fp16"),
    (dict(B=-1), b"num_seqs must be >= 0"),
    (dict(fixed=-1), b"seq_len must be >= 0"),
    (dict(q=None), b"null pointer argument"),
    (dict(q=8), b"q must be 16-byte aligned"),
    (dict(qh=100), b"q must be 16-byte aligned"),
]


@pytest.mark.parametrize("kw,msg", PAGED_VALIDATION)
def test_paged_decode_validation(lib, kw, msg):
    assert _paged(lib, **kw) == _native.ERR_INVALID
    assert msg in lib.slmt_last_error()


def test_empty_batch_is_a_no_op(lib):
    assert _paged(lib, B=0, q=None, out=None) == _native.OK


def test_single_request_entry_validates_like_the_reference(lib):
    """slmt_decode_paged (one request, int64 block row) shares the batched checks."""
    f = ctypes.c_void_p(16)
    assert lib.slmt_decode_paged(f, f, 4, 16, f, -1, 32, 8, 128, f, None, 0, None) == _native.ERR_INVALID
    assert b"seq_len must be >= 0" in lib.slmt_last_error()
    assert lib.slmt_decode_paged(f, f, 4, 16, f, 5, 32, 8, 80 + 16, f, None, 0, None) == _native.ERR_INVALID
    assert b"head_dim must be 64/80/128" in lib.slmt_last_error()
    assert lib.slmt_decode_paged(f, f, 4, 16, f, 5, 30, 8, 128, f, None, 0, None) == _native.ERR_INVALID
    assert b"H not divisible by num_kv_heads" in lib.slmt_last_error()


def test_store_and_quantizer_validation(lib):
    assert lib.slmt_quantize_store(16, 1024, 16, 1024, 16, 4, 16, 16, 1, 8, 96, None) == _native.ERR_INVALID
    assert b"store: head_dim must be 64/80/128" in lib.slmt_last_error()
    assert lib.slmt_quantize_store(None, 1024, None, 1024, None, 4, 16, None, 0, 8, 128, None) == _native.OK
    assert lib.slmt_quantize_store(16, 100, 16, 1024, 16, 4, 16, 16, 1, 8, 128, None) == _native.ERR_INVALID
    assert b"token stride smaller than KV*D" in lib.slmt_last_error()
    assert lib.slmt_quantize_per_channel(16, 2, 0, 64, 16, 16, 16, None) == _native.ERR_INVALID
    assert b"need KV >= 0 and S >= 1" in lib.slmt_last_error()


def test_fixed_ruler_quantizer_validation(lib):
    q = lib.slmt_quantize_with_rulers
    assert q(16, 4096, 64, 2, 8, 96, 16, 16, 16, 256, 32, None) == _native.ERR_INVALID
    assert b"quantize_tensor: head_dim must be 64/80/128" in lib.slmt_last_error()
    assert q(None, 0, 0, 2, 0, 64, None, None, None, 0, 0, None) == _native.OK      # nothing to do
    assert q(16, 4096, 64, 2, 8, 64, None, 16, 16, 256, 32, None) == _native.ERR_INVALID
    assert b"null pointer" in lib.slmt_last_error()
    assert q(16, 4096, 63, 2, 8, 64, 16, 16, 16, 256, 32, None) == _native.ERR_INVALID
    assert b"4-byte aligned" in lib.slmt_last_error()
    assert q(16, 4096, 32, 2, 8, 64, 16, 16, 16, 256, 32, None) == _native.ERR_INVALID
    assert b"strides smaller than a row" in lib.slmt_last_error()
    assert q(16, 4096, 64, 2, 8, 64, 16, 16, 16, 256, 16, None) == _native.ERR_INVALID
    assert b"strides smaller than a row" in lib.slmt_last_error()


def test_contiguous_entry_points_validate_block_sizes(lib):
    f = ctypes.c_void_p(16)
    assert lib.slmt_decode_per_token(f, f, f, f, f, f, f, 8, 2, 2, 4, 64, 48, f, None, 0, None) \
        == _native.ERR_INVALID
    assert b"BLOCK_N must be 32 or 64" in lib.slmt_last_error()
    assert lib.slmt_decode_per_channel(f, f, f, f, f, f, f, 8, 2, 2, 4, 64, 16, 1, f, None, 0, None) \
        == _native.ERR_INVALID
    assert b"kv_dequant_decode: BLOCK_N must be 32 or 64" in lib.slmt_last_error()


def _fast(lib):
    f = _native.fast()
    if f is None:
        pytest.fail("kernels/_slmt_fast is not built: run `python slm-turbo_amd/build_lib.py`")
    return f


@pytest.mark.parametrize("kw,msg", PAGED_VALIDATION)
def test_fastcall_decode_reaches_the_same_checks(lib, kw, msg):
    """The METH_FASTCALL binding passes all 22 arguments through unchanged:
    each bad one is rejected by the library with the same status and message
    as through ctypes (None is the null pointer 0 there)."""
    f = _fast(lib)
    args = [0 if v is None else v for v in _paged_args(**kw)]
    assert f.decode_paged_batched(*args) == _native.ERR_INVALID
    assert msg in lib.slmt_last_error()
    assert f.decode_paged_batched(*[0 if v is None else v for v in _paged_args(B=0, q=None, out=None)]) == _native.OK


def test_fastcall_store_reaches_the_same_checks(lib):
    f = _fast(lib)
    assert f.quantize_store(16, 1024, 16, 1024, 16, 4, 16, 16, 1, 8, 96, 0) == _native.ERR_INVALID
    assert b"store: head_dim must be 64/80/128" in lib.slmt_last_error()
    assert f.quantize_store(16, 100, 16, 1024, 16, 4, 16, 16, 1, 8, 128, 0) == _native.ERR_INVALID
    assert b"token stride smaller than KV*D" in lib.slmt_last_error()
    assert f.quantize_store(0, 1024, 0, 1024, 0, 4, 16, 0, 0, 8, 128, 0) == _native.OK
    with pytest.raises(TypeError):
        f.quantize_store(1, 2, 3)
    with pytest.raises(TypeError):
        f.quantize_store("x", 1024, 16, 1024, 16, 4, 16, 16, 1, 8, 128, 0)
    with pytest.raises(TypeError):
        f.decode_paged_batched(*range(21))
