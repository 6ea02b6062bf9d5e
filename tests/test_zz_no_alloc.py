"""GPU: slmt_decode_paged_batched_noalloc through the C ABI against
slmt_decode_paged_batched (same kernels, caller-owned workspace).

Two calls in a row on each shape, the second with a smaller batch, so the
second call runs on the static scratch the first call left behind.  Shapes
cover the whole-row kernel (no arrival counters) and the per-wave fallback,
whose last-arriver merges count pieces in the scratch.  Outputs must be
bit-identical to the workspace entry point's and within 2e-3 / 1e-2 of the
float64 oracle.  Invalid arguments and unsupported sizes fail with the
workspace entry point's status and message; a request whose workspace would
exceed the scratch fails with SLMT_ERR_UNSUPPORTED, which on a 256-CU MI355X
no supported head layout reaches (the scratch holds the largest workspace).
"""
import ctypes

import numpy as np
import pytest
import torch

from common import assert_close, make_paged_case, paged_reference
from kernels import _native

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _call(lib, case, noalloc):
    q = case.q.to(DEV)
    cache = torch.from_numpy(case.kv_cache).to(DEV)
    tables = case.block_tables.to(DEV)
    lens = case.seq_lens.to(DEV)
    B, H, D = q.shape
    out = torch.full((B, H, D), float("nan"), dtype=torch.float32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    args = [ctypes.c_void_p(q.data_ptr()), q.stride(0), q.stride(1), ctypes.c_void_p(cache.data_ptr()),
            cache.size(0), case.block_size, ctypes.c_void_p(tables.data_ptr()), 32, tables.stride(0),
            ctypes.c_void_p(lens.data_ptr()), 0, B, H, case.num_kv_heads, D, ctypes.c_void_p(out.data_ptr()),
            _native.OUT_F32, out.stride(0), out.stride(1)]
    if noalloc:
        rc = lib.slmt_decode_paged_batched_noalloc(*args, stream)
    else:
        nbytes = lib.slmt_attention_workspace_bytes(B, H, case.num_kv_heads, D)
        assert nbytes > 0, _native.last_error(lib)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        rc = lib.slmt_decode_paged_batched(*args, ctypes.c_void_p(ws.data_ptr()), nbytes, stream)
    _native.check(lib, rc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (32, 4, 64), (64, 8, 128), (8, 8, 80), (12, 3, 128)])
def test_noalloc_matches_workspace_entry_point(H, KV, D):
    lib = _native.load()
    big = make_paged_case(seed=H + D, B=9, H=H, KV=KV, D=D, len_range=(1, 3000))
    small = make_paged_case(seed=H + D + 1, B=3, H=H, KV=KV, D=D, len_range=(1, 900))
    for case in (big, small):
        print(f"no-alloc decode H={H} KV={KV} D={D} B={case.q.shape[0]}", flush=True)
        got = _call(lib, case, noalloc=True)
        ref_ws = _call(lib, case, noalloc=False)
        assert np.array_equal(got, ref_ws), f"differs from the workspace entry point (max {np.nanmax(np.abs(got - ref_ws))})"
        assert_close(got, paged_reference(case), what=f"no-alloc H={H} KV={KV} D={D}")


def test_noalloc_scratch_holds_every_workspace():
    """The static scratch (16 MiB) covers the workspace of every head layout the
    decode supports on this device, so no valid call is refused here: the
    workspace is 4 MiB of counters plus partials for the workgroups of one
    launch, which shrink as the head count grows."""
    lib = _native.load()
    worst = 0
    for D in (64, 80, 128):
        for KV in (1, 2, 3, 4, 6, 8, 16, 32):
            for G in (1, 2, 4, 8, 16):
                for B in (1, 64, 4096):
                    need = lib.slmt_attention_workspace_bytes(B, KV * G, KV, D)
                    assert need > 0, _native.last_error(lib)
                    worst = max(worst, need)
    print(f"largest workspace: {worst} bytes", flush=True)
    assert worst <= 16 * 1024 * 1024


def _noalloc_status(lib, B, H, KV, D):
    """Status and message of a no-alloc call that fails its checks before any
    pointer is used (null pointers everywhere)."""
    null = ctypes.c_void_p(0)
    rc = lib.slmt_decode_paged_batched_noalloc(null, H * D, D, null, 1, 16, null, 32, 1, null, 1, B, H, KV, D,
                                               null, _native.OUT_F32, H * D, D, null)
    return rc, _native.last_error(lib)


def test_noalloc_reports_the_sizing_status():
    """Bad arguments give SLMT_ERR_INVALID; more than 2^20 (sequence, head group)
    pairs give SLMT_ERR_UNSUPPORTED, the same status and message as the
    workspace entry point's sizing."""
    lib = _native.load()
    rc, msg = _noalloc_status(lib, 4, 30, 8, 128)                   # 30 heads over 8 KV heads
    assert rc == _native.ERR_INVALID and "divisible" in msg
    rc, msg = _noalloc_status(lib, 4, 32, 8, 96)
    assert rc == _native.ERR_INVALID and "head_dim" in msg
    B = (1 << 20) + 1
    assert lib.slmt_attention_workspace_bytes(B, 32, 8, 128) == -1
    ws_msg = _native.last_error(lib)
    rc, msg = _noalloc_status(lib, B, 32, 8, 128)
    assert rc == _native.ERR_UNSUPPORTED and msg == ws_msg and "2^20" in msg
