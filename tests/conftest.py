"""pytest configuration: import paths and the ``gpu`` marker.

Tests marked ``gpu`` need an MI355X (HIP) device; without one they are
skipped.  Everything else runs on the CPU.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "slm-turbo_amd", ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) GPU; skipped without one")


def pytest_sessionfinish(session, exitstatus):
    """With SLMT_ENVELOPE_OUT set, write every parity check's largest error and
    the share of the tolerance it used (the measured precision envelope)."""
    import os

    path = os.environ.get("SLMT_ENVELOPE_OUT")
    if not path:
        return
    import json

    from common import ENVELOPE

    Path(path).parent.mkdir(parents=True, exist_ok=True)
    Path(path).write_text(json.dumps(ENVELOPE, indent=0))


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(params=["mfma", "valu"])
def paged_kernel(request, monkeypatch):
    """Runs a paged-decode test through both whole-row kernels: the matrix-core
    one (the default) and the vector-ALU one (SLMT_PAGED_DECODE=valu).  The
    library reads the variable on every call.  Shapes outside the whole-row
    kernels take the per-wave kernel either way."""
    if request.param == "valu":
        monkeypatch.setenv("SLMT_PAGED_DECODE", "valu")
    else:
        monkeypatch.delenv("SLMT_PAGED_DECODE", raising=False)
    return request.param
