import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "triton-metal_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libtm_hip.so")


@pytest.fixture(scope="session")
def kats():
    """Reference known-answer tests replayed by tests/golden/make_golden.py."""
    meta = json.loads((GOLDEN / "reference_kats.json").read_text())
    data = np.load(GOLDEN / "reference_kats.npz")
    out = {}
    for name, m in meta.items():
        arrs = {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}
        out[name] = (m, arrs)
    return out


@pytest.fixture(scope="session")
def dev():
    """The HIP device; GPU tests fail (not skip) when the library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    import triton_metal_amd._lib as L
    L.lib()  # raises NativeLibraryMissing if not built
    return torch.device("cuda", 0)


def pytest_report_header(config):
    return f"repo: {ROOT}"
