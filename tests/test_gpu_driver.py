"""Generic loader / launcher (HipUtils, the MetalUtils counterpart) on the GPU,
plus the MFMA lane layouts the library's kernels are written against."""
from pathlib import Path

import numpy as np
import pytest
import torch

PROBE = Path(__file__).resolve().parent / "kernels" / "probe.hsaco"

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def utils(dev):
    from triton_metal_amd.driver import HipUtils
    return HipUtils()


def test_load_binary_returns_five_tuple_and_launches(utils, dev):
    assert PROBE.exists(), "probe.hsaco not built (run __graft_entry__.build())"
    mod, fn, n_regs, n_spills, n_max = utils.load_binary("probe_axpy", PROBE.read_bytes(), 0)
    assert n_regs > 0 and n_spills == 0 and n_max >= 256
    n = 1000
    x = torch.arange(n, dtype=torch.float32, device=dev)
    y = torch.ones(n, dtype=torch.float32, device=dev)
    utils.launch(fn, ((n + 255) // 256,), (256,), [y, x, 2.0, n], sync=True)
    assert torch.equal(y.cpu(), 2 * torch.arange(n, dtype=torch.float32) + 1)
    utils.unload(mod)


def test_load_binary_errors(utils):
    from triton_metal_amd.errors import KernelLoadError
    with pytest.raises(KernelLoadError):
        utils.load_binary("probe_axpy", b"\0" * 256, 0)
    with pytest.raises(KernelLoadError, match="not found"):
        utils.load_binary("no_such_kernel", PROBE.read_bytes(), 0)


def test_mfma16x16x32_layout(utils, dev):
    _, fn, *_ = utils.load_binary("probe_mfma16_layout", PROBE.read_bytes(), 0)
    out = torch.zeros(64 * 4, dtype=torch.float32, device=dev)
    utils.launch(fn, (1,), (64,), [out], sync=True)
    got = out.cpu().numpy().reshape(64, 4)
    l = np.arange(64)[:, None]
    e = np.arange(4)[None, :]
    expect = 100 * (4 * (l // 16) + e) + (l % 16)          # D[4(l/16)+e][l%16]
    assert np.array_equal(got, expect.astype(np.float32))


def test_mfma32x32x16_layout(utils, dev):
    _, fn, *_ = utils.load_binary("probe_mfma32_layout", PROBE.read_bytes(), 0)
    out = torch.zeros(64 * 16, dtype=torch.float32, device=dev)
    utils.launch(fn, (1,), (64,), [out], sync=True)
    got = out.cpu().numpy().reshape(64, 16)
    l = np.arange(64)[:, None]
    e = np.arange(16)[None, :]
    row = 8 * (e // 4) + 4 * (l // 32) + (e % 4)          # D[8(e/4)+4(l/32)+e%4][l%32]
    expect = 100 * row + (l % 32)
    # only rows < 16 have a non-zero identity entry in A (k < 16)
    expect = np.where(row < 16, expect, 0)
    assert np.array_equal(got, expect.astype(np.float32))


def test_mfma16x16x4_f32_layout(utils, dev):
    _, fn, *_ = utils.load_binary("probe_mfma16x4_f32_layout", PROBE.read_bytes(), 0)
    out = torch.zeros(64 * 4, dtype=torch.float32, device=dev)
    utils.launch(fn, (1,), (64,), [out], sync=True)
    got = out.cpu().numpy().reshape(64, 4)
    l = np.arange(64)[:, None]
    e = np.arange(4)[None, :]
    i = 4 * (l // 16) + e                                   # D[4(l/16)+e][l%16]
    expect = (1 + i // 4) * (100 * (i % 4) + (l % 16))
    assert np.array_equal(got, expect.astype(np.float32))
