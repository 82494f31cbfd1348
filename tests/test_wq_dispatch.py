"""W-only kernel selection and code-object hygiene, on the CPU.

* Every W-only matmul kernel built into libtm_hip.so is reachable: some case of
  tests/wq_cases.py (each of which tests/test_gpu_wq.py runs on the GPU)
  selects it through tm_wq_plan, the selection the launch path uses.
* No hot-path kernel uses scratch memory (private_segment_fixed_size == 0, so
  no register spills to memory), read from the built code objects' metadata.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

import triton_metal_amd as tm

from wq_cases import CASES, case_id, plan

ROOT = Path(__file__).resolve().parent.parent
BUILD = ROOT / "triton-metal_amd" / "_build"
LLVM = Path("/opt/rocm/llvm/bin")

# fallback kernels that hold per-lane arrays indexed at run time (the general
# FlashAttention kernel for head dims other than 32 / 64 / 128 layouts)
SCRATCH_ALLOWED = {"flash_fwd_general_d64", "flash_fwd_general_d128"}


def _kernel_metadata(hsaco: Path, tmp: Path):
    """[(name, private_segment_fixed_size, vgpr_count)] of a bundled code object."""
    bundler, readelf = LLVM / "clang-offload-bundler", LLVM / "llvm-readelf"
    if not (bundler.exists() and readelf.exists()):
        pytest.skip("ROCm LLVM tools not found")
    co = tmp / (hsaco.stem + ".co")
    subprocess.run([str(bundler), "--unbundle", "--type=o", f"--input={hsaco}",
                    f"--output={co}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950"], check=True)
    notes = subprocess.run([str(readelf), "--notes", str(co)], check=True, capture_output=True,
                           text=True).stdout
    out, cur = [], {}
    for line in notes.splitlines():
        m = re.match(r"\s+\.(name|private_segment_fixed_size|vgpr_count):\s+(\S+)", line)
        if not m:
            continue
        k, v = m.groups()
        if k == "name" and "name" in cur:
            out.append(cur)
            cur = {}
        cur[k] = v
    if cur:
        out.append(cur)
    return [(d["name"], int(d.get("private_segment_fixed_size", 0)), int(d.get("vgpr_count", 0)))
            for d in out if "name" in d]


def _built(stem):
    p = BUILD / f"{stem}.hsaco"
    if not p.exists():
        pytest.skip(f"{p} not built (run __graft_entry__.build())")
    return p


@pytest.fixture(scope="module")
def wq_kernels(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("co")
    names = set()
    stems = ["wq_gemm", "wq_gemvp", "wq_splitk"] + sorted(
        p.stem for p in (ROOT / "triton-metal_amd" / "csrc" / "kernels").glob("wq_streamk*.hip"))
    for stem in stems:
        names |= {n for n, _, _ in _kernel_metadata(_built(stem), tmp)}
    # the dequantised tile, the GEMV's pure-read twin (a measurement kernel)
    # and the split-K reduction (launched after every split-K kernel)
    return {n for n in names if n != "wq_dequant" and not n.startswith("wq_read_twin")
            and not n.startswith("wq_splitk_reduce")}


def test_cases_cover_every_wq_kernel(wq_kernels):
    reached = {plan(c) for c in CASES}
    missing = sorted(wq_kernels - reached)
    assert not missing, f"W-only kernels no GPU case reaches: {missing}"
    assert reached <= wq_kernels, sorted(reached - wq_kernels)


@pytest.mark.parametrize("c", [c for c in CASES if c[1] == 1 and c[3] == 4096 and c[0] == 4],
                         ids=case_id)
def test_m1_k4096_branches(c):
    """int4 M = 1, K = 4096: the persistent kernel up to N = 16384 on 256 CUs,
    the linear GEMV beyond."""
    name = plan(c)
    assert name.startswith("wq_gemv4p_" if c[2] <= 16384 else "wq_gemv4l_"), name


def test_split_k_plans():
    """Split-K only with a workspace: the plan's slices, grid rows and
    workspace bytes (fp32 slice sums), and the plain C entry points' choice."""
    d = tm.wq_kernel_for(4, 24, 1040, 20480, zero_dtype=torch.float16, details=True)
    assert d["name"].endswith("_x16m_c16_k") and d["splits"] == 2
    assert d["workspace_bytes"] == 2 * 24 * 1040 * 4
    d0 = tm.wq_kernel_for(4, 24, 1024, 20480, zero_dtype=torch.float16, with_workspace=False,
                          details=True)
    assert d0["name"].startswith("wq_tiled_") and d0["splits"] == 1 and d0["workspace_bytes"] == 0
    # int4 K = 11008 (43 units of 256, K % 512 != 0): the wide kernel's split
    # form in slices of whole units, the last one shorter; uint8 zero-points
    # (whose split gathers need 512-k slices) and bf16 activations take the
    # tiled kernel, split when its tiles fill fewer than the CUs
    d = tm.wq_kernel_for(4, 128, 4096, 11008, zero_dtype=torch.float16, details=True)
    assert d["name"] == "wq_wide_q4_f16_zs_k" and d["splits"] == 4
    assert d["workspace_bytes"] == 4 * 128 * 4096 * 4
    d = tm.wq_kernel_for(4, 512, 4096, 11008, zero_dtype=torch.float16, details=True)
    assert d["name"] == "wq_wide_q4_f16_zs_k" and d["splits"] == 3
    d = tm.wq_kernel_for(4, 128, 4096, 11008, zero_dtype=torch.uint8, details=True)
    assert d["name"] == "wq_tiled_q4_f16_zu_k" and d["splits"] == 4
    d = tm.wq_kernel_for(4, 512, 4096, 11008, act_dtype=torch.bfloat16, details=True)
    assert d["name"] == "wq_tiled_q4_bf16_zn" and d["splits"] == 1
    d = tm.wq_kernel_for(8, 80, 64, 4352, details=True)
    assert d["name"] == "wq_tiled_q8_f16_zn_k" and d["splits"] == 9
    # shapes a single launch covers never split, with or without a workspace
    for args in ((4, 16, 4096, 14336), (8, 16, 4096, 14336), (4, 1, 14336, 4096)):
        d = tm.wq_kernel_for(*args, details=True)
        assert d["splits"] == 1 and d["workspace_bytes"] == 0, (args, d)


def test_plan_depends_on_cu_count():
    # 14336 rows need 256 workgroups of 56; with 128 CUs the persistent grid
    # would take a second round, so the plan moves to the linear GEMV
    c = (4, 1, 14336, 4096, 128, torch.float16, "s", True)
    assert plan(c, 256) == "wq_gemv4p_f16_zs_r14"
    assert plan(c, 128).startswith("wq_gemv4l_")


def test_no_scratch_in_hot_path_kernels(tmp_path):
    if shutil.which(str(LLVM / "llvm-readelf")) is None and not (LLVM / "llvm-readelf").exists():
        pytest.skip("llvm-readelf not found")
    bad = []
    for hsaco in sorted(BUILD.glob("*.hsaco")):
        for name, priv, _ in _kernel_metadata(hsaco, tmp_path):
            if priv and name not in SCRATCH_ALLOWED:
                bad.append((hsaco.stem, name, priv))
    if not list(BUILD.glob("*.hsaco")):
        pytest.skip("code objects not built")
    assert not bad, bad
