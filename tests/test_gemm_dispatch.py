"""Dense kernel selection, on the CPU: every dense kernel built into
libtm_hip.so (other than the device-sizes family, which its own entry points
select) is reachable -- some case of tests/gemm_cases.py, each of which
tests/test_gpu_gemm.py runs on the GPU, selects it through tm_gemm_plan, the
selection the launch path uses."""
import pytest
import torch

import triton_metal_amd as tm
from triton_metal_amd import _lib

from gemm_cases import CASES, case_id, plan
from test_wq_dispatch import _built, _kernel_metadata


@pytest.fixture(scope="module")
def gemm_kernels(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("co")
    names = set()
    for stem in ("gemm", "gemm_big", "gemm_f32"):
        names |= {n for n, _, _ in _kernel_metadata(_built(stem), tmp)}
    # gemm_general is selected only for K = 0 (tests/test_gpu_gemm.py runs it)
    return {n for n in names if n.startswith("gemm_") and not n.startswith("gemm_dd_")
            and n != "gemm_general"}


def test_cases_cover_every_dense_kernel(gemm_kernels):
    reached = {plan(c) for c in CASES}
    missing = sorted(gemm_kernels - reached)
    assert not missing, f"dense kernels no GPU case reaches: {missing}"
    assert reached <= gemm_kernels | {"tm_dot"}, sorted(reached - gemm_kernels)


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_case_reaches_its_family(case):
    from gemm_cases import F32_SHAPES, FAMILIES
    form, M, N, K, dt, out, bias = case
    fam = next((f for f, s in FAMILIES.items() if s == (M, N, K)), "general")
    if dt == torch.float32:
        fam = next(f for f, s in F32_SHAPES.items() if s == (M, N, K))
    name = plan(case)
    assert name.startswith(f"gemm_{fam}_") if fam != "general" else name == "tm_dot", name


def test_plan_follows_alignment_and_leading_dimensions():
    # unaligned A / B, or a leading dimension that is not a multiple of 8,
    # leave the dense tile kernels for tm_dot's (grid and block tm_dot's own);
    # an unaligned C leaves the 32-tile K-split kernel
    assert tm.gemm_kernel_for(512, 512, 512, align=_lib.TM_GEMM_ALIGN_C16) == ("tm_dot", 0, 0)
    # fp32 inputs take the fp32-MFMA kernels whatever the alignment: 16-byte
    # pieces for aligned operands with leading dimensions multiples of 4
    f32 = torch.float32
    assert tm.gemm_kernel_for(5, 7, 3, in_dtype=f32, align=0)[0] == "gemm_f32t64u_nn_f32"
    assert tm.gemm_kernel_for(5, 8, 4, in_dtype=f32)[0] == "gemm_f32t64_nn_f32"
    assert tm.gemm_kernel_for(5, 8, 4, in_dtype=f32, align=_lib.TM_GEMM_ALIGN_C16)[0] == \
        "gemm_f32t64u_nn_f32"
    assert tm.gemm_kernel_for(5, 7, 4, in_dtype=f32, trans_b=True)[0] == "gemm_f32t64_nt_f32"
    assert tm.gemm_kernel_for(5, 7, 4, in_dtype=f32, ldb=6, trans_b=True)[0] == \
        "gemm_f32t64u_nt_f32"
    assert tm.gemm_kernel_for(512, 512, 512, lda=516)[0] == "tm_dot"
    assert tm.gemm_kernel_for(512, 512, 512)[0] == "gemm_s32k128_nn_f16_same"
    assert tm.gemm_kernel_for(512, 512, 512, align=_lib.TM_GEMM_ALIGN_AB16)[0].startswith(
        "gemm_t32k_")
    # 31 tiles of 256 take smaller tiles, 32 the 256 tiles
    assert tm.gemm_kernel_for(256 * 31, 256, 64)[0].startswith("gemm_t64_")
    assert tm.gemm_kernel_for(256 * 32, 256, 64)[0].startswith("gemm_t256_")
    name, grid, block = tm.gemm_kernel_for(2048, 1024, 128, trans_b=True, bias=True,
                                           out_dtype=torch.float32)
    assert (name, grid, block) == ("gemm_t256_nt_f16_f32_bias", 32, 512)


def test_plan_rejects_bad_calls():
    with pytest.raises(Exception):
        tm.gemm_kernel_for(0, 8, 8)
    with pytest.raises(Exception):
        tm.gemm_kernel_for(8, 8, 8, lda=4)
