"""One dense matmul / linear case per kernel the selection of tm_matmul /
tm_linear can make (ops_gemm.cpp gemm_plan), for torch-allocated (aligned,
contiguous) buffers.

Each case is (form, M, N, K, dtype, out_dtype, bias): form "nn" (tm_matmul,
B [K, N]) or "nt" (tm_linear, weight [N, K]); out_dtype the input dtype or
fp32; bias only for "nt".  tests/test_gemm_dispatch.py checks on the CPU that
the cases reach every instantiated dense kernel (tm_gemm_plan);
tests/test_gpu_gemm.py runs every case on the GPU against the oracle.
"""
import torch

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32

# one (M, N, K) per tile family, from the selection's conditions
FAMILIES = {
    "t256": (2048, 1024, 128),   # M, N multiples of 256, 32 tiles, K % 64 == 0
    "s32k64": (256, 256, 256),   # < 256 tiles of 128, M, N % 32 == 0, K == 256
    "s32k128": (256, 192, 512),  # the same with K == 512
    "t128": (2048, 2176, 64),    # >= 256 tiles of 128 (N not a multiple of 256)
    "t64": (1024, 832, 64),      # < 256 tiles of 128, >= 192 of 64
    "t32k": (100, 72, 40),       # fewer tiles, K <= 512
    "t32": (100, 72, 1000),      # fewer tiles, K > 512
}

CASES = []
for fam, (M, N, K) in FAMILIES.items():
    for dt in (F16, BF16):
        for out in (dt, F32):
            CASES.append(("nn", M, N, K, dt, out, False))
            for bias in (False, True):
                CASES.append(("nt", M, N, K, dt, out, bias))
# fp32 inputs (the fp32-MFMA 64-tile kernels), every output dtype, sizes that
# are not multiples of its tiles: leading dimensions multiples of 4 (16-byte
# operand pieces, gemm_f32t64) and not (element loads, gemm_f32t64u)
F32_SHAPES = {"f32t64": (150, 132, 68), "f32t64u": (150, 130, 70)}
for shape in F32_SHAPES.values():
    for out in (F32, F16, BF16):
        CASES.append(("nn", *shape, F32, out, False))
        for bias in (False, True):
            CASES.append(("nt", *shape, F32, out, bias))
# 16-bit inputs with K % 8 != 0: tm_dot's tile kernels
CASES += [("nn", 37, 53, 29, F16, F16, False), ("nt", 40, 48, 20, BF16, F32, True)]


def case_id(c):
    form, M, N, K, dt, out, bias = c
    name = lambda t: str(t).split(".")[-1]
    return f"{form}-{M}x{N}x{K}-{name(dt)}-{name(out)}" + ("-bias" if bias else "")


def plan(c):
    """Kernel name for a case (tm_gemm_plan through gemm_kernel_for)."""
    import triton_metal_amd as tm
    form, M, N, K, dt, out, bias = c
    return tm.gemm_kernel_for(M, N, K, trans_b=form == "nt", bias=bias, in_dtype=dt,
                              out_dtype=out)[0]
