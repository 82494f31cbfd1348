"""One W-only matmul case per kernel the dispatcher of tm_int4_matmul /
tm_int8_matmul can select (ops_gemm.cpp wq_plan), for torch-allocated
(aligned) buffers on a 256-CU MI355X.

Each case is (qbits, M, N, K, G, act, zeros, ws); zeros is None, "s" (the
scale dtype) or "u8"; ws says whether the call supplies a workspace (the
Python operators, tm_wq_matmul_ws: split-K plans allowed) or not (the plain C
entry points).  tests/test_wq_dispatch.py checks on the CPU that the cases
reach every instantiated W-only kernel; tests/test_gpu_wq.py runs every case
on the GPU against the oracle.
"""
import torch

ACTS = (torch.float16, torch.bfloat16)
ZEROS = (None, "s", "u8")


def _each(qbits, M, N, K, G=128, acts=ACTS, zeros=ZEROS, ws=True):
    return [(qbits, M, N, K, G, a, z, ws) for a in acts for z in zeros]


CASES = []
# wide kernels (M > 64): int4 (fp16) every zero form, int8 (fp16, bf16) none;
# their one-launch forms through the plain C entry points (with a workspace
# these few tiles would split K)
CASES += _each(4, 80, 256, 1024, acts=(torch.float16,), ws=False)
CASES += _each(8, 80, 256, 512, zeros=(None,), ws=False)
# their split-K forms (with a workspace): few tiles (16 slices), and int4 K
# past 4096 (K = 14336 at N = 4096: 4 slices)
CASES += _each(4, 96, 1024, 8192, acts=(torch.float16,))
CASES += _each(8, 96, 1024, 4096, zeros=(None,))
CASES += _each(4, 128, 4096, 14336, acts=(torch.float16,), zeros=("s",))
# int4 K % 512 == 256 (fp16 or no zero-points): one launch (K = 3840), and
# split-K into slices of 256-k units with a shorter last one (K = 11008 = 43
# units: 4 slices of 11, 11, 11, 10)
CASES += _each(4, 80, 256, 3840, acts=(torch.float16,), zeros=(None, "s"), ws=False)
CASES += _each(4, 128, 256, 11008, acts=(torch.float16,), zeros=(None, "s"))
# two-tile int4 GEMV, 2 <= M <= 6, K = 4096
CASES += _each(4, 3, 64, 4096)
# streaming kernels: x8s (M <= 8), x16s (M <= 16), x16m (M <= 64 / 128)
for M, K in ((8, 1024), (12, 2048), (40, 512)):
    CASES += _each(4, M, 64, K)
    CASES += _each(8, M, 48, K)
# persistent int4 GEMV, M = 1, K = 4096: one N per rows-per-wave count
for N in (1024, 7168, 8192, 11264, 12288, 14336, 16384):
    CASES += _each(4, 1, N, 4096)
# persistent int4 GEMV for other K: KS segments of 2048 k (the last one
# partial for K = 1536, 2176, 9216, 11008); per KS one N per row-group shape
# (RG, RW) = (1, 8), (1, 16), (2, 16), (4, 16) (the last for KS <= 4), the
# last workgroup shifted back (N not a multiple of the workgroup's rows)
GEMV4K = {1: 1536, 2: 2176, 3: 6144, 4: 8192, 5: 9216, 6: 11008, 7: 14336, 8: 16384}
for ks, K in GEMV4K.items():
    for N in (2048 - 16, 4096 - 16, 8192 - 16, 16384 - 16)[: 4 if ks <= 4 else 3]:
        CASES += _each(4, 1, N, K)
# linear int4 GEMV: K = 4096 / 8192 past the persistent kernels' reach (N >
# 16384 / 16384 on 256 CUs, e.g. a fused gate/up projection)
CASES += _each(4, 1, 16400, 4096)
CASES += _each(4, 1, 28672, 4096, acts=(torch.float16,))
CASES += _each(4, 1, 16400, 8192)
# long-K streaming kernel (M <= 64, K > 4096): tiles per workgroup NT = 1 / 2
# (N / 16 <= 256 or not), activation rows staged XR = 8 / 16 in one pass (M <=
# 8 / 16) or 16 over several (M > 16, NT = 1; int4 K <= 16384), chunks per
# wave NCH (int4 8 / 16 / 32, int8 16 / 32); K = 11008, 16512: the last round
# of chunks partly past K
STREAMK = {
    4: ((5, 6144, 1040), (3, 5120, 8176), (8, 11008, 4096), (7, 16384, 8176), (2, 20480, 1024),
        (6, 28672, 8192), (16, 8192, 2048), (9, 6144, 5120), (12, 14336, 4096), (16, 11008, 8176),
        (13, 24576, 2048), (10, 16512, 4112), (40, 6144, 1024), (24, 14336, 1040)),
    8: ((4, 6144, 1040), (8, 5120, 4112), (3, 14336, 2048), (1, 11008, 4112), (16, 8192, 512),
        (12, 4608, 4112), (9, 16384, 1024), (14, 9216, 4112), (33, 6144, 256), (64, 12288, 512)),
}
for qb, shapes in STREAMK.items():
    for M, K, N in shapes:
        CASES += _each(qb, M, N, K)
# its split-K forms (with a workspace): K past the single-launch limits in
# two slices, one tile per workgroup; int4 x8 / x16 (K > 32768), x16m
# (M > 16, K > 16384); int8 x8 / x16 / x16m (K > 16384)
for qb, M, K in ((4, 5, 40960), (4, 12, 36864), (4, 24, 20480), (8, 4, 20480), (8, 16, 24576),
                 (8, 40, 32768)):
    CASES += _each(qb, M, 1040, K)
# the same kind of shape through the plain C entry points (no workspace, no
# split): the tiled kernel
CASES += _each(4, 24, 1024, 20480, acts=(torch.float16,), zeros=("s",), ws=False)
CASES += _each(8, 16, 1024, 24576, acts=(torch.bfloat16,), zeros=(None,), ws=False)
# int4 GEMV at K = 8192, 2 <= M <= 8
CASES += _each(4, 4, 64, 8192)
# int8 GEMVs, M = 1, K = 4096: linear (fp16) and 8-wave (bf16)
CASES += _each(8, 1, 64, 4096)
# skinny (M <= 8, other K or G): int4 without and with vector scale loads
# (G = 256; K past the long-K kernel's 32768, no workspace), int8
CASES += _each(4, 2, 64, 5120, G=256)
CASES += _each(4, 2, 64, 36864, ws=False)
CASES += _each(8, 1, 64, 1024)
# tiled (M > 64 with K past the streaming kernels' 4096; int4 M > 16 with K
# past 16384 and no workspace): one launch without a workspace, split-K with
# one (fewer tiles than CUs: 16 slices of 2 steps at K = 8192; 9 slices, the
# last of one step, at K = 4352; 15 slices, the last of one step, at
# K = 11008)
CASES += _each(4, 80, 64, 8192, ws=False)
CASES += _each(4, 20, 64, 20480, acts=(torch.bfloat16,), ws=False)
CASES += _each(8, 80, 64, 4352, ws=False)
CASES += _each(4, 80, 64, 8192)
CASES += _each(8, 80, 64, 4352)
CASES += _each(4, 128, 256, 11008, acts=(torch.float16,), zeros=("s",))
# general fp32 kernel
CASES += [(4, 3, 40, 100, 32, torch.float32, None, True),
          (8, 3, 40, 100, 1, torch.float32, "s", True)]


def case_id(c):
    q, M, N, K, G, a, z, ws = c
    return f"q{q}-M{M}-N{N}-K{K}-G{G}-{str(a).split('.')[-1]}-z{z}" + ("" if ws else "-nows")


def plan(c, cu_count=256):
    """Kernel name for a case (tm_wq_plan through wq_kernel_for)."""
    import triton_metal_amd as tm
    q, M, N, K, G, a, z, ws = c
    zdt = None if z is None else (torch.uint8 if z == "u8" else a)
    return tm.wq_kernel_for(q, M, N, K, G, act_dtype=a, zero_dtype=zdt, cu_count=cu_count,
                            with_workspace=ws)[0]
