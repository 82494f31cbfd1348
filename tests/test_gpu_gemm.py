"""Dense matmul / fused linear parity on the GPU against the oracle.

fp16/bf16 outputs within atol 2e-2 / rtol 1e-2 of the oracle's fp64 product
of the same (rounded) inputs; the reference's known-answer tests with the
reference's own tolerances.
"""
import numpy as np
import pytest
import torch

import oracle
import triton_metal_amd as tm

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2

MATMUL_KATS = ["matmul_seed789", "matmul_seed101r", "matmul_seed202", "matmul_seed42",
               "matmul_seed101g", "simdgroup_seed88", "simdgroup_seed303", "simdgroup_seed404",
               "simdgroup_seed505", "simdgroup_f16_seed707", "simdgroup_f16_seed808"]


@pytest.mark.parametrize("name", MATMUL_KATS)
@pytest.mark.parametrize("out_dtype", ["same", "f32"])
def test_matmul_reference_kat(kats, dev, name, out_dtype):
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    dt = torch.float16 if m["in_dtype"] == "fp16" else torch.float32
    A = torch.tensor(a["A"], dtype=dt, device=dev).reshape(M, K)
    B = torch.tensor(a["B"], dtype=dt, device=dev).reshape(K, N)
    C = torch.empty(M, N, dtype=dt if out_dtype == "same" else torch.float32, device=dev)
    kern = (tm.make_simdgroup_matmul_kernel(m["in_dtype"]) if name.startswith("simdgroup")
            else tm.make_matmul_kernel())
    kern(A, B, C, M, N, K)
    got = C.float().cpu().numpy().ravel()
    sel = np.zeros((M, N), bool)
    sel[::m["spot"], ::m["spot"]] = True
    err = np.abs(got - a["expected"])[sel.ravel()].max()
    assert err < m["tol"]
    # the same inputs through the MFMA path (fp16) stay inside the reference tolerance too
    if dt == torch.float32:
        A16, B16 = A.half(), B.half()
        C16 = torch.empty(M, N, dtype=torch.float32, device=dev)
        tm.matmul(A16, B16, C16, M, N, K)
        ref = oracle.matmul(A16.float().cpu().numpy(), B16.float().cpu().numpy())
        np.testing.assert_allclose(C16.cpu().numpy(), ref, atol=1e-3, rtol=1e-4)


DEVICE_SIZE_KATS = ["matmul2d_seed1001", "matmul2d_seed1002", "matmul2d_seed1003",
                    "swizzled_seed2001", "swizzled_seed2002"]


@pytest.mark.parametrize("name", DEVICE_SIZE_KATS)
@pytest.mark.parametrize("sizes", ["device", "int", "capacity"])
def test_device_sizes_reference_kat(kats, dev, name, sizes):
    """make_matmul_2d_kernel / make_matmul_swizzled_kernel with M, N, K in
    uint32 device buffers (the templates' buffer(3..5)), as Python ints, and
    with a larger launch capacity than the sizes on the device; the reference
    tests' tolerance on their sampled entries, and every entry within 1e-4 of
    the oracle (fp32 in, fp32 out)."""
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    A = torch.tensor(a["A"], dtype=torch.float32, device=dev)
    B = torch.tensor(a["B"], dtype=torch.float32, device=dev)
    if m["kind"] == "matmul_2d":
        kern = tm.make_matmul_2d_kernel(32, 32, 32)
    else:
        kern = tm.make_matmul_swizzled_kernel(32, 32, 32, group_size=m["group_size"])
    if sizes == "int":
        C = torch.empty(M * N, dtype=torch.float32, device=dev)
        kern(A, B, C, M, N, K)
    else:
        u32 = lambda v: torch.tensor([v], dtype=torch.int32, device=dev).view(torch.uint32)
        if sizes == "device":
            C = torch.empty(M * N, dtype=torch.float32, device=dev)
            kern(A, B, C, u32(M), u32(N), u32(K))
        else:
            C = torch.full((200 * 200,), 7.0, dtype=torch.float32, device=dev)
            kern(A, B, C, u32(M), u32(N), u32(K), max_m=200, max_n=200)
            assert torch.all(C[M * N:] == 7.0)  # nothing written past M x N
            C = C[:M * N]
    got = C.cpu().numpy().astype(np.float64)
    sel = np.zeros((M, N), bool)
    sel[::m["spot_m"], ::m["spot"]] = True
    assert np.abs(got - a["expected"])[sel.ravel()].max() < m["tol"]
    ref = oracle.matmul(a["A"].reshape(M, K), a["B"].reshape(K, N)).ravel()
    np.testing.assert_allclose(got, ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dt,out", [(torch.float16, torch.float16), (torch.bfloat16, torch.float32),
                                    (torch.float32, torch.float32)])
@pytest.mark.parametrize("group", [0, 1, 3])
def test_device_sizes_shapes(dev, dt, out, group):
    """Ragged sizes across several 64 x 64 tiles, both tile orders (a run of
    3 tile rows leaves a shorter last run), against the oracle; sizes on the
    device smaller than the capacity."""
    M, N, K = 200, 150, 77
    A = _rand((M, K), 61, dt)
    B = _rand((K, N), 62, dt)
    C = torch.empty(256 * 160, dtype=out, device=dev)  # holds the capacity
    dims = torch.tensor([M, N, K], dtype=torch.int32, device=dev)
    tm.matmul_device_sizes(A.to(dev), B.to(dev), C, dims[0:1], dims[1:2], dims[2:3],
                           max_m=256, max_n=160, group_size=group)
    ref = oracle.matmul(A.double().numpy(), B.double().numpy())
    tol = (1e-4, 1e-4) if out == torch.float32 else (ATOL, RTOL)
    np.testing.assert_allclose(C[:M * N].double().cpu().numpy().reshape(M, N), ref,
                               atol=tol[0], rtol=tol[1])


def test_device_sizes_past_the_buffers_do_nothing(dev):
    """Sizes on the device that the buffers cannot hold (here K larger than A
    and B allow, then M larger than C) make the launch write nothing; with
    fitting sizes the same launch computes."""
    M, N, K = 16, 16, 16
    A = torch.randn(M * K, device=dev)
    B = torch.randn(K * N, device=dev)
    C = torch.full((M * N,), 7.0, device=dev)
    dims = torch.tensor([M, N, 1000], dtype=torch.int32, device=dev)
    tm.matmul_device_sizes(A, B, C, dims[0:1], dims[1:2], dims[2:3], max_m=M, max_n=N)
    torch.cuda.synchronize()
    assert torch.all(C == 7.0)
    dims = torch.tensor([64, N, K], dtype=torch.int32, device=dev)
    tm.matmul_device_sizes(A, B, C, dims[0:1], dims[1:2], dims[2:3], max_m=64, max_n=N)
    torch.cuda.synchronize()
    assert torch.all(C == 7.0)
    dims = torch.tensor([M, N, K], dtype=torch.int32, device=dev)
    tm.matmul_device_sizes(A, B, C, dims[0:1], dims[1:2], dims[2:3], max_m=M, max_n=N)
    ref = oracle.matmul(A.double().cpu().numpy().reshape(M, K), B.double().cpu().numpy().reshape(K, N))
    np.testing.assert_allclose(C.double().cpu().numpy().reshape(M, N), ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("name", ["linear_seed1111", "linear_seed2222"])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_fused_linear_reference_kat(kats, dev, name, dt):
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    x = torch.tensor(a["input"], dtype=dt, device=dev).reshape(M, K)
    W = torch.tensor(a["weight"], dtype=dt, device=dev).reshape(N, K)
    C = torch.empty(M, N, dtype=dt, device=dev)
    if m["has_bias"]:
        b = torch.tensor(a["bias"], dtype=dt, device=dev)
        tm.make_fused_linear_kernel(True)(x, W, C, b, M, N, K)
    else:
        tm.make_fused_linear_kernel(False)(x, W, C, M, N, K)
    err = np.abs(C.float().cpu().numpy().ravel() - a["expected"]).max()
    assert err < (m["tol"] if dt == torch.float32 else max(m["tol"], 5e-2))


def test_identity_fp16(dev):
    # tests/test_emitter.py:4849 test_matmul_fp16_identity
    A = torch.eye(16, dtype=torch.float16, device=dev)
    B = torch.arange(1, 17, dtype=torch.float16, device=dev).repeat(16, 1).contiguous()
    C = torch.empty(16, 16, dtype=torch.float16, device=dev)
    tm.matmul(A, B, C, 16, 16, 16)
    assert torch.equal(C, B)


def _rand(shape, seed, dt):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dt)


@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (256, 384, 1024), (100, 72, 40),
                                   (1, 64, 64), (33, 8, 520), (2048, 2048, 256)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_matmul_shapes(dev, M, N, K, dt):
    A, B = _rand((M, K), 1, dt), _rand((K, N), 2, dt)
    C = torch.empty(M, N, dtype=dt, device=dev)
    tm.matmul(A.to(dev), B.to(dev), C, M, N, K)
    ref = oracle.matmul(A.float().numpy(), B.float().numpy())
    np.testing.assert_allclose(C.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_matmul_c1_fp16_fp32_out(dev):
    M = N = K = 512
    A, B = _rand((M, K), 3, torch.float16), _rand((K, N), 4, torch.float16)
    C = torch.empty(M, N, dtype=torch.float32, device=dev)
    tm.matmul(A.to(dev), B.to(dev), C, M, N, K)
    ref = oracle.matmul(A.float().numpy(), B.float().numpy())
    np.testing.assert_allclose(C.cpu().numpy(), ref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("M,N,K", [(64, 128, 256), (1000, 520, 64), (7, 24, 48)])
@pytest.mark.parametrize("bias", [False, True])
def test_linear_shapes(dev, M, N, K, bias):
    x, W = _rand((M, K), 5, torch.float16), _rand((N, K), 6, torch.float16)
    b = _rand((N,), 7, torch.float16) if bias else None
    C = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.fused_linear(x.to(dev), W.to(dev), C, None if b is None else b.to(dev), M, N, K)
    ref = oracle.linear(x.float().numpy(), W.float().numpy(),
                        None if b is None else b.float().numpy())
    np.testing.assert_allclose(C.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


# --- 32 x 32 tiles with K split over 4 waves (M, N % 32 == 0, K = 256 or 512) --------
@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (1024, 512, 256), (96, 160, 512),
                                   (32, 32, 256)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out32", [False, True])
def test_matmul_small_tiles(dev, M, N, K, dt, out32):
    A, B = _rand((M, K), 21, dt), _rand((K, N), 22, dt)
    C = torch.empty(M, N, dtype=torch.float32 if out32 else dt, device=dev)
    tm.matmul(A.to(dev), B.to(dev), C, M, N, K)
    ref = oracle.matmul(A.float().numpy(), B.float().numpy())
    np.testing.assert_allclose(C.float().cpu().numpy(), ref, atol=1e-3 if out32 else ATOL,
                               rtol=1e-4 if out32 else RTOL)


@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (64, 96, 256)])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_linear_small_tiles(dev, M, N, K, bias, dt):
    x, W = _rand((M, K), 23, dt), _rand((N, K), 24, dt)
    b = _rand((N,), 25, dt) if bias else None
    C = torch.empty(M, N, dtype=dt, device=dev)
    tm.fused_linear(x.to(dev), W.to(dev), C, None if b is None else b.to(dev), M, N, K)
    ref = oracle.linear(x.float().numpy(), W.float().numpy(),
                        None if b is None else b.float().numpy())
    np.testing.assert_allclose(C.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("ldc_pad", [32, 2])
def test_matmul_small_tiles_padded_leading_dims(dev, ldc_pad):
    """The C ABI with row strides above the logical widths on the 32 x 32 K-split
    kernel (ldc_pad 32), and with an ldc that is not a multiple of 4 (ldc_pad 2),
    which the host sends to another kernel."""
    import ctypes
    from triton_metal_amd import _lib
    M, N, K = 512, 256, 512
    lda, ldb, ldc = K + 64, N + 128, N + ldc_pad
    Ap, Bp = _rand((M, lda), 26, torch.float16), _rand((K, ldb), 27, torch.float16)
    Cp = torch.zeros(M, ldc, dtype=torch.float16, device=dev)
    Ad, Bd = Ap.to(dev), Bp.to(dev)
    L = _lib.lib()
    rc = L.tm_matmul(ctypes.c_void_p(Ad.data_ptr()), ctypes.c_void_p(Bd.data_ptr()),
                     ctypes.c_void_p(Cp.data_ptr()), M, N, K, lda, ldb, ldc,
                     _lib.TM_DT_F16, _lib.TM_DT_F16, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    ref = oracle.matmul(Ap[:, :K].float().numpy(), Bp[:, :N].float().numpy())
    got = Cp.float().cpu().numpy()
    np.testing.assert_allclose(got[:, :N], ref, atol=ATOL, rtol=RTOL)
    assert (got[:, N:] == 0).all()  # the padding columns of C are untouched


# --- 256 x 256 tiles (M, N multiples of 256 with at least 32 tiles, K % 64 == 0) -----
def _sample(n, k, seed):
    return np.sort(np.random.default_rng(seed).choice(n, k, replace=False))


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 128), (3072, 4096, 192), (2048, 1024, 320)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out32", [False, True])
def test_matmul_large_tiles(dev, M, N, K, dt, out32):
    A, B = _rand((M, K), 11, dt), _rand((K, N), 12, dt)
    C = torch.empty(M, N, dtype=torch.float32 if out32 else dt, device=dev)
    tm.matmul(A.to(dev), B.to(dev), C, M, N, K)
    rows, cols = _sample(M, 256, 1), _sample(N, 256, 2)
    ref = oracle.matmul(A.float().numpy()[rows], B.float().numpy()[:, cols])
    got = C.float().cpu().numpy()[np.ix_(rows, cols)]
    atol = 1e-3 if out32 else ATOL
    np.testing.assert_allclose(got, ref, atol=atol, rtol=1e-4 if out32 else RTOL)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_linear_large_tiles(dev, bias, dt):
    M, N, K = 3072, 4096, 256
    x, W = _rand((M, K), 13, dt), _rand((N, K), 14, dt)
    b = _rand((N,), 15, dt) if bias else None
    C = torch.empty(M, N, dtype=dt, device=dev)
    tm.fused_linear(x.to(dev), W.to(dev), C, None if b is None else b.to(dev), M, N, K)
    rows, cols = _sample(M, 256, 3), _sample(N, 256, 4)
    ref = oracle.linear(x.float().numpy()[rows], W.float().numpy()[cols],
                        None if b is None else b.float().numpy()[cols])
    got = C.float().cpu().numpy()[np.ix_(rows, cols)]
    np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)


def test_matmul_large_tiles_padded_leading_dims(dev):
    """The C ABI with row strides above the logical widths (lda > K, ldb > N,
    ldc > N) on the 256 x 256-tile kernel: views into padded buffers."""
    import ctypes
    from triton_metal_amd import _lib
    M, N, K = 4096, 3072, 128
    lda, ldb, ldc = K + 64, N + 256, N + 128
    Ap, Bp = _rand((M, lda), 16, torch.float16), _rand((K, ldb), 17, torch.float16)
    Cp = torch.zeros(M, ldc, dtype=torch.float16, device=dev)
    Ad, Bd = Ap.to(dev), Bp.to(dev)
    L = _lib.lib()
    rc = L.tm_matmul(ctypes.c_void_p(Ad.data_ptr()), ctypes.c_void_p(Bd.data_ptr()),
                     ctypes.c_void_p(Cp.data_ptr()), M, N, K, lda, ldb, ldc,
                     _lib.TM_DT_F16, _lib.TM_DT_F16, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    rows, cols = _sample(M, 256, 5), _sample(N, 256, 6)
    ref = oracle.matmul(Ap[:, :K].float().numpy()[rows], Bp[:, :N].float().numpy()[:, cols])
    got = Cp.float().cpu().numpy()
    np.testing.assert_allclose(got[np.ix_(rows, cols)], ref, atol=ATOL, rtol=RTOL)
    assert (got[:, N:] == 0).all()  # the padding columns of C are untouched


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("form", ["nn", "nt", "nt_bias"])
def test_off_tile_shapes_run_the_dot_tiles(dev, dt, form):
    """16-bit shapes the dense tile kernels do not take run tm_dot's tile
    kernels (tm_gemm_plan: "tm_dot"): K not a multiple of 8 (large and odd),
    A one element off 16-byte alignment, a leading dimension not a multiple
    of 8 (tm_matmul), with fp32 output and the linear bias."""
    import ctypes
    from triton_metal_amd import _lib
    L = _lib.lib()
    bt, bias = form != "nn", form == "nt_bias"
    code = _lib.TM_DT_BF16 if dt == torch.bfloat16 else _lib.TM_DT_F16
    # (M, N, K, lda, element offset of A, out dtype); tm_linear rows are contiguous
    cases = ((300, 260, 1001, 1001, 0, dt), (130, 96, 64, 64 if bt else 68, 1, dt),
             (64, 200, 36, 36 if bt else 44, 0, torch.float32))
    for M, N, K, lda, off, out in cases:
        ldb = K if bt else N
        Ap = _rand((M * lda + off,), M + K, dt)
        B = _rand((N, K) if bt else (K, N), N + K, dt)
        b = _rand((N,), N, dt) if bias else None
        C = torch.full((M, N), 7.0, dtype=out, device=dev)
        Ad, Bd = Ap.to(dev), B.to(dev)
        bd = None if b is None else b.to(dev)
        a_ptr = ctypes.c_void_p(Ad.data_ptr() + off * Ad.element_size())
        ocode = _lib.TM_DT_F32 if out == torch.float32 else code
        align = _lib.TM_GEMM_ALIGN_C16 | (0 if off else _lib.TM_GEMM_ALIGN_AB16)
        name = tm.gemm_kernel_for(M, N, K, lda=lda, ldb=ldb, trans_b=bt, bias=bias, in_dtype=dt,
                                  out_dtype=out, align=align)[0]
        assert name == "tm_dot", (M, N, K, name)
        if bt:
            rc = L.tm_linear(a_ptr, ctypes.c_void_p(Bd.data_ptr()),
                             None if bd is None else ctypes.c_void_p(bd.data_ptr()),
                             ctypes.c_void_p(C.data_ptr()), M, N, K, code, ocode, None)
        else:
            rc = L.tm_matmul(a_ptr, ctypes.c_void_p(Bd.data_ptr()), ctypes.c_void_p(C.data_ptr()),
                             M, N, K, lda, ldb, N, code, ocode, None)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        A = Ap[off:off + M * lda].reshape(M, lda)[:, :K].float().numpy()
        if bt:
            ref = oracle.linear(A, B.float().numpy(), None if b is None else b.float().numpy())
        else:
            ref = oracle.matmul(A, B.float().numpy())
        atol, rtol = (1e-3, 1e-4) if out == torch.float32 else (max(ATOL, 1e-3 * K ** 0.5), RTOL)
        np.testing.assert_allclose(C.float().cpu().numpy(), ref, atol=atol, rtol=rtol)


def test_k_zero_runs_the_general_kernel(dev):
    """K = 0: a product of zeros (plus the linear bias) on gemm_general."""
    import ctypes
    from triton_metal_amd import _lib
    L = _lib.lib()
    M, N = 5, 24
    A = torch.zeros(8, dtype=torch.float16, device=dev)
    B = torch.zeros(8, dtype=torch.float16, device=dev)
    b = _rand((N,), 3, torch.float16).to(dev)
    C = torch.full((M, N), 7.0, dtype=torch.float16, device=dev)
    rc = L.tm_matmul(ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(B.data_ptr()),
                     ctypes.c_void_p(C.data_ptr()), M, N, 0, 0, N, N, _lib.TM_DT_F16,
                     _lib.TM_DT_F16, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert (C == 0).all()
    C.fill_(7.0)
    rc = L.tm_linear(ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(B.data_ptr()),
                     ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(C.data_ptr()), M, N, 0,
                     _lib.TM_DT_F16, _lib.TM_DT_F16, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(C, b.expand(M, N))


def test_fp32_general_path(dev):
    M, N, K = 13, 17, 19
    A, B = _rand((M, K), 8, torch.float32), _rand((K, N), 9, torch.float32)
    C = torch.empty(M, N, dtype=torch.float32, device=dev)
    tm.matmul(A.to(dev), B.to(dev), C, M, N, K)
    np.testing.assert_allclose(C.cpu().numpy(), oracle.matmul(A.numpy(), B.numpy()),
                               atol=1e-5, rtol=1e-5)


# --- every dense kernel the selection can make (tests/gemm_cases.py) ------------
from gemm_cases import CASES as DENSE_CASES, case_id as dense_case_id, plan as dense_plan  # noqa: E402


@pytest.mark.parametrize("case", DENSE_CASES, ids=[dense_case_id(c) for c in DENSE_CASES])
def test_dispatch_case(dev, case):
    form, M, N, K, dt, out, bias = case
    print(f"[dense] {dense_case_id(case)} -> {dense_plan(case)}", flush=True)
    seed = M + 3 * N + 7 * K
    A = _rand((M, K), seed, dt)
    B = _rand((N, K) if form == "nt" else (K, N), seed + 1, dt)
    b = _rand((N,), seed + 2, dt) if bias else None
    C = torch.full((M, N), 3.0, dtype=out, device=dev)
    if form == "nt":
        tm.fused_linear(A.to(dev), B.to(dev), C, None if b is None else b.to(dev), M, N, K)
        ref = oracle.linear(A.float().numpy(), B.float().numpy(),
                            None if b is None else b.float().numpy())
    else:
        tm.matmul(A.to(dev), B.to(dev), C, M, N, K)
        ref = oracle.matmul(A.float().numpy(), B.float().numpy())
    torch.cuda.synchronize()
    atol, rtol = (1e-3, 1e-4) if out == torch.float32 else (ATOL, RTOL)
    np.testing.assert_allclose(C.float().cpu().numpy(), ref, atol=atol, rtol=rtol)
