"""tl.dot in general form on the GPU against oracle.dot: strided, transposed
and column-major views, batched 3-D operands, every epilogue, fp16 / bf16 /
fp32 and the five FP8 formats.

Tolerances: fp16 / bf16 outputs atol 2e-2 / rtol 1e-2.  fp32 outputs (fp32
accumulation of exact products): |err| <= 1e-4 |ref| + 2^-16 (|A| @ |B|), the
accumulation bound with the magnitude of the terms (the FP8 tests draw codes
across each format's whole range, subnormals and extremes included).
"""
import numpy as np
import pytest
import torch

import oracle
import triton_metal_amd as tm

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2
FP8 = ["fp8e4nv", "fp8e5", "fp8e4b15", "fp8e4b8", "fp8e5b16"]


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _rand(shape, seed, dt):
    return torch.randn(*shape, generator=_gen(seed)).to(dt)


def _np(t):
    return t.double().cpu().numpy()


def _check(got, ref, out_dt, absA=None, absB=None):
    got = got.double().cpu().numpy()
    if out_dt == torch.float32:
        bound = 1e-4 * np.abs(ref) + (2.0 ** -16 * (absA @ absB) if absA is not None else 1e-5)
        err = np.abs(got - ref)
        assert (err <= bound + 1e-30).all(), f"max err {err.max():.3e}, worst {(err / (bound + 1e-30)).max():.2f}"
    else:
        np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)


def _views(M, N, K, dt, layout, seed, batch=None, dev="cuda"):
    """a [.., M, K], b [.., K, N] as views of the requested layout; returns the
    device views and their CPU copies (logical values)."""
    bs = () if batch is None else (batch,)
    a = _rand(bs + (M, K), seed, dt)
    b = _rand(bs + (K, N), seed + 1, dt)
    if layout == "row":
        da, db = a.to(dev), b.to(dev)
    elif layout == "trans_a":      # A stored [K, M] (column-major A)
        da = a.transpose(-1, -2).contiguous().to(dev).transpose(-1, -2)
        db = b.to(dev)
    elif layout == "trans_b":      # B stored [N, K]
        da = a.to(dev)
        db = b.transpose(-1, -2).contiguous().to(dev).transpose(-1, -2)
    elif layout == "strided":      # every second element of wider buffers
        ap = torch.zeros(bs + (M, 2 * K + 3), dtype=dt)
        ap[..., : 2 * K : 2] = a
        bp = torch.zeros(bs + (2 * K, N + 5), dtype=dt)
        bp[..., ::2, :N] = b
        da = ap.to(dev)[..., : 2 * K : 2]
        db = bp.to(dev)[..., ::2, :N]
    else:
        raise ValueError(layout)
    return da, db, a, b


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["row", "trans_a", "trans_b", "strided"])
@pytest.mark.parametrize("M,N,K", [(64, 64, 32), (100, 72, 136), (7, 130, 50)])
def test_dot_layouts(dev, dt, layout, M, N, K):
    da, db, a, b = _views(M, N, K, dt, layout, seed=M + N + K)
    c = torch.empty(M, N, dtype=dt, device=dev)
    tm.dot(da, db, c)
    _check(c, oracle.dot(_np(a), _np(b)), dt)


@pytest.mark.parametrize("layout", ["row", "trans_a", "trans_b", "strided"])
@pytest.mark.parametrize("M,N,K", [(64, 64, 32), (100, 72, 136), (7, 130, 50), (300, 260, 520)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_dot_fp32_layouts(dev, layout, M, N, K, out):
    """fp32 inputs without an epilogue: k- and n-contiguous rows (row, trans_b)
    run the fp32-MFMA dense kernel, the other layouts the strided fp32-MFMA
    tile kernel."""
    da, db, a, b = _views(M, N, K, torch.float32, layout, seed=M + 2 * N + K)
    c = torch.empty(M, N, dtype=out, device=dev)
    tm.dot(da, db, c)
    _check(c, oracle.dot(_np(a), _np(b)), out, np.abs(_np(a)), np.abs(_np(b)))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(5, 3, 40), (7, 70, 130), (130, 6, 33)])
def test_dot_row_contiguous_operands_with_few_rows(dev, dt, M, N, K):
    """Row-contiguous operands (A stored [K, M], B [K, N]) with fewer rows
    than one 16-byte piece holds, as narrow views of buffers whose leading
    dimension is a multiple of 8: the 16-byte loads read past the operand
    inside the buffer's rows, and those elements must not reach C."""
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    lda, ldb = (M + 7) // 8 * 8, (N + 7) // 8 * 8
    Ab = torch.randn(K, lda, generator=g).to(dt)
    Bb = torch.randn(K, ldb, generator=g).to(dt)
    a, b = Ab[:, :M].t(), Bb[:, :N]  # logical [M, K] and [K, N] views
    c = torch.empty(M, N, dtype=torch.float32, device=dev)
    tm.dot(Ab.to(dev)[:, :M].t(), Bb.to(dev)[:, :N], c)
    _check(c, oracle.dot(_np(a), _np(b)), torch.float32, np.abs(_np(a)), np.abs(_np(b)))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_dot_column_major_output(dev, dt):
    """The reference's "trans" case: C written through column-major strides."""
    M, N, K = 96, 80, 64
    da, db, a, b = _views(M, N, K, dt, "row", seed=5)
    cbuf = torch.zeros(N, M, dtype=dt, device=dev)
    tm.dot(da, db, cbuf.t())
    _check(cbuf.t(), oracle.dot(_np(a), _np(b)), dt, np.abs(_np(a)), np.abs(_np(b)))


@pytest.mark.parametrize("layout", ["row", "trans_a", "trans_b", "strided"])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_dot_batched_3d(dev, layout, dt):
    B, M, N, K = 3, 70, 40, 96
    da, db, a, b = _views(M, N, K, dt, layout, seed=17, batch=B)
    c = torch.empty(B, M, N, dtype=torch.float32, device=dev)
    tm.dot(da, db, c)
    ref = oracle.dot(_np(a), _np(b))
    _check(c, ref, torch.float32, np.abs(_np(a)), np.abs(_np(b)))


@pytest.mark.parametrize("epilogue", ["add-matrix", "add-rows", "add-cols"])
@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
@pytest.mark.parametrize("batch", [None, 2])
def test_dot_add_epilogues(dev, epilogue, dt, batch):
    M, N, K = 90, 66, 48
    da, db, a, b = _views(M, N, K, dt, "trans_b", seed=23, batch=batch)
    bs = () if batch is None else (batch,)
    z = _rand(bs + (M, N), 29, dt)
    c = torch.empty(bs + (M, N), dtype=dt, device=dev)
    tm.dot(da, db, c, epilogue, z=z.to(dev))
    _check(c, oracle.dot(_np(a), _np(b), epilogue, Z=_np(z)), dt,
           np.abs(_np(a)), np.abs(_np(b)))


@pytest.mark.parametrize("epilogue", ["add-matrix", "add-rows"])
@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_dot_bias_read_in_place(dev, epilogue, dt):
    """Z is the output buffer itself, as in the reference's test kernels."""
    M, N, K = 130, 70, 64
    da, db, a, b = _views(M, N, K, dt, "row", seed=31)
    z = _rand((M, N), 37, dt)
    c = z.to(dev)
    tm.dot(da, db, c, epilogue, z=c)
    _check(c, oracle.dot(_np(a), _np(b), epilogue, Z=_np(z)), dt, np.abs(_np(a)),
           np.abs(_np(b)))


def test_dot_add_cols_in_place_rejected_for_many_rows(dev):
    M, N, K = 8, 16, 16
    da, db, _, _ = _views(M, N, K, torch.float16, "row", seed=41)
    c = torch.zeros(M, N, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="add-cols"):
        tm.dot(da, db, c, "add-cols", z=c)


def test_dot_add_matrix_aliasing_view_rejected(dev):
    """add-matrix in place is defined only when Z is C element for element; a
    transposed view of C as Z would race between workgroups and is refused."""
    M = N = K = 64
    da, db, _, _ = _views(M, N, K, torch.float16, "row", seed=43)
    c = torch.zeros(M, N, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="add-matrix"):
        tm.dot(da, db, c, "add-matrix", z=c.t())
    wide = torch.zeros(M, N + 1, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="add-matrix"):
        tm.dot(da, db, wide[:, :N], "add-matrix", z=wide[:, 1:])


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("side", ["a", "b"])
def test_dot_batch_one_broadcast_3d(dev, dt, side):
    """A 3-D operand of batch 1 is broadcast over the other operand's batch
    (np.matmul's rule, which oracle.dot follows): [1, M, K] @ [B, K, N] and
    [B, M, K] @ [1, K, N]."""
    B, M, N, K = 3, 70, 40, 96
    a = _rand((1 if side == "a" else B, M, K), 51, dt)
    b = _rand((B if side == "a" else 1, K, N), 52, dt)
    c = torch.empty(B, M, N, dtype=torch.float32, device=dev)
    tm.dot(a.to(dev), b.to(dev), c)
    ref = oracle.dot(_np(a), _np(b))
    assert ref.shape == (B, M, N)
    _check(c, ref, torch.float32, np.abs(_np(a)), np.abs(_np(b)))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N", [40, 1500])
def test_dot_softmax(dev, dt, N):
    M, K = 33, 2100  # two pieces of A's row, two column groups at N = 1500
    da, db, a, b = _views(M, N, K, dt, "trans_a", seed=43)
    c = torch.empty(M, N, dtype=torch.float32, device=dev)
    # scale so that the softmax is neither uniform nor one-hot
    da = (da.float() * 0.05).to(dt)
    a = (a.float() * 0.05).to(dt)
    tm.dot(da, db, c, "softmax")
    ref = oracle.dot(_np(a), _np(b), "softmax")
    np.testing.assert_allclose(c.cpu().numpy(), ref, atol=1e-6, rtol=1e-4)
    np.testing.assert_allclose(c.sum(-1).cpu().numpy(), 1.0, rtol=1e-5)


@pytest.mark.parametrize("layout", ["row", "trans_a", "trans_b", "strided"])
@pytest.mark.parametrize("out", [torch.float32, torch.float16])
def test_dot_softmax_batched(dev, layout, out):
    """Batched softmax: an fp32 output takes the tile kernels and the in-place
    row softmax (dot_softmax_rows), a 16-bit one dot_softmax16; both against
    the softmax of the fp64 product."""
    B, M, N, K = 3, 70, 300, 96
    da, db, a, b = _views(M, N, K, torch.bfloat16, layout, seed=47, batch=B)
    c = torch.empty(B, M, N, dtype=out, device=dev)
    tm.dot(da, db, c, "softmax")
    ref = oracle.dot(_np(a), _np(b), "softmax")
    if out == torch.float32:
        np.testing.assert_allclose(c.cpu().numpy(), ref, atol=1e-6, rtol=1e-4)
    else:
        np.testing.assert_allclose(c.float().cpu().numpy(), ref, atol=1e-3, rtol=1e-2)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N", [40, 700, 2048, 2049])
@pytest.mark.parametrize("out", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["trans_b", "row"])
def test_dot_softmax_16bit_output(dev, dt, N, out, layout):
    """softmax into a 16-bit C: rows of N <= 2048 on dot_softmax16 (16 whole
    fp32 product rows on chip; a row-major 16-bit B with N % 8 == 0 read in
    16-byte pieces, N = 40 leaving most of its one chunk past N), N = 2049 on
    dot_rows; against the softmax of the fp64 product, rounded once (half an
    ulp relative; fp16 subnormals absolute)."""
    B, M, K = 2, 37, 72
    da, db, a, b = _views(M, N, K, dt, layout, seed=N + 3, batch=B)
    da, a = (da.float() * 0.1).to(dt), (a.float() * 0.1).to(dt)
    c = torch.empty(B, M, N, dtype=out, device=dev)
    tm.dot(da, db, c, "softmax")
    ref = oracle.dot(_np(a), _np(b), "softmax")
    rel = 2.0 ** -11 if out == torch.float16 else 2.0 ** -8
    err = np.abs(c.double().cpu().numpy() - ref)
    assert (err <= (1e-4 + rel) * ref + 1e-7).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_dot_chain(dev, dt):
    M, N, K, L = 50, 64, 80, 24
    da, db, a, b = _views(M, N, K, dt, "strided", seed=47)
    w = _rand((N, L), 53, dt)
    c = torch.empty(M, L, dtype=torch.float32, device=dev)
    tm.dot(da, db, c, "chain-dot", w=w.to(dev).t().contiguous().t())  # W column-major
    ref = oracle.dot(_np(a), _np(b), "chain-dot", W=_np(w))
    absP = np.abs(_np(a)) @ np.abs(_np(b))
    bound = 1e-4 * np.abs(ref) + 2.0 ** -16 * (absP @ np.abs(_np(w)))
    assert (np.abs(c.cpu().numpy() - ref) <= bound).all()


def _chain_check(c, ref, absPW):
    """fp32 accumulation bound of both products; a 16-bit C adds its rounding
    (half an ulp: 2^-11 fp16, 2^-8 bf16 relative)."""
    got = c.double().cpu().numpy()
    rel = {torch.float32: 0.0, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[c.dtype]
    bound = (1e-4 + rel) * np.abs(ref) + 2.0 ** -16 * absPW
    err = np.abs(got - ref)
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst {(err / bound).max():.2f}"


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["row", "trans_a", "trans_b", "strided"])
@pytest.mark.parametrize("batch,M,N,K,L", [(None, 50, 64, 80, 24), (3, 70, 200, 96, 130),
                                           (3, 1100, 130, 40, 140)])
@pytest.mark.parametrize("out", ["f32", "in"])
def test_dot_chain_fused(dev, dt, layout, batch, M, N, K, L, out):
    """chain-dot on the fused kernel (C apart from A, B and W):
    ragged N and L (several 64-wide L tiles), batches, both C tile heights
    (16 rows; 32 once those make a workgroup per CU: 3 x 35 x 3 tiles), W of
    another dtype and layout, C in fp32 and in the input dtype."""
    da, db, a, b = _views(M, N, K, dt, layout, seed=M + N + L, batch=batch)
    wdt = torch.bfloat16 if dt == torch.float16 else torch.float32
    w = _rand((N, L), 59, wdt)
    dw = w.to(dev) if layout == "row" else w.t().contiguous().to(dev).t()
    odt = torch.float32 if out == "f32" else dt
    c = torch.empty(((batch,) if batch else ()) + (M, L), dtype=odt, device=dev)
    tm.dot(da, db, c, "chain-dot", w=dw)
    ref = oracle.dot(_np(a), _np(b), "chain-dot", W=_np(w))
    absPW = (np.abs(_np(a)) @ np.abs(_np(b))) @ np.abs(_np(w))
    _chain_check(c, ref.reshape(c.shape), absPW.reshape(c.shape))


@pytest.mark.parametrize("fmt", FP8)
def test_dot_chain_fused_fp8(dev, fmt):
    """chain-dot with FP8 inputs (codes over each format's whole range) on the
    fused kernel: P from the exactly decoded codes, unrounded, times an fp16 W."""
    M, N, K, L = 96, 150, 72, 40
    a = _fp8_codes((M, K), fmt, 81)
    b = _fp8_codes((K, N), fmt, 83)
    w = _rand((N, L), 85, torch.float16)
    c = torch.empty(M, L, dtype=torch.float32, device=dev)
    tm.dot(a.to(dev), b.t().contiguous().to(dev).t(), c, "chain-dot", w=w.to(dev), fp8_format=fmt)
    av, bv = oracle.fp8_decode(a.numpy(), fmt), oracle.fp8_decode(b.numpy(), fmt)
    ref = oracle.dot(av, bv, "chain-dot", W=_np(w))
    _chain_check(c, ref.reshape(c.shape), (np.abs(av) @ np.abs(bv)) @ np.abs(_np(w)))


@pytest.mark.parametrize("fmt", FP8)
@pytest.mark.parametrize("wlayout", ["row", "col"])
def test_dot_chain_fp8_w(dev, fmt, wlayout):
    """chain-dot with fp16 operands and an FP8 W (codes over the whole format):
    the fused kernel loads the aligned 4-byte word holding each code and
    decodes the code at its byte offset (all four occur in both layouts)."""
    M, N, K, L = 40, 90, 48, 37
    da, db, a, b = _views(M, N, K, torch.float16, "row", seed=89)
    w = _fp8_codes((N, L), fmt, 97)
    dw = w.to(dev) if wlayout == "row" else w.t().contiguous().to(dev).t()
    c = torch.empty(M, L, dtype=torch.float32, device=dev)
    tm.dot(da, db, c, "chain-dot", w=dw, fp8_format=fmt)
    wv = oracle.fp8_decode(w.numpy(), fmt)
    ref = oracle.dot(_np(a), _np(b), "chain-dot", W=wv)
    _chain_check(c, ref, (np.abs(_np(a)) @ np.abs(_np(b))) @ np.abs(wv))


def _fp8_codes(shape, fmt, seed):
    """Codes over the whole format, NaN / inf codes replaced by 0."""
    c = torch.randint(0, 256, shape, generator=_gen(seed), dtype=torch.uint8)
    v = oracle.fp8_decode(c.numpy(), fmt)
    c[torch.from_numpy(~np.isfinite(v))] = 0
    return c


@pytest.mark.parametrize("fmt", FP8)
@pytest.mark.parametrize("layout", ["row", "trans_b"])
def test_dot_fp8_formats(dev, fmt, layout):
    M, N, K = 96, 80, 160
    a = _fp8_codes((M, K), fmt, 61)
    b = _fp8_codes((K, N), fmt, 67)
    da = a.to(dev)
    db = b.to(dev) if layout == "row" else b.t().contiguous().to(dev).t()
    c = torch.empty(M, N, dtype=torch.float32, device=dev)
    tm.dot(da, db, c, fp8_format=fmt)
    av, bv = oracle.fp8_decode(a.numpy(), fmt), oracle.fp8_decode(b.numpy(), fmt)
    ref = oracle.dot(av, bv)
    _check(c, ref, torch.float32, np.abs(av), np.abs(bv))


@pytest.mark.parametrize("tdt,fmt", [(torch.float8_e4m3fn, "fp8e4nv"),
                                     (torch.float8_e5m2, "fp8e5")])
def test_matmul_fp8_c1_shape(dev, tdt, fmt):
    """tm_matmul with FP8 inputs (the reference's FP8 make_matmul_kernel: fp32
    output) at the C1 shape, torch's FP8 dtypes."""
    M = N = K = 512
    a = (torch.randn(M, K, generator=_gen(71)) * 2).to(tdt)
    b = (torch.randn(K, N, generator=_gen(73)) * 2).to(tdt)
    c = torch.empty(M, N, dtype=torch.float32, device=dev)
    tm.matmul(a.to(dev), b.to(dev), c, M, N, K)
    av, bv = a.double().numpy(), b.double().numpy()
    _check(c, av @ bv, torch.float32, np.abs(av), np.abs(bv))
