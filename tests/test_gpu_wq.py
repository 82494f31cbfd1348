"""W8A16 / W4A16 parity on the GPU against the oracle.

Tolerances: fp16/bf16 outputs within atol 2e-2 / rtol 1e-2 of the oracle's
fp32-dequant, fp64-accumulated result; dequantised weights bit-exact.
The reference's own known-answer tests run with the reference's tolerances.
"""
import numpy as np
import pytest
import torch

import oracle
import triton_metal_amd as tm
from triton_metal_amd import _lib

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def make_int4_problem(M, N, K, G, seed, act=torch.float16, zeros="f16"):
    g = _gen(seed)
    x = torch.randn(M, K, generator=g).to(act)
    q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_int4(q.numpy()))
    ng = (K + G - 1) // G
    s = (torch.rand(N, ng, generator=g) * 0.019 + 0.001).to(act)
    zi = torch.randint(0, 16, (N, ng), generator=g)
    z = None if zeros is None else (zi.to(torch.uint8) if zeros == "u8" else zi.to(act))
    return x, q, packed, s, z


def make_int8_problem(M, N, K, seed, act=torch.float16, zeros=None):
    g = _gen(seed)
    x = torch.randn(M, K, generator=g).to(act)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) * 0.019 + 0.001).to(act)
    z = None if zeros is None else torch.randint(-3, 4, (N,), generator=g).to(act)
    return x, w, s, z


def np32(t):
    return None if t is None else t.float().numpy()


def check_close(got, ref, atol=ATOL, rtol=RTOL):
    got = got.float().cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got, ref, atol=atol, rtol=rtol)


# --- reference known-answer tests ---------------------------------------------
@pytest.mark.parametrize("name", ["int4_seed7070", "int4_seed44"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_int4_reference_kat(kats, dev, name, dtype):
    m, a = kats[name]
    M, N, K, G = m["M"], m["N"], m["K"], m["G"]
    x = torch.tensor(a["input"], dtype=dtype, device=dev).reshape(M, K)
    w = torch.tensor(a["packed"].astype(np.uint8), device=dev).reshape(N, K // 2)
    s = torch.tensor(a["scales"], dtype=dtype, device=dev)
    z = torch.tensor(a["zeros"], dtype=dtype, device=dev)
    out = torch.empty(M, N, dtype=dtype, device=dev)
    tm.make_int4_matmul_kernel(group_size=G)(x, w, out, s, z, M, N, K)
    torch.cuda.synchronize()
    err = np.abs(out.float().cpu().numpy().ravel() - a["expected"]).max()
    assert err < m["tol"]
    if dtype == torch.float32:
        assert err < 1e-4


@pytest.mark.parametrize("name", ["int8_seed8888", "int8_seed66"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_int8_reference_kat(kats, dev, name, dtype):
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    x = torch.tensor(a["input"], dtype=dtype, device=dev).reshape(M, K)
    w = torch.tensor(a["weight"].astype(np.int8), device=dev).reshape(N, K)
    s = torch.tensor(a["scales"], dtype=dtype, device=dev)
    z = torch.tensor(a["zeros"], dtype=dtype, device=dev)
    out = torch.empty(M, N, dtype=dtype, device=dev)
    tm.make_int8_matmul_kernel()(x, w, out, s, z, M, N, K)
    torch.cuda.synchronize()
    err = np.abs(out.float().cpu().numpy().ravel() - a["expected"]).max()
    assert err < m["tol"]
    if dtype == torch.float32:
        assert err < 1e-4


# --- dequantised weights are bit-exact ------------------------------------------
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int4_dequant_tile_bit_exact(dev, act):
    N, K, G = 96, 512, 128
    _, q, packed, s, z = make_int4_problem(1, N, K, G, seed=11, act=act)
    ref = torch.from_numpy(oracle.dequant_int4(packed.numpy(), np32(s), np32(z), K, G)).to(act)
    got = tm.wq_dequant(packed.to(dev), s.to(dev), z.to(dev), N, K, 4, G, out_dtype=act)
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


# (M, K, N) of each kernel kind: the stream kernel takes 1 < M <= 64 with
# K <= 4096; the GEMV M = 1 and K = 8192; the two-tile GEMV int4 2 <= M <= 6
# at K = 4096 with N % 32 == 0; skinny the remaining M <= 8 shapes with
# K % 512 == 0; wide M > 64 with fp16 activations and N % 128 == 0 (int8: no
# zero-points); tiled the other M > 64 shapes.
INT4_KINDS = {"skinny": (8, 5120, 64), "gemv": (1, 4096, 64), "gemv8k": (8, 8192, 64),
              "gemv2t": (4, 4096, 64),
              "stream8": (8, 4096, 64), "stream16": (16, 2048, 64),
              "stream_multi": (40, 2048, 64), "tiled": (72, 512, 64), "wide": (100, 1024, 256)}
INT8_KINDS = {"skinny": (8, 768, 64), "gemv": (1, 4096, 64), "stream8": (8, 2048, 64),
              "stream16": (16, 2048, 64),
              "stream_multi": (40, 1024, 64), "tiled": (72, 512, 64), "wide": (100, 1024, 256)}


@pytest.mark.parametrize("kind", list(INT4_KINDS))
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int4_in_register_dequant_bit_exact(dev, kind, act):
    """One-hot activation rows make each output equal one dequantised weight,
    so the GEMM's in-register dequantisation is compared bit for bit."""
    G = 128
    M, K, N = INT4_KINDS[kind]
    _, q, packed, s, z = make_int4_problem(M, N, K, G, seed=12, act=act)
    ks = torch.randperm(K, generator=_gen(3))[:M]
    x = torch.zeros(M, K, dtype=act)
    x[torch.arange(M), ks] = 1.0
    ref = torch.from_numpy(oracle.dequant_int4(packed.numpy(), np32(s), np32(z), K, G)).to(act)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    assert torch.equal(out.cpu().view(torch.int16), ref[:, ks].T.contiguous().view(torch.int16))


@pytest.mark.parametrize("kind", list(INT8_KINDS))
def test_int8_in_register_dequant_bit_exact(dev, kind):
    M, K, N = INT8_KINDS[kind]
    _, w, s, _ = make_int8_problem(M, N, K, seed=13)
    ks = torch.randperm(K, generator=_gen(4))[:M]
    x = torch.zeros(M, K, dtype=torch.float16)
    x[torch.arange(M), ks] = 1.0
    ref = torch.from_numpy(oracle.dequant_int8(w.numpy(), np32(s), None)).half()
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None, M, N, K)
    assert torch.equal(out.cpu().view(torch.int16), ref[:, ks].T.contiguous().view(torch.int16))


# --- fused bias (nn.Linear form) on every kernel kind ------------------------------
@pytest.mark.parametrize("kind", list(INT4_KINDS))
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int4_linear_bias(dev, kind, act):
    G = 128
    M, K, N = INT4_KINDS[kind]
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=40 + M, act=act)
    bias = (torch.randn(N, generator=_gen(41)) * 4).to(act)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int4_linear(x.to(dev), packed.to(dev), bias.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref + np32(bias)[None, :].astype(np.float64))
    # without a bias the linear entry is the matmul, bit for bit
    plain = torch.empty_like(out)
    tm.int4_matmul(x.to(dev), packed.to(dev), plain, s.to(dev), z.to(dev), M, N, K, G)
    tm.int4_linear(x.to(dev), packed.to(dev), None, out, s.to(dev), z.to(dev), M, N, K, G)
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))


@pytest.mark.parametrize("kind", list(INT8_KINDS))
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int8_linear_bias(dev, kind, act):
    M, K, N = INT8_KINDS[kind]
    x, w, s, _ = make_int8_problem(M, N, K, seed=50 + M, act=act)
    bias = (torch.randn(N, generator=_gen(51)) * 4).to(act)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int8_linear(x.to(dev), w.to(dev), bias.to(dev), out, s.to(dev), None, M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), None, M, N, K)
    check_close(out.cpu(), ref + np32(bias)[None, :].astype(np.float64))


def test_int4_linear_fp32_general_kernel(dev):
    """fp32 activations take the fp32 kernel; its bias is fp32 too."""
    M, N, K, G = 3, 48, 256, 64
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=61, act=torch.float32)
    bias = torch.randn(N, generator=_gen(62))
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    tm.int4_linear(x.to(dev), packed.to(dev), bias.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    np.testing.assert_allclose(out.cpu().numpy(), ref + bias.numpy()[None, :], rtol=1e-4,
                               atol=1e-4)


def test_linear_bias_dtype_checked(dev):
    x, q, packed, s, z = make_int4_problem(2, 64, 256, 128, seed=63)
    out = torch.empty(2, 64, dtype=torch.float16, device=dev)
    with pytest.raises(TypeError):
        tm.int4_linear(x.to(dev), packed.to(dev), torch.zeros(64, device=dev), out, s.to(dev),
                       z.to(dev), 2, 64, 256, 128)
    with pytest.raises(ValueError):
        tm.int4_linear(x.to(dev), packed.to(dev), torch.zeros(8, dtype=torch.float16, device=dev),
                       out, s.to(dev), z.to(dev), 2, 64, 256, 128)


# --- benchmark configurations (a column subset is checked against the oracle) ----
def _cols(N, n=384, seed=0):
    return np.sort(np.random.default_rng(seed).choice(N, n, replace=False))


@pytest.mark.parametrize("M,K,zeros", [(2, 8192, "f16"), (3, 4096, "u8"), (5, 4096, None),
                                       (1, 8192, None), (1, 4096, "u8"), (1, 4096, None),
                                       (1, 8192, "u8")])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int4_gemv_shapes(dev, M, K, zeros, act):
    N, G = 1024, 128
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=M * 31 + K, zeros=zeros, act=act)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref)


# The persistent GEMV (M = 1, K = 4096, G = 128) picks rows per wave RW from
# {4, 7, 8, 11, 12, 14, 16} so that ceil(N / 4 RW) workgroups fit the CUs; these
# N reach every RW on a 256-CU part, a grid of one workgroup, and a last
# workgroup shifted back over its neighbour's rows (N not a multiple of 4 RW).
@pytest.mark.parametrize("N", [16, 48, 1040, 4112, 8208, 11008, 12304, 14336, 16384])
@pytest.mark.parametrize("zeros,act", [("f16", torch.float16), (None, torch.float16),
                                       ("u8", torch.bfloat16), ("f16", torch.bfloat16)])
def test_int4_persistent_gemv(dev, N, zeros, act):
    K, G = 4096, 128
    x, q, packed, s, z = make_int4_problem(1, N, K, G, seed=N + 7, zeros=zeros, act=act)
    bias = (torch.randn(N, generator=_gen(N)) * 0.5).to(act)
    out = torch.empty(1, N, dtype=act, device=dev)
    tm.int4_linear(x.to(dev), packed.to(dev), bias.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), 1, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), 1, N, K, G)
    check_close(out.cpu(), ref + np32(bias)[None, :].astype(np.float64))


@pytest.mark.parametrize("M", [1, 8, 32, 128])
def test_w4a16_config_c3(dev, M):
    """C3 at full size, every output column against the oracle."""
    N, K, G = 14336, 4096, 128
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=100 + M)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref)


@pytest.mark.parametrize("M", [1, 16, 128])
def test_w8a16_config_c2(dev, M):
    """C2 at full size, every output column against the oracle."""
    N, K = 11008, 4096
    x, w, s, _ = make_int8_problem(M, N, K, seed=200 + M)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None, M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), None, M, N, K)
    check_close(out.cpu(), ref)


# --- edge cases -------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K,G", [(3, 48, 512, 128), (5, 64, 1024, 64), (9, 64, 512, 32),
                                     (17, 128, 768, 128), (65, 64, 256, 128), (1, 40, 512, 128),
                                     (2, 64, 200, 40), (4, 24, 64, 16)])
@pytest.mark.parametrize("zeros", ["f16", "u8", None])
def test_int4_shapes_and_zero_types(dev, M, N, K, G, zeros):
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=M * 7 + N, zeros=zeros)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref)


@pytest.mark.parametrize("M,N", [(4, 64), (80, 256)])
def test_int4_fractional_zero_points(dev, M, N):
    """Non-integer zero-points take the fp32 formula path (lane by lane in the
    skinny kernels, per chunk in the wide kernel)."""
    K, G = 1024, 128
    x, q, packed, s, _ = make_int4_problem(M, N, K, G, seed=21)
    z = (torch.rand(N, K // G, generator=_gen(22)) * 8).half()
    z[::2] = z[::2].round()  # mix integral and fractional rows
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref)
    deq = tm.wq_dequant(packed.to(dev), s.to(dev), z.to(dev), N, K, 4, G)
    refd = torch.from_numpy(oracle.dequant_int4(packed.numpy(), np32(s), np32(z), K, G)).half()
    assert torch.equal(deq.cpu().view(torch.int16), refd.view(torch.int16))


@pytest.mark.parametrize("M", [1, 7, 33])
def test_int4_bf16_activations(dev, M):
    N, K, G = 128, 1024, 128
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=31, act=torch.bfloat16)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (16, 128, 512), (3, 40, 100), (70, 64, 256)])
@pytest.mark.parametrize("zeros", [False, True])
def test_int8_shapes(dev, M, N, K, zeros):
    x, w, s, z = make_int8_problem(M, N, K, seed=M + N + K, zeros=zeros or None)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None if z is None else z.to(dev),
                   M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K)
    check_close(out.cpu(), ref)


# --- int8 GEMV (M = 1, K = 4096): every zero-point form, both activation dtypes,
# the full int8 range (-128 included) and a fused bias
@pytest.mark.parametrize("zeros", [None, "f16", "u8"])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int8_gemv_zero_forms(dev, zeros, act):
    M, N, K = 1, 1040, 4096
    g = _gen(77)
    x = torch.randn(M, K, generator=g).to(act)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    w[:, :64] = -128
    w[:, 64:128] = 127
    s = (torch.rand(N, generator=g) * 0.019 + 0.001).to(act)
    zi = torch.randint(0, 9, (N,), generator=g)
    z = None if zeros is None else (zi.to(torch.uint8) if zeros == "u8" else (zi - 4).to(act))
    bias = (torch.randn(N, generator=g) * 4).to(act)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None if z is None else z.to(dev),
                   M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K)
    check_close(out.cpu(), ref)
    tm.int8_linear(x.to(dev), w.to(dev), bias.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), M, N, K)
    check_close(out.cpu(), ref + np32(bias)[None, :].astype(np.float64))


# --- two-tile GEMV (int4, 2 <= M <= 6, K = 4096, N % 32 == 0) --------------------
@pytest.mark.parametrize("M,N", [(2, 32), (3, 96), (5, 64), (6, 160)])
@pytest.mark.parametrize("zeros", ["f16", "u8", None])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int4_two_tile_gemv_shapes(dev, M, N, zeros, act):
    K, G = 4096, 128
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=M * 17 + N, act=act, zeros=zeros)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref, atol=ATOL)


def test_int4_two_tile_gemv_fractional_zero_points(dev):
    """The zero-point enters the correction in fp32, so non-integer values
    are exact as in the reference formula."""
    M, N, K, G = 6, 64, 4096, 128
    x, q, packed, s, _ = make_int4_problem(M, N, K, G, seed=23)
    z = (torch.rand(N, K // G, generator=_gen(24)) * 8).half()
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev), z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref)


# --- stream kernel (1 < M <= 128 for int4, 64 for int8; K = 512..4096 by 512) -----
# N not a multiple of the workgroup's columns (int4: 64, int8: 48) leaves a
# partial last workgroup.
@pytest.mark.parametrize("M,N,K", [(2, 64, 512), (8, 80, 4096), (9, 128, 1024), (16, 128, 4096),
                                   (17, 80, 2048), (32, 128, 1536), (33, 64, 4096),
                                   (64, 128, 1024), (100, 64, 1024), (128, 80, 2048)])
@pytest.mark.parametrize("zeros", ["f16", "u8", None])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int4_stream_shapes(dev, M, N, K, zeros, act):
    G = 128
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=M * 13 + K + N, act=act, zeros=zeros)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(2, 48, 512), (8, 208, 4096), (9, 32, 1024), (16, 96, 4096),
                                   (31, 64, 2048), (64, 32, 1536)])
@pytest.mark.parametrize("zeros", [False, True])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int8_stream_shapes(dev, M, N, K, zeros, act):
    x, w, s, z = make_int8_problem(M, N, K, seed=M + N + K, act=act, zeros=zeros or None)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None if z is None else z.to(dev),
                   M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K)
    check_close(out.cpu(), ref, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(65, 128, 512), (128, 256, 4096), (200, 384, 2048),
                                   (300, 128, 1024)])
@pytest.mark.parametrize("zeros", ["f16", "u8", None])
def test_int4_wide_shapes(dev, M, N, K, zeros):
    G = 128
    x, q, packed, s, z = make_int4_problem(M, N, K, G, seed=M * 5 + N + K, zeros=zeros)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_matmul(x.to(dev), packed.to(dev), out, s.to(dev),
                   None if z is None else z.to(dev), M, N, K, G)
    ref = oracle.int4_matmul(np32(x), packed.numpy(), np32(s), np32(z), M, N, K, G)
    check_close(out.cpu(), ref)


@pytest.mark.parametrize("M,N,K", [(65, 128, 256), (100, 256, 1024), (128, 128, 4096),
                                   (257, 384, 768)])
def test_int8_wide_shapes(dev, M, N, K):
    x, w, s, _ = make_int8_problem(M, N, K, seed=M + 3 * N + K)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None, M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), None, M, N, K)
    check_close(out.cpu(), ref)


@pytest.mark.parametrize("N", [16, 208])
@pytest.mark.parametrize("zeros", [False, True])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_int8_gemv_shapes(dev, N, zeros, act):
    """The int8 GEMV (M = 1, K = 4096), with and without per-channel zero-points."""
    M, K = 1, 4096
    x, w, s, z = make_int8_problem(M, N, K, seed=N + 7 * zeros, act=act, zeros=zeros or None)
    out = torch.empty(M, N, dtype=act, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), None if z is None else z.to(dev),
                   M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K)
    check_close(out.cpu(), ref, atol=ATOL)


def test_int8_stream_u8_zero_points(dev):
    """int8 with uint8 zero-points through the stream kernel (one per channel)."""
    M, N, K = 12, 80, 1024
    x, w, s, _ = make_int8_problem(M, N, K, seed=5)
    z = torch.randint(0, 5, (N,), generator=_gen(6), dtype=torch.uint8)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int8_matmul(x.to(dev), w.to(dev), out, s.to(dev), z.to(dev), M, N, K)
    ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K)
    check_close(out.cpu(), ref)


def test_empty_and_errors(dev):
    x = torch.zeros(0, 512, dtype=torch.float16, device=dev)
    w = torch.zeros(64, 256, dtype=torch.uint8, device=dev)
    s = torch.ones(64, 4, dtype=torch.float16, device=dev)
    out = torch.empty(0, 64, dtype=torch.float16, device=dev)
    tm.int4_matmul(x, w, out, s, None, 0, 64, 512, 128)  # no-op
    with pytest.raises(TypeError):
        tm.int4_matmul(x.float(), w, out, s, None, 0, 64, 512, 128)
    with pytest.raises(ValueError):
        tm.int4_matmul(x.cpu(), w, out, s, None, 0, 64, 512, 128)


# --- GPTQ / AWQ checkpoints into the int4 layout -------------------------------------
@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2", "awq"])
@pytest.mark.parametrize("N,K,G", [(64, 256, 128), (1000, 520, 8), (512, 4096, 128)])
def test_checkpoint_repack_bit_exact(dev, fmt, N, K, G):
    rng = np.random.default_rng(N + K)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    ng = (K + G - 1) // G
    z = rng.integers(1, 16, size=(N, ng))
    s = (rng.random((ng, N)) * 0.02 + 0.001).astype(np.float16)
    if fmt == "awq":
        qw, qz = oracle.pack_awq(q, z)
        ref = oracle.awq_to_ref(qw, qz, s, N, K, G)
        got = tm.from_awq(torch.from_numpy(qw).to(dev), torch.from_numpy(qz).to(dev),
                          torch.from_numpy(s).to(dev), group_size=G)
    else:
        off = 1 if fmt == "gptq" else 0
        qw, qz = oracle.pack_gptq(q, z, zero_offset=off)
        ref = oracle.gptq_to_ref(qw, qz, s, N, K, G, zero_offset=off)
        got = tm.from_gptq(torch.from_numpy(qw).to(dev), torch.from_numpy(qz).to(dev),
                           torch.from_numpy(s).to(dev), group_size=G, zero_offset=off)
    torch.cuda.synchronize()
    assert np.array_equal(got[0].cpu().numpy(), ref[0])
    assert np.array_equal(got[1].cpu().numpy(), ref[1])
    assert np.array_equal(got[2].cpu().numpy().astype(np.int64), ref[2])


def test_gptq_checkpoint_through_the_gemv(dev):
    """A GPTQ checkpoint loaded with from_gptq runs through the M = 1 GEMV and
    matches (q - z) s of the checkpoint."""
    N, K, G, M = 256, 4096, 128, 1
    rng = np.random.default_rng(5)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    z = rng.integers(1, 16, size=(N, K // G))
    s = (rng.random((K // G, N)) * 0.019 + 0.001).astype(np.float16)
    qw, qz = oracle.pack_gptq(q, z, zero_offset=1)
    w, sc, zz = tm.from_gptq(torch.from_numpy(qw).to(dev), torch.from_numpy(qz).to(dev),
                             torch.from_numpy(s).to(dev), group_size=G)
    x = torch.randn(M, K, generator=_gen(6)).half()
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_matmul(x.to(dev), w, out, sc, zz, M, N, K, G)
    ref = oracle.int4_matmul(np32(x), oracle.pack_int4(q), s.T.astype(np.float32),
                             z.astype(np.float32), M, N, K, G)
    check_close(out.cpu(), ref)


def test_act_order_checkpoint_rejected(dev):
    N, K, G = 64, 256, 128
    qw = torch.zeros(K // 8, N, dtype=torch.int32, device=dev)
    s = torch.ones(K // G, N, dtype=torch.float16, device=dev)
    trivial = torch.arange(K, dtype=torch.int32, device=dev) // G
    tm.from_gptq(qw, None, s, group_size=G, g_idx=trivial)
    with pytest.raises(ValueError):
        tm.from_gptq(qw, None, s, group_size=G, g_idx=trivial.flip(0))


# --- every W-only kernel the dispatcher can select (tests/wq_cases.py) -----------
from wq_cases import CASES, case_id, plan  # noqa: E402


@pytest.fixture(scope="module")
def cu_count(dev):
    return torch.cuda.get_device_properties(dev).multi_processor_count


def _plain_c_call(qbits, x, w, bias, out, s, z, M, N, K, G=128):
    """The call through tm_int{4,8}_linear (bias NULL: the plain matmul), the C
    entry points without a workspace."""
    L = _lib.lib()
    dts = {torch.float16: _lib.TM_DT_F16, torch.bfloat16: _lib.TM_DT_BF16,
           torch.float32: _lib.TM_DT_F32, torch.uint8: _lib.TM_DT_U8, None: _lib.TM_DT_NONE}
    p = lambda t: None if t is None else t.data_ptr()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    zdt = dts[None if z is None else z.dtype]
    if qbits == 4:
        rc = L.tm_int4_linear(p(x), p(w), p(bias), p(out), p(s), p(z), M, N, K, G, dts[x.dtype],
                              dts[s.dtype], zdt, stream)
    else:
        rc = L.tm_int8_linear(p(x), p(w), p(bias), p(out), p(s), p(z), M, N, K, dts[x.dtype],
                              dts[s.dtype], zdt, stream)
    _lib.check(rc, "plain C call")
    torch.cuda.synchronize()


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_dispatch_case(dev, cu_count, case):
    """Each case against the oracle (a column sample when N is large), with the
    bias form on alternate cases; the kernel it reaches is named by tm_wq_plan
    for this device, and on a 256-CU part is the kernel the CPU coverage test
    counts."""
    qbits, M, N, K, G, act, zeros, ws = case
    name = plan(case, cu_count)
    if cu_count == 256:
        assert name == plan(case)
    print(f"[wq case] {case_id(case)} -> {name}", flush=True)
    seed = (M * 131 + N * 7 + K) % 100003
    use_bias = seed % 2 == 0
    bias = (torch.randn(N, generator=_gen(seed)) * 0.5).to(act) if use_bias else None
    out = torch.empty(M, N, dtype=act, device=dev)
    cols = _cols(N) if N > 2048 else np.arange(N)
    if qbits == 4:
        g = _gen(seed)
        x = torch.randn(M, K, generator=g).to(act)
        packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
        ng = (K + G - 1) // G
        s = (torch.rand(N, ng, generator=g) * 0.019 + 0.001).to(act)
        zi = torch.randint(0, 16, (N, ng), generator=g)
        z = None if zeros is None else zi.to(torch.uint8 if zeros == "u8" else act)
        args = (packed.to(dev), out, s.to(dev), None if z is None else z.to(dev), M, N, K, G)
        if not ws:
            _plain_c_call(4, x.to(dev), args[0], None if bias is None else bias.to(dev), *args[1:])
        elif use_bias:
            tm.int4_linear(x.to(dev), args[0], bias.to(dev), *args[1:])
        else:
            tm.int4_matmul(x.to(dev), *args)
        ref = oracle.int4_matmul(np32(x), packed.numpy()[cols], np32(s)[cols],
                                 None if z is None else np32(z)[cols], M, len(cols), K, G)
    else:
        x, w, s, _ = make_int8_problem(M, N, K, seed=seed, act=act)
        z = None
        if zeros == "s":
            z = torch.randint(-3, 4, (N,), generator=_gen(seed + 1)).to(act)
        elif zeros == "u8":
            z = torch.randint(0, 5, (N,), generator=_gen(seed + 1)).to(torch.uint8)
        args = (w.to(dev), out, s.to(dev), None if z is None else z.to(dev), M, N, K)
        if not ws:
            _plain_c_call(8, x.to(dev), args[0], None if bias is None else bias.to(dev), *args[1:])
        elif use_bias:
            tm.int8_linear(x.to(dev), args[0], bias.to(dev), *args[1:])
        else:
            tm.int8_matmul(x.to(dev), *args)
        ref = oracle.int8_matmul(np32(x), w.numpy()[cols], np32(s)[cols],
                                 None if z is None else np32(z)[cols], M, len(cols), K)
    if use_bias:
        ref = ref + np32(bias)[cols][None, :].astype(np.float64)
    check_close(out.cpu()[:, cols], ref)


# --- split-K: the workspace contract and graph replays -----------------------------
SPLIT_SHAPES = {"streamk": (24, 1040, 20480), "wide": (128, 1024, 14336)}


def _split_problem(dev, shape, seed):
    M, N, K = shape
    x, _, packed, s, z = make_int4_problem(M, N, K, 128, seed=seed)
    return [t.to(dev) for t in (x, packed, s, z)]


@pytest.mark.parametrize("kind", list(SPLIT_SHAPES))
def test_split_k_workspace_contract(dev, kind):
    """tm_wq_matmul_ws: a split-K plan refuses a workspace smaller than
    tm_wq_workspace_bytes (nothing launched), runs with exactly that many
    bytes, and without a workspace takes the single-launch plan; the three
    results agree with the oracle, and the split and unsplit sums to within
    the output rounding."""
    M, N, K = SPLIT_SHAPES[kind]
    x, packed, s, z = _split_problem(dev, SPLIT_SHAPES[kind], seed=61)
    L = _lib.lib()
    args = (_lib.TM_DT_F16, _lib.TM_DT_F16, _lib.TM_DT_F16)
    need = L.tm_wq_workspace_bytes(4, x.data_ptr(), packed.data_ptr(), s.data_ptr(), z.data_ptr(),
                                   M, N, K, 128, *args)
    assert need == tm.wq_kernel_for(4, M, N, K, zero_dtype=torch.float16,
                                    details=True)["workspace_bytes"] > 0
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = torch.full((M, N), 7.0, dtype=torch.float16, device=dev)
    small = torch.empty(need - 16, dtype=torch.uint8, device=dev)
    rc = L.tm_wq_matmul_ws(4, x.data_ptr(), packed.data_ptr(), None, out.data_ptr(), s.data_ptr(),
                           z.data_ptr(), M, N, K, 128, *args, small.data_ptr(), need - 16, stream)
    torch.cuda.synchronize()
    assert rc == _lib.TM_ERR_INVALID_ARG and "workspace" in _lib.last_error()
    assert bool((out == 7.0).all()), "nothing may run when the workspace is refused"
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    rc = L.tm_wq_matmul_ws(4, x.data_ptr(), packed.data_ptr(), None, out.data_ptr(), s.data_ptr(),
                           z.data_ptr(), M, N, K, 128, *args, ws.data_ptr(), need, stream)
    assert rc == 0
    plain = torch.empty_like(out)
    _plain_c_call(4, x, packed, None, plain, s, z, M, N, K)
    ref = oracle.int4_matmul(np32(x.cpu()), packed.cpu().numpy(), np32(s.cpu()), np32(z.cpu()),
                             M, N, K, 128)
    check_close(out.cpu(), ref)
    check_close(plain.cpu(), ref)
    diff = (out.float() - plain.float()).abs().max().item()
    assert diff <= 2 ** -10 * plain.float().abs().max().item() + 1e-3, diff


@pytest.mark.parametrize("kind", list(SPLIT_SHAPES))
def test_split_k_output_view_off_8_byte_alignment(dev, kind):
    """The split-K reduction writes an output view that starts 2 bytes into
    its buffer (so its 4-output groups are not 8-byte aligned), with a bias:
    bit for bit the aligned call's result, and the element before the view is
    untouched."""
    M, N, K = SPLIT_SHAPES[kind]
    x, packed, s, z = _split_problem(dev, SPLIT_SHAPES[kind], seed=67)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(68)) * 0.1).half().to(dev)
    assert tm.wq_kernel_for(4, M, N, K, zero_dtype=torch.float16, details=True)["splits"] > 1
    ref = torch.empty(M, N, dtype=torch.float16, device=dev)
    tm.int4_linear(x, packed, bias, ref, s, z, M, N, K, 128)
    buf = torch.full((M * N + 1,), 3.0, dtype=torch.float16, device=dev)
    out = buf[1:].view(M, N)
    assert out.data_ptr() % 8 == 2
    tm.int4_linear(x, packed, bias, out, s, z, M, N, K, 128)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert buf[0].item() == 3.0


@pytest.mark.parametrize("kind", list(SPLIT_SHAPES))
def test_split_k_graph_replays_track_new_inputs(dev, kind):
    """A split-K call (two launches and the workspace the plan holds) captured
    in a HIP graph and replayed three times with new inputs copied in and eager
    work in between: every replay equals the eager call bit for bit."""
    M, N, K = SPLIT_SHAPES[kind]
    x, packed, s, z = _split_problem(dev, SPLIT_SHAPES[kind], seed=71)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    plan = tm.plan_int4_matmul(x, packed, out, s, z, M, N, K, 128)
    assert plan._keep is not None  # the split plan's workspace
    plan()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=cap):
        plan(torch.cuda.current_stream().cuda_stream)
    for seed in (72, 73, 74):
        new = _split_problem(dev, SPLIT_SHAPES[kind], seed=seed)
        for dst, src in zip((x, packed, s, z), new):
            dst.copy_(src)
        eager = torch.empty_like(out)
        tm.int4_matmul(*new[:2], eager, *new[2:], M, N, K, 128)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {seed}"
    del graph
