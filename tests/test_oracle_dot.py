"""Pins of oracle.fp8_decode and oracle.dot (CPU only).

fp8_decode: all 256 codes of every format against a scalar per-code decoder
written from the format definition with math.ldexp (a second formulation),
against torch's own float8_e4m3fn / float8_e5m2 decoders, and at each
format's closed-form extremes.  dot: brute-force loops over (b, m, n, k) for
every epilogue; a planted mistake in each epilogue must be caught.
"""
import math

import numpy as np
import pytest
import torch

import oracle


def scalar_decode(code: int, ebits: int, mbits: int, bias: int, has_inf: bool) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> mbits) & ((1 << ebits) - 1)
    m = code & ((1 << mbits) - 1)
    if e == (1 << ebits) - 1:
        if has_inf:
            return s * math.inf if m == 0 else math.nan
        if m == (1 << mbits) - 1:
            return math.nan
    if e == 0:
        return s * math.ldexp(m, 1 - bias - mbits)
    return s * math.ldexp((1 << mbits) + m, e - bias - mbits)


@pytest.mark.parametrize("fmt", sorted(oracle.FP8_FORMATS))
def test_fp8_decode_all_codes(fmt):
    eb, mb, bias, inf = oracle.FP8_FORMATS[fmt]
    got = oracle.fp8_decode(np.arange(256), fmt)
    want = np.array([scalar_decode(c, eb, mb, bias, inf) for c in range(256)])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    # every finite value is exactly representable in fp16 (the kernels decode to fp16)
    fin = np.isfinite(got)
    assert np.array_equal(got[fin].astype(np.float16).astype(np.float64), got[fin])


@pytest.mark.parametrize("fmt,tdt", [("fp8e4nv", torch.float8_e4m3fn),
                                     ("fp8e5", torch.float8_e5m2)])
def test_fp8_decode_matches_torch(fmt, tdt):
    tv = torch.arange(256, dtype=torch.uint8).view(tdt).double().numpy()
    ov = oracle.fp8_decode(np.arange(256), fmt)
    assert np.array_equal(np.isnan(tv), np.isnan(ov))
    assert np.array_equal(tv[~np.isnan(tv)], ov[~np.isnan(ov)])


def test_fp8_decode_extremes():
    d = oracle.fp8_decode
    assert d([0x7E], "fp8e4nv")[0] == 448.0 and np.isnan(d([0x7F], "fp8e4nv")[0])
    assert d([0x01], "fp8e4nv")[0] == 2.0 ** -9
    assert d([0x7B], "fp8e5")[0] == 57344.0 and d([0x7C], "fp8e5")[0] == np.inf
    assert d([0x01], "fp8e5")[0] == 2.0 ** -16
    assert d([0x7E], "fp8e4b15")[0] == 1.75 and d([0x01], "fp8e4b15")[0] == 2.0 ** -17
    assert d([0x7E], "fp8e4b8")[0] == 224.0 and d([0x01], "fp8e4b8")[0] == 2.0 ** -10
    assert d([0x7B], "fp8e5b16")[0] == 57344.0 / 2 and d([0x01], "fp8e5b16")[0] == 2.0 ** -17
    assert d([0x80], "fp8e4nv")[0] == 0.0 and math.copysign(1, d([0x80], "fp8e4nv")[0]) < 0


def brute_dot(A, B, epilogue, Z=None, W=None):
    """Loops over (b, m, n, k) in the order of the reference's strided template."""
    A3 = A[None] if A.ndim == 2 else A
    B3 = B[None] if B.ndim == 2 else B
    Z3 = None if Z is None else (Z[None] if Z.ndim == 2 else Z)
    nb, M, K = A3.shape
    N = B3.shape[2]
    out = np.zeros((nb, M, N if epilogue != "chain-dot" else W.shape[1]))
    for b in range(nb):
        P = np.zeros((M, N))
        for m in range(M):
            for n in range(N):
                acc = 0.0
                if epilogue == "add-matrix":
                    acc = Z3[b, m, n]
                elif epilogue == "add-rows":
                    acc = Z3[b, m, 0]
                elif epilogue == "add-cols":
                    acc = Z3[b, 0, n]
                for k in range(K):
                    acc += A3[b, m, k] * B3[b, k, n]
                P[m, n] = acc
        if epilogue == "softmax":
            for m in range(M):
                mx = max(P[m])
                den = sum(math.exp(x - mx) for x in P[m])
                out[b, m] = [math.exp(x - mx) / den for x in P[m]]
        elif epilogue == "chain-dot":
            L = W.shape[1]
            for m in range(M):
                for l in range(L):
                    out[b, m, l] = sum(P[m, n] * W[n, l] for n in range(N))
        else:
            out[b] = P
    return out if A.ndim == 3 else out[0]


@pytest.mark.parametrize("epilogue", oracle.DOT_EPILOGUES)
@pytest.mark.parametrize("batched", [False, True])
def test_dot_brute_force(epilogue, batched):
    rng = np.random.default_rng(3)
    shp = (2,) if batched else ()
    M, N, K, L = 5, 7, 6, 4
    A = rng.standard_normal(shp + (M, K))
    B = rng.standard_normal(shp + (K, N))
    Z = rng.standard_normal(shp + (M, N))
    W = rng.standard_normal((N, L))
    got = oracle.dot(A, B, epilogue, Z=Z, W=W)
    want = brute_dot(A, B, epilogue, Z=Z, W=W)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    if epilogue == "softmax":
        np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-12)


def test_dot_planted_mistakes_are_caught():
    rng = np.random.default_rng(4)
    A, B = rng.standard_normal((5, 6)), rng.standard_normal((6, 7))
    Z, W = rng.standard_normal((5, 7)), rng.standard_normal((7, 3))
    P = A @ B
    wrong = {
        "add-rows": P + Z[:1, :5].T,            # a row of Z read as the row bias
        "add-cols": P + Z[:, :1],               # rows and columns swapped
        "softmax": np.exp(P) / np.exp(P).sum(0, keepdims=True),  # over the wrong axis
        "chain-dot": P @ W[::-1],               # W rows reversed
        "add-matrix": P - Z,                    # wrong sign
    }
    for epi, w in wrong.items():
        want = brute_dot(A, B, epi, Z=Z, W=W)
        assert not np.allclose(w, want), epi
        np.testing.assert_allclose(oracle.dot(A, B, epi, Z=Z, W=W), want, rtol=1e-12, atol=1e-12)
