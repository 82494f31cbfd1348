"""Pin the oracle's dense matmul / linear (CPU only)."""
import numpy as np
import pytest

import oracle

MATMUL_KATS = ["matmul_seed789", "matmul_seed101r", "matmul_seed202", "matmul_seed42",
               "matmul_seed101g", "simdgroup_seed88", "simdgroup_seed303", "simdgroup_seed404",
               "simdgroup_seed505", "simdgroup_f16_seed707", "simdgroup_f16_seed808",
               "matmul2d_seed1001", "matmul2d_seed1002", "matmul2d_seed1003",
               "swizzled_seed2001", "swizzled_seed2002"]


@pytest.mark.parametrize("name", MATMUL_KATS)
def test_matmul_oracle_matches_reference_kat(kats, name):
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    out = oracle.matmul(a["A"].reshape(M, K), a["B"].reshape(K, N))
    np.testing.assert_allclose(out.ravel(), a["expected"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", ["linear_seed1111", "linear_seed2222"])
def test_linear_oracle_matches_reference_kat(kats, name):
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    out = oracle.linear(a["input"].reshape(M, K), a["weight"].reshape(N, K), a.get("bias"))
    np.testing.assert_allclose(out.ravel(), a["expected"], rtol=1e-12, atol=1e-12)


def test_identity_closed_form():
    # tests/test_emitter.py:4849 (I @ B = B) and tests/test_integration.py:346-377
    B = np.tile(np.arange(1, 17, dtype=np.float64), (16, 1))
    assert np.array_equal(oracle.matmul(np.eye(16), B), B)


def test_brute_force_non_symmetric():
    rng = np.random.default_rng(5)
    A, B = rng.standard_normal((3, 5)), rng.standard_normal((5, 4))
    C = oracle.matmul(A, B)
    for i in range(3):
        for j in range(4):
            assert abs(C[i, j] - sum(A[i, k] * B[k, j] for k in range(5))) < 1e-12
    # a transposed operand would not even have this shape
    assert C.shape == (3, 4)
