"""Pin the oracle's KDA chunked gated delta rule (CPU only).

The reference has no KDA, so its parity is unpinned by the reference; the
oracle is pinned by two independent restatements agreeing (token recurrence
vs chunk-parallel WY form) and by closed forms.
"""
import numpy as np
import pytest

import oracle


def _inputs(B, T, H, Dk, Dv, seed, decay=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, H, Dk))
    k = rng.standard_normal((B, T, H, Dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, H, Dv))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    g = -decay * np.log1p(np.exp(rng.standard_normal((B, T, H, Dk))))
    return q, k, v, g, beta


@pytest.mark.parametrize("T,chunk", [(64, 64), (100, 16), (37, 8), (130, 64)])
def test_chunked_matches_recurrent(T, chunk):
    q, k, v, g, beta = _inputs(2, T, 3, 16, 8, seed=T)
    s0 = np.random.default_rng(9).standard_normal((2, 3, 16, 8))
    o1, s1 = oracle.kda_recurrent(q, k, v, g, beta, initial_state=s0)
    o2, s2 = oracle.kda_chunked(q, k, v, g, beta, initial_state=s0, chunk_size=chunk)
    np.testing.assert_allclose(o2, o1, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(s2, s1, rtol=1e-9, atol=1e-10)


def test_beta_zero_gives_zero_state_and_output():
    q, k, v, g, beta = _inputs(1, 20, 2, 8, 8, seed=1)
    o, s = oracle.kda_chunked(q, k, v, g, np.zeros_like(beta), chunk_size=8)
    assert np.abs(o).max() == 0 and np.abs(s).max() == 0


def test_single_step_closed_form():
    q, k, v, g, beta = _inputs(1, 1, 1, 8, 4, seed=2)
    g[:] = 0.0
    beta[:] = 1.0
    o, s = oracle.kda_recurrent(q, k, v, g, beta)
    np.testing.assert_allclose(s[0, 0], np.outer(k[0, 0, 0], v[0, 0, 0]), atol=1e-12)
    np.testing.assert_allclose(o[0, 0, 0], (q[0, 0, 0] @ k[0, 0, 0]) * 8 ** -0.5 * v[0, 0, 0],
                               atol=1e-12)


def test_orthonormal_keys_exact_retrieval():
    Dk, Dv, T = 8, 5, 8
    rng = np.random.default_rng(3)
    keys = np.linalg.qr(rng.standard_normal((Dk, Dk)))[0].T  # rows orthonormal
    k = keys[None, :, None, :]
    v = rng.standard_normal((1, T, 1, Dv))
    g = np.zeros((1, T, 1, Dk))
    beta = np.ones((1, T, 1))
    q = k.copy()
    o, s = oracle.kda_chunked(q, k, v, g, beta, scale=1.0, chunk_size=4)
    # S = sum_t k_t v_t^T, and querying with k_t returns v_t at step t
    np.testing.assert_allclose(o[0, :, 0], v[0, :, 0], atol=1e-10)
    np.testing.assert_allclose(keys @ s[0, 0], v[0, :, 0], atol=1e-10)


def test_infinite_decay_is_memoryless():
    q, k, v, g, beta = _inputs(1, 12, 1, 8, 4, seed=4)
    g[:] = -1e4
    o, _ = oracle.kda_chunked(q, k, v, g, beta, chunk_size=4)
    for t in range(12):
        kt, vt, bt, qt = k[0, t, 0], v[0, t, 0], beta[0, t, 0], q[0, t, 0]
        expect = (qt @ kt) * 8 ** -0.5 * bt * vt
        np.testing.assert_allclose(o[0, t, 0], expect, atol=1e-10)


def test_planted_wrong_decay_sign_breaks_agreement():
    q, k, v, g, beta = _inputs(1, 32, 1, 8, 4, seed=5)
    o1, _ = oracle.kda_recurrent(q, k, v, g, beta)
    o2, _ = oracle.kda_chunked(q, k, v, -g, beta, chunk_size=8)
    assert np.abs(o1 - o2).max() > 1e-3
