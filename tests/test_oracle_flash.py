"""Pin the oracle's flash attention forward (CPU only).

Pins: the reference tests' seeded known answers, torch's scaled_dot_product_
attention (an independent library routine, CPU fp64), torch.logsumexp for the
LSE, and closed forms (uniform scores -> mean of V; causal row 0 -> V_0).
"""
import math

import numpy as np
import pytest
import torch

import oracle

FLASH_KATS = ["flash_seed555", "flash_seed666", "flash_seed1234", "flash_seed123"]


@pytest.mark.parametrize("name", FLASH_KATS)
def test_flash_oracle_matches_reference_kat(kats, name):
    m, a = kats[name]
    S, D = m["S"], m["D"]
    o, _ = oracle.flash_attention(a["Q"].reshape(S, D), a["K"].reshape(S, D),
                                  a["V"].reshape(S, D), 1.0 / math.sqrt(D), m["causal"])
    np.testing.assert_allclose(o.ravel(), a["expected"], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_flash_oracle_matches_sdpa_and_logsumexp(causal):
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 3, 37, 16, generator=g, dtype=torch.float64) for _ in range(3))
    scale = 0.3
    o, lse = oracle.flash_attention(q.numpy(), k.numpy(), v.numpy(), scale, causal)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal,
                                                           scale=scale)
    np.testing.assert_allclose(o, ref.numpy(), rtol=1e-10, atol=1e-12)
    s = (q @ k.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(37, 37, dtype=torch.bool), 1), -math.inf)
    np.testing.assert_allclose(lse, torch.logsumexp(s, -1).numpy(), rtol=1e-12, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(1)
    S, D = 9, 4
    v = rng.standard_normal((S, D))
    q = np.zeros((S, D))
    k = rng.standard_normal((S, D))
    o, lse = oracle.flash_attention(q, k, v, 1.0, False)   # all scores 0
    np.testing.assert_allclose(o, np.tile(v.mean(0), (S, 1)), atol=1e-12)
    np.testing.assert_allclose(lse, np.full(S, math.log(S)), atol=1e-12)
    q = rng.standard_normal((S, D))
    o, lse = oracle.flash_attention(q, k, v, 0.5, True)    # row 0 sees only key 0
    np.testing.assert_allclose(o[0], v[0], atol=1e-12)
    np.testing.assert_allclose(lse[0], 0.5 * q[0] @ k[0], atol=1e-12)


def test_planted_reversed_causal_mask_fails_kat(kats):
    m, a = kats["flash_seed1234"]
    S, D = m["S"], m["D"]
    q, k, v = (a[x].reshape(S, D) for x in "QKV")
    # attend to the future instead of the past
    o, _ = oracle.flash_attention(q[::-1], k[::-1], v[::-1], 1 / math.sqrt(D), True)
    assert np.abs(o[::-1].ravel() - a["expected"]).max() > 1e-2
