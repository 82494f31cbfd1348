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


# --- decode attention ------------------------------------------------------------------
def _decode_problem(seed, B=2, Hq=6, Hkv=3, D=8, S=11):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, D))
    K = rng.standard_normal((B, Hkv, S, D))
    V = rng.standard_normal((B, Hkv, S, D))
    return q, K, V


def test_decode_matches_flash_attention_on_one_row():
    q, K, V = _decode_problem(0)
    lens = [11, 5]
    O, L = oracle.decode_attention(q, K, V, lens, 0.3)
    for b in range(2):
        for h in range(6):
            kvh = h // 2
            o_f, l_f = oracle.flash_attention(q[b, h][None], K[b, kvh, :lens[b]],
                                              V[b, kvh, :lens[b]], 0.3, False)
            np.testing.assert_allclose(O[b, h], o_f[0], rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(L[b, h], l_f[0], rtol=1e-12)


def test_decode_paged_equals_dense_gather():
    q, K, V = _decode_problem(1, B=2, Hkv=3, S=12)
    ps = 4
    # scatter the dense cache into shuffled pages, then read it back paged
    rng = np.random.default_rng(2)
    perm = rng.permutation(2 * 3)
    Kp = np.zeros((6, ps, 3, 8)); Vp = np.zeros_like(Kp)
    table = perm.reshape(2, 3)
    for b in range(2):
        for i in range(3):
            Kp[table[b, i]] = K[b, :, ps * i:ps * i + ps].transpose(1, 0, 2)
            Vp[table[b, i]] = V[b, :, ps * i:ps * i + ps].transpose(1, 0, 2)
    lens = [12, 7]
    O1, L1 = oracle.decode_attention(q, K, V, lens, 0.5)
    O2, L2 = oracle.decode_attention(q, Kp, Vp, lens, 0.5, page_table=table)
    np.testing.assert_allclose(O1, O2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(L1, L2, rtol=1e-12)


def test_decode_brute_force_phase_loops():
    q, K, V = _decode_problem(3, B=1, Hq=2, Hkv=1, D=3, S=4)
    O, _ = oracle.decode_attention(q, K, V, [4], 0.7)
    for h in range(2):
        sc = [sum(q[0, h, d] * K[0, 0, p, d] for d in range(3)) * 0.7 for p in range(4)]
        mx = max(sc)
        tot = sum(math.exp(x - mx) for x in sc)
        for d in range(3):
            want = sum(math.exp(sc[p] - mx) / tot * V[0, 0, p, d] for p in range(4))
            assert abs(O[0, h, d] - want) < 1e-12


def test_decode_closed_forms():
    q, K, V = _decode_problem(4)
    O, L = oracle.decode_attention(q, K, V, [1, 0], 0.3)
    np.testing.assert_allclose(O[0], V[0, np.arange(6) // 2, 0], rtol=1e-12)   # one position
    assert (O[1] == 0).all() and np.isneginf(L[1]).all()                       # no position
    O, _ = oracle.decode_attention(np.zeros_like(q), K, V, [11, 11], 0.3)       # uniform scores
    np.testing.assert_allclose(O, V.mean(axis=2)[:, np.arange(6) // 2], rtol=1e-12)
