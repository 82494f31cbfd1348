"""Pin the oracle's int4/int8 unpack, dequant and matmul (CPU only).

Pins: hand-built nibble words (nibble order), the reference tests' seeded
known answers (tests/golden), per-group closed forms (group index), and
planted mistakes that each pin must catch.
"""
import numpy as np
import pytest

import oracle


def test_unpack_nibble_order_hand_built():
    # bytes little-endian 0x10, 0x32, 0x54, 0x76 -> k = 0..7 hold 0..7
    word = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    q = oracle.unpack_int4(word.view(np.uint8), 16)
    assert q.tolist() == [list(range(16))]
    # single byte 0xA5: k even (low nibble) = 5, k odd = 10 (_msl_templates.py:2727-2731)
    q = oracle.unpack_int4(np.array([[0xA5]], np.uint8), 2)
    assert q.tolist() == [[5, 10]]


def test_pack_unpack_round_trip():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(7, 40), dtype=np.uint8)
    assert np.array_equal(oracle.unpack_int4(oracle.pack_int4(q), 40), q)


def test_uint32_view_equals_byte_layout():
    # nibble i of uint32 word j  <->  k = 8j + i  (little-endian bytes)
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(3, 64), dtype=np.uint8)
    words = np.zeros((3, 8), np.uint32)
    for j in range(8):
        for i in range(8):
            words[:, j] |= q[:, 8 * j + i].astype(np.uint32) << (4 * i)
    assert np.array_equal(words.view(np.uint8), oracle.pack_int4(q))


def test_dequant_group_index_closed_form():
    N, K, G = 3, 64, 16
    q = np.ones((N, K), np.uint8)
    ng = K // G
    s = np.tile(np.arange(1, ng + 1, dtype=np.float32), (N, 1))
    w = oracle.dequant_int4(oracle.pack_int4(q), s, None, K, G)
    assert np.array_equal(w, np.tile((np.arange(K) // G + 1).astype(np.float32), (N, 1)))
    # z = q gives exactly zero
    q = np.random.default_rng(2).integers(0, 16, size=(N, K), dtype=np.uint8)
    z = np.zeros((N, ng), np.float32)
    w = oracle.dequant_int4(oracle.pack_int4(q), np.ones((N, ng), np.float32), z, K, G)
    assert np.array_equal(w, q.astype(np.float32))


def test_dequant_is_q_minus_z_times_s_not_q_times_s_minus_z():
    q = np.array([[3, 12]], np.uint8)
    w = oracle.dequant_int4(oracle.pack_int4(q), np.array([[0.5]], np.float32),
                            np.array([[2.0]], np.float32), 2, 2)
    assert w.tolist() == [[0.5, 5.0]]


@pytest.mark.parametrize("name", ["int4_seed7070", "int4_seed44"])
def test_int4_oracle_matches_reference_kat(kats, name):
    m, a = kats[name]
    M, N, K, G = m["M"], m["N"], m["K"], m["G"]
    packed = a["packed"].astype(np.uint8).reshape(N, K // 2)
    assert np.array_equal(oracle.unpack_int4(packed, K), a["q"].reshape(N, K))
    out = oracle.int4_matmul(a["input"], packed, a["scales"], a["zeros"], M, N, K, G)
    np.testing.assert_allclose(out.ravel(), a["expected"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", ["int8_seed8888", "int8_seed66"])
def test_int8_oracle_matches_reference_kat(kats, name):
    m, a = kats[name]
    M, N, K = m["M"], m["N"], m["K"]
    w = a["weight"].astype(np.int8).reshape(N, K)
    out = oracle.int8_matmul(a["input"], w, a["scales"], a["zeros"], M, N, K)
    np.testing.assert_allclose(out.ravel(), a["expected"], rtol=1e-5, atol=1e-6)


def test_int4_matmul_brute_force():
    rng = np.random.default_rng(3)
    M, N, K, G = 3, 5, 32, 8
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.uniform(0.01, 0.1, (N, K // G)).astype(np.float32)
    z = rng.integers(0, 16, (N, K // G)).astype(np.float32)
    x = rng.standard_normal((M, K))
    out = oracle.int4_matmul(x, oracle.pack_int4(q), s, z, M, N, K, G)
    for i in range(M):
        for j in range(N):
            ref = 0.0
            for k in range(K):
                ref += x[i, k] * float((np.float32(q[j, k]) - z[j, k // G]) * s[j, k // G])
            assert abs(out[i, j] - ref) < 1e-9


# --- planted mistakes: each must be caught by a pin above -------------------
def _kat_error(kats, name, unpack):
    m, a = kats[name]
    M, N, K, G = m["M"], m["N"], m["K"], m["G"]
    packed = a["packed"].astype(np.uint8).reshape(N, K // 2)
    q = unpack(packed, K).astype(np.float32)
    ng = (K + G - 1) // G
    s = a["scales"].astype(np.float32).reshape(N, ng)
    z = a["zeros"].astype(np.float32).reshape(N, ng)
    g = np.arange(K) // G
    w = (q - z[:, g]) * s[:, g]
    out = a["input"].reshape(M, K) @ w.T.astype(np.float64)
    return np.abs(out.ravel() - a["expected"]).max()


def test_planted_swapped_nibbles_fail_kat(kats):
    def swapped(packed, K):
        b = packed.view(np.uint8).reshape(-1, K // 2)
        out = np.empty((b.shape[0], K), np.uint8)
        out[:, 0::2] = (b >> 4) & 0xF
        out[:, 1::2] = b & 0xF
        return out
    assert _kat_error(kats, "int4_seed44", oracle.unpack_int4) < 1e-6
    assert _kat_error(kats, "int4_seed44", swapped) > 0.1


# --- GPTQ / AWQ checkpoint formats (restated; not in the reference) ------------------
# Second, independent formulations of the published unpacking, written the way
# the formats' own loaders state it (a shift table over the packed axis; for
# AWQ a reverse-order column gather), so that a wrong nibble order, axis or
# offset in the oracle's packers fails here.
def _gptq_unpack_shift_table(qweight, K, N):
    wf = np.arange(0, 32, 4, dtype=np.uint32)                    # [8]
    u = qweight.view(np.uint32)                                  # [K/8, N]
    t = (u[:, None, :] >> wf[None, :, None]) & 0xF               # [K/8, 8, N]
    return t.reshape(K, N).astype(np.uint8)                      # q^T [K, N]


def _awq_unpack_reverse_order(qweight, K, N):
    rev = [0, 4, 1, 5, 2, 6, 3, 7]
    u = qweight.view(np.uint32)                                  # [K, N/8]
    t = (u[:, :, None] >> np.arange(0, 32, 4, dtype=np.uint32)) & 0xF   # [K, N/8, 8] nibble order
    return t[:, :, rev].reshape(K, N).astype(np.uint8)           # q^T [K, N]


def _problem(seed, N=32, K=64, G=16, zlo=0):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    z = rng.integers(zlo, 16, size=(N, K // G))
    s = (rng.random((K // G, N)) * 0.02 + 0.001).astype(np.float16)
    return q, z, s


def test_gptq_pack_matches_shift_table_unpacking():
    q, z, _ = _problem(1, zlo=1)
    qw, qz = oracle.pack_gptq(q, z, zero_offset=1)
    assert qw.shape == (64 // 8, 32) and qz.shape == (4, 32 // 8)
    assert np.array_equal(_gptq_unpack_shift_table(qw, 64, 32), q.T)
    zt = ((qz.view(np.uint32)[:, :, None] >> np.arange(0, 32, 4, dtype=np.uint32)) & 0xF)
    assert np.array_equal(zt.reshape(4, 32).T + 1, z)           # stored minus one


def test_awq_pack_matches_reverse_order_unpacking():
    q, z, _ = _problem(2)
    qw, qz = oracle.pack_awq(q, z)
    assert qw.shape == (64, 32 // 8)
    assert np.array_equal(_awq_unpack_reverse_order(qw, 64, 32), q.T)
    assert np.array_equal(_awq_unpack_reverse_order(qz, 4, 32), z.T)
    # columns 0..7 holding their own index pack to the format's signature word
    ident = np.repeat(np.arange(8, dtype=np.uint8)[:, None], 8, axis=1)
    w, _ = oracle.pack_awq(ident, np.zeros((8, 1), int))
    assert int(w.view(np.uint32)[0, 0]) == 0x75316420


@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2", "awq"])
def test_checkpoint_to_ref_preserves_dequant(fmt):
    N, K, G = 32, 64, 16
    q, z, s = _problem(3, N, K, G, zlo=1)
    if fmt == "awq":
        qw, qz = oracle.pack_awq(q, z)
        packed, s_ref, z_ref = oracle.awq_to_ref(qw, qz, s, N, K, G)
        qt = _awq_unpack_reverse_order(qw, K, N)
    else:
        off = 1 if fmt == "gptq" else 0
        qw, qz = oracle.pack_gptq(q, z, zero_offset=off)
        packed, s_ref, z_ref = oracle.gptq_to_ref(qw, qz, s, N, K, G, zero_offset=off)
        qt = _gptq_unpack_shift_table(qw, K, N)
    # dequant through the reference layout == (q - z) s of the checkpoint
    got = oracle.dequant_int4(packed, s_ref.astype(np.float32), z_ref.astype(np.float32), K, G)
    gi = np.arange(K) // G
    want = (qt.T.astype(np.float32) - z[:, gi]) * s.T.astype(np.float32)[:, gi]
    np.testing.assert_array_equal(got, want)


def test_gptq_original_format_cannot_hold_zero_point_zero():
    # the original format stores z - 1 in 4 bits: z = 0 wraps to 16 (a property
    # of the format the conversion reproduces, not a conversion error)
    q = np.zeros((8, 8), np.uint8)
    qw, qz = oracle.pack_gptq(q, np.zeros((8, 1), int), zero_offset=1)
    _, _, z = oracle.gptq_to_ref(qw, qz, np.ones((1, 8)), 8, 8, 8, zero_offset=1)
    assert (z == 16).all()
