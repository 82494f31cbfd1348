"""CPU oracle for the hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of the reference kernels the
library replaces.  It exists to check the HIP kernels: only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg may import it, and
never as the thing measured or shipped.  The product path (triton_metal_amd)
must not import it.

Every function cites the reference file:line it follows (paths relative to the
reference tree bledden/triton-metal).  How each function is pinned (golden
vectors / known-answer tests / closed forms) is listed in PINNING below; the
tests in tests/test_oracle_*.py carry out those checks.

KDA has no counterpart in the reference (no linear attention anywhere in
bledden/triton-metal), so kda_recurrent / kda_chunked restate the published
gated delta rule of Kimi Delta Attention; they are pinned only by closed forms
and by agreeing with each other.
"""
from __future__ import annotations

import numpy as np

PINNING = {
    "unpack_int4": "hand-built nibble words (order), ported KATs seeds 7070/44",
    "pack_int4": "round trip with unpack_int4; packing of tests/test_emitter.py:3027-3032",
    "dequant_int4": "closed form per-group scales (group index), z=q -> 0, KATs 7070/44",
    "dequant_int8": "closed form, KATs 8888/66",
    "int4_matmul": "KATs 7070/44 (expected values of the reference tests), brute force",
    "int8_matmul": "KATs 8888/66, brute force",
    "matmul": "KATs 42/789/101/202/303/404/505/707/808, I@B=B, brute-force triple loop",
    "flash_attention": "KATs 555/666/1234/123, torch SDPA (CPU, fp64), logsumexp, "
                       "uniform-score and causal-row-0 closed forms",
    "kda_recurrent": "closed forms (beta=0, T=1, orthonormal retrieval, memoryless); "
                     "agreement with kda_chunked (parity unpinned by the reference)",
    "kda_chunked": "agreement with kda_recurrent; same closed forms (parity unpinned by "
                   "the reference)",
    "pack_gptq": "round trip with the shift-table unpacking of the published format; "
                 "dequant equivalence through gptq_to_ref (format not in the reference)",
    "pack_awq": "inverse of the published reverse-order unpacking; identity-column word "
                "0x75316420; dequant equivalence through awq_to_ref",
    "decode_attention": "flash_attention on one query row (dense and gathered pages), "
                        "brute-force phase loops, closed forms (one position -> V[0], "
                        "zero query -> mean of V)",
    "gptq_to_ref": "dequant_int4 of the result equals (q - z) s of the unpacked checkpoint",
    "fp8_decode": "every one of the 256 codes of each format against an independent "
                  "bit-field formula, torch's float8_e4m3fn / float8_e5m2 decoders, the "
                  "formats' closed-form extremes (max normal, min subnormal, NaN / inf codes)",
    "dot": "brute-force loops over (b, m, n, k) for every epilogue, strided and transposed "
           "views equal to the contiguous product of the same matrices, softmax rows sum "
           "to one, chain-dot equal to two plain products, add-* equal to the plain "
           "product plus the broadcast bias",
    "awq_to_ref": "dequant_int4 of the result equals (q - z) s of the unpacked checkpoint",
}


# ---------------------------------------------------------------------------
# int4 / int8 weight-only quantisation
# ---------------------------------------------------------------------------
def unpack_int4(packed: np.ndarray, K: int) -> np.ndarray:
    """[N, K/2] bytes -> [N, K] nibbles, even k in the low nibble.

    _msl_templates.py:2724-2732: ``byte = weight[col*(K/2) + k/2]``;
    ``w4 = k%2==0 ? byte & 0xF : (byte >> 4) & 0xF``."""
    b = np.ascontiguousarray(packed).view(np.uint8).reshape(-1, K // 2)
    out = np.empty((b.shape[0], K), dtype=np.uint8)
    out[:, 0::2] = b & 0x0F
    out[:, 1::2] = (b >> 4) & 0x0F
    return out


def pack_int4(q: np.ndarray) -> np.ndarray:
    """[N, K] values 0..15 -> [N, K/2] bytes, ``lo | (hi << 4)``.

    tests/test_emitter.py:3027-3032 and 6198-6204."""
    q = np.asarray(q, dtype=np.uint8)
    return (q[:, 0::2] & 0x0F) | ((q[:, 1::2] & 0x0F) << 4)


def dequant_int4(packed, scales, zeros, K: int, group_size: int) -> np.ndarray:
    """w[n, k] = (float(q) - z[n, k/G]) * s[n, k/G] in fp32.

    _msl_templates.py:2734-2739 (``group_idx = k / GROUP_SIZE``;
    ``n_groups = ceil(K / G)``; ``w = (float(w4) - z) * s``)."""
    q = unpack_int4(packed, K).astype(np.float32)
    N = q.shape[0]
    ng = (K + group_size - 1) // group_size
    s = np.asarray(scales, dtype=np.float32).reshape(N, ng)
    z = (np.zeros((N, ng), np.float32) if zeros is None
         else np.asarray(zeros, dtype=np.float32).reshape(N, ng))
    g = np.arange(K) // group_size
    return ((q - z[:, g]) * s[:, g]).astype(np.float32)


def dequant_int8(weight, scales, zeros) -> np.ndarray:
    """w[n, k] = (float(W[n, k]) - z[n]) * s[n] in fp32 (_msl_templates.py:2671)."""
    w = np.asarray(weight).view(np.int8).astype(np.float32)
    N = w.shape[0]
    s = np.asarray(scales, dtype=np.float32).reshape(N, 1)
    z = np.zeros((N, 1), np.float32) if zeros is None else np.asarray(
        zeros, dtype=np.float32).reshape(N, 1)
    return ((w - z) * s).astype(np.float32)


def int4_matmul(x, packed, scales, zeros, M, N, K, group_size) -> np.ndarray:
    """out[M, N] = x @ dequant_int4(...)^T, accumulated in float64.

    make_int4_matmul_kernel, _msl_templates.py:2704-2744 (the reference
    accumulates in fp32 per output; fp64 here is the tighter answer both are
    checked against)."""
    w = dequant_int4(packed, scales, zeros, K, group_size).astype(np.float64)
    return np.asarray(x, dtype=np.float64).reshape(M, K) @ w.T


def int8_matmul(x, weight, scales, zeros, M, N, K) -> np.ndarray:
    """out[M, N] = x @ dequant_int8(...)^T (_msl_templates.py:2652-2678)."""
    w = dequant_int8(np.asarray(weight).reshape(N, K), scales, zeros).astype(np.float64)
    return np.asarray(x, dtype=np.float64).reshape(M, K) @ w.T


# ---------------------------------------------------------------------------
# dense matmul
# ---------------------------------------------------------------------------
def matmul(A, B) -> np.ndarray:
    """C = A @ B with A [M, K], B [K, N] row-major, float64 accumulation.

    make_matmul_kernel _msl_templates.py:512-585 (``acc += tileA[row][k] *
    tileB[k][col]``); make_simdgroup_matmul_kernel 3501-3667 (same product)."""
    return np.asarray(A, dtype=np.float64) @ np.asarray(B, dtype=np.float64)


def linear(x, W, bias=None) -> np.ndarray:
    """out = x @ W^T (+ bias) (make_fused_linear_kernel, _msl_templates.py:4013-4135)."""
    out = np.asarray(x, dtype=np.float64) @ np.asarray(W, dtype=np.float64).T
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None, :]
    return out


# ---------------------------------------------------------------------------
# flash attention forward
# ---------------------------------------------------------------------------
def flash_attention(Q, K, V, scale: float, causal: bool):
    """Attention over [..., S, D] heads in float64; returns (O, LSE).

    make_flash_attention_kernel _msl_templates.py:1568-1767: scores
    ``S = Q.K^T * scale``; a score is -inf when ``kv_pos >= seq_len`` or, if
    causal, ``kv_pos > q_pos`` (1610-1619); softmax by row; ``O /= l`` only when
    ``l > 0`` (1747-1754), so a fully masked row yields O = 0.  LSE (natural
    log, no reference counterpart) = logsumexp of the masked scores, -inf for a
    fully masked row."""
    q = np.asarray(Q, dtype=np.float64)
    k = np.asarray(K, dtype=np.float64)
    v = np.asarray(V, dtype=np.float64)
    s = np.einsum("...qd,...kd->...qk", q, k) * scale
    Sq, Sk = s.shape[-2], s.shape[-1]
    if causal:
        mask = np.arange(Sk)[None, :] > np.arange(Sq)[:, None]
        s = np.where(mask, -np.inf, s)
    m = np.max(s, axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m_safe)
    l = np.sum(p, axis=-1, keepdims=True)
    o = np.einsum("...qk,...kd->...qd", p, v)
    o = np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0)
    with np.errstate(divide="ignore"):
        lse = np.where(l[..., 0] > 0, m_safe[..., 0] + np.log(l[..., 0]), -np.inf)
    return o, lse


# ---------------------------------------------------------------------------
# decode attention (one query token per head over a KV cache)
# ---------------------------------------------------------------------------
def decode_attention(q, K, V, lens, scale: float, page_table=None):
    """The reference's decode templates in float64; returns (O [B, Hq, D], LSE [B, Hq]).

    Per (batch b, query head h): KV head kvh = h // (Hq // Hkv)
    (make_gqa_attention_kernel _msl_templates.py:2098-2101); positions
    p < lens[b] (make_batched_kv_decode_kernel 2201-2207); three phases as the
    templates: max of scale * q.K[p] (1995-2004), sum of exp(score - max)
    (2017-2026), weights * V (2039-2050).  Dense caches are [B, Hkv, S, D];
    with page_table [B, max_pages] the caches are pages [n, page_size, Hkv, D]
    and position p is slot p % page_size of page page_table[b][p // page_size]
    (make_multi_head_paged_attention_kernel 2448-2455).  No position: O = 0,
    LSE = -inf."""
    q = np.asarray(q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    B, Hq, D = q.shape
    Hkv = K.shape[2] if page_table is not None else K.shape[1]
    group = Hq // Hkv
    O = np.zeros((B, Hq, D))
    LSE = np.full((B, Hq), -np.inf)
    for b in range(B):
        n = int(lens[b])
        if n == 0:
            continue
        pos = np.arange(n)
        for h in range(Hq):
            kvh = h // group
            if page_table is not None:
                ps = K.shape[1]
                pages = np.asarray(page_table)[b][pos // ps]
                kr, vr = K[pages, pos % ps, kvh], V[pages, pos % ps, kvh]
            else:
                kr, vr = K[b, kvh, :n], V[b, kvh, :n]
            sc = kr @ q[b, h] * scale
            m = sc.max()
            e = np.exp(sc - m)
            tot = e.sum()
            O[b, h] = (e / tot) @ vr
            LSE[b, h] = m + np.log(tot)
    return O, LSE


# ---------------------------------------------------------------------------
# KDA (Kimi Delta Attention) chunked gated delta rule -- no reference code
# ---------------------------------------------------------------------------
def kda_recurrent(q, k, v, g, beta, scale=None, initial_state=None):
    """Token-by-token gated delta rule with per-key-channel decay, float64.

    Layout [B, T, H, D] (q, k: Dk; v: Dv), g [B, T, H, Dk] (log decay),
    beta [B, T, H].  Per head, S in R^{Dk x Dv}:
        S <- diag(exp(g_t)) S
        S <- S + beta_t k_t (v_t - S^T k_t)^T
        o_t = S^T (q_t * scale)
    Returns (o [B, T, H, Dv], S_T [B, H, Dk, Dv])."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    if scale is None:
        scale = Dk ** -0.5
    S = (np.zeros((B, H, Dk, Dv)) if initial_state is None
         else np.array(initial_state, np.float64).reshape(B, H, Dk, Dv))
    o = np.zeros((B, T, H, Dv))
    for t in range(T):
        S = S * np.exp(g[:, t])[..., None]
        kt = k[:, t]
        u = beta[:, t][..., None] * (v[:, t] - np.einsum("bhkv,bhk->bhv", S, kt))
        S = S + np.einsum("bhk,bhv->bhkv", kt, u)
        o[:, t] = np.einsum("bhkv,bhk->bhv", S, q[:, t] * scale)
    return o, S


def kda_chunked(q, k, v, g, beta, scale=None, initial_state=None, chunk_size=64):
    """Chunk-parallel form of kda_recurrent (independent restatement), float64.

    Within a chunk with inclusive cumulative log decay G_t (per channel) and
    pairwise decays D[t, s, c] = exp(G_tc - G_sc) for s <= t (never > 1):
        A[t, s]   = beta_t sum_c k_tc k_sc D[t, s, c]   (s < t),  T = (I + A)^-1
        Aqk[t, s] = sum_c q_tc k_sc D[t, s, c] * scale  (s <= t)
        U  = T diag(beta) (V - (k * exp(G)) S0)
        O  = (q * scale * exp(G)) S0 + Aqk U
        S1 = diag(exp(G_C)) S0 + (k * exp(G_C - G))^T U
    The pairwise form never multiplies exp(G) by exp(-G), so it stays finite
    for any decay."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    if scale is None:
        scale = Dk ** -0.5
    S = (np.zeros((B, H, Dk, Dv)) if initial_state is None
         else np.array(initial_state, np.float64).reshape(B, H, Dk, Dv))
    o = np.zeros((B, T, H, Dv))
    for b in range(B):
        for h in range(H):
            St = S[b, h].copy()
            for c0 in range(0, T, chunk_size):
                c1 = min(T, c0 + chunk_size)
                kc, vc, qc = k[b, c0:c1, h], v[b, c0:c1, h], q[b, c0:c1, h] * scale
                bc = beta[b, c0:c1, h]
                G = np.cumsum(g[b, c0:c1, h], axis=0)
                n = c1 - c0
                incl = np.tril(np.ones((n, n), bool))
                expo = np.where(incl[:, :, None], G[:, None, :] - G[None, :, :], -np.inf)
                Dts = np.exp(expo)                                   # [t, s, c]
                A = np.where(np.tril(incl, -1),
                             bc[:, None] * np.einsum("tc,sc,tsc->ts", kc, kc, Dts), 0.0)
                Aqk = np.einsum("tc,sc,tsc->ts", qc, kc, Dts)
                Tm = np.linalg.inv(np.eye(n) + A)
                eG = np.exp(G)
                U = Tm @ (bc[:, None] * (vc - (kc * eG) @ St))
                o[b, c0:c1, h] = (qc * eG) @ St + Aqk @ U
                St = eG[-1][:, None] * St + (kc * np.exp(G[-1][None, :] - G)).T @ U
            S[b, h] = St
    return o, S


# ---------------------------------------------------------------------------
# On-disk int4 checkpoint formats -> the int4 layout of the reference template
# (W [N, K/2] bytes, even k in the low nibble; scales / zeros [N, K/G]:
# _msl_templates.py:2687-2697).  The formats themselves are not in the
# reference; they are restated from their published definitions:
#   GPTQ (AutoGPTQ checkpoints): qweight int32 [K/8, N], nibble i of word
#     (j, n) = q[n, 8 j + i]; qzeros int32 [K/G, N/8], nibble i of word (g, b)
#     = z[8 b + i, g] - zero_offset (1 in the original format, which stores
#     zero-points minus one; 0 in its "v2" variant); scales fp16 [K/G, N].
#   AWQ (AutoAWQ GEMM checkpoints): qweight int32 [K, N/8], nibble p of word
#     (k, b) = q[8 b + AWQ_ORDER[p], k]; qzeros int32 [K/G, N/8] in the same
#     order (no offset); scales fp16 [K/G, N].
# ---------------------------------------------------------------------------
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _pack_nibbles(vals: np.ndarray) -> np.ndarray:
    """[..., 8] values 0..15 -> uint32 words, value i in nibble i."""
    v = np.asarray(vals, np.uint32) & 0xF
    return (v << (4 * np.arange(8, dtype=np.uint32))).sum(axis=-1, dtype=np.uint64).astype(
        np.uint32)


def pack_gptq(q: np.ndarray, zeros: np.ndarray, zero_offset: int = 1):
    """q uint8 [N, K] (0..15), zeros int [N, ng] -> (qweight int32 [K/8, N],
    qzeros int32 [ng, N/8])."""
    N, K = q.shape
    qw = _pack_nibbles(np.asarray(q).T.reshape(K // 8, 8, N).transpose(0, 2, 1))
    zs = (np.asarray(zeros, np.int64).T - zero_offset) & 0xF          # [ng, N]
    qz = _pack_nibbles(zs.reshape(zs.shape[0], N // 8, 8))
    return np.ascontiguousarray(qw).view(np.int32), np.ascontiguousarray(qz).view(np.int32)


def pack_awq(q: np.ndarray, zeros: np.ndarray):
    """q uint8 [N, K], zeros int [N, ng] -> (qweight int32 [K, N/8],
    qzeros int32 [ng, N/8]) in the AWQ column order."""
    N, K = q.shape
    order = np.array(AWQ_ORDER)
    qt = np.asarray(q).T.reshape(K, N // 8, 8)[:, :, order]           # nibble p <- col ORDER[p]
    zt = np.asarray(zeros, np.int64).T.reshape(-1, N // 8, 8)[:, :, order]
    return (np.ascontiguousarray(_pack_nibbles(qt)).view(np.int32),
            np.ascontiguousarray(_pack_nibbles(zt)).view(np.int32))


def _unpack_words(w: np.ndarray) -> np.ndarray:
    u = np.asarray(w).view(np.uint32)
    return ((u[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).astype(np.uint8)


def gptq_to_ref(qweight, qzeros, scales, N: int, K: int, group_size: int, zero_offset: int = 1):
    """GPTQ checkpoint -> (packed [N, K/2] uint8, scales [N, ng] as given, zeros
    [N, ng] as integers), the reference int4 layout."""
    q = _unpack_words(qweight).transpose(0, 2, 1).reshape(K, N).T        # [N, K]
    ng = (K + group_size - 1) // group_size
    z = _unpack_words(qzeros).reshape(ng, N).T.astype(np.int64) + zero_offset
    return pack_int4(q), np.asarray(scales).T.copy(), z


def awq_to_ref(qweight, qzeros, scales, N: int, K: int, group_size: int):
    """AWQ checkpoint -> (packed [N, K/2] uint8, scales [N, ng], zeros [N, ng])."""
    inv = np.argsort(AWQ_ORDER)                                         # column i at nibble inv[i]
    q = _unpack_words(qweight)[:, :, inv].reshape(K, N).T
    ng = (K + group_size - 1) // group_size
    z = _unpack_words(qzeros)[:, :, inv].reshape(ng, N).T.astype(np.int64)
    return pack_int4(q), np.asarray(scales).T.copy(), z


# ---------------------------------------------------------------------------
# FP8 formats: the decoders of triton_metal/codegen/msl_builtins.py
# ---------------------------------------------------------------------------
# (exponent bits, mantissa bits, bias, has inf) per Triton dtype name:
#   fp8e4nv  FP8_E4M3_TO_FLOAT    msl_builtins.py:53-66   (exp 15 / mant 7 = NaN)
#   fp8e5    FP8_E5M2_TO_FLOAT    msl_builtins.py:95-109  (exp 31: inf / NaN)
#   fp8e4b15 FP8_E4M3B15_TO_FLOAT msl_builtins.py:140-153
#   fp8e4b8  FP8_E4M3B8_TO_FLOAT  msl_builtins.py:182-195
#   fp8e5b16 FP8_E5M2B16_TO_FLOAT msl_builtins.py:223-237
# (the dtype map is msl_builtins.py:264-272)
FP8_FORMATS = {
    "fp8e4nv": (4, 3, 7, False),
    "fp8e5": (5, 2, 15, True),
    "fp8e4b15": (4, 3, 15, False),
    "fp8e4b8": (4, 3, 8, False),
    "fp8e5b16": (5, 2, 16, True),
}


def fp8_decode(codes, fmt: str) -> np.ndarray:
    """uint8 codes -> float64 values as the reference's MSL decoders compute
    them: exponent field 0 is subnormal (mant / 2^mbits * 2^(1 - bias)); the
    all-ones exponent is NaN with mantissa all ones (4-bit exponent formats) or
    inf / NaN (5-bit formats); otherwise (1 + mant / 2^mbits) * 2^(exp - bias);
    the sign bit negates."""
    eb, mb, bias, has_inf = FP8_FORMATS[fmt]
    c = np.asarray(codes, np.uint8).astype(np.int64)
    sign = (c >> 7) & 1
    e = (c >> mb) & ((1 << eb) - 1)
    m = c & ((1 << mb) - 1)
    emax = (1 << eb) - 1
    val = np.where(e == 0, m / (1 << mb) * 2.0 ** (1 - bias),
                   (1 + m / (1 << mb)) * 2.0 ** (e.astype(np.float64) - bias))
    if has_inf:
        val = np.where(e == emax, np.where(m == 0, np.inf, np.nan), val)
    else:
        val = np.where((e == emax) & (m == (1 << mb) - 1), np.nan, val)
    return np.where(sign == 1, -val, val)


# ---------------------------------------------------------------------------
# tl.dot with strides, batches and epilogues
# ---------------------------------------------------------------------------
DOT_EPILOGUES = ("none", "add-matrix", "add-rows", "add-cols", "softmax", "chain-dot")


def dot(A, B, epilogue: str = "none", Z=None, W=None) -> np.ndarray:
    """The strided tl.dot template of _lowerer_templates.py:1116-1540, float64.

    A [.., M, K] @ B [.., K, N] (a leading batch dimension for the 3-D dot,
    1151-1160 and 1453-1470), accumulated from zero or from the epilogue's bias
    (1429-1438): add-matrix Z[.., m, n], add-rows Z[.., m, 0], add-cols
    Z[.., 0, n] (the bias loads of 1395-1420); softmax over each row of the
    product, exp(x - rowmax) / sum (1488-1505); chain-dot (A @ B) @ W with W
    [N, L] from the unrounded product (1506-1522).  Strides only select which
    elements are read and written, so the restatement takes the logical
    matrices."""
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    P = A @ B
    if epilogue == "none":
        return P
    Z = None if Z is None else np.asarray(Z, np.float64)
    if epilogue == "add-matrix":
        return P + Z
    if epilogue == "add-rows":
        return P + Z[..., :, :1]
    if epilogue == "add-cols":
        return P + Z[..., :1, :]
    if epilogue == "softmax":
        mx = P.max(axis=-1, keepdims=True)
        e = np.exp(P - mx)
        return e / e.sum(axis=-1, keepdims=True)
    if epilogue == "chain-dot":
        return P @ np.asarray(W, np.float64)
    raise ValueError(f"unknown epilogue {epilogue}")
