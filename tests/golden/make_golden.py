"""Regenerate the reference's seeded known-answer tests as fixtures.

The reference ships no fixture files; its hot-path tests draw inputs from the
stdlib Mersenne Twister (``random.seed(s)``, platform-stable) and compute the
expected values with explicit Python loops.  This script replays exactly
those draws (same seed, same call order, same distributions) and the same
expected-value loops, without importing the reference, and stores inputs,
expected outputs and the reference's tolerance in reference_kats.npz /
reference_kats.json next to this file.

Each entry names the reference test it comes from (tests/test_emitter.py).

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import random
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _ref_matmul(A, B, M, N, K):
    # tests/test_emitter.py:1238-1247 and 5937-5946
    C = [0.0] * (M * N)
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += A[i * K + k] * B[k * N + j]
            C[i * N + j] = s
    return C


def _softmax(row):
    mx = max(row)
    ex = [math.exp(s - mx) if s > float("-inf") else 0.0 for s in row]
    t = sum(ex)
    return [e / t if t > 0 else 0.0 for e in ex]


def _attention(Q, K, V, S, D, scale, causal):
    # tests/test_emitter.py:1890-1920 (non-causal), 2332-2350 (causal),
    # 5579-5612 (_ref_softmax / _ref_dot)
    out = [0.0] * (S * D)
    for i in range(S):
        row = []
        for j in range(S):
            if causal and j > i:
                row.append(float("-inf"))
            else:
                row.append(sum(Q[i * D + d] * K[j * D + d] for d in range(D)) * scale)
        P = _softmax(row)
        for d in range(D):
            out[i * D + d] = sum(P[j] * V[j * D + d] for j in range(S))
    return out


def matmul_kat(name, test, seed, M, N, K, dist, lo, hi, tol, in_dtype="fp32", spot=1,
               kind="matmul", spot_m=None, extra=None):
    random.seed(seed)
    draw = (lambda: random.uniform(lo, hi)) if dist == "uniform" else (
        lambda: random.gauss(lo, hi))
    A = [draw() for _ in range(M * K)]
    B = [draw() for _ in range(K * N)]
    C = _ref_matmul(A, B, M, N, K)
    # checked entries: rows ::spot_m (default spot), columns ::spot
    meta = dict(kind=kind, test=test, seed=seed, M=M, N=N, K=K, tol=tol, in_dtype=in_dtype,
                spot=spot, spot_m=spot if spot_m is None else spot_m, **(extra or {}))
    return name, meta, dict(A=A, B=B, expected=C)


def linear_kat(name, test, seed, M, N, K, bias, tol):
    random.seed(seed)
    x = [random.uniform(-1.0, 1.0) for _ in range(M * K)]
    W = [random.uniform(-1.0, 1.0) for _ in range(N * K)]
    b = [random.uniform(-0.5, 0.5) for _ in range(N)] if bias else None
    exp = []
    for i in range(M):
        for j in range(N):
            v = sum(x[i * K + k] * W[j * K + k] for k in range(K))
            exp.append(v + (b[j] if b else 0.0))
    arrays = dict(input=x, weight=W, expected=exp)
    if b:
        arrays["bias"] = b
    return name, dict(kind="linear", test=test, seed=seed, M=M, N=N, K=K, tol=tol,
                      has_bias=bias), arrays


def int8_kats():
    out = []
    # tests/test_emitter.py:2576-2649
    M, N, K = 16, 16, 32
    random.seed(8888)
    x = [random.uniform(-1.0, 1.0) for _ in range(M * K)]
    w = [random.randint(-10, 10) for _ in range(N * K)]
    s, z = [0.1] * N, [0.0] * N
    exp = [sum(x[i * K + k] * (float(w[j * K + k]) - 0.0) * 0.1 for k in range(K))
           for i in range(M) for j in range(N)]
    out.append(("int8_seed8888", dict(kind="int8", test="test_emitter.py:2576 test_int8_matmul",
                                      seed=8888, M=M, N=N, K=K, tol=0.5),
                dict(input=x, weight=w, scales=s, zeros=z, expected=exp)))
    # tests/test_emitter.py:6101-6153
    M, N, K = 2, 4, 8
    random.seed(66)
    x = [random.gauss(0, 1) for _ in range(M * K)]
    w = [random.randint(-5, 5) for _ in range(N * K)]
    s = [random.uniform(0.1, 0.5) for _ in range(N)]
    z = [random.uniform(-1, 1) for _ in range(N)]
    exp = []
    for i in range(M):
        for j in range(N):
            acc = 0.0
            for k in range(K):
                acc += x[i * K + k] * ((float(w[j * K + k]) - z[j]) * s[j])
            exp.append(acc)
    out.append(("int8_seed66", dict(kind="int8", test="test_emitter.py:6101 test_int8_matmul_gpu",
                                    seed=66, M=M, N=N, K=K, tol=0.01),
                dict(input=x, weight=w, scales=s, zeros=z, expected=exp)))
    return out


def int4_kats():
    out = []
    # tests/test_emitter.py:3009-3079
    M, N, K, G = 8, 8, 16, 16
    random.seed(7070)
    x = [random.uniform(-1.0, 1.0) for _ in range(M * K)]
    q = [random.randint(0, 15) for _ in range(N * K)]
    packed = []
    for n in range(N):
        for kp in range(K // 2):
            packed.append((q[n * K + 2 * kp + 1] << 4) | q[n * K + 2 * kp])
    ng = (K + G - 1) // G
    s, z = [0.1] * (N * ng), [8.0] * (N * ng)
    exp = [sum(x[i * K + k] * (float(q[j * K + k]) - 8.0) * 0.1 for k in range(K))
           for i in range(M) for j in range(N)]
    out.append(("int4_seed7070", dict(kind="int4", test="test_emitter.py:3009 test_int4_matmul",
                                      seed=7070, M=M, N=N, K=K, G=G, tol=0.5),
                dict(input=x, q=q, packed=packed, scales=s, zeros=z, expected=exp)))
    # tests/test_emitter.py:6157-6219
    M, N, K, G = 2, 4, 8, 8
    random.seed(44)
    x = [random.gauss(0, 1) for _ in range(M * K)]
    q = [random.randint(0, 15) for _ in range(N * K)]
    ng = (K + G - 1) // G
    s = [random.uniform(0.1, 0.5) for _ in range(N * ng)]
    z = [random.uniform(0, 8) for _ in range(N * ng)]
    exp = []
    for i in range(M):
        for j in range(N):
            acc = 0.0
            for k in range(K):
                g = k // G
                acc += x[i * K + k] * ((float(q[j * K + k]) - z[j * ng + g]) * s[j * ng + g])
            exp.append(acc)
    packed = []
    for j in range(N):
        for k in range(0, K, 2):
            packed.append((q[j * K + k] & 0x0F) | ((q[j * K + k + 1] & 0x0F) << 4))
    out.append(("int4_seed44", dict(kind="int4", test="test_emitter.py:6157 test_int4_matmul_gpu",
                                    seed=44, M=M, N=N, K=K, G=G, tol=0.1),
                dict(input=x, q=q, packed=packed, scales=s, zeros=z, expected=exp)))
    return out


def fa_kat(name, test, seed, S, D, sigma, causal, tol_abs, tol_rel, pos_step, dim_step):
    random.seed(seed)
    n = S * D
    Q = [random.gauss(0, sigma) for _ in range(n)]
    K = [random.gauss(0, sigma) for _ in range(n)]
    V = [random.gauss(0, sigma) for _ in range(n)]
    O = _attention(Q, K, V, S, D, 1.0 / math.sqrt(D), causal)
    return name, dict(kind="flash", test=test, seed=seed, S=S, D=D, causal=causal,
                      tol_abs=tol_abs, tol_rel=tol_rel, pos_step=pos_step,
                      dim_step=dim_step), dict(Q=Q, K=K, V=V, expected=O)


def all_kats():
    kats = []
    kats.append(matmul_kat("matmul_seed789", "test_emitter.py:481 test_matmul_small", 789,
                           16, 16, 16, "uniform", -1.0, 1.0, 1e-2))
    kats.append(matmul_kat("matmul_seed101r", "test_emitter.py:538 test_matmul_rectangular",
                           101, 24, 16, 32, "uniform", -1.0, 1.0, 1e-2))
    kats.append(matmul_kat("matmul_seed202", "test_emitter.py:592 test_matmul_multi_tile", 202,
                           64, 64, 64, "uniform", -0.5, 0.5, 1e-1, spot=8))
    kats.append(matmul_kat("matmul_seed42", "test_emitter.py:5950 test_matmul_gpu", 42,
                           8, 8, 8, "gauss", 0.0, 1.0, 0.01))
    kats.append(matmul_kat("matmul_seed101g", "test_emitter.py:6000 test_matmul_non_square_gpu",
                           101, 4, 8, 16, "gauss", 0.0, 0.5, 0.05))
    kats.append(matmul_kat("simdgroup_seed88", "test_emitter.py:6050 test_simdgroup_matmul_gpu",
                           88, 32, 32, 32, "gauss", 0.0, 0.5, 0.1))
    kats.append(matmul_kat("simdgroup_seed303", "test_emitter.py:1251 test_simdgroup_matmul_32x32",
                           303, 32, 32, 32, "uniform", -1.0, 1.0, 1e-2))
    kats.append(matmul_kat("simdgroup_seed404", "test_emitter.py:1286 test_simdgroup_matmul_64x64",
                           404, 64, 64, 64, "uniform", -0.5, 0.5, 1e-1, spot=4))
    kats.append(matmul_kat("simdgroup_seed505",
                           "test_emitter.py:1322 test_simdgroup_matmul_rectangular", 505,
                           64, 64, 32, "uniform", -1.0, 1.0, 1e-1, spot=4))
    kats.append(matmul_kat("simdgroup_f16_seed707",
                           "test_emitter.py:1370 test_simdgroup_matmul_fp16_32x32", 707,
                           32, 32, 32, "uniform", -1.0, 1.0, 0.1, in_dtype="fp16"))
    kats.append(matmul_kat("simdgroup_f16_seed808",
                           "test_emitter.py:1408 test_simdgroup_matmul_fp16_64x64", 808,
                           64, 64, 64, "uniform", -0.5, 0.5, 0.15, in_dtype="fp16", spot=4))
    # the sizes-in-device-memory templates (2-D dispatch and grouped order)
    kats.append(matmul_kat("matmul2d_seed1001", "test_emitter.py:651 test_matmul_2d_small", 1001,
                           16, 16, 16, "uniform", -1.0, 1.0, 1e-2, kind="matmul_2d"))
    kats.append(matmul_kat("matmul2d_seed1002", "test_emitter.py:705 test_matmul_2d_multi_tile",
                           1002, 64, 64, 64, "uniform", -0.5, 0.5, 1e-1, spot=8,
                           kind="matmul_2d"))
    kats.append(matmul_kat("matmul2d_seed1003", "test_emitter.py:758 test_matmul_2d_rectangular",
                           1003, 48, 64, 32, "uniform", -1.0, 1.0, 1e-1, spot=8, spot_m=6,
                           kind="matmul_2d"))
    kats.append(matmul_kat("swizzled_seed2001", "test_emitter.py:815 test_matmul_swizzled_small",
                           2001, 16, 16, 16, "uniform", -1.0, 1.0, 1e-2, kind="matmul_swizzled",
                           extra=dict(group_size=4)))
    kats.append(matmul_kat("swizzled_seed2002", "test_emitter.py:869 test_matmul_swizzled_large",
                           2002, 128, 128, 64, "uniform", -0.5, 0.5, 1e-1, spot=16,
                           kind="matmul_swizzled", extra=dict(group_size=4)))
    kats.append(linear_kat("linear_seed1111", "test_emitter.py:2402 test_fused_linear_no_bias",
                           1111, 32, 32, 32, False, 1e-2))
    kats.append(linear_kat("linear_seed2222", "test_emitter.py:2439 test_fused_linear_with_bias",
                           2222, 32, 32, 32, True, 1e-1))
    kats += int8_kats()
    kats += int4_kats()
    kats.append(fa_kat("flash_seed555", "test_emitter.py:1849 test_flash_attention_single_head",
                       555, 16, 64, 0.5, False, 1e-3, 1e-2, 1, 1))
    kats.append(fa_kat("flash_seed666", "test_emitter.py:1926 test_flash_attention_multi_block",
                       666, 48, 64, 0.3, False, 1e-2, 0.05, 4, 8))
    kats.append(fa_kat("flash_seed1234", "test_emitter.py:2291 test_flash_attention_causal",
                       1234, 16, 64, 0.5, True, 1e-3, 0.02, 1, 8))
    kats.append(fa_kat("flash_seed123", "test_emitter.py:5579 test_flash_attention_gpu",
                       123, 8, 8, 0.3, False, 0.1, 0.0, 1, 1))
    return kats


def main():
    arrays, meta = {}, {}
    for name, m, arr in all_kats():
        meta[name] = m
        for k, v in arr.items():
            dt = np.int64 if k in ("weight", "q", "packed") and m["kind"] in ("int8", "int4") \
                else np.float64
            arrays[f"{name}/{k}"] = np.asarray(v, dtype=dt)
    np.savez_compressed(HERE / "reference_kats.npz", **arrays)
    (HERE / "reference_kats.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print(f"wrote {len(meta)} KATs")


if __name__ == "__main__":
    main()
