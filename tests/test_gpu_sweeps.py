"""Seeded random-shape sweeps on the GPU.

Each entry point runs over problem shapes drawn (with a fixed seed) across its
dispatch plan -- the fast kernels, the edges of their shape conditions and the
general fallbacks -- and is checked against the oracle at the tolerances of
the per-kernel tests: fp16/bf16 outputs atol 2e-2 / rtol 1e-2, fp32 outputs
1e-4 (attention) or the reference templates' 1e-3 scale, LSE within 1e-3.
The case lists are fixed by the seeds, so a failure names a reproducible case;
each test prints the kernel the plan picked.
"""
import ctypes as C
import math

import numpy as np
import pytest
import torch

import oracle
import triton_metal_amd as tm
from triton_metal_amd import _lib

pytestmark = pytest.mark.gpu
F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
DT_CODE = {F32: _lib.TM_DT_F32, F16: _lib.TM_DT_F16, BF16: _lib.TM_DT_BF16}


def _tol(dt):
    return (1e-4, 1e-4) if dt == F32 else (2e-2, 1e-2)


# --- weight-only matmuls ------------------------------------------------------
def _wq_cases(n=64, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        qbits = int(rng.choice([4, 8]))
        act = [F16, BF16, F16, BF16, F16, BF16, F16, F32][int(rng.integers(8))]
        M = int(rng.choice([1, int(rng.integers(2, 9)), int(rng.integers(9, 17)),
                            int(rng.integers(17, 65)), int(rng.integers(65, 161))]))
        G = 128 if qbits == 8 or rng.random() < 0.8 else int(rng.choice([64, 32, 256]))
        if rng.random() < 0.85:  # the fast kernels' K (and past their limits)
            K = int(rng.choice([512, 1024, 2048, 3072, 4096, 4096, 5120, 6144, 8192, 11008,
                                14336, 20480]))
        else:
            K = 2 * int(rng.integers(1, 2048))
        if qbits == 4 and K % G and rng.random() < 0.5:
            K = G * max(1, K // G)
        if rng.random() < 0.85:
            N = 16 * int(rng.integers(1, 129)) * (8 if rng.random() < 0.3 else 1)
        else:
            N = int(rng.integers(1, 700))
        zeros = [None, "s", "u8"][int(rng.integers(3))]
        ws = bool(rng.random() < 0.7)
        bias = bool(rng.random() < 0.3)
        if M * N * K > 2.5e9 or N * K > 4.5e7:
            continue
        out.append((qbits, M, N, K, G, act, zeros, ws, bias))
    return out


def _wq_fast_cases(n=24, seed=515):
    """Shapes inside the fast kernels' conditions, sizes drawn at random: the
    wide kernel (M > 64, N % 128 == 0) with and without split-K, the
    persistent GEMV (M = 1, K = 4096) and the long-K kernel past its
    single-launch K."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        z = [None, "s", "u8"][int(rng.integers(3))]
        ws, b = bool(rng.random() < 0.7), bool(rng.random() < 0.3)
        kind = i % 3
        if kind == 0:
            qbits = int(rng.choice([4, 8]))
            act = F16 if qbits == 4 else [F16, BF16][int(rng.integers(2))]
            M, N = int(rng.integers(65, 200)), 128 * int(rng.integers(1, 17))
            K = 512 * int(rng.integers(1, 17)) if qbits == 4 else 128 * int(rng.integers(1, 40))
            z = z if qbits == 4 else None
        elif kind == 1:
            qbits, act, M, K = 4, [F16, BF16][int(rng.integers(2))], 1, 4096
            N = 16 * int(rng.integers(1, 1025))
        else:
            qbits = int(rng.choice([4, 8]))
            act = [F16, BF16][int(rng.integers(2))]
            M = int(rng.integers(1, 65))
            K = 128 * int(rng.integers(129, 321))
            N = 16 * int(rng.integers(1, 80))
        out.append((qbits, M, N, K, 128, act, z, ws, b))
    return out


WQ_CASES = _wq_cases() + _wq_fast_cases()


def _wq_id(c):
    q, M, N, K, G, a, z, ws, b = c
    return (f"q{q}-M{M}-N{N}-K{K}-G{G}-{str(a).split('.')[-1]}-z{z}"
            + ("" if ws else "-nows") + ("-bias" if b else ""))


@pytest.mark.parametrize("case", WQ_CASES, ids=[_wq_id(c) for c in WQ_CASES])
def test_wq_random_shapes(dev, case):
    qbits, M, N, K, G, act, zeros, ws, use_bias = case
    g = torch.Generator().manual_seed(M * 7919 + N * 31 + K)
    x = torch.randn(M, K, generator=g).to(act)
    if qbits == 4:
        ng = (K + G - 1) // G
        q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
        w = torch.from_numpy(oracle.pack_int4(q.numpy()))
        s = (torch.rand(N, ng, generator=g) * 0.019 + 0.001).to(act)
        zi = torch.randint(0, 16, (N, ng), generator=g)
    else:
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        s = (torch.rand(N, generator=g) * 0.019 + 0.001).to(act)
        zi = torch.randint(-3, 4, (N,), generator=g)
        if zeros == "u8":
            zi = zi.abs()
    z = None if zeros is None else (zi.to(torch.uint8) if zeros == "u8" else zi.to(act))
    bias = (torch.randn(N, generator=g) * 0.5).to(act) if use_bias else None
    zdt = None if z is None else z.dtype
    plan = tm.wq_kernel_for(qbits, M, N, K, G, act_dtype=act, zero_dtype=zdt,
                            with_workspace=ws, details=True)
    print(f"[sweep] {_wq_id(case)} -> {plan['name']} splits={plan['splits']}", flush=True)
    d = lambda t: None if t is None else t.to(dev)
    out = torch.full((M, N), 5.0, dtype=act, device=dev)
    if ws:
        if qbits == 4:
            tm.int4_linear(d(x), d(w), d(bias), out, d(s), d(z), M, N, K, G)
        else:
            tm.int8_linear(d(x), d(w), d(bias), out, d(s), d(z), M, N, K)
    else:
        L = _lib.lib()
        p = lambda t: None if t is None else t.data_ptr()
        xd, wd, sd, zd, bd = d(x), d(w), d(s), d(z), d(bias)
        zc = _lib.TM_DT_NONE if z is None else (_lib.TM_DT_U8 if z.dtype == torch.uint8
                                                 else DT_CODE[act])
        adt = DT_CODE[act]
        stream = torch.cuda.current_stream(dev).cuda_stream
        if qbits == 4:
            rc = L.tm_int4_linear(p(xd), p(wd), p(bd), p(out), p(sd), p(zd), M, N, K, G, adt, adt,
                                  zc, stream)
        else:
            rc = L.tm_int8_linear(p(xd), p(wd), p(bd), p(out), p(sd), p(zd), M, N, K, adt, adt,
                                  zc, stream)
        assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    np32 = lambda t: None if t is None else t.float().numpy()
    if qbits == 4:
        ref = oracle.int4_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K, G)
    else:
        ref = oracle.int8_matmul(np32(x), w.numpy(), np32(s), np32(z), M, N, K)
    if bias is not None:
        ref = ref + np32(bias)[None, :].astype(np.float64)
    atol, rtol = (1e-3, 1e-4) if act == F32 else (2e-2, 1e-2)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=atol, rtol=rtol)


# --- dense matmul / linear ----------------------------------------------------
def _dense_cases(n=36, seed=4242):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = [F16, BF16, F16, BF16, F32][int(rng.integers(5))]
        out32 = bool(rng.random() < 0.4) and dt != F32
        form = ["matmul", "matmul", "linear", "strided"][int(rng.integers(4))]
        r = rng.random()
        if r < 0.15:  # the 256-tile kernel: multiples of 256, >= 32 tiles
            M, N = 256 * int(rng.integers(4, 9)), 256 * int(rng.integers(8, 13))
            K = 64 * int(rng.integers(1, 4))
        elif r < 0.45:  # multiples of 32 (small-tile kernels)
            M, N = 32 * int(rng.integers(1, 33)), 32 * int(rng.integers(1, 33))
            K = int(rng.choice([256, 512, 8 * int(rng.integers(1, 200))]))
        else:
            M, N, K = (int(v) for v in rng.integers(1, 700, size=3))
        out.append((form, M, N, K, dt, out32, bool(rng.random() < 0.5)))
    return out


DENSE_CASES = _dense_cases()


@pytest.mark.parametrize("case", DENSE_CASES,
                         ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-{str(c[4]).split('.')[-1]}"
                              + ("-out32" if c[5] else "") + ("-bias" if c[6] else "")
                              for c in DENSE_CASES])
def test_dense_random_shapes(dev, case):
    form, M, N, K, dt, out32, use_bias = case
    g = torch.Generator().manual_seed(M * 131 + N * 7 + K)
    odt = F32 if out32 else dt
    atol, rtol = (1e-3, 1e-4) if odt == F32 else (2e-2, 1e-2)
    if dt != F32:
        atol = max(atol, 1e-3 * math.sqrt(K))  # bf16 / fp16 inputs, fp32 sums of K terms
    if form == "linear":
        x, W = torch.randn(M, K, generator=g).to(dt), torch.randn(N, K, generator=g).to(dt)
        b = torch.randn(N, generator=g).to(dt) if use_bias else None
        C_ = torch.empty(M, N, dtype=dt, device=dev)
        tm.fused_linear(x.to(dev), W.to(dev), C_, None if b is None else b.to(dev), M, N, K)
        ref = oracle.linear(x.float().numpy(), W.float().numpy(),
                            None if b is None else b.float().numpy())
        atol, rtol = (1e-3, 1e-4) if dt == F32 else (max(2e-2, 1e-3 * math.sqrt(K)), 1e-2)
    elif form == "matmul":
        A, B = torch.randn(M, K, generator=g).to(dt), torch.randn(K, N, generator=g).to(dt)
        C_ = torch.empty(M, N, dtype=odt, device=dev)
        tm.matmul(A.to(dev), B.to(dev), C_, M, N, K)
        ref = oracle.matmul(A.float().numpy(), B.float().numpy())
    else:  # the C ABI with leading dimensions past the logical widths
        pad = lambda n: n + 8 * int(1 + (M + N + K) % 5)
        lda, ldb, ldc = pad(K), pad(N), pad(N)
        A = torch.randn(M, lda, generator=g).to(dt)
        B = torch.randn(K, ldb, generator=g).to(dt)
        Cp = torch.zeros(M, ldc, dtype=odt, device=dev)
        Ad, Bd = A.to(dev), B.to(dev)
        rc = _lib.lib().tm_matmul(C.c_void_p(Ad.data_ptr()), C.c_void_p(Bd.data_ptr()),
                                  C.c_void_p(Cp.data_ptr()), M, N, K, lda, ldb, ldc,
                                  DT_CODE[dt], DT_CODE[odt], None)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        ref = oracle.matmul(A[:, :K].float().numpy(), B[:, :N].float().numpy())
        got = Cp.float().cpu().numpy()
        assert (got[:, N:] == 0).all()
        np.testing.assert_allclose(got[:, :N], ref, atol=atol, rtol=rtol)
        return
    torch.cuda.synchronize()
    np.testing.assert_allclose(C_.float().cpu().numpy(), ref, atol=atol, rtol=rtol)


# --- tl.dot in general form ---------------------------------------------------
def _dot_cases(n=40, seed=9090):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = [F16, BF16, F32, F32][int(rng.integers(4))]
        odt = dt if rng.random() < 0.5 else F32
        epi = ["none", "none", "add-matrix", "add-rows", "add-cols"][int(rng.integers(5))]
        batch = None if rng.random() < 0.5 else int(rng.integers(1, 5))
        la = ["row", "col", "strided"][int(rng.integers(3))]
        lb = ["row", "col", "strided"][int(rng.integers(3))]
        if rng.random() < 0.3:
            M, N, K = (64 * int(v) for v in rng.integers(1, 6, size=3))
        else:
            M, N, K = (int(v) for v in rng.integers(1, 400, size=3))
        out.append((dt, odt, epi, batch, la, lb, M, N, K))
    return out


def _operand(rows, cols, bs, dt, layout, g, dev):
    """A [.., rows, cols] view on the device in the given layout and its CPU
    values: row-major, column-major (a transposed copy) or every second
    element of a wider row."""
    x = torch.randn(*bs, rows, cols, generator=g).to(dt)
    if layout == "row":
        return x.to(dev), x
    if layout == "col":
        return x.transpose(-1, -2).contiguous().to(dev).transpose(-1, -2), x
    buf = torch.zeros(*bs, rows, 2 * cols + 1, dtype=dt)
    buf[..., : 2 * cols : 2] = x
    return buf.to(dev)[..., : 2 * cols : 2], x


DOT_CASES = _dot_cases()


@pytest.mark.parametrize("case", DOT_CASES,
                         ids=[f"{str(c[0]).split('.')[-1]}-{str(c[1]).split('.')[-1]}-{c[2]}"
                              f"-b{c[3]}-{c[4]}-{c[5]}-{c[6]}x{c[7]}x{c[8]}" for c in DOT_CASES])
def test_dot_random_layouts(dev, case):
    """tm.dot with mixed operand layouts, batches and add-* epilogues against
    oracle.dot; fp32 outputs within 1e-4 |ref| + 2^-16 (|A| @ |B|) (fp32
    accumulation of exact products), 16-bit outputs atol 2e-2 / rtol 1e-2."""
    dt, odt, epi, batch, la, lb, M, N, K = case
    g = torch.Generator().manual_seed(M * 977 + N * 31 + K)
    bs = () if batch is None else (batch,)
    a, a_cpu = _operand(M, K, bs, dt, la, g, dev)
    b, b_cpu = _operand(K, N, bs, dt, lb, g, dev)
    z = z_cpu = None
    if epi != "none":
        z_cpu = torch.randn(*bs, M, N, generator=g).to(dt)
        z = z_cpu.to(dev)
    c = torch.empty(*bs, M, N, dtype=odt, device=dev)
    tm.dot(a, b, c, epi, z=z)
    torch.cuda.synchronize()
    an, bn = a_cpu.double().numpy(), b_cpu.double().numpy()
    ref = oracle.dot(an, bn, epi, Z=None if z_cpu is None else z_cpu.double().numpy())
    got = c.double().cpu().numpy()
    if odt == F32:
        bound = 1e-4 * np.abs(ref) + 2.0 ** -16 * (np.abs(an) @ np.abs(bn))
        err = np.abs(got - ref)
        assert (err <= bound + 1e-30).all(), f"max err {err.max():.3e}"
    else:
        np.testing.assert_allclose(got, ref, atol=2e-2, rtol=1e-2)


# --- flash attention ----------------------------------------------------------
def _fa_cases(n=28, seed=777):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
        S = int(rng.choice([int(rng.integers(1, 130)), int(rng.integers(130, 700)),
                            128 * int(rng.integers(1, 6))]))
        D = int(rng.choice([32, 64, 128, 128, 64, 48, 80, 96]))
        dt = [F16, BF16, BF16, F32][int(rng.integers(4))]
        out.append((B, H, S, D, dt, bool(rng.random() < 0.5), bool(rng.random() < 0.3)))
    return out


FA_CASES = _fa_cases()


@pytest.mark.parametrize("case", FA_CASES,
                         ids=[f"B{c[0]}-H{c[1]}-S{c[2]}-D{c[3]}-{str(c[4]).split('.')[-1]}"
                              + ("-causal" if c[5] else "") + ("-strided" if c[6] else "")
                              for c in FA_CASES])
def test_flash_random_shapes(dev, case):
    B, H, S, D, dt, causal, strided = case
    g = torch.Generator().manual_seed(B * 1000 + H * 100 + S + D)
    if strided:  # [B, S, H, D] storage seen as [B, H, S, D]
        mk = lambda: torch.randn(B, S, H, D, generator=g).to(dt).to(dev).transpose(1, 2)
    else:
        mk = lambda: torch.randn(B, H, S, D, generator=g).to(dt).to(dev)
    q, k, v = mk(), mk(), mk()
    o, lse = tm.attention(q, k, v, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.flash_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                          v.float().cpu().numpy(), 1.0 / math.sqrt(D), causal)
    atol, rtol = _tol(dt)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=atol, rtol=rtol)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)


# --- decode attention ---------------------------------------------------------
def _decode_cases(n=30, seed=99):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        B = int(rng.integers(1, 6))
        Hkv = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4, 8, 16, 32]))
        D = int(rng.choice([64, 128, 128, 96]))
        S = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 3000))]))
        cache = [F16, BF16, F16, F32][int(rng.integers(4))]
        qdt = F32 if (cache != F32 and rng.random() < 0.25) else cache
        paged = bool(rng.random() < 0.4)
        ps = int(rng.choice([8, 16, 32, 64, 24])) if paged else 0
        ragged = bool(rng.random() < 0.6)
        out.append((B, Hkv, group, D, S, cache, qdt, ps, ragged))
    return out


DECODE_CASES = _decode_cases()


@pytest.mark.parametrize("case", DECODE_CASES,
                         ids=[f"B{c[0]}-kv{c[1]}-g{c[2]}-D{c[3]}-S{c[4]}-"
                              f"{str(c[5]).split('.')[-1]}-q{str(c[6]).split('.')[-1]}"
                              + (f"-page{c[7]}" if c[7] else "") + ("-ragged" if c[8] else "")
                              for c in DECODE_CASES])
def test_decode_random_shapes(dev, case):
    B, Hkv, group, D, S, cache, qdt, ps, ragged = case
    Hq = Hkv * group
    rng = np.random.default_rng(B * 100000 + Hq * 1000 + S)
    g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    lens = [int(x) for x in rng.integers(0, S + 1, size=B)] if ragged else [S] * B
    q = torch.randn(B, Hq, D, generator=g).to(qdt)
    scale = D ** -0.5
    o = torch.empty(B, Hq, D, dtype=qdt, device=dev)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    if ps:
        max_pages = (S + ps - 1) // ps
        npages = B * max_pages + 3
        kp = torch.randn(npages, ps, Hkv, D, generator=g).to(cache)
        vp = torch.randn(npages, ps, Hkv, D, generator=g).to(cache)
        table = torch.from_numpy(rng.permutation(npages)[:B * max_pages].reshape(B, max_pages)
                                 .astype(np.int32))
        tm.decode_attention(q.to(dev), kp.to(dev), vp.to(dev), seq_lens=sl, seq_len=S,
                            page_table=table.to(dev), scale=scale, o=o, lse=lse)
        ref_o, ref_l = oracle.decode_attention(q.float().numpy(), kp.float().numpy(),
                                               vp.float().numpy(), lens, scale,
                                               page_table=table.numpy())
    else:
        k = torch.randn(B, Hkv, S, D, generator=g).to(cache)
        v = torch.randn(B, Hkv, S, D, generator=g).to(cache)
        tm.decode_attention(q.to(dev), k.to(dev), v.to(dev), seq_lens=sl, seq_len=S,
                            scale=scale, o=o, lse=lse)
        ref_o, ref_l = oracle.decode_attention(q.float().numpy(), k.float().numpy(),
                                               v.float().numpy(), lens, scale)
    torch.cuda.synchronize()
    atol, rtol = _tol(qdt)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref_o, atol=atol, rtol=rtol)
    got_l = lse.cpu().numpy()
    fin = np.isfinite(ref_l)
    assert (np.isneginf(got_l) == ~fin).all()
    np.testing.assert_allclose(got_l[fin], ref_l[fin], atol=1e-3, rtol=1e-4)
