"""Decode attention parity on the GPU against the oracle (fp64 on the same
rounded inputs).  Tolerances: fp16/bf16 outputs atol 2e-2 / rtol 1e-2, fp32
outputs 1e-4; LSE (natural log) within 1e-3."""
import numpy as np
import pytest
import torch

import oracle
import triton_metal_amd as tm

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _problem(B, Hq, Hkv, D, S, dtype, seed):
    g = _gen(seed)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    return q, k, v


def _tol(dtype):
    return (1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 1e-2)


def _check(dev, q, k, v, lens, scale, dtype, page_table=None, kp=None, vp=None, seq_len=None):
    B, Hq, D = q.shape
    o = torch.empty(B, Hq, D, dtype=dtype, device=dev)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=dev)
    sl = None if lens is None else torch.tensor(lens, dtype=torch.int32).to(dev)
    if page_table is None:
        tm.decode_attention(q.to(dev), k.to(dev), v.to(dev), seq_lens=sl, seq_len=seq_len,
                            scale=scale, o=o, lse=lse)
        ref_o, ref_l = oracle.decode_attention(q.float().numpy(), k.float().numpy(),
                                               v.float().numpy(),
                                               lens if lens is not None else [k.shape[2]] * B,
                                               scale)
    else:
        tm.decode_attention(q.to(dev), kp.to(dev), vp.to(dev), seq_lens=sl, seq_len=seq_len,
                            page_table=page_table.to(dev), scale=scale, o=o, lse=lse)
        ref_o, ref_l = oracle.decode_attention(q.float().numpy(), kp.float().numpy(),
                                               vp.float().numpy(), lens, scale,
                                               page_table=page_table.numpy())
    torch.cuda.synchronize()
    atol, rtol = _tol(dtype)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref_o, atol=atol, rtol=rtol)
    got_l = lse.cpu().numpy()
    fin = np.isfinite(ref_l)
    assert (np.isneginf(got_l) == ~fin).all()
    np.testing.assert_allclose(got_l[fin], ref_l[fin], atol=1e-3, rtol=1e-4)


# (B, Hq, Hkv, D, S): MFMA kernels (D 64/128, 16-bit caches) with one slice and
# with many slices (long S, few heads: up to 32 slices merge in one round of
# loads, (1, 2, 1, 128, 9000) makes 36 and takes the looped merge), GQA groups
# below / above 16, D 96 in the 128 layout, and the general kernel (D 40)
SHAPES = [(1, 8, 8, 128, 1000), (2, 32, 8, 128, 4096), (3, 12, 4, 64, 300),
          (1, 40, 2, 128, 700), (2, 4, 4, 96, 100), (1, 2, 1, 64, 17), (1, 2, 1, 128, 9000),
          (2, 4, 4, 40, 100)]


# head dims 48 / 80 / 96 / 112 on the MFMA kernel in the 64 / 128 layout
# (decode_attn_d<64|128>v<D>): one slice and many, a GQA group above 16
@pytest.mark.parametrize("D", [48, 80, 96, 112])
@pytest.mark.parametrize("shape", [(2, 8, 2, 300), (1, 4, 1, 5000), (1, 24, 1, 700)],
                         ids=["B2-S300", "B1-S5000", "G24-S700"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_inlaid_head_dims(dev, D, shape, dtype):
    B, Hq, Hkv, S = shape
    q, k, v = _problem(B, Hq, Hkv, D, S, dtype, seed=D + S)
    lens = [S] + [S // 2 + 1] * (B - 1)
    _check(dev, q, k, v, lens, D ** -0.5, dtype)


@pytest.mark.parametrize("D", [80, 96])
def test_decode_inlaid_head_dims_paged_and_fp32_query(dev, D):
    """Paged caches (16-position pages) and an fp32 query over an fp16 cache
    (the hi + lo split form), D in the 128 layout."""
    B, Hq, Hkv, S = 2, 8, 2, 700
    q, k, v = _problem(B, Hq, Hkv, D, S, torch.float16, seed=D)
    kp, vp, table = _paged(k, v, 16, seed=D + 1)
    _check(dev, q, k, v, [S, 333], D ** -0.5, torch.float16, page_table=table, kp=kp, vp=vp)
    q32 = torch.randn(B, Hq, D, generator=_gen(D + 2))
    o = torch.empty(B, Hq, D, dtype=torch.float32, device=dev)
    tm.decode_attention(q32.to(dev), k.to(dev), v.to(dev), scale=D ** -0.5, o=o)
    ref, _ = oracle.decode_attention(q32.numpy(), k.float().numpy(), v.float().numpy(), [S] * B,
                                     D ** -0.5)
    torch.cuda.synchronize()
    np.testing.assert_allclose(o.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_contiguous(dev, shape, dtype):
    B, Hq, Hkv, D, S = shape
    q, k, v = _problem(B, Hq, Hkv, D, S, dtype, seed=B + Hq + S)
    rng = np.random.default_rng(S)
    lens = [int(x) for x in rng.integers(1, S + 1, size=B)]
    lens[0] = S
    _check(dev, q, k, v, lens, D ** -0.5, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_decode_empty_and_single_positions(dev, dtype):
    q, k, v = _problem(4, 8, 2, 128, 64, dtype, seed=3)
    _check(dev, q, k, v, [0, 1, 2, 64], 0.1, dtype)


def test_decode_fp32_cache_general_kernel(dev):
    q, k, v = _problem(2, 6, 3, 64, 300, torch.float32, seed=4)
    _check(dev, q, k, v, [300, 123], 64 ** -0.5, torch.float32)


@pytest.mark.parametrize("D", [32, 48, 80, 96, 112, 128])
@pytest.mark.parametrize("S", [300, 5000])
def test_decode_fp32_mfma_head_dims(dev, D, S):
    """fp32 caches and queries on the fp32-MFMA kernel (decode_attn_f32_d<D>,
    head dims multiples of 16), one slice and many, within 1e-4."""
    q, k, v = _problem(2, 8, 2, D, S, torch.float32, seed=D + S)
    _check(dev, q, k, v, [S, S // 3], D ** -0.5, torch.float32)


def test_decode_no_workspace_single_slice(dev):
    """Without room for slice partials the MFMA kernel runs one slice per wave."""
    B, Hq, Hkv, D, S = 1, 8, 8, 128, 3000
    q, k, v = _problem(B, Hq, Hkv, D, S, torch.float16, seed=5)
    o = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    tm.plan_decode_attention(q.to(dev), k.to(dev), v.to(dev), o,
                             workspace=torch.empty(16, dtype=torch.uint8, device=dev))()
    ref, _ = oracle.decode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                     [S], D ** -0.5)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)


def _paged(k, v, ps, seed):
    """Scatter dense [B, Hkv, S, D] caches into shuffled pages [n, ps, Hkv, D]."""
    B, Hkv, S, D = k.shape
    npb = (S + ps - 1) // ps
    rng = np.random.default_rng(seed)
    perm = rng.permutation(B * npb + 3)[:B * npb]
    table = torch.tensor(perm.reshape(B, npb), dtype=torch.int32)
    kp = torch.zeros(B * npb + 3, ps, Hkv, D, dtype=k.dtype)
    vp = torch.zeros_like(kp)
    for b in range(B):
        for i in range(npb):
            n = min(ps, S - ps * i)
            kp[table[b, i], :n] = k[b, :, ps * i:ps * i + n].transpose(0, 1)
            vp[table[b, i], :n] = v[b, :, ps * i:ps * i + n].transpose(0, 1)
    return kp, vp, table


@pytest.mark.parametrize("ps", [16, 32, 48, 1])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_paged(dev, ps, dtype):
    B, Hq, Hkv, D, S = 3, 16, 4, 128, 1200 if ps > 1 else 200
    q, k, v = _problem(B, Hq, Hkv, D, S, dtype, seed=ps)
    kp, vp, table = _paged(k, v, ps, seed=ps + 1)
    _check(dev, q, k, v, [S, S // 2 + 3, 1], D ** -0.5, dtype, page_table=table, kp=kp, vp=vp)


def test_decode_paged_fp32_general(dev):
    q, k, v = _problem(2, 4, 2, 64, 100, torch.float32, seed=9)
    kp, vp, table = _paged(k, v, 16, seed=10)
    _check(dev, q, k, v, [100, 37], 0.125, torch.float32, page_table=table, kp=kp, vp=vp)


# --- the reference templates' buffer orders -------------------------------------
def test_reference_template_wrappers(dev):
    D, S = 64, 200
    g = _gen(11)
    # kv_cache_attention: Q [H, D], caches [H, seq_len, D]
    H = 4
    Q = torch.randn(H, D, generator=g).half(); Kc = torch.randn(H, S, D, generator=g).half()
    Vc = torch.randn(H, S, D, generator=g).half()
    O = torch.empty(H, D, dtype=torch.float16, device=dev)
    tm.make_kv_cache_attention_kernel(D)(Q.to(dev), Kc.to(dev), Vc.to(dev), O, S, 0.2)
    ref, _ = oracle.decode_attention(Q[None].float().numpy(), Kc[None].float().numpy(),
                                     Vc[None].float().numpy(), [S], 0.2)
    np.testing.assert_allclose(O.float().cpu().numpy(), ref[0], atol=2e-2, rtol=1e-2)
    # gqa_attention: 8 query heads over 2 KV heads
    Q = torch.randn(8, D, generator=g).half(); Kc = torch.randn(2, S, D, generator=g).half()
    Vc = torch.randn(2, S, D, generator=g).half()
    O = torch.empty(8, D, dtype=torch.float16, device=dev)
    tm.make_gqa_attention_kernel(D, n_q_per_kv=4)(Q.to(dev), Kc.to(dev), Vc.to(dev), O, S, 0.2)
    ref, _ = oracle.decode_attention(Q[None].float().numpy(), Kc[None].float().numpy(),
                                     Vc[None].float().numpy(), [S], 0.2)
    np.testing.assert_allclose(O.float().cpu().numpy(), ref[0], atol=2e-2, rtol=1e-2)
    # batched_kv_decode: [B, H, max_seq_len, D], per-batch lengths, scale 1/sqrt(D)
    B, H = 3, 4
    Q = torch.randn(B, H, D, generator=g).half(); Kc = torch.randn(B, H, S, D, generator=g).half()
    Vc = torch.randn(B, H, S, D, generator=g).half()
    lens = torch.tensor([S, 50, 0], dtype=torch.int32)
    O = torch.empty(B, H, D, dtype=torch.float16, device=dev)
    tm.make_batched_kv_decode_kernel(H, D)(Q.to(dev), Kc.to(dev), Vc.to(dev), O, lens.to(dev), S, B)
    ref, _ = oracle.decode_attention(Q.float().numpy(), Kc.float().numpy(), Vc.float().numpy(),
                                     lens.tolist(), D ** -0.5)
    np.testing.assert_allclose(O.float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)
    # paged_attention (one head) and multi_head_paged_attention
    ps, n_pages = 16, (S + 15) // 16
    for heads in (1, 4):
        Q = torch.randn(heads, D, generator=g).half()
        Kd = torch.randn(1, heads, S, D, generator=g).half()
        Vd = torch.randn(1, heads, S, D, generator=g).half()
        kp, vp, table = _paged(Kd, Vd, ps, seed=heads)
        O = torch.empty(heads, D, dtype=torch.float16, device=dev)
        if heads == 1:
            tm.make_paged_attention_kernel(D, ps)(Q[0].to(dev), kp[:, :, 0].contiguous().to(dev),
                                                   vp[:, :, 0].contiguous().to(dev),
                                                   table[0].to(dev), O[0], S, n_pages)
        else:
            tm.make_multi_head_paged_attention_kernel(heads, D, ps)(
                Q.to(dev), kp.to(dev), vp.to(dev), table[0].to(dev), O, S, n_pages)
        ref, _ = oracle.decode_attention(Q[None].float().numpy(), Kd.float().numpy(),
                                         Vd.float().numpy(), [S], D ** -0.5)
        np.testing.assert_allclose(O.float().cpu().numpy(), ref[0], atol=2e-2, rtol=1e-2)
    # fp16_kv_attention: fp32 query and output, fp16 cache
    Q = torch.randn(D, generator=g); Kc = torch.randn(S, D, generator=g).half()
    Vc = torch.randn(S, D, generator=g).half()
    O = torch.empty(D, dtype=torch.float32, device=dev)
    tm.make_fp16_kv_attention_kernel(D)(Q.to(dev), Kc.to(dev), Vc.to(dev), O, 150)
    ref, _ = oracle.decode_attention(Q[None, None].numpy(), Kc[None, None].float().numpy(),
                                     Vc[None, None].float().numpy(), [150], D ** -0.5)
    # the reference computes in fp32 throughout (an fp32 query against float(half K))
    np.testing.assert_allclose(O.cpu().numpy(), ref[0, 0], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D,S", [(64, 150), (128, 3000)])
def test_decode_fp32_query_exact(dev, kv_dtype, D, S):
    """fp32 queries and outputs over a 16-bit cache (the fp16_kv_attention
    contract) keep fp32 accuracy on the MFMA path, one slice and many, GQA."""
    g = _gen(21)
    B, Hq, Hkv = 2, 8, 2
    q = torch.randn(B, Hq, D, generator=g) * 2.0
    k = torch.randn(B, Hkv, S, D, generator=g).to(kv_dtype)
    v = torch.randn(B, Hkv, S, D, generator=g).to(kv_dtype)
    lens = torch.tensor([S, S // 3], dtype=torch.int32)
    o = torch.empty(B, Hq, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=dev)
    tm.decode_attention(q.to(dev), k.to(dev), v.to(dev), seq_lens=lens.to(dev), o=o, lse=lse)
    ref, ref_l = oracle.decode_attention(q.numpy(), k.float().numpy(), v.float().numpy(),
                                         lens.tolist(), D ** -0.5)
    np.testing.assert_allclose(o.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_l, atol=1e-4, rtol=1e-5)


def test_reference_wrappers_capacity_beyond_seq_len(dev):
    """kv_cache_attention / gqa_attention space heads by seq_len as the
    reference does (head_offset_kv = pid * seq_len * D), also when the buffers
    hold more positions than seq_len."""
    D, S, cap = 64, 100, 160
    g = _gen(23)
    H = 4
    Q = torch.randn(H, D, generator=g).half()
    flatK = torch.randn(H * cap * D, generator=g).half()
    flatV = torch.randn(H * cap * D, generator=g).half()
    O = torch.empty(H, D, dtype=torch.float16, device=dev)
    tm.make_kv_cache_attention_kernel(D)(Q.to(dev), flatK.to(dev), flatV.to(dev), O, S, 0.2)
    Kr = flatK[:H * S * D].view(H, S, D)
    Vr = flatV[:H * S * D].view(H, S, D)
    ref, _ = oracle.decode_attention(Q[None].float().numpy(), Kr[None].float().numpy(),
                                     Vr[None].float().numpy(), [S], 0.2)
    np.testing.assert_allclose(O.float().cpu().numpy(), ref[0], atol=2e-2, rtol=1e-2)
    Hq, n = 8, 4
    Q = torch.randn(Hq, D, generator=g).half()
    O = torch.empty(Hq, D, dtype=torch.float16, device=dev)
    tm.make_gqa_attention_kernel(D, n_q_per_kv=n)(Q.to(dev), flatK.to(dev), flatV.to(dev), O, S,
                                                  0.2)
    Kr = flatK[:(Hq // n) * S * D].view(Hq // n, S, D)
    Vr = flatV[:(Hq // n) * S * D].view(Hq // n, S, D)
    ref, _ = oracle.decode_attention(Q[None].float().numpy(), Kr[None].float().numpy(),
                                     Vr[None].float().numpy(), [S], 0.2)
    np.testing.assert_allclose(O.float().cpu().numpy(), ref[0], atol=2e-2, rtol=1e-2)


def test_decode_fp32_query_beyond_fp16_range(dev):
    """An fp32 query with elements past the largest finite half (65504) over an
    fp16 cache stays finite and exact: the hi part saturates at 65504 and the
    lo part carries the remainder (70000 = 65504 + 4496, -100000 = -65504 -
    34496, both halves exact), as the reference's fp32 arithmetic gives."""
    g = _gen(31)
    B, Hq, Hkv, D, S = 1, 4, 1, 64, 200
    q = torch.randn(B, Hq, D, generator=g)
    q[0, 0, 3] = 70000.0
    q[0, 1, 10] = -100000.0
    q[0, 2, 0] = 65504.0
    k = torch.randn(B, Hkv, S, D, generator=g).half()
    v = torch.randn(B, Hkv, S, D, generator=g).half()
    scale = 1e-5
    o = torch.empty(B, Hq, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=dev)
    tm.decode_attention(q.to(dev), k.to(dev), v.to(dev), scale=scale, o=o, lse=lse)
    ref, ref_l = oracle.decode_attention(q.numpy(), k.float().numpy(), v.float().numpy(),
                                         [S], scale)
    got = o.cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_l, atol=1e-4, rtol=1e-5)
