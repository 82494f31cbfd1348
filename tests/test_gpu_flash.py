"""FlashAttention forward parity on the GPU against the oracle.

bf16/fp16 outputs within atol 2e-2 / rtol 1e-2 of the oracle's fp64 attention
on the same (rounded) inputs; LSE (fp32) within 1e-3; the reference's own
known-answer tests with the reference's tolerances.
"""
import math

import numpy as np
import pytest
import torch

import oracle
import triton_metal_amd as tm

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2


def _rand(shape, seed, dt, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dt).to(dev)


def _ref(q, k, v, causal, scale=None):
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    return oracle.flash_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                  v.float().cpu().numpy(), scale, causal)


# --- reference known-answer tests (fp32 template ABI, [n_heads*seq, D]) -------
@pytest.mark.parametrize("name", ["flash_seed555", "flash_seed666", "flash_seed1234",
                                  "flash_seed123"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_flash_reference_kat(kats, dev, name, dtype):
    m, a = kats[name]
    S, D = m["S"], m["D"]
    Q, K, V = (torch.tensor(a[x], dtype=dtype, device=dev).reshape(S, D) for x in "QKV")
    O = torch.empty_like(Q)
    kern = tm.make_flash_attention_kernel(head_dim=D, causal=m["causal"])
    kern(Q, K, V, O, S, 1.0 / math.sqrt(D))
    got = O.float().cpu().numpy().reshape(S, D)
    exp = a["expected"].reshape(S, D)
    sel = np.zeros((S, D), bool)
    sel[::m["pos_step"], ::m["dim_step"]] = True
    tol = np.maximum(m["tol_abs"], np.abs(exp) * m["tol_rel"])
    if dtype != torch.float32:
        tol = np.maximum(tol, ATOL + RTOL * np.abs(exp))
    assert np.all(np.abs(got - exp)[sel] < tol[sel])


# --- @triton.jit signature (tests/test_flash_attention.py shapes, seed 42) ----
FA_SHAPES_NC = [(1, 1, 32, 32), (1, 1, 64, 32), (1, 1, 64, 64), (1, 2, 64, 32), (2, 2, 64, 32),
                (1, 1, 128, 32)]
FA_SHAPES_C = [(1, 1, 32, 32), (1, 1, 64, 32), (1, 1, 64, 64), (1, 2, 64, 32), (1, 1, 128, 32)]


@pytest.mark.parametrize("causal,shape", [(False, s) for s in FA_SHAPES_NC] +
                                         [(True, s) for s in FA_SHAPES_C])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flash_attn_fwd_signature(dev, causal, shape, dtype):
    Z, H, N, D = shape
    torch.manual_seed(42)
    q = torch.randn(Z, H, N, D, dtype=torch.float32)
    k = torch.randn(Z, H, N, D, dtype=torch.float32)
    v = torch.randn(Z, H, N, D, dtype=torch.float32)
    q, k, v = (t.to(dtype).to(dev) for t in (q, k, v))
    out = torch.empty_like(q)
    tm.flash_attn_fwd(q, k, v, out, *q.stride(), *k.stride(), *v.stride(), *out.stride(),
                      Z, H, N, BLOCK_M=min(32, N), BLOCK_N=min(32, N), HEAD_DIM=D,
                      IS_CAUSAL=causal)
    ref, _ = _ref(q, k, v, causal)
    err = np.abs(out.float().cpu().numpy() - ref)
    if dtype == torch.float32:
        assert err.max() < 0.01   # the reference test's bound
    else:
        assert np.all(err <= ATOL + RTOL * np.abs(ref))


# --- MFMA path: shapes, partial tiles, LSE ---------------------------------------
@pytest.mark.parametrize("S", [1, 17, 64, 100, 128, 257, 511, 777, 1025])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flash_mfma_shapes(dev, S, D, causal, dtype):
    B, H = 2, 3
    q, k, v = (_rand((B, H, S, D), s, dtype, dev) for s in (1, 2, 3))
    o, lse = tm.attention(q, k, v, causal=causal, return_lse=True)
    ref, ref_lse = _ref(q, k, v, causal)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("S", [1, 100, 257, 777])
@pytest.mark.parametrize("D", [48, 80, 96, 112])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flash_mfma_inlaid_head_dims(dev, S, D, causal, dtype):
    """Head dims 48 / 80 / 96 / 112 on the MFMA kernel in the 64 / 128 layout
    (flash_fwd_d<64|128>v<D>): the chunks past D are neither copied nor read,
    and the output columns past D are not written (checked against a sentinel
    in a wider buffer)."""
    B, H = 2, 3
    q, k, v = (_rand((B, H, S, D), s, dtype, dev) for s in (11, 12, 13))
    wide = torch.full((B, H, S, D + 16), 5.0, dtype=dtype, device=dev)
    o = wide[..., :D]
    lse = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    tm.plan_flash_attention(q, k, v, o, lse, causal=causal)()
    torch.cuda.synchronize()
    ref, ref_lse = _ref(q, k, v, causal)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)
    assert (wide[..., D:] == 5.0).all()


@pytest.mark.parametrize("S", [1, 100, 257])
@pytest.mark.parametrize("D", [32, 48, 64, 80, 96, 112, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_fp32_mfma_head_dims(dev, S, D, causal):
    """fp32 (the reference template's dtype) on the fp32-MFMA kernel,
    flash_fwd_f32_d<D>: within 1e-4 of the oracle, LSE within 1e-4."""
    B, H = 2, 3
    q, k, v = (_rand((B, H, S, D), s, torch.float32, dev) for s in (21, 22, 23))
    o, lse = tm.attention(q, k, v, causal=causal, return_lse=True)
    ref, ref_lse = _ref(q, k, v, causal)
    np.testing.assert_allclose(o.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=1e-4, rtol=1e-5)


def test_flash_inlaid_head_dim_strided_views(dev):
    """D = 96 through views of a packed [B, S, 3, H, D] tensor (row strides
    3 H D), causal."""
    B, S, H, D = 2, 200, 4, 96
    qkv = _rand((B, S, 3, H, D), 17, torch.bfloat16, dev)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    o = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=dev).transpose(1, 2)
    tm.plan_flash_attention(q, k, v, o, causal=True)()
    ref, _ = _ref(q, k, v, True)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_flash_strided_views(dev):
    """q, k, v as views into a packed [B, S, 3, H, D] tensor."""
    B, S, H, D = 2, 96, 4, 64
    qkv = _rand((B, S, 3, H, D), 7, torch.bfloat16, dev)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    o = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=dev).transpose(1, 2)
    tm.plan_flash_attention(q, k, v, o, causal=True)()
    ref, _ = _ref(q, k, v, True)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_flash_custom_scale_and_closed_forms(dev):
    B, H, S, D = 1, 2, 130, 128
    v = _rand((B, H, S, D), 9, torch.bfloat16, dev)
    k = _rand((B, H, S, D), 10, torch.bfloat16, dev)
    q = torch.zeros_like(k)                       # uniform scores
    o, lse = tm.attention(q, k, v, causal=False, scale=0.3, return_lse=True)
    np.testing.assert_allclose(o.float().cpu().numpy(),
                               v.float().mean(2, keepdim=True).expand_as(v).cpu().numpy(),
                               atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(lse.cpu().numpy(), math.log(S), atol=1e-4)
    q = _rand((B, H, S, D), 11, torch.bfloat16, dev)
    o = tm.attention(q, k, v, causal=True, scale=0.3)
    assert torch.equal(o[:, :, 0], v[:, :, 0])    # row 0 sees only key 0


@pytest.mark.parametrize("B,H", [(1, 24), (2, 8), (1, 40)])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_every_head_xcd_pairing(dev, B, H, causal):
    """B*H a multiple of 8 takes the work order that gives each XCD its heads
    two at a time (3 and 5 heads per XCD leave the last one alone, 2 pairs
    them): every (batch, head) and every query block against the oracle."""
    S, D = 300, 128
    q, k, v = (_rand((B, H, S, D), s, torch.bfloat16, dev) for s in (31, 32, 33))
    o, lse = tm.attention(q, k, v, causal=causal, return_lse=True)
    ref, ref_lse = _ref(q, k, v, causal)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)


# --- benchmark configuration C4 (sampled rows against the oracle) -----------------
@pytest.mark.parametrize("causal", [True, False])
def test_flash_config_c4(dev, causal):
    """C4 at full size: every one of the 128 (batch, head) pairs on 24 rows
    sampled across the sequence (the last row always), and three heads on 128
    rows, against the fp64 softmax of the same bf16 inputs."""
    B, H, S, D = 4, 32, 4096, 128
    q, k, v = (_rand((B, H, S, D), s, torch.bfloat16, dev) for s in (21, 22, 23))
    o, lse = tm.attention(q, k, v, causal=causal, return_lse=True)
    rng = np.random.default_rng(0)
    heads = [(b, h, 24) for b in range(B) for h in range(H)]
    heads += [(0, 0, 128), (3, 31, 128), (2, 17, 128)]
    for b, h, nrow in heads:
        rows = np.sort(rng.choice(S, nrow, replace=False))
        rows[-1] = S - 1
        qs = q[b, h, rows].float().cpu().numpy()
        kk, vv = k[b, h].float().cpu().numpy(), v[b, h].float().cpu().numpy()
        s = (qs @ kk.T) / math.sqrt(D)
        if causal:
            s = np.where(np.arange(S)[None, :] > rows[:, None], -np.inf, s)
        mx = s.max(1, keepdims=True)
        p = np.exp(s - mx)
        ref = (p @ vv) / p.sum(1, keepdims=True)
        ref_lse = mx[:, 0] + np.log(p.sum(1))
        np.testing.assert_allclose(o[b, h, rows].float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(lse[b, h, rows].cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)


# --- the second signature: _fa_fwd_strided_kernel (tests/test_cpp_backend.py) ---
@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fa_fwd_strided_signature(dev, D, dtype):
    """The reference's N_CTX = 64 cases (test_cpp_flash_attention_head32 /
    head64: seed 42, [N_CTX, D] fp32, sm_scale 1/sqrt(D), no mask) against
    the oracle; fp32 within the reference's 5e-2 and within 1e-4."""
    N = 64
    torch.manual_seed(42)
    q, k, v = (torch.randn(N, D) for _ in range(3))
    q, k, v = (t.to(dtype).to(dev) for t in (q, k, v))
    out = torch.zeros(N, D, dtype=dtype, device=dev)
    tm.fa_fwd_strided(q, k, v, out, q.stride(0), q.stride(1), k.stride(0), k.stride(1),
                      v.stride(0), v.stride(1), out.stride(0), out.stride(1),
                      1.0 / math.sqrt(D), N, D, 32, 32)
    ref, _ = _ref(q[None, None], k[None, None], v[None, None], False)
    err = np.abs(out.float().cpu().numpy() - ref[0, 0])
    assert err.max() < 5e-2
    if dtype == torch.float32:
        assert err.max() < 1e-4
    else:
        assert np.all(err <= ATOL + RTOL * np.abs(ref[0, 0]))


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attn_fwd_strided_head_dim(dev, causal):
    """stride_qk / stride_kk / stride_vk / stride_ok other than 1 (the head
    dimension interleaved with another tensor, and a column-major output)."""
    Z, H, N, D = 2, 3, 80, 64
    qk2 = _rand((Z, H, N, D, 2), 11, torch.bfloat16, dev)   # q and k interleaved per element
    q, k = qk2[..., 0], qk2[..., 1]
    v = _rand((Z, H, N, D), 12, torch.bfloat16, dev)
    obuf = torch.zeros(Z, H, D, N, dtype=torch.bfloat16, device=dev)
    out = obuf.transpose(2, 3)  # [Z, H, N, D] with stride_ok = N
    assert q.stride(3) == 2 and out.stride(3) == N
    tm.flash_attn_fwd(q, k, v, out, *q.stride(), *k.stride(), *v.stride(), *out.stride(),
                      Z, H, N, HEAD_DIM=D, IS_CAUSAL=causal)
    ref, _ = _ref(q, k, v, causal)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
