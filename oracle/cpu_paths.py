"""The reference's CPU path for each hot-path op, in torch fp32 -- TEST
INFRASTRUCTURE ONLY (bench.py's CPU-baseline leg times these; tests pin them
against oracle.py).  Never imported by the product path.

Each function restates the test-side CPU reference the reference's own tests
compare their kernels against, in torch fp32 on the host's threads:
  dense        tests/test_integration.py:613 (expected = a @ b), fp16 inputs
               upcast (PERFORMANCE_METRICS.md:32 times torch on the CPU)
  w8a16        tests/test_emitter.py:6117-6125 (w = q * s per output channel,
               then x @ w^T), the arithmetic of _msl_templates.py:2652-2678
  w4a16        tests/test_emitter.py:6174-6185 (unpack even-k-low nibbles,
               w = (q - z) * s per group, then x @ w^T), _msl_templates.py:
               2704-2744
  attention    _ref_attention, tests/test_flash_attention.py:107-118 (scale
               q k^T, causal mask, softmax, nan_to_num, @ v) per (b, h) head,
               plus the row logsumexp
  kda          the per-token gated delta rule (no counterpart in the
               reference; the same recurrence as oracle.kda_recurrent)
"""
from __future__ import annotations

import torch


def dense(a, b):
    return (a.float() @ b.float()).half()


def w8a16_dequant(q, s):
    return q.float() * s.float()[:, None]


def w8a16(x, q, s):
    return (x.float() @ w8a16_dequant(q, s).T).half()


def unpack_int4(packed, K):
    """[N, K/2] uint8 -> [N, K] nibbles (even k in the low nibble)."""
    p = packed.view(torch.uint8).reshape(packed.shape[0], K // 2)
    q = torch.empty(p.shape[0], K, dtype=torch.uint8)
    q[:, 0::2] = p & 0x0F
    q[:, 1::2] = p >> 4
    return q


def w4a16_dequant(packed, s, z, K, G):
    q = unpack_int4(packed, K).float()
    N = q.shape[0]
    ng = (K + G - 1) // G
    qg = q.reshape(N, ng, G)
    return ((qg - z.float()[:, :, None]) * s.float()[:, :, None]).reshape(N, K)


def w4a16(x, packed, s, z, K, G):
    return (x.float() @ w4a16_dequant(packed, s, z, K, G).T).half()


def ref_attention(q, k, v, causal):
    """One or more (b, h) heads [.., S, D]: returns (o, lse) in fp32."""
    q, k, v = q.float(), k.float(), v.float()
    scale = 1.0 / (q.shape[-1] ** 0.5)
    attn = torch.matmul(q * scale, k.transpose(-2, -1))
    if causal:
        n = attn.shape[-1]
        mask = torch.tril(torch.ones(n, n, dtype=torch.bool))
        attn = attn.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(attn, dim=-1)
    p = torch.nan_to_num(torch.softmax(attn, dim=-1), nan=0.0)
    return torch.matmul(p, v), lse


def kda(q, k, v, g, beta, scale=None):
    """Per-token recurrence over [B, T, H, D] inputs, every (b, h) head at once;
    returns (o fp32 [B, T, H, Dv], final state fp32 [B, H, Dk, Dv])."""
    q, k, v, g, beta = (t.float() for t in (q, k, v, g, beta))
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    scale = Dk ** -0.5 if scale is None else scale
    S = torch.zeros(B, H, Dk, Dv)
    o = torch.empty(B, T, H, Dv)
    for t in range(T):
        S = S * torch.exp(g[:, t])[..., None]
        kt = k[:, t]
        u = beta[:, t][..., None] * (v[:, t] - torch.einsum("bhkv,bhk->bhv", S, kt))
        S = S + kt[..., None] * u[..., None, :]
        o[:, t] = torch.einsum("bhkv,bhk->bhv", S, q[:, t] * scale)
    return o, S
