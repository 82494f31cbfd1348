"""The torch fp32 CPU paths timed as bench.py's CPU baseline agree with the
oracle (CPU only)."""
import numpy as np
import torch
import torch.nn.functional as F

import oracle
from oracle import cpu_paths


def test_dense_and_wonly_paths():
    g = torch.Generator().manual_seed(0)
    a, b = torch.randn(33, 64, generator=g).half(), torch.randn(64, 40, generator=g).half()
    np.testing.assert_allclose(cpu_paths.dense(a, b).float().numpy(),
                               oracle.matmul(a.float().numpy(), b.float().numpy()),
                               atol=2e-2, rtol=1e-2)
    N, K, G = 24, 256, 128
    x = torch.randn(3, K, generator=g).half()
    q8 = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s8 = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
    np.testing.assert_allclose(
        cpu_paths.w8a16(x, q8, s8).float().numpy(),
        oracle.int8_matmul(x.float().numpy(), q8.numpy(), s8.float().numpy(), None, 3, N, K),
        atol=2e-2, rtol=1e-2)
    q4 = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_int4(q4.numpy()))
    s4 = (torch.rand(N, K // G, generator=g) * 0.019 + 0.001).half()
    z4 = torch.randint(0, 16, (N, K // G), generator=g).half()
    np.testing.assert_array_equal(cpu_paths.unpack_int4(packed, K).numpy(), q4.numpy())
    np.testing.assert_allclose(
        cpu_paths.w4a16(x, packed, s4, z4, K, G).float().numpy(),
        oracle.int4_matmul(x.float().numpy(), packed.numpy(), s4.float().numpy(),
                           z4.float().numpy(), 3, N, K, G), atol=2e-2, rtol=1e-2)


def test_attention_path():
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(2, 50, 16, generator=g) for _ in range(3))
    for causal in (False, True):
        o, lse = cpu_paths.ref_attention(q, k, v, causal)
        ro, rl = oracle.flash_attention(q.numpy()[None], k.numpy()[None], v.numpy()[None],
                                        16 ** -0.5, causal)
        np.testing.assert_allclose(o.numpy(), ro[0], atol=1e-5, rtol=1e-5)
        np.testing.assert_allclose(lse.numpy(), rl[0], atol=1e-5, rtol=1e-5)


def test_kda_path():
    g = torch.Generator().manual_seed(2)
    B, T, H = 1, 40, 2
    q = F.normalize(torch.randn(B, T, H, 128, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, 128, generator=g), dim=-1)
    v = torch.randn(B, T, H, 128, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gl = -F.softplus(torch.randn(B, T, H, 128, generator=g))
    o, S = cpu_paths.kda(q, k, v, gl, beta)
    ro, rS = oracle.kda_recurrent(*(t.numpy() for t in (q, k, v, gl, beta)))
    np.testing.assert_allclose(o.numpy(), ro, atol=1e-5, rtol=1e-4)
    np.testing.assert_allclose(S.numpy(), rS, atol=1e-5, rtol=1e-4)
