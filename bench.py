#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X.

Headline (``value``): W4A16 GEMV, M=1, K=4096, N=14336, group 128 (BASELINE
configs[2]) in GB/s of algorithmic bytes, with every input resident in HBM and
the weight sets rotated so that the 256 MB Infinity Cache cannot serve them.
The other BASELINE configurations (W4A16 M=8/32/128, W8A16, dense 512^3,
FlashAttention fwd, KDA) are measured in the same run and reported under
``workloads``.

A "step" is one call of the hot-path op on one batch of synthetic input.
Timing: W untimed warm-up steps, then K steps bracketed by synchronisation,
timed with HIP events recorded on the stream the kernels are launched on.
The K steps are captured into one HIP graph and replayed (how a decode loop
issues them); the same K steps enqueued eagerly from Python are reported as
``eager_us_per_call``.

The CPU baseline times the reference's own CPU path for every configuration
(its test-side references restated in torch fp32, oracle/cpu_paths.py) on the
host's threads, after the GPU measurements; attention and KDA on a stated
sample of heads / steps.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME ...]
                       [--no-cpu] [--list]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "triton-metal_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "W4A16 GEMM GB/s & %HBM roofline (M=1..128); FA-fwd TFLOP/s & %MFMA peak"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_PEAK_TFLOPS = 2516.6      # MI355X dense fp16/bf16 MFMA, TFLOP/s
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA, TFLOP/s
ROTATE_BYTES = 600 << 20       # > 256 MB Infinity Cache


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# workloads: each returns dict(launches, bytes, flops, bound, config, dtype)
# ---------------------------------------------------------------------------
def _nsets(per_set_bytes):
    return max(2, min(64, -(-ROTATE_BYTES // max(1, per_set_bytes))))


def w4a16(dev, M, K=4096, N=14336, G=128):
    import torch
    import triton_metal_amd as tm
    ng = K // G
    per = N * K // 2 + 2 * N * ng * 2
    R = _nsets(per)
    g = torch.Generator(device=dev).manual_seed(2)
    Ws = [torch.randint(0, 256, (N, K // 2), device=dev, dtype=torch.uint8, generator=g)
          for _ in range(R)]
    Ss = [(torch.rand(N, ng, device=dev, generator=g) * 0.019 + 0.001).half() for _ in range(R)]
    Zs = [torch.randint(0, 16, (N, ng), device=dev, generator=g).half() for _ in range(R)]
    x = torch.randn(M, K, device=dev, generator=g).half()
    y = torch.empty(M, N, device=dev, dtype=torch.float16)
    launches = [tm.plan_int4_matmul(x, Ws[j], y, Ss[j], Zs[j], M, N, K, G) for j in range(R)]

    nbytes = N * K // 2 + 2 * N * ng + 2 * N * ng + 2 * M * K + 2 * M * N
    flops = 2 * M * N * K
    bound = "hbm" if M <= 32 else "mfma"
    return dict(launches=launches, keep=(Ws, Ss, Zs, x, y), bytes=nbytes, flops=flops,
                bound=bound, dtype="fp16",
                config={"workload": f"w4a16_m{M}", "M": M, "K": K, "N": N, "group_size": G,
                        "weight_sets_rotated": R})


def w8a16(dev, M, K=4096, N=11008):
    import torch
    import triton_metal_amd as tm
    per = N * K + 2 * N
    R = _nsets(per)
    g = torch.Generator(device=dev).manual_seed(3)
    Ws = [torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=g)
          for _ in range(R)]
    Ss = [(torch.rand(N, device=dev, generator=g) * 0.019 + 0.001).half() for _ in range(R)]
    x = torch.randn(M, K, device=dev, generator=g).half()
    y = torch.empty(M, N, device=dev, dtype=torch.float16)
    launches = [tm.plan_int8_matmul(x, Ws[j], y, Ss[j], None, M, N, K) for j in range(R)]

    nbytes = N * K + 2 * N + 2 * M * K + 2 * M * N
    flops = 2 * M * N * K
    bound = "hbm" if M <= 32 else "mfma"
    return dict(launches=launches, keep=(Ws, Ss, x, y), bytes=nbytes, flops=flops,
                bound=bound, dtype="fp16",
                config={"workload": f"w8a16_m{M}", "M": M, "K": K, "N": N,
                        "weight_sets_rotated": R})


def dense(dev, M=512, N=512, K=512):
    import torch
    import triton_metal_amd as tm
    g = torch.Generator(device=dev).manual_seed(1)
    A = torch.randn(M, K, device=dev, generator=g).half()
    B = torch.randn(K, N, device=dev, generator=g).half()
    C = torch.empty(M, N, device=dev, dtype=torch.float16)
    launches = [tm.plan_matmul(A, B, C, M, N, K)]
    return dict(launches=launches, keep=(A, B, C), bytes=2 * (M * K + K * N + M * N),
                flops=2 * M * N * K, bound="mfma", dtype="fp16", config={"workload": f"dense_{M}x{N}x{K}", "M": M, "N": N, "K": K})


def dot_general(dev, layout, dt_name, M, N, K, batch=None, epilogue="none"):
    """tm_dot (the strided tl.dot template) on layouts the dense kernels do not
    take: "colmajor_a" (A stored [K, M]), "batched" (row-major [batch, M, K] @
    [batch, K, N]) or "trans_b" with an add-matrix epilogue; "row" with the
    chain-dot epilogue: (A @ B) @ W, W [N, L = K] in the input dtype, C [M, L]
    in fp32; "row" with the softmax epilogue into C in the input dtype."""
    import torch
    import triton_metal_amd as tm
    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dt_name]
    g = torch.Generator(device=dev).manual_seed(5)
    bs = () if batch is None else (batch,)
    A = torch.randn(*bs, M, K, device=dev, generator=g).to(dt)
    B = torch.randn(*bs, K, N, device=dev, generator=g).to(dt)
    if layout == "colmajor_a":
        A = A.transpose(-1, -2).contiguous().transpose(-1, -2)
    elif layout == "trans_b":
        B = B.transpose(-1, -2).contiguous().transpose(-1, -2)
    chain = epilogue == "chain-dot"
    L = K
    C = torch.empty(*bs, M, L if chain else N, device=dev,
                    dtype=torch.float32 if chain else dt)
    Z = (torch.randn(*bs, M, N, device=dev, generator=g).to(dt)
         if epilogue not in ("none", "chain-dot") else None)
    W = torch.randn(N, L, device=dev, generator=g).to(dt) if chain else None
    launches = [tm.plan_dot(A, B, C, epilogue, z=Z, w=W)]
    nb = batch or 1
    esz = A.element_size()
    w = dict(launches=launches, keep=(A, B, C, Z, W), bytes=esz * nb * (M * K + K * N + M * N),
             flops=2 * nb * M * N * (K + L if chain else K), bound="mfma", dtype=dt_name,
             config={"workload": f"dot_{dt_name}_{layout}", "M": M, "N": N, "K": K,
                     "batch": batch, "epilogue": epilogue})
    if dt == torch.float32:
        w["peak_tflops"] = MFMA_F32_PEAK_TFLOPS
    return w


def flash(dev, causal, B=4, H=32, S=4096, D=128, const_data=False):
    """C4.  const_data: every element of q, k, v the same value (0.5), the
    same kernel and work with no bit toggling in the MFMA operands - the
    measurement that shows the clock the random data costs."""
    import torch
    import triton_metal_amd as tm
    g = torch.Generator(device=dev).manual_seed(4)
    if const_data:
        q, k, v = (torch.full((B, H, S, D), 0.5, device=dev, dtype=torch.bfloat16)
                   for _ in range(3))
    else:
        q, k, v = (torch.randn(B, H, S, D, device=dev, generator=g).bfloat16() for _ in range(3))
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=dev, dtype=torch.float32)
    launches = [tm.plan_flash_attention(q, k, v, o, lse, causal=causal)]
    flops = 4 * B * H * S * S * D // (2 if causal else 1)
    nbytes = 2 * 4 * B * H * S * D + 4 * B * H * S
    return dict(launches=launches, keep=(q, k, v, o, lse), bytes=nbytes, flops=flops,
                bound="mfma", dtype="bf16",
                config={"workload": f"flash_fwd_{'causal' if causal else 'full'}"
                        + ("_constdata" if const_data else ""), "B": B,
                        "H": H, "S": S, "D": D, "causal": causal,
                        "flops_convention": "4*B*H*S^2*D, halved when causal"})


def kda(dev, B=1, H=16, T=8192, D=128, C=64):
    import torch
    import torch.nn.functional as F
    import triton_metal_amd as tm
    # q, k, v, o bf16 + g fp32 + beta fp32 + final state fp32
    nbytes = 4 * B * T * H * D * 2 + B * T * H * D * 4 + B * T * H * 4 + B * H * D * D * 4
    R = _nsets(nbytes)  # input sets rotated past the 256 MB Infinity Cache
    g = torch.Generator(device=dev).manual_seed(5)
    ws = torch.empty(tm.kda_workspace_size(B, T, H), dtype=torch.uint8, device=dev)
    launches, keep = [], [ws]
    for _ in range(R):
        q = F.normalize(torch.randn(B, T, H, D, device=dev, generator=g).bfloat16().float(),
                        dim=-1).bfloat16()
        k = F.normalize(torch.randn(B, T, H, D, device=dev, generator=g).bfloat16().float(),
                        dim=-1).bfloat16()
        v = torch.randn(B, T, H, D, device=dev, generator=g).bfloat16()
        beta = torch.sigmoid(torch.randn(B, T, H, device=dev, generator=g))
        gl = -F.softplus(torch.randn(B, T, H, D, device=dev, generator=g))
        o = torch.empty_like(v)
        st = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
        launches.append(tm.plan_chunk_kda(q, k, v, gl, beta, o, final_state=st, workspace=ws))
        keep += [q, k, v, beta, gl, o, st]
    nc = -(-T // C)
    per_chunk = 2 * C * C * D * 3 + 2 * C * C * D * 2 + 2 * C * D * D * 3 + C ** 3 // 3
    return dict(launches=launches, keep=keep, bytes=nbytes,
                flops=per_chunk * nc * B * H, bound="hbm", dtype="bf16",
                config={"workload": "kda_chunk_fwd", "B": B, "H": H, "T": T, "Dk": D,
                        "Dv": D, "chunk": C, "input_sets_rotated": R})


def kda_decode(dev, B=16, H=16, D=128):
    """One decoding step of KDA for B sequences x H heads (the token-by-token
    form continuing from a state, updated in place); state sets rotated past
    the Infinity Cache."""
    import torch
    import torch.nn.functional as F
    import triton_metal_amd as tm
    g = torch.Generator(device=dev).manual_seed(6)
    per = 2 * B * H * D * D * 4
    R = _nsets(per)
    q = F.normalize(torch.randn(B, 1, H, D, device=dev, generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, 1, H, D, device=dev, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, 1, H, D, device=dev, generator=g).bfloat16()
    beta = torch.sigmoid(torch.randn(B, 1, H, device=dev, generator=g))
    gl = -F.softplus(torch.randn(B, 1, H, D, device=dev, generator=g))
    o = torch.empty_like(v)
    sts = [torch.randn(B, H, D, D, device=dev, generator=g) * 0.1 for _ in range(R)]
    launches = [tm.plan_fused_recurrent_kda(q, k, v, gl, beta, o, initial_state=s, final_state=s)
                for s in sts]
    # state read + written (fp32), q, k, v, o bf16, g fp32, beta fp32
    nbytes = 2 * B * H * D * D * 4 + 4 * B * H * D * 2 + B * H * D * 4 + B * H * 4
    flops = B * H * 6 * D * D
    return dict(launches=launches, keep=(q, k, v, beta, gl, o, sts), bytes=nbytes, flops=flops,
                bound="hbm", dtype="fp32",
                config={"workload": "kda_recurrent_decode", "B": B, "H": H, "T": 1, "Dk": D,
                        "Dv": D, "state_sets_rotated": R})


def decode_attn(dev, paged=False, B=8, Hq=32, Hkv=8, D=128, S=8192, page_size=16):
    """Decode attention over an fp16 KV cache (one query token per head);
    caches rotated past the Infinity Cache."""
    import torch
    import triton_metal_amd as tm
    g = torch.Generator(device=dev).manual_seed(7)
    per = 2 * B * Hkv * S * D * 2
    R = _nsets(per)
    q = torch.randn(B, Hq, D, device=dev, generator=g).half()
    o = torch.empty_like(q)
    launches, keep = [], [q, o]
    for _ in range(R):
        if paged:
            npb = S // page_size
            kc = torch.randn(B * npb, page_size, Hkv, D, device=dev, generator=g).half()
            vc = torch.randn(B * npb, page_size, Hkv, D, device=dev, generator=g).half()
            table = torch.randperm(B * npb, device=dev, generator=g).int().reshape(B, npb)
            launches.append(tm.plan_decode_attention(q, kc, vc, o, page_table=table))
            keep += [kc, vc, table]
        else:
            kc = torch.randn(B, Hkv, S, D, device=dev, generator=g).half()
            vc = torch.randn(B, Hkv, S, D, device=dev, generator=g).half()
            launches.append(tm.plan_decode_attention(q, kc, vc, o))
            keep += [kc, vc]
    nbytes = 2 * B * Hkv * S * D * 2 + 2 * B * Hq * D * 2
    flops = 4 * B * Hq * S * D
    return dict(launches=launches, keep=keep, bytes=nbytes, flops=flops, bound="hbm",
                dtype="fp16",
                config={"workload": "decode_attention_paged" if paged else "decode_attention",
                        "B": B, "q_heads": Hq, "kv_heads": Hkv, "D": D, "seq_len": S,
                        "page_size": page_size if paged else None, "cache_sets_rotated": R})


WORKLOADS = {
    "w4a16_m1": lambda d: w4a16(d, 1),
    "w4a16_m8": lambda d: w4a16(d, 8),
    "w4a16_m32": lambda d: w4a16(d, 32),
    "w4a16_m128": lambda d: w4a16(d, 128),
    "w8a16_m1": lambda d: w8a16(d, 1),
    "w8a16_m16": lambda d: w8a16(d, 16),
    "w8a16_m128": lambda d: w8a16(d, 128),
    "dense_512": lambda d: dense(d),
    "dense_4096": lambda d: dense(d, 4096, 4096, 4096),
    "flash_causal": lambda d: flash(d, True),
    "flash_full": lambda d: flash(d, False),
    "kda": lambda d: kda(d),
    "kda_decode": lambda d: kda_decode(d),
    "decode_attn": lambda d: decode_attn(d),
    "decode_attn_paged": lambda d: decode_attn(d, paged=True),
}
HEADLINE = "w4a16_m1"


def hbm_copy(dev, nbytes=512 << 20):
    """Plain device copy of a known size: the calibration kernel for the
    FETCH_SIZE / WRITE_SIZE counters (not part of the default run)."""
    import torch
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)

    def run(stream=None):
        if stream is None:
            dst.copy_(src)
        else:
            with torch.cuda.stream(torch.cuda.ExternalStream(stream)):
                dst.copy_(src)
    return dict(launches=[run], keep=(src, dst), bytes=2 * nbytes, flops=0, bound="hbm",
                dtype="bf16", config={"workload": "hbm_copy", "bytes_read": nbytes,
                                      "bytes_written": nbytes})


def w4a16_read_twin(dev, weights_only=False, K=4096, N=14336, G=128):
    """The headline GEMV's pure-read twin (wq_read_twin_r14, wq_gemvp.hip): the
    same grid of 256 workgroups x 56 rows and the same weight loads, plus the
    scale and zero-point rows (or the weights alone), reduced to nothing - the
    time that streaming the GEMV's bytes with its grid takes by itself.  Bytes:
    what it reads.  Weight sets rotated as the headline."""
    import torch
    from triton_metal_amd.driver import HipUtils
    ng = K // G
    rw = 14
    per = N * K // 2 + 2 * N * ng * 2
    R = _nsets(per)
    g = torch.Generator(device=dev).manual_seed(2)
    Ws = [torch.randint(0, 256, (N, K // 2), device=dev, dtype=torch.uint8, generator=g)
          for _ in range(R)]
    Ss = [(torch.rand(N, ng, device=dev, generator=g) * 0.019 + 0.001).half() for _ in range(R)]
    Zs = [torch.randint(0, 16, (N, ng), device=dev, generator=g).half() for _ in range(R)]
    grid = -(-N // (4 * rw))
    sink = torch.zeros(grid, device=dev, dtype=torch.int32)
    hu = HipUtils()
    name = f"wq_read_twin_{'w_' if weights_only else ''}r{rw}"
    fn = hu.builtin_function(name, dev)

    class Twin:
        def __init__(self, j):
            self.j = j

        def __call__(self, stream=None):
            hu.launch(fn, (grid,), (512,), [Ws[self.j], Ss[self.j], Zs[self.j], sink, N], 0,
                      stream)
    nbytes = N * K // 2 + (0 if weights_only else 2 * N * ng * 2)
    return dict(launches=[Twin(j) for j in range(R)], keep=(Ws, Ss, Zs, sink), bytes=nbytes,
                flops=0, bound="hbm", dtype="u8",
                config={"workload": "w4a16_m1_read_twin" + ("_w" if weights_only else ""),
                        "kernel": name, "grid": grid, "rows_per_workgroup": 4 * rw, "K": K,
                        "N": N, "weight_sets_rotated": R})


def w4a16_wide_k(dev, M, K=14336, N=4096, G=128):
    """A W4A16 shape off the bench configurations: the down projection
    (K = 14336 -> N = 4096) of the same model family, M = 1 or 16, to measure
    the kernels that shapes other than K = 4096 reach."""
    import torch
    import triton_metal_amd as tm
    w = w4a16(dev, M, K=K, N=N, G=G)
    w["config"]["workload"] = f"w4a16_m{M}_k{K}"
    d = tm.wq_kernel_for(4, M, N, K, G, zero_dtype=torch.float16, details=True)
    w["config"]["kernel"] = d["name"]
    if d["splits"] > 1:
        w["config"]["k_slices"] = d["splits"]
    return w


def w8a16_wide_k(dev, M, K=14336, N=4096):
    """The W8A16 counterpart of w4a16_wide_k (per-channel scales, no zero-points)."""
    import triton_metal_amd as tm
    w = w8a16(dev, M, K=K, N=N)
    w["config"]["workload"] = f"w8a16_m{M}_k{K}"
    d = tm.wq_kernel_for(8, M, N, K, details=True)
    w["config"]["kernel"] = d["name"]
    if d["splits"] > 1:
        w["config"]["k_slices"] = d["splits"]
    return w


# opt-in workloads (--only NAME), not part of the default run
EXTRA = {"hbm_copy": hbm_copy,
         "w4a16_m1_read_twin": lambda d: w4a16_read_twin(d),
         "w4a16_m1_read_twin_w": lambda d: w4a16_read_twin(d, weights_only=True),
         "flash_causal_constdata": lambda d: flash(d, True, const_data=True),
         "flash_full_constdata": lambda d: flash(d, False, const_data=True),
         # 256 x 256 tiles with fewer workgroups than CUs (40 and 32 tiles)
         "dense_2560x4096x4096": lambda d: dense(d, 2560, 4096, 4096),
         "dense_2048x4096x4096": lambda d: dense(d, 2048, 4096, 4096),
         "w4a16_m1_k14336": lambda d: w4a16_wide_k(d, 1),
         "w4a16_m16_k14336": lambda d: w4a16_wide_k(d, 16),
         "w4a16_m8_k14336": lambda d: w4a16_wide_k(d, 8),
         "w4a16_m4_k11008": lambda d: w4a16_wide_k(d, 4, K=11008),
         "w4a16_m32_k14336": lambda d: w4a16_wide_k(d, 32),
         "w4a16_m64_k14336": lambda d: w4a16_wide_k(d, 64),
         "w4a16_m8_k28672": lambda d: w4a16_wide_k(d, 8, K=28672, N=8192),
         # tm_dot on layouts the dense kernels do not take (dot_tile*)
         "dot_fp16_colmajor_a_4096": lambda d: dot_general(d, "colmajor_a", "fp16", 4096, 4096, 4096),
         "dot_bf16_batched_8x1024": lambda d: dot_general(d, "batched", "bf16", 1024, 1024, 1024,
                                                          batch=8),
         "dot_fp16_chain_1024": lambda d: dot_general(d, "row", "fp16", 1024, 1024, 64,
                                                      epilogue="chain-dot"),
         "dot_fp16_chain_4096x1024x128": lambda d: dot_general(d, "row", "fp16", 4096, 1024, 128,
                                                               epilogue="chain-dot"),
         "dot_fp16_softmax_4096x1024x128": lambda d: dot_general(d, "row", "fp16", 4096, 1024,
                                                                 128, epilogue="softmax"),
         "dot_fp16_addmatrix_2048": lambda d: dot_general(d, "trans_b", "fp16", 2048, 2048, 2048,
                                                          epilogue="add-matrix"),
         "dot_fp32_colmajor_a_4096": lambda d: dot_general(d, "colmajor_a", "fp32", 4096, 4096, 4096),
         # int4 K = 11008 (43 units of 256 k): the wide kernel's split form in
         # uneven slices (the tiled kernel with uint8 zero-points or bf16)
         "w4a16_m128_k11008": lambda d: w4a16_wide_k(d, 128, K=11008),
         "w4a16_m512_k11008": lambda d: w4a16_wide_k(d, 512, K=11008),
         "w8a16_m1_k14336": lambda d: w8a16_wide_k(d, 1),
         "w8a16_m16_k14336": lambda d: w8a16_wide_k(d, 16),
         # split-K plans (the Python operators pass a workspace)
         "w4a16_m128_k14336": lambda d: w4a16_wide_k(d, 128),
         "w8a16_m128_k14336": lambda d: w8a16_wide_k(d, 128),
         "w4a16_m32_k28672": lambda d: w4a16_wide_k(d, 32, K=28672, N=8192),
         "w8a16_m16_k28672": lambda d: w8a16_wide_k(d, 16, K=28672, N=8192)}


def time_workload(w, steps, warmup, graph=True, budget_s=2.0, min_replays=100):
    """ms per step.  W warm-up steps, then the K steps captured into one HIP
    graph (the launch pattern of a captured decode loop) and replayed: each
    replay is bracketed by synchronisation and timed with HIP events on the
    launch stream; the per-step time is the median over the replays (at
    least min_replays while one replay is short, fewer when replays are long,
    within about budget_s).  The same K steps enqueued eagerly from Python
    are timed once (eager_ms).  Returns (median_ms, mean_ms, eager_ms,
    replays)."""
    import statistics

    import torch
    L = w["launches"]
    R = len(L)
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        L[i % R]()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        L[(warmup + i) % R]()
    end.record(stream)
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(end) / steps
    if not graph:
        return eager_ms, eager_ms, eager_ms, 1
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=cap):
        sp = torch.cuda.current_stream().cuda_stream
        for i in range(steps):
            L[i % R](sp)
    g.replay()
    torch.cuda.synchronize()
    replays = max(3, min(min_replays, int(budget_s / max(1e-6, eager_ms * 1e-3 * steps))))
    per_step = []
    for _ in range(replays):
        torch.cuda.synchronize()
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        per_step.append(start.elapsed_time(end) / steps)
    del g
    return statistics.median(per_step), statistics.fmean(per_step), eager_ms, replays


def summarize(w, ms, mean_ms, eager_ms, replays):
    s = ms * 1e-3
    gbs = w["bytes"] / s / 1e9
    tfl = w["flops"] / s / 1e12
    if w["bound"] == "hbm":
        roof = dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(gbs / HBM_PEAK_GBS, 4))
    else:
        peak = w.get("peak_tflops", MFMA_PEAK_TFLOPS)
        roof = dict(bound="mfma", achieved=round(tfl, 2), peak=peak, unit="TFLOP/s",
                    frac=round(tfl / peak, 4))
    return dict(us_per_call=round(ms * 1e3, 3), mean_us_per_call=round(mean_ms * 1e3, 3),
                replays=replays, eager_us_per_call=round(eager_ms * 1e3, 3),
                GBps=round(gbs, 1), TFLOPs=round(tfl, 3), roofline=roof, config=w["config"])


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own CPU path for each op (its test-side
# references, restated in torch fp32 in oracle/cpu_paths.py) on the host's
# threads, outside every GPU timed region
# ---------------------------------------------------------------------------
def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, reps=3, budget_s=4.0):
    """1 warm-up, then at least `reps` timed runs (more while under budget_s);
    median wall seconds and the count."""
    import statistics
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < reps or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline():
    """Every BASELINE configuration through the reference's CPU path (torch
    fp32).  W-only matmuls are timed with and without their dequantisation;
    attention and KDA run on a stated sample of heads.  Units as the GPU
    numbers: GB/s for W-only and KDA, TFLOP/s for dense and attention."""
    import torch
    import torch.nn.functional as F

    from oracle import cpu_paths
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    out = {}

    def rec(name, secs, n, units_per_call, unit, sample):
        rate = units_per_call / secs / (1e9 if unit == "GB/s" else 1e12)
        out[name] = dict(value=round(rate, 4), unit=unit, ms=round(secs * 1e3, 2), reps=n,
                         sample=sample)

    # C1 dense 512^3, fp16 inputs
    A, Bm = torch.randn(512, 512, generator=g).half(), torch.randn(512, 512, generator=g).half()
    t, n = _median_time(lambda: cpu_paths.dense(A, Bm))
    rec("dense_512", t, n, 2 * 512 ** 3, "TFLOP/s", "full workload")
    # C3 W4A16, M in {1, 8, 32, 128}
    K, N, G = 4096, 14336, 128
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    s4 = (torch.rand(N, K // G, generator=g) * 0.019 + 0.001).half()
    z4 = torch.randint(0, 16, (N, K // G), generator=g).half()
    w4 = cpu_paths.w4a16_dequant(packed, s4, z4, K, G)
    for M in (1, 8, 32, 128):
        x = torch.randn(M, K, generator=g).half()
        nbytes = N * K // 2 + 4 * N * (K // G) + 2 * M * K + 2 * M * N
        t, n = _median_time(lambda: cpu_paths.w4a16(x, packed, s4, z4, K, G))
        rec(f"w4a16_m{M}", t, n, nbytes, "GB/s", "full workload, unpack + dequantise + matmul")
        t, n = _median_time(lambda: (x.float() @ w4.T).half())
        rec(f"w4a16_m{M}_matmul_only", t, n, nbytes, "GB/s",
            "full workload, matmul on the pre-dequantised fp32 weight")
    del w4
    # C2 W8A16, M in {1, 16, 128}
    N8 = 11008
    q8 = torch.randint(-127, 128, (N8, K), generator=g, dtype=torch.int8)
    s8 = (torch.rand(N8, generator=g) * 0.019 + 0.001).half()
    w8 = cpu_paths.w8a16_dequant(q8, s8)
    for M in (1, 16, 128):
        x = torch.randn(M, K, generator=g).half()
        nbytes = N8 * K + 2 * N8 + 2 * M * K + 2 * M * N8
        t, n = _median_time(lambda: cpu_paths.w8a16(x, q8, s8))
        rec(f"w8a16_m{M}", t, n, nbytes, "GB/s", "full workload, dequantise + matmul")
        t, n = _median_time(lambda: (x.float() @ w8.T).half())
        rec(f"w8a16_m{M}_matmul_only", t, n, nbytes, "GB/s",
            "full workload, matmul on the pre-dequantised fp32 weight")
    del w8
    # C4 attention, S=4096, D=128: 2 of the 128 (b, h) heads per variant
    S, D, nh = 4096, 128, 2
    q, k, v = (torch.randn(1, nh, S, D, generator=g).bfloat16() for _ in range(3))
    for causal in (True, False):
        t, n = _median_time(lambda: cpu_paths.ref_attention(q, k, v, causal), budget_s=6.0)
        flops = 4 * nh * S * S * D // (2 if causal else 1)
        rec(f"flash_{'causal' if causal else 'full'}", t, n, flops, "TFLOP/s",
            f"{nh} of the 128 (b, h) heads, _ref_attention in fp32 + logsumexp")
    # C5 KDA: every head of the workload, the first 1024 of its 8192 steps
    T, H = 1024, 16
    qk = [F.normalize(torch.randn(1, T, H, D, generator=g), dim=-1).bfloat16() for _ in range(2)]
    vk = torch.randn(1, T, H, D, generator=g).bfloat16()
    bk = torch.sigmoid(torch.randn(1, T, H, generator=g))
    gk = -F.softplus(torch.randn(1, T, H, D, generator=g))
    t, n = _median_time(lambda: cpu_paths.kda(qk[0], qk[1], vk, gk, bk), reps=3, budget_s=1.0)
    nbytes = 4 * T * H * D * 2 + T * H * D * 4 + T * H * 4 + H * D * D * 4
    rec("kda", t, n, nbytes, "GB/s",
        f"all 16 heads, the first {T} of the 8192 steps (per-token recurrence in fp32; the "
        f"build's restatement, the reference has none)")
    head = out["w4a16_m1"]
    return dict(value=head["value"], unit="GB/s", cores=cores, kind="port",
                sample=f"W4A16 M=1 K=4096 N=14336 G=128, full workload: the reference's CPU "
                       f"path (unpack, dequantise, x @ w^T) in torch fp32, median of "
                       f"{head['reps']} reps, {head['ms']} ms",
                threads=torch.get_num_threads(), cpu_model=_cpu_model(),
                configs={k: v for k, v in out.items() if k != "w4a16_m1"})


TRAFFIC_PROFILE = ROOT / "profiles" / "wq_gemv4p_w4a16_m1_hbm_traffic.md"


def profiled_traffic():
    """HBM bytes per launch of the headline kernel, from the calibrated
    FETCH_SIZE / WRITE_SIZE passes committed under profiles/ (None if absent)."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", nargs="*", default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--list", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="time eagerly enqueued calls only (no HIP graph)")
    args = ap.parse_args()
    if args.list:
        print("\n".join(list(WORKLOADS) + [f"{n} (opt-in)" for n in EXTRA]))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(every kernel here runs on one GPU's share of a sharded problem: W-only and "
              "dense matmuls split over N, attention over batch x heads, KDA over heads)",
              file=sys.stderr)
        return 2

    import torch
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    names = args.only or list(WORKLOADS)
    if HEADLINE not in names:
        names = [HEADLINE] + names
    results = {}
    for name in names:
        log(f"[bench] {name}: setup")
        w = (WORKLOADS.get(name) or EXTRA[name])(dev)
        ms, mean_ms, eager_ms, replays = time_workload(w, args.steps, args.warmup,
                                                       graph=not args.eager)
        results[name] = summarize(w, ms, mean_ms, eager_ms, replays)
        log(f"[bench] {name}: {results[name]['us_per_call']} us/call "
            f"{results[name]['GBps']} GB/s {results[name]['TFLOPs']} TFLOP/s")
        del w
        torch.cuda.empty_cache()
        if name == HEADLINE:
            head_ms = ms

    head = results[HEADLINE]
    line = {
        "metric": METRIC,
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "timing": "eager" if args.eager else "K steps captured in one HIP graph, each replay "
                  "synchronised and timed with HIP events; per-step time = median over the "
                  "replays; eager_us_per_call is the same loop enqueued from Python",
        "config": head["config"],
        "roofline": dict(head["roofline"], traffic=profiled_traffic()),
        "workloads": {k: v for k, v in results.items() if k != HEADLINE},
    }
    if not args.no_cpu:
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
