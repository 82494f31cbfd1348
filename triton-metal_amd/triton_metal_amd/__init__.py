"""MI355X (gfx950) native kernels for triton-metal's hot path.

Dense fp16/bf16/FP8 matmul and tl.dot in general form (strides, batches,
epilogues), W8A16 and W4A16 weight-only
matmul, FlashAttention forward and KDA chunked forward, as hand-written HIP
kernels behind the C ABI of libtm_hip.so (include/tm_hip.h).
"""
from . import errors
from .errors import HipLaunchError, KernelLoadError, NativeLibraryMissing, NoDeviceError
from .ops import (
    Kernel,
    Launch,
    attention,
    decode_attention,
    dot,
    plan_dot,
    DOT_EPILOGUES,
    plan_decode_attention,
    kv_cache_attention,
    gqa_attention,
    batched_kv_decode,
    paged_attention,
    multi_head_paged_attention,
    fp16_kv_attention,
    make_kv_cache_attention_kernel,
    make_gqa_attention_kernel,
    make_batched_kv_decode_kernel,
    make_paged_attention_kernel,
    make_multi_head_paged_attention_kernel,
    make_fp16_kv_attention_kernel,
    chunk_kda,
    fused_recurrent_kda,
    kda_workspace_size,
    plan_chunk_kda,
    plan_fused_recurrent_kda,
    flash_attention,
    flash_attn_fwd,
    make_flash_attention_kernel,
    plan_flash_attention,
    plan_int4_linear,
    plan_int4_matmul,
    plan_int8_linear,
    plan_int8_matmul,
    plan_matmul,
    from_awq,
    from_gptq,
    fused_linear,
    int4_linear,
    int4_matmul,
    int8_linear,
    int8_matmul,
    make_fused_linear_kernel,
    make_int4_matmul_kernel,
    make_int8_matmul_kernel,
    make_matmul_kernel,
    make_simdgroup_matmul_kernel,
    matmul,
    wq_dequant,
)

__all__ = [
    "errors", "HipLaunchError", "KernelLoadError", "NativeLibraryMissing", "NoDeviceError",
    "Kernel", "Launch", "attention", "decode_attention", "dot", "plan_dot", "DOT_EPILOGUES", "plan_decode_attention", "kv_cache_attention", "gqa_attention", "batched_kv_decode", "paged_attention", "multi_head_paged_attention", "fp16_kv_attention", "make_kv_cache_attention_kernel", "make_gqa_attention_kernel", "make_batched_kv_decode_kernel", "make_paged_attention_kernel", "make_multi_head_paged_attention_kernel", "make_fp16_kv_attention_kernel", "chunk_kda", "fused_recurrent_kda", "kda_workspace_size", "plan_chunk_kda", "plan_fused_recurrent_kda", "flash_attention", "flash_attn_fwd",
    "make_flash_attention_kernel", "plan_flash_attention", "plan_int4_linear", "plan_int4_matmul", "plan_int8_linear", "plan_int8_matmul", "plan_matmul", "from_awq", "from_gptq", "fused_linear", "int4_linear", "int4_matmul", "int8_linear", "int8_matmul", "make_fused_linear_kernel",
    "make_int4_matmul_kernel", "make_int8_matmul_kernel", "make_matmul_kernel",
    "make_simdgroup_matmul_kernel", "matmul", "wq_dequant",
]
