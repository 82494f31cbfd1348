/*
 * tm_hip.h -- C ABI of the MI355X (gfx950) kernel library libtm_hip.so.
 *
 * Plain C: pointers, sizes and ints only.  Every function returns 0 on
 * success; a positive value is the hipError_t that the HIP runtime returned,
 * a negative value is one of the TM_ERR_* codes below.  tm_last_error() gives
 * a thread-local message for the last failure on the calling thread.
 *
 * All typed entry points are asynchronous on `stream` (a hipStream_t passed as
 * void*, NULL = the null stream) and launch on the calling thread's current
 * HIP device.  Every buffer is allocated and owned by the caller; the library
 * owns only the code objects it loads.
 *
 * The library binds to the HIP runtime already loaded in the process (for
 * example PyTorch's), and loads the system libamdhip64 only when none is.
 */
#ifndef TM_HIP_H
#define TM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* ---- error codes --------------------------------------------------------- */
#define TM_OK 0
#define TM_ERR_INVALID_ARG (-1)   /* bad shape, dtype, pointer or size */
#define TM_ERR_UNSUPPORTED (-2)   /* valid request this build cannot serve */
#define TM_ERR_NO_RUNTIME (-3)    /* no usable HIP runtime / no GPU */
#define TM_ERR_NOT_FOUND (-4)     /* kernel name not present in a module */
#define TM_ERR_LOAD (-5)          /* code object rejected by the runtime */

/* ---- dtype codes ----------------------------------------------------------- */
#define TM_DT_NONE (-1) /* absent optional tensor (e.g. zero-points) */
#define TM_DT_F32 0
#define TM_DT_F16 1
#define TM_DT_BF16 2
#define TM_DT_U8 3
/* FP8 inputs of the dot / matmul entry points, decoded as the reference's
 * converters (triton_metal/codegen/msl_builtins.py, dtype map 264-272):
 * Triton's fp8e4nv (OCP E4M3, bias 7, 0x7F/0xFF NaN), fp8e5 (E5M2, bias 15,
 * inf and NaN), fp8e4b15, fp8e4b8 and fp8e5b16 (bias 15 / 8 / 16). */
#define TM_DT_FP8_E4M3 4
#define TM_DT_FP8_E5M2 5
#define TM_DT_FP8_E4M3B15 6
#define TM_DT_FP8_E4M3B8 7
#define TM_DT_FP8_E5M2B16 8

/* ---- dot epilogues (tm_dot) --------------------------------------------- */
#define TM_EPI_NONE 0
#define TM_EPI_ADD_MATRIX 1 /* C = A@B + Z[b, m, n]                      */
#define TM_EPI_ADD_ROWS 2   /* C = A@B + Z[b, m, 0]                      */
#define TM_EPI_ADD_COLS 3   /* C = A@B + Z[b, 0, n]                      */
#define TM_EPI_SOFTMAX 4    /* C = softmax over n of A@B                 */
#define TM_EPI_CHAIN_DOT 5  /* C = (A@B) @ W, W [N, L]                   */

/* ---- library / device ------------------------------------------------------ */
/* Resolve the HIP runtime.  Called implicitly by every entry point. */
int tm_init(void);
/* Message for the last failure on this thread ("" if none). */
const char* tm_last_error(void);
/* Library version string. */
const char* tm_version(void);
/* Device properties: gcn arch name (e.g. "gfx950:sramecc+:xnack-"), CU count,
 * max shared memory per block, L2 bytes.  Any out pointer may be NULL.
 * Replaces triton_metal/backend/device_detect.py:239 get_device_info(). */
int tm_device_info(int device, char* arch, size_t arch_len, int* cu_count,
                   int* max_shared_per_block, int* l2_bytes);
/* Number of built-in kernels and the name of kernel i (for introspection). */
int tm_num_builtin_modules(void);
const char* tm_builtin_module_name(int i);

/* ---- generic code-object loader / launcher --------------------------------
 * Replaces MetalUtils.load_binary (triton_metal/backend/driver.py:114-162),
 * which returns (library, pipeline_state, n_regs, n_spills, n_max_threads),
 * and MetalUtils.launch (driver.py:164-227).  Unlike the Metal path the launch
 * does not wait: call tm_synchronize to block. */
typedef struct tm_module_opaque* tm_module_t;
typedef struct tm_function_opaque* tm_function_t;

/* Load a gfx950 code object (hsaco bytes) on the current device. */
int tm_module_load(const void* image, size_t nbytes, tm_module_t* out);
int tm_module_unload(tm_module_t module);
/* Look up `name`; the out values mirror load_binary's n_regs, n_spills
 * (private segment bytes per lane) and n_max_threads.  NULL outs ignored. */
int tm_module_get_function(tm_module_t module, const char* name, tm_function_t* out,
                           int* n_regs, int* n_spills, int* max_threads, int* shared_bytes);
/* A kernel of the library's own embedded code objects by name, resolved on
 * the current device (loading them there on first use), for launching with
 * tm_launch: the built-in counterpart of tm_module_get_function, as
 * MetalUtils.load_binary (triton_metal/backend/driver.py:114-162) returns a
 * function from a compiled library. */
int tm_builtin_get_function(const char* name, tm_function_t* out);
/* Launch with kernel arguments as an array of pointers to each argument
 * (hipModuleLaunchKernel's kernelParams convention). */
int tm_launch(tm_function_t fn, unsigned grid_x, unsigned grid_y, unsigned grid_z,
              unsigned block_x, unsigned block_y, unsigned block_z, unsigned shared_bytes,
              void* stream, void** args);
int tm_synchronize(void* stream);

/* ---- weight-only quantized matmul --------------------------------------------
 * Buffer order follows the reference template ABI
 *   input, weight, output, scales, zeros, M, N, K
 * of make_int8_matmul_kernel (triton_metal/codegen/_msl_templates.py:2652-2661)
 * and make_int4_matmul_kernel (_msl_templates.py:2704-2713, group size a
 * template parameter there, an argument here).
 *
 *   output[m, n] = sum_k input[m, k] * (q(n, k) - zeros[g]) * scales[g]
 *
 * int8: weight int8 [N, K]; scales/zeros [N] (per output channel).
 * int4: weight bytes [N, K/2] (even k in the low nibble; equivalently uint32
 *       [N, K/8] with nibble i of word j = k 8j+i); scales/zeros
 *       [N, ceil(K/group_size)].
 * input/output: [M, K] / [M, N] row-major in act_dtype (F32, F16 or BF16).
 * scales: F32/F16/BF16.  zeros: TM_DT_NONE (zero), F32/F16/BF16 or U8.
 * Accumulation is fp32.  fp16/bf16 activations with scales in the activation
 * dtype run on MFMA kernels; other combinations on an fp32 kernel. */
int tm_int8_matmul(const void* input, const void* weight, void* output, const void* scales,
                   const void* zeros, int M, int N, int K, int act_dtype, int scale_dtype,
                   int zero_dtype, void* stream);
int tm_int4_matmul(const void* input, const void* weight, void* output, const void* scales,
                   const void* zeros, int M, int N, int K, int group_size, int act_dtype,
                   int scale_dtype, int zero_dtype, void* stream);
/* Fused linear forms of the two: output[m, n] = (the sum above) + bias[n],
 * the bias added to the fp32 sum before the output rounding, as
 * make_fused_linear_kernel (_msl_templates.py:4013-4135) adds its bias to a
 * dense product.  bias [N] in act_dtype; NULL gives the plain matmul.  The
 * reference's quantized templates have no bias; these are the nn.Linear form
 * of the same kernels. */
int tm_int8_linear(const void* input, const void* weight, const void* bias, void* output,
                   const void* scales, const void* zeros, int M, int N, int K, int act_dtype,
                   int scale_dtype, int zero_dtype, void* stream);
int tm_int4_linear(const void* input, const void* weight, const void* bias, void* output,
                   const void* scales, const void* zeros, int M, int N, int K, int group_size,
                   int act_dtype, int scale_dtype, int zero_dtype, void* stream);
/* The same four operations (qbits 4 or 8; bias NULL for the plain matmul;
 * group_size ignored for int8) with a caller-provided device workspace:
 * shapes whose kernel would leave the GPU underfilled or exceed a kernel's K
 * (long-K down projections at M >= 17, int8 K > 16384, ...) then run split-K
 * (fp32 slice sums in the workspace, then one reduction launch).  workspace:
 * 16-byte aligned, at least tm_wq_workspace_bytes(...) bytes, used only by
 * this call's launches on `stream` (overlapping calls must not share one);
 * NULL / 0 behaves as tm_int4_matmul / tm_int8_matmul / the linear forms, which
 * never split.  The Python operators (int4_matmul, ...) pass a torch-allocated
 * workspace this way.  No counterpart in the reference, whose templates run
 * one threadgroup per output tile over the whole of K. */
int tm_wq_matmul_ws(int qbits, const void* input, const void* weight, const void* bias,
                    void* output, const void* scales, const void* zeros, int M, int N, int K,
                    int group_size, int act_dtype, int scale_dtype, int zero_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);
/* Workspace bytes tm_wq_matmul_ws needs for this call on the current device
 * (0: no split-K; then any workspace, or none, will do).  The pointers are
 * only inspected for their alignment. */
size_t tm_wq_workspace_bytes(int qbits, const void* input, const void* weight,
                             const void* scales, const void* zeros, int M, int N, int K,
                             int group_size, int act_dtype, int scale_dtype, int zero_dtype);
/* Kernel selection of the entry points above, without launching: the name of
 * the gfx950 kernel a call with these sizes and dtypes would run, its grid,
 * block and dynamic LDS bytes, its k-slices (1: no split-K; the grid is then
 * (grid, splits) and wq_splitk_reduce_<act> follows) and workspace bytes,
 * for a device with cu_count CUs and max_lds bytes of dynamic LDS per
 * workgroup (MI355X: 256, 163840), with or without a workspace.  align_flags:
 * TM_WQ_ALIGN_* bits for the pointer alignments of the call.  A diagnostic with
 * no counterpart in the reference (which compiles one kernel per template); it
 * lets tests show which kernel family a shape reaches.  Touches no device.
 * Any of the output pointers may be NULL. */
#define TM_WQ_ALIGN_XW16 1u /* input and weight 16-byte aligned */
#define TM_WQ_ALIGN_S16 2u  /* scales 16-byte aligned */
#define TM_WQ_ALIGN_Z16 4u  /* zeros 16-byte aligned (or no zeros) */
#define TM_WQ_ALIGN_SZ4 8u  /* scales and zeros 4-byte aligned */
int tm_wq_plan(int qbits, int M, int N, int K, int group_size, int act_dtype, int scale_dtype,
               int zero_dtype, unsigned align_flags, int cu_count, size_t max_lds,
               int with_workspace, char* name, size_t name_len, unsigned* grid, unsigned* block,
               unsigned* lds_bytes, unsigned* splits, size_t* workspace_bytes);
/* Dequantised weight tile out[n, k] = round_out((float(q) - z) * s), the
 * per-element arithmetic of _msl_templates.py:2671 (int8) / 2738-2739 (int4).
 * qbits 4 or 8; out_dtype F32/F16/BF16. */
int tm_wq_dequant(const void* weight, const void* scales, const void* zeros, void* out, int N,
                  int K, int group_size, int qbits, int scale_dtype, int zero_dtype,
                  int out_dtype, void* stream);

/* int4 checkpoints in the GPTQ and AWQ on-disk formats -> the int4 layout of
 * tm_int4_matmul (weight [N, K/2] bytes, even k in the low nibble, as
 * make_int4_matmul_kernel's layout, _msl_templates.py:2687-2697; scales /
 * zeros [N, ceil(K/group_size)]).  No counterpart in the reference, which
 * takes that layout as given; these load real checkpoints into it.
 *   GPTQ: qweight int32 [K/8, N] (nibble i of word (j, n) = q[n, 8j+i]);
 *         qzeros int32 [ngroups, N/8] (nibble i of word (g, b) =
 *         z[8b+i, g] - zero_offset: 1 for the original format, 0 for v2).
 *   AWQ:  qweight int32 [K, N/8] (nibble p of word (k, b) = q[8b + ORDER[p],
 *         k], ORDER = 0 2 4 6 1 3 5 7); qzeros [ngroups, N/8] the same way.
 *   scales: 16-bit [ngroups, N] (fp16 as stored) -> [N, ngroups].
 * weight_out: N*K/2 bytes; zeros_out: uint8 [N, ngroups]; scales_out: 16-bit
 * [N, ngroups].  qzeros / scales may be NULL together with their output.
 * N and K multiples of 8; act-order (g_idx) checkpoints are not representable
 * in this layout and are rejected by the Python layer. */
int tm_wq_repack_gptq(const void* qweight, const void* qzeros, const void* scales, int N, int K,
                      int group_size, int zero_offset, void* weight_out, void* scales_out,
                      void* zeros_out, void* stream);
int tm_wq_repack_awq(const void* qweight, const void* qzeros, const void* scales, int N, int K,
                     int group_size, void* weight_out, void* scales_out, void* zeros_out,
                     void* stream);

/* ---- dense matmul -----------------------------------------------------------
 * C[M, N] = A[M, K] @ B[K, N], row-major with leading dimensions lda/ldb/ldc
 * (elements).  Replaces make_matmul_kernel (_msl_templates.py:447-585; buffer
 * order A, B, C, M, N, K) and make_simdgroup_matmul_kernel (3501-3667; fp16
 * in, fp32 out).  in_dtype F16/BF16 (MFMA), an FP8 code (MFMA on the exact
 * fp16 values; the reference's FP8 matmul writes fp32, _msl_templates.py:
 * 475-476) or F32; out_dtype F32/F16/BF16. */
int tm_matmul(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb,
              int ldc, int in_dtype, int out_dtype, void* stream);
/* Dense matmul with its sizes in device memory: C[M, N] = A[M, K] @ B[K, N],
 * row-major with leading dimensions K, N, N; M, N, K are one uint32 each on
 * the device, the buffer(3..5) arguments of make_matmul_2d_kernel
 * (_msl_templates.py:588-679) and make_matmul_swizzled_kernel (682-781).
 * max_m / max_n: the host-known capacity the launch covers; M and N read on
 * the device are clamped to it (rows / columns beyond are not written), so a
 * captured launch serves any M <= max_m, N <= max_n.  a_elems / b_elems /
 * c_elems: the element counts of A, B and C; sizes on the device whose M K,
 * K N or M N exceed them make the launch do nothing (the reference trusts the
 * buffers; here nothing past them is read or written).  in_dtype F32, F16 or
 * BF16; out_dtype in_dtype or F32; fp32 accumulation.  tm_matmul_2d walks the
 * output tiles on a 2-D grid; tm_matmul_swizzled in runs of group_size tile
 * rows (64-row tiles), column by column within a run. */
int tm_matmul_2d(const void* A, const void* B, void* C, const unsigned* M, const unsigned* N,
                 const unsigned* K, int max_m, int max_n, size_t a_elems, size_t b_elems,
                 size_t c_elems, int in_dtype, int out_dtype, void* stream);
int tm_matmul_swizzled(const void* A, const void* B, void* C, const unsigned* M,
                       const unsigned* N, const unsigned* K, int max_m, int max_n,
                       size_t a_elems, size_t b_elems, size_t c_elems, int group_size,
                       int in_dtype, int out_dtype, void* stream);
/* tl.dot in general form: the strided dot template of the reference,
 * _lower_dot_via_prebuilt_template (triton_metal/codegen/_lowerer_templates.py:
 * 1116-1540), with the epilogue detection of _detect_dot_epilogue
 * (_lowerer_detection.py:763-805).  For b < batch, m < M, n < N:
 *   P[b, m, n] = sum_k A[b, m, k] * B[b, k, n]      (fp32 accumulation)
 *   C[b, m, n] = P + Z[b, m, n] | P + Z[b, m, 0] | P + Z[b, 0, n]
 *                | exp(P - max_n P) / sum_n exp(P - max_n P)
 *   C[b, m, l] = sum_n P[b, m, n] * W[n, l]         (chain-dot, l < L)
 * Every operand is addressed by element strides, so transposed and
 * column-major views need no copy:
 *   strides[14] = {A: batch, m, k;  B: batch, k, n;  C: batch, m, n (l);
 *                  Z: batch, m, n;  W: n, l}   (non-negative).
 * in_dtype F16 / BF16 / FP8 (MFMA; FP8 decoded exactly to fp16) or F32
 * (fp32 FMA); out_dtype F32 / F16 / BF16 (the reference writes FP8 products
 * as fp32).  z_dtype / w_dtype: the dtypes of Z / W (any input dtype), or
 * TM_DT_NONE when unused.  Z may be C itself (the reference reads the bias
 * from the output buffer): add-matrix and add-rows are defined in place;
 * add-cols in place only for batch * M == 1.  Softmax and chain-dot keep a
 * product row on chip: N <= 8192. */
int tm_dot(const void* A, const void* B, void* C, const void* Z, const void* W, int batch, int M,
           int N, int K, int L, const long long* strides, int epilogue, int in_dtype,
           int out_dtype, int z_dtype, int w_dtype, void* stream);
/* output[M, N] = input[M, K] @ weight[N, K]^T (+ bias[N]); bias may be NULL.
 * Replaces make_fused_linear_kernel (_msl_templates.py:4013-4135; buffer order
 * input, weight, C, [bias], M, N, K). */
int tm_linear(const void* input, const void* weight, const void* bias, void* output, int M,
              int N, int K, int in_dtype, int out_dtype, void* stream);
/* The kernel a tm_matmul (trans_b = 0: B [K, N]) or tm_linear (trans_b = 1:
 * weight [N, K], has_bias) call of these sizes, leading dimensions, dtypes and
 * pointer alignment runs, with its grid and block: the selection those entry
 * points make, as a pure function (no device is touched).  No counterpart in
 * the reference, whose callers pick a template; for tests and callers that
 * want to know the path.  FP8 inputs (the general dot) give
 * TM_ERR_UNSUPPORTED.  16-bit shapes the dense tile kernels do not take (K
 * or a leading dimension not a multiple of 8, unaligned A / B) run tm_dot's
 * tile kernels: name "tm_dot", grid and block 0 (tm_dot picks them).
 * tm_linear's leading dimensions are K, K, N. */
#define TM_GEMM_ALIGN_AB16 1u /* A and B 16-byte aligned */
#define TM_GEMM_ALIGN_C16 2u  /* C 16-byte aligned */
#define TM_GEMM_ALIGN_ALL 3u
int tm_gemm_plan(int M, int N, int K, int lda, int ldb, int ldc, int trans_b, int has_bias,
                 int in_dtype, int out_dtype, unsigned align_flags, char* name, size_t name_len,
                 unsigned* grid, unsigned* block);

/* ---- flash attention forward -------------------------------------------------
 * O = softmax(scale * Q K^T [+ causal mask]) V per (batch, head), fp32 softmax
 * and accumulation; lse (may be NULL) receives the natural-log logsumexp of
 * each row as fp32 [batch, heads, seq_len].
 * q, k, v, o: [batch, heads, seq_len, head_dim] with element strides
 * strides[12] = {q_b, q_h, q_s, k_b, k_h, k_s, v_b, v_h, v_s, o_b, o_h, o_s}
 * (NULL = contiguous); the head dimension must be contiguous.
 * Masking follows make_flash_attention_kernel (_msl_templates.py:1610-1619):
 * key j is excluded when j >= seq_len or (causal) j > i; a row with no key
 * gives O = 0 and lse = -inf (1747-1754).  Replaces the template's buffer ABI
 * Q, K, V, O, seq_len, scale (1624-1634) and the @triton.jit _flash_attn_fwd
 * signature (tests/test_flash_attention.py:24-33).
 * dtype F16/BF16 (MFMA kernel for head_dim 32, 48, 64, 80, 96, 112, 128) or
 * F32 (MFMA kernel for head_dim a multiple of 16 from 32 to 128); other head
 * dims (<= 128) and strides on a one-thread-per-row kernel. */
int tm_flash_attention(const void* q, const void* k, const void* v, void* o, float* lse,
                       int batch, int heads, int seq_len, int head_dim,
                       const long long* strides, float scale, int causal, int dtype,
                       void* stream);

/* ---- decode attention ---------------------------------------------------------
 * One query token per (batch, query head) over a KV cache:
 *   o[b, h] = softmax_p(scale * q[b, h] . K[b, h / (q_heads / kv_heads), p]) V[...]
 * over positions p < len(b), fp32 softmax; lse (may be NULL) receives the
 * natural-log logsumexp [batch, q_heads].  A batch entry with no position
 * gives o = 0, lse = -inf.  Replaces the reference's decode templates
 * (_msl_templates.py): make_kv_cache_attention_kernel (1949-2048),
 * make_gqa_attention_kernel (2049-2160), make_batched_kv_decode_kernel
 * (2161-2278), make_paged_attention_kernel (2279-2404),
 * make_multi_head_paged_attention_kernel (2405-2532) and
 * make_fp16_kv_attention_kernel (2533-2629).
 * q, o: [batch, q_heads, head_dim] in q_dtype / o_dtype; the cache in
 * kv_dtype, head dim contiguous; kv_strides = {batch (paged: page), kv head,
 * position (paged: slot)} in elements, NULL for
 *   contiguous [batch][kv_heads][seq_len][head_dim], or
 *   paged      [pages][page_size][kv_heads][head_dim].
 * seq_lens: int32 [batch] on the device (clamped to seq_len) or NULL (every
 * batch entry has seq_len positions); seq_len bounds the positions.
 * page_table: int32 [batch, max_pages] on the device, or NULL (contiguous);
 * position p sits in page page_table[b][p / page_size], slot p % page_size.
 * workspace: scratch for per-slice partials of long sequences, at least
 * tm_decode_attention_workspace_size(...) bytes (NULL or smaller: no slices).
 * fp16 / bf16 caches with head_dim 48, 64, 80, 96, 112 or 128, and fp32 caches
 * with fp32 queries and head_dim a multiple of 16 from 32 to 128, run on MFMA
 * kernels; everything else (head_dim <= 256) on an fp32 kernel.  With a query dtype other than
 * the cache's (an fp32 query over a 16-bit cache, as
 * make_fp16_kv_attention_kernel, _msl_templates.py:2558-2576, computes it) the
 * MFMA kernels carry the query and the softmax weights as hi + lo pairs of
 * cache-dtype operands, keeping fp32-level accuracy.  Over an fp16 cache the
 * pair spans |q| <= 131008 (hi saturates at 65504 and lo carries the rest);
 * query elements beyond that saturate at +-131008. */
size_t tm_decode_attention_workspace_size(int batch, int q_heads, int kv_heads, int head_dim,
                                          int seq_len, int page_size);
int tm_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* o,
                        float* lse, int batch, int q_heads, int kv_heads, int head_dim,
                        const int* seq_lens, int seq_len, const long long* kv_strides,
                        const int* page_table, int page_size, int max_pages, float scale,
                        int q_dtype, int kv_dtype, int o_dtype, void* workspace,
                        size_t workspace_bytes, void* stream);

/* tm_decode_attention without the workspace arguments, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  It has no counterpart in the
 * reference.  It allocates nothing: the per-slice partials go to a static
 * device array of TM_DECODE_SCRATCH_BYTES, one per device, held from the
 * library's first use on that device until the process ends.  A call whose
 * slice plan needs more (tm_decode_attention_workspace_size(...) bytes) fails
 * with TM_ERR_INVALID_ARG before launching anything.  Every call on a device
 * shares that device's array: calls that overlap on one device (other
 * streams, other threads) race and must be serialised by the caller.  Nothing
 * in the array needs clearing between calls; each call writes every partial
 * it reads. */
#define TM_DECODE_SCRATCH_BYTES (8u << 20)
int tm_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache, void* o,
                                float* lse, int batch, int q_heads, int kv_heads, int head_dim,
                                const int* seq_lens, int seq_len, const long long* kv_strides,
                                const int* page_table, int page_size, int max_pages, float scale,
                                int q_dtype, int kv_dtype, int o_dtype, void* stream);

/* ---- KDA chunked forward -----------------------------------------------------
 * No counterpart in the reference (it has no linear attention): the gated
 * delta rule of Kimi Delta Attention in the [B, T, H, D] layout of its chunked
 * operator.  Per (batch, head), with S in R^{key_dim x value_dim}:
 *   S <- diag(exp(g_t)) S;  S <- S + beta_t k_t (v_t - S^T k_t)^T;
 *   o_t = S^T (scale q_t).
 * q, k: bf16 [batch, seq_len, heads, key_dim]; v, o: bf16 [.., value_dim];
 * g: fp32 [batch, seq_len, heads, key_dim] (log decay, finite);
 * beta: [batch, seq_len, heads], beta_dtype F32 or BF16;
 * initial_state, final_state: fp32 [batch, heads, key_dim, value_dim], either
 * may be NULL (zero initial state / final state not returned).
 * key_dim = value_dim = 128 and chunk_size = 64 (else TM_ERR_UNSUPPORTED).
 * workspace: 16-byte aligned device memory of at least
 * tm_kda_workspace_size(...) bytes; its contents are scratch. */
size_t tm_kda_workspace_size(int batch, int seq_len, int heads, int key_dim, int value_dim,
                             int chunk_size);
int tm_kda_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                     const void* beta, const float* initial_state, void* o, float* final_state,
                     int batch, int seq_len, int heads, int key_dim, int value_dim,
                     int chunk_size, float scale, int beta_dtype, void* workspace,
                     size_t workspace_bytes, void* stream);
/* The same rule token by token (the recurrent form; no counterpart in the
 * reference either): for decoding one or a few tokens that continue from a
 * state, e.g. the final_state of tm_kda_chunk_fwd.  Arguments as
 * tm_kda_chunk_fwd without chunk size and workspace; the state lives in
 * registers across the seq_len steps.  initial_state and final_state may be
 * the same buffer (an in-place update).  key_dim = value_dim = 128. */
int tm_kda_recurrent_fwd(const void* q, const void* k, const void* v, const float* g,
                         const void* beta, const float* initial_state, void* o,
                         float* final_state, int batch, int seq_len, int heads, int key_dim,
                         int value_dim, float scale, int beta_dtype, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif
#endif /* TM_HIP_H */
