// Typed entry point for decode-time attention (one query token per head over
// a contiguous or paged KV cache): decode_attn_d<D>_<dt> or, for head dims
// 48 / 80 / 96 / 112, decode_attn_d<64|128>v<D>_<dt> (16-bit caches) or
// decode_attn_f32_d<D> (fp32), + decode_attn_combine when the sequence is
// split into slices, or decode_attn_general.
#include <cmath>
#include <cstdio>
#include <cstring>

#include "runtime.h"

using namespace tmhip;

namespace {

// Kernel argument block; must match struct DecodeParams in decode_attn.hip.
struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  const int* seq_lens;
  const int* page_table;
  float* ws;
  long long sB, sH, sS;
  int B, Hq, Hkv, D;
  int seq_len;
  int page_size, max_pages;
  int page_shift;
  int nsplit, split_len;
  float sl2;
  int q_dt, kv_dt, o_dt;
};

bool is16(int dt) { return dt == TM_DT_F16 || dt == TM_DT_BF16; }

// Slices of the positions for the MFMA kernel: about one resident round of
// waves (B * kv_heads * head blocks * slices ~ 768: three 48 KB rings per CU)
// with at least 256 positions per slice, a multiple of 32 (and, paged, whole
// pages, at most 64 of them).
void plan_split(int batch, int q_heads, int kv_heads, int cap, int page_size, bool paged,
                int* nsplit, int* split_len) {
  const int group = q_heads / kv_heads, hbn = (group + 15) / 16;
  const long long waves = (long long)batch * kv_heads * hbn;
  int want = (int)std::max<long long>(1, (768 + waves - 1) / waves);
  int sl = std::max(256, (cap + want - 1) / want);
  sl = (sl + 31) / 32 * 32;
  if (paged) {
    int g = 32, r = page_size;  // unit = lcm(page_size, 32)
    while (r) { const int t = g % r; g = r; r = t; }
    const int unit = page_size / g * 32;
    sl = (sl + unit - 1) / unit * unit;
    const long long maxsl = 64LL * page_size / 32 * 32;  // 64 pages, whole tiles
    if (sl > maxsl) sl = (int)(maxsl / unit * unit);
  }
  if (sl <= 0) sl = 32;
  *split_len = sl;
  *nsplit = (cap + sl - 1) / sl;
}

}  // namespace

extern "C" size_t tm_decode_attention_workspace_size(int batch, int q_heads, int kv_heads,
                                                     int head_dim, int seq_len, int page_size) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || head_dim <= 0 ||
      seq_len <= 0)
    return 0;
  int ns = 1, sl = 0;
  plan_split(batch, q_heads, kv_heads, seq_len, page_size > 0 ? page_size : 1, page_size > 0,
             &ns, &sl);
  return ns > 1 ? (size_t)batch * q_heads * ns * (head_dim + 4) * sizeof(float) : 0;
}

// Both entry points.  noalloc: the slice partials go to the device's
// tm_decode_scratch array (no workspace argument); a plan that needs more than
// it holds is rejected instead of falling back to one slice per wave.
static int decode_attention(const char* op, bool noalloc, const void* q, const void* k_cache,
                            const void* v_cache, void* o, float* lse, int batch, int q_heads,
                            int kv_heads, int head_dim, const int* seq_lens, int seq_len,
                            const long long* kv_strides, const int* page_table, int page_size,
                            int max_pages, float scale, int q_dtype, int kv_dtype, int o_dtype,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || seq_len < 0)
    return fail(TM_ERR_INVALID_ARG, "%s: batch=%d q_heads=%d kv_heads=%d head_dim=%d seq_len=%d",
                op, batch, q_heads, kv_heads, head_dim, seq_len);
  if (q_heads % kv_heads)
    return fail(TM_ERR_INVALID_ARG, "%s: q_heads=%d not a multiple of kv_heads=%d", op, q_heads,
                kv_heads);
  if (head_dim > 256) return fail(TM_ERR_UNSUPPORTED, "%s: head_dim=%d > 256", op, head_dim);
  if (!is_float(q_dtype) || !is_float(kv_dtype) || !is_float(o_dtype))
    return fail(TM_ERR_INVALID_ARG, "%s: dtypes %d %d %d", op, q_dtype, kv_dtype, o_dtype);
  if (!std::isfinite(scale)) return fail(TM_ERR_INVALID_ARG, "%s: scale", op);
  const bool paged = page_table != nullptr;
  if (paged && (page_size <= 0 || max_pages <= 0 || (long long)page_size * max_pages < seq_len))
    return fail(TM_ERR_INVALID_ARG, "%s: page_size=%d max_pages=%d for seq_len=%d", op,
                page_size, max_pages, seq_len);
  if (batch == 0) return 0;
  if (!q || !o || (seq_len > 0 && (!k_cache || !v_cache)))
    return fail(TM_ERR_INVALID_ARG, "%s: null buffer", op);
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();

  DecodeParams p;
  memset(&p, 0, sizeof p);
  p.q = q; p.k = k_cache; p.v = v_cache; p.o = o; p.lse = lse;
  p.seq_lens = seq_lens; p.page_table = page_table;
  const long long D = head_dim;
  if (kv_strides) {
    p.sB = kv_strides[0]; p.sH = kv_strides[1]; p.sS = kv_strides[2];
  } else if (paged) {  // [pages][page_size][kv_heads][D]
    p.sS = kv_heads * D; p.sH = D; p.sB = (long long)page_size * kv_heads * D;
  } else {             // [batch][kv_heads][seq_len][D]
    p.sS = D; p.sH = (long long)seq_len * D; p.sB = (long long)kv_heads * seq_len * D;
  }
  p.B = batch; p.Hq = q_heads; p.Hkv = kv_heads; p.D = head_dim;
  p.seq_len = seq_len;
  p.page_size = paged ? page_size : 1; p.max_pages = paged ? max_pages : 0;
  p.page_shift = -1;
  if (paged && (page_size & (page_size - 1)) == 0)
    for (int s = 0; s < 31; ++s)
      if ((1 << s) == page_size) p.page_shift = s;
  p.sl2 = scale * 1.4426950408889634f;
  p.q_dt = q_dtype; p.kv_dt = kv_dtype; p.o_dt = o_dtype;

  const bool rows16 = p.sB % 8 == 0 && p.sH % 8 == 0 && p.sS % 8 == 0;
  // fp32 caches with fp32 queries (the reference templates' dtype): the fp32
  // MFMA kernel, same slices, partials and combine
  const bool f32 = kv_dtype == TM_DT_F32 && q_dtype == TM_DT_F32 && head_dim % 16 == 0 &&
                   head_dim >= 32 && head_dim <= 128 && p.sB % 4 == 0 && p.sH % 4 == 0 &&
                   p.sS % 4 == 0 && aligned16(k_cache) && aligned16(v_cache) && aligned16(q) &&
                   seq_len > 0;
  // 16-bit caches: head dims 64 / 128, and 48 / 80 / 96 / 112 in the layout
  // of 64 / 128 (the kernel skips the pieces past the head dim)
  const bool inlaid = head_dim == 48 || head_dim == 80 || head_dim == 96 || head_dim == 112;
  bool mfma = f32 || (is16(kv_dtype) && (head_dim == 64 || head_dim == 128 || inlaid) &&
                      rows16 && aligned16(k_cache) && aligned16(v_cache) && seq_len > 0 &&
                      (q_dtype == kv_dtype ? aligned16(q) : true));
  if (mfma) {
    int ns = 1, sl = 0;
    plan_split(batch, q_heads, kv_heads, seq_len, p.page_size, paged, &ns, &sl);
    const size_t need = (size_t)batch * q_heads * ns * (head_dim + 4) * sizeof(float);
    if (noalloc && ns > 1) {
      static DeviceGlobal scratch("tm_decode_scratch");
      void* ptr = nullptr;
      size_t bytes = 0;
      int rc = scratch.get(&ptr, &bytes);
      if (rc) return rc;
      if (need > bytes)
        return fail(TM_ERR_INVALID_ARG,
                    "%s: this call needs %zu bytes of slice scratch, more than the %zu bytes "
                    "of the static scratch array; use tm_decode_attention with a workspace",
                    op, need, bytes);
      workspace = ptr;
      workspace_bytes = bytes;
    }
    if (ns > 1 && (!workspace || workspace_bytes < need || !aligned16(workspace))) {
      // no room for slice partials: one slice per wave (paged: only while it
      // spans at most 64 pages)
      ns = 1;
      sl = (seq_len + 31) / 32 * 32;
      if (paged && (long long)sl > 64LL * page_size) mfma = false;
    }
    if (mfma) {
      p.nsplit = ns; p.split_len = sl;
      p.ws = (float*)workspace;
      const int group = q_heads / kv_heads, hbn = (group + 15) / 16;
      // [head dim][cache dtype][query dtype other than the cache's: hi + lo split]
      static Kernel* kd[2][2][2] = {
          {{new Kernel("decode_attn_d64_f16"), new Kernel("decode_attn_d64_f16_x")},
           {new Kernel("decode_attn_d64_bf16"), new Kernel("decode_attn_d64_bf16_x")}},
          {{new Kernel("decode_attn_d128_f16"), new Kernel("decode_attn_d128_f16_x")},
           {new Kernel("decode_attn_d128_bf16"), new Kernel("decode_attn_d128_bf16_x")}}};
      // fp32: head dims 32, 48, ..., 128
      static Kernel* kf[7] = {new Kernel("decode_attn_f32_d32"), new Kernel("decode_attn_f32_d48"),
                              new Kernel("decode_attn_f32_d64"), new Kernel("decode_attn_f32_d80"),
                              new Kernel("decode_attn_f32_d96"), new Kernel("decode_attn_f32_d112"),
                              new Kernel("decode_attn_f32_d128")};
      // inlaid head dims [48, 80, 96, 112][cache dtype][split query]
      static Kernel* kv[4][2][2] = {
          {{new Kernel("decode_attn_d64v48_f16"), new Kernel("decode_attn_d64v48_f16_x")},
           {new Kernel("decode_attn_d64v48_bf16"), new Kernel("decode_attn_d64v48_bf16_x")}},
          {{new Kernel("decode_attn_d128v80_f16"), new Kernel("decode_attn_d128v80_f16_x")},
           {new Kernel("decode_attn_d128v80_bf16"), new Kernel("decode_attn_d128v80_bf16_x")}},
          {{new Kernel("decode_attn_d128v96_f16"), new Kernel("decode_attn_d128v96_f16_x")},
           {new Kernel("decode_attn_d128v96_bf16"), new Kernel("decode_attn_d128v96_bf16_x")}},
          {{new Kernel("decode_attn_d128v112_f16"), new Kernel("decode_attn_d128v112_f16_x")},
           {new Kernel("decode_attn_d128v112_bf16"), new Kernel("decode_attn_d128v112_bf16_x")}}};
      const int bf = kv_dtype == TM_DT_BF16, xq = q_dtype != kv_dtype;
      const int vi = head_dim == 48 ? 0 : head_dim == 80 ? 1 : head_dim == 96 ? 2 : 3;
      Kernel& kk = f32      ? *kf[head_dim / 16 - 2]
                   : inlaid ? *kv[vi][bf][xq]
                            : *kd[head_dim == 128][bf][xq];
      // 16-bit: a 3-slot ring of 32-position K and V tiles in the layout's
      // head dim; fp32: a 2-slot ring of 16-position tiles with rows padded by
      // 4 floats
      const unsigned layout_d = head_dim <= 64 ? 64u : 128u;
      const unsigned lds = f32 ? 2u * 2u * 16u * (unsigned)(head_dim + 4) * 4u
                               : 3u * 2u * 32u * layout_d * 2u;
      int rc = launch(kk, dim3(ns, kv_heads * hbn, batch), dim3(64), lds, stream, p);
      if (rc || ns == 1) return rc;
      static Kernel comb("decode_attn_combine");
      return launch(comb, dim3((unsigned)((long long)batch * q_heads)), dim3(64), 0, stream, p);
    }
  }
  static Kernel gen("decode_attn_general");
  p.nsplit = 1; p.split_len = seq_len;
  return launch(gen, dim3((unsigned)((long long)batch * q_heads)), dim3(256), 0, stream, p);
}

extern "C" int tm_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                                   void* o, float* lse, int batch, int q_heads, int kv_heads,
                                   int head_dim, const int* seq_lens, int seq_len,
                                   const long long* kv_strides, const int* page_table,
                                   int page_size, int max_pages, float scale, int q_dtype,
                                   int kv_dtype, int o_dtype, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  return decode_attention("tm_decode_attention", false, q, k_cache, v_cache, o, lse, batch,
                          q_heads, kv_heads, head_dim, seq_lens, seq_len, kv_strides, page_table,
                          page_size, max_pages, scale, q_dtype, kv_dtype, o_dtype, workspace,
                          workspace_bytes, stream);
}

extern "C" int tm_decode_attention_noalloc(const void* q, const void* k_cache,
                                           const void* v_cache, void* o, float* lse, int batch,
                                           int q_heads, int kv_heads, int head_dim,
                                           const int* seq_lens, int seq_len,
                                           const long long* kv_strides, const int* page_table,
                                           int page_size, int max_pages, float scale,
                                           int q_dtype, int kv_dtype, int o_dtype, void* stream) {
  return decode_attention("tm_decode_attention_noalloc", true, q, k_cache, v_cache, o, lse,
                          batch, q_heads, kv_heads, head_dim, seq_lens, seq_len, kv_strides,
                          page_table, page_size, max_pages, scale, q_dtype, kv_dtype, o_dtype,
                          nullptr, 0, stream);
}
