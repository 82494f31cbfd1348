// Typed entry point for FlashAttention forward.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>

#include "runtime.h"

using namespace tmhip;

namespace {

// Kernel argument block; must match struct FlashParams in kernels/flash_params.h.
struct FlashParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  long long sqb, sqh, sqs;
  long long skb, skh, sks;
  long long svb, svh, svs;
  long long sob, soh, sos;
  int B, H, S, D;
  float sl2;
  int causal;
  int dtype;
};

Kernel& flash_kernel(const char* name) {
  static std::mutex mu;
  static std::map<std::string, Kernel*> table;
  std::lock_guard<std::mutex> lk(mu);
  auto it = table.find(name);
  if (it != table.end()) return *it->second;
  Kernel* k = new Kernel(strdup(name));
  table[name] = k;
  return *k;
}

}  // namespace

extern "C" int tm_flash_attention(const void* q, const void* k, const void* v, void* o,
                                  float* lse, int batch, int heads, int seq_len, int head_dim,
                                  const long long* strides, float scale, int causal, int dtype,
                                  void* stream) {
  if (batch < 0 || heads < 0 || seq_len < 0 || head_dim <= 0)
    return fail(TM_ERR_INVALID_ARG, "tm_flash_attention: B=%d H=%d S=%d D=%d", batch, heads,
                seq_len, head_dim);
  if (batch == 0 || heads == 0 || seq_len == 0) return 0;
  if (!q || !k || !v || !o) return fail(TM_ERR_INVALID_ARG, "tm_flash_attention: null buffer");
  if (!is_float(dtype)) return fail(TM_ERR_INVALID_ARG, "tm_flash_attention: dtype %d", dtype);
  if (head_dim > 128)
    return fail(TM_ERR_UNSUPPORTED, "tm_flash_attention: head_dim %d > 128", head_dim);
  if (!std::isfinite(scale)) return fail(TM_ERR_INVALID_ARG, "tm_flash_attention: scale");
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  FlashParams p;
  memset(&p, 0, sizeof p);
  p.q = q; p.k = k; p.v = v; p.o = o; p.lse = lse;
  const long long sd = head_dim, ss = (long long)seq_len * head_dim,
                  sh = (long long)heads * seq_len * head_dim;
  long long st[12] = {sh, ss, sd, sh, ss, sd, sh, ss, sd, sh, ss, sd};
  if (strides) memcpy(st, strides, sizeof st);
  p.sqb = st[0]; p.sqh = st[1]; p.sqs = st[2];
  p.skb = st[3]; p.skh = st[4]; p.sks = st[5];
  p.svb = st[6]; p.svh = st[7]; p.svs = st[8];
  p.sob = st[9]; p.soh = st[10]; p.sos = st[11];
  p.B = batch; p.H = heads; p.S = seq_len; p.D = head_dim;
  p.sl2 = scale * 1.4426950408889634f;
  p.causal = causal ? 1 : 0;
  p.dtype = dtype;

  // the MFMA kernel keeps per-lane source offsets of a 64-key block in 32 bits
  const bool small_rows = 64LL * std::max(std::llabs(st[5]), std::llabs(st[8])) < (1LL << 31);
  bool st8 = small_rows;
  for (int i = 0; i < 12; ++i) st8 &= (st[i] % 8) == 0;
  // head dims 32 / 64 / 128, and 48 / 80 / 96 / 112 in the layout of 64 / 128
  const bool exact = head_dim == 32 || head_dim == 64 || head_dim == 128;
  const bool inlaid = head_dim == 48 || head_dim == 80 || head_dim == 96 || head_dim == 112;
  const bool mfma = is_half(dtype) && (exact || inlaid) && st8 && aligned16(q) && aligned16(k) &&
                    aligned16(v) && aligned16(o);
  if (mfma) {
    char name[64];
    if (exact)
      snprintf(name, sizeof name, "flash_fwd_d%d_%s_%s", head_dim,
               dtype == TM_DT_BF16 ? "bf16" : "f16", causal ? "causal" : "full");
    else
      snprintf(name, sizeof name, "flash_fwd_d%dv%d_%s_%s", head_dim <= 64 ? 64 : 128, head_dim,
               dtype == TM_DT_BF16 ? "bf16" : "f16", causal ? "causal" : "full");
    // causal: one workgroup per pair of query blocks (i, nqb - 1 - i)
    const long long nqb = (seq_len + 127) / 128;
    const long long grid = (causal ? (nqb + 1) / 2 : nqb) * (long long)batch * heads;
    if (grid > 0x7fffffffLL) return fail(TM_ERR_UNSUPPORTED, "tm_flash_attention: grid");
    return launch(flash_kernel(name), dim3((unsigned)grid), dim3(256), 0, stream, p);
  }
  // fp32 (the reference template's dtype): the fp32-MFMA kernel for head dims
  // 32, 48, ..., 128 with 16-byte aligned rows
  bool st4 = true;
  for (int i = 0; i < 12; ++i) st4 &= (st[i] % 4) == 0;
  if (dtype == TM_DT_F32 && head_dim % 16 == 0 && head_dim >= 32 && head_dim <= 128 && st4 &&
      aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o)) {
    char name[64];
    snprintf(name, sizeof name, "flash_fwd_f32_d%d_%s", head_dim, causal ? "causal" : "full");
    const long long grid = (long long)((seq_len + 63) / 64) * batch * heads;
    if (grid > 0x7fffffffLL) return fail(TM_ERR_UNSUPPORTED, "tm_flash_attention: grid");
    const unsigned lds = 2u * 2u * 32u * (unsigned)(head_dim + 4) * 4u;
    return launch(flash_kernel(name), dim3((unsigned)grid), dim3(256), lds, stream, p);
  }
  const char* gname = head_dim <= 32 ? "flash_fwd_general_d32"
                      : head_dim <= 64 ? "flash_fwd_general_d64" : "flash_fwd_general_d128";
  if ((long long)batch * heads > 65535)
    return fail(TM_ERR_UNSUPPORTED, "tm_flash_attention: batch*heads > 65535 (general kernel)");
  return launch(flash_kernel(gname), dim3((seq_len + 63) / 64, batch * heads), dim3(64), 0,
                stream, p);
}
