// Typed entry points for KDA: the chunked forward (kda_intra + kda_state) and
// the token-by-token recurrent form (kda_recurrent).
#include <algorithm>
#include <cmath>
#include <cstring>

#include "runtime.h"

using namespace tmhip;

namespace {

constexpr int kChunk = 64, kKeyDim = 128, kValueDim = 128;
constexpr size_t kChunkBytes = 74240;  // workspace bytes per (head, chunk)

// Kernel argument block; must match struct KdaParams in kda.hip.
struct KdaParams {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const void* beta;
  const float* s0;
  void* o;
  float* st;
  void* ws;
  int B, T, H, NC;
  int c0, c1;
  float scale;
  int beta_bf16;
};

Kernel& intra_kernel() {
  static Kernel k("kda_intra");
  return k;
}
Kernel& state_kernel() {
  static Kernel k("kda_state");
  return k;
}
Kernel& recurrent_kernel() {
  static Kernel k("kda_recurrent");
  return k;
}
Kernel& recurrent_v4_kernel() {
  static Kernel k("kda_recurrent_v4");
  return k;
}

}  // namespace

extern "C" size_t tm_kda_workspace_size(int batch, int seq_len, int heads, int key_dim,
                                        int value_dim, int chunk_size) {
  if (batch < 0 || seq_len < 0 || heads < 0 || key_dim != kKeyDim || value_dim != kValueDim ||
      chunk_size != kChunk)
    return 0;
  const size_t nc = ((size_t)seq_len + kChunk - 1) / kChunk;
  return (size_t)batch * heads * nc * kChunkBytes;
}

extern "C" int tm_kda_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                                const void* beta, const float* initial_state, void* o,
                                float* final_state, int batch, int seq_len, int heads,
                                int key_dim, int value_dim, int chunk_size, float scale,
                                int beta_dtype, void* workspace, size_t workspace_bytes,
                                void* stream) {
  if (batch < 0 || seq_len < 0 || heads < 0 || key_dim <= 0 || value_dim <= 0 || chunk_size <= 0)
    return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: B=%d T=%d H=%d Dk=%d Dv=%d chunk=%d",
                batch, seq_len, heads, key_dim, value_dim, chunk_size);
  if (key_dim != kKeyDim || value_dim != kValueDim || chunk_size != kChunk)
    return fail(TM_ERR_UNSUPPORTED,
                "tm_kda_chunk_fwd: key_dim=%d value_dim=%d chunk_size=%d (supported: 128, 128, 64)",
                key_dim, value_dim, chunk_size);
  if (beta_dtype != TM_DT_F32 && beta_dtype != TM_DT_BF16)
    return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: beta_dtype %d", beta_dtype);
  if (!std::isfinite(scale)) return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: scale");
  if (batch == 0 || heads == 0) return 0;
  if (seq_len > 0 && (!q || !k || !v || !g || !beta || !o))
    return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: null buffer");
  const size_t need = tm_kda_workspace_size(batch, seq_len, heads, key_dim, value_dim, chunk_size);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: workspace of %zu bytes, need %zu",
                workspace_bytes, need);
  if (seq_len == 0 && !final_state) return 0;
  for (const void* ptr : {q, k, v, (const void*)g, (const void*)o, (const void*)workspace})
    if (ptr && !aligned16(ptr))
      return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: buffers must be 16-byte aligned");
  if ((initial_state && !aligned16(initial_state)) || (final_state && !aligned16(final_state)))
    return fail(TM_ERR_INVALID_ARG, "tm_kda_chunk_fwd: state buffers must be 16-byte aligned");
  const long long nc = ((long long)seq_len + kChunk - 1) / kChunk;
  const long long bh = (long long)batch * heads;
  if (bh * nc > 0x7fffffffLL || (long long)batch * seq_len * heads > 0x7fffffffLL)
    return fail(TM_ERR_UNSUPPORTED, "tm_kda_chunk_fwd: problem too large for 32-bit indexing");
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();

  KdaParams p;
  memset(&p, 0, sizeof p);
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta;
  p.s0 = initial_state; p.o = o; p.st = final_state; p.ws = workspace;
  p.B = batch; p.T = seq_len; p.H = heads; p.NC = (int)nc;
  p.scale = scale;
  p.beta_bf16 = beta_dtype == TM_DT_BF16 ? 1 : 0;

  if (nc > 0) {
    // two workgroups per CU (their LDS and registers admit no third), each
    // walking its share of the chunks
    p.c0 = 0; p.c1 = (int)nc;
    const long long grid = std::min<long long>(bh * nc, 2LL * cu_count());
    const int rc = launch(intra_kernel(), dim3((unsigned)grid), dim3(256), 0, stream, p);
    if (rc) return rc;
  }
  p.c0 = 0; p.c1 = (int)nc;
  return launch(state_kernel(), dim3((unsigned)(bh * (kValueDim / 16))), dim3(192), 0, stream, p);
}

extern "C" int tm_kda_recurrent_fwd(const void* q, const void* k, const void* v, const float* g,
                                    const void* beta, const float* initial_state, void* o,
                                    float* final_state, int batch, int seq_len, int heads,
                                    int key_dim, int value_dim, float scale, int beta_dtype,
                                    void* stream) {
  if (batch < 0 || seq_len < 0 || heads < 0 || key_dim <= 0 || value_dim <= 0)
    return fail(TM_ERR_INVALID_ARG, "tm_kda_recurrent_fwd: B=%d T=%d H=%d Dk=%d Dv=%d", batch,
                seq_len, heads, key_dim, value_dim);
  if (key_dim != kKeyDim || value_dim != kValueDim)
    return fail(TM_ERR_UNSUPPORTED,
                "tm_kda_recurrent_fwd: key_dim=%d value_dim=%d (supported: 128, 128)", key_dim,
                value_dim);
  if (beta_dtype != TM_DT_F32 && beta_dtype != TM_DT_BF16)
    return fail(TM_ERR_INVALID_ARG, "tm_kda_recurrent_fwd: beta_dtype %d", beta_dtype);
  if (!std::isfinite(scale)) return fail(TM_ERR_INVALID_ARG, "tm_kda_recurrent_fwd: scale");
  if (batch == 0 || heads == 0) return 0;
  if (seq_len > 0 && (!q || !k || !v || !g || !beta || !o))
    return fail(TM_ERR_INVALID_ARG, "tm_kda_recurrent_fwd: null buffer");
  if (seq_len == 0 && !final_state) return 0;
  for (const void* ptr : {q, k, v, (const void*)g})
    if (ptr && !aligned16(ptr))
      return fail(TM_ERR_INVALID_ARG, "tm_kda_recurrent_fwd: q, k, v, g must be 16-byte aligned");
  if ((long long)batch * seq_len * heads * kKeyDim > 0x7fffffffffffLL ||
      (long long)batch * heads * (kValueDim / 16) > 0x7fffffffLL)
    return fail(TM_ERR_UNSUPPORTED, "tm_kda_recurrent_fwd: problem too large");
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  KdaParams p;
  memset(&p, 0, sizeof p);
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta;
  p.s0 = initial_state; p.o = o; p.st = final_state;
  p.B = batch; p.T = seq_len; p.H = heads;
  p.scale = scale;
  p.beta_bf16 = beta_dtype == TM_DT_BF16 ? 1 : 0;
  // one wave per (head, 16 value columns), or per (head, 32 value columns)
  // with 16-byte state accesses when both state buffers (or null) are 16-byte
  // aligned
  const bool v4 = ((reinterpret_cast<uintptr_t>(initial_state) |
                    reinterpret_cast<uintptr_t>(final_state)) & 15) == 0;
  const long long waves = (long long)batch * heads * (kValueDim / (v4 ? 32 : 16));
  return launch(v4 ? recurrent_v4_kernel() : recurrent_kernel(), dim3((unsigned)waves), dim3(64),
                0, stream, p);
}
