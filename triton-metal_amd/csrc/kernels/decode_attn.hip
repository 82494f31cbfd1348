// Decode-time attention: one query token per (batch, query head) attending to
// a KV cache, softmax in fp32.
//
//   O[b, h, :] = sum_p softmax_p(scale * q[b, h, :] . K[b, kvh(h), p, :]) V[b, kvh(h), p, :]
//   over positions p < len(b);  kvh(h) = h / (q_heads / kv_heads)  (GQA)
//
// Semantics follow the reference's decode templates (_msl_templates.py):
// make_kv_cache_attention_kernel (1949-2048), make_gqa_attention_kernel
// (2049-2160: query head h reads KV head h / n_q_per_kv),
// make_batched_kv_decode_kernel (2161-2278: per-batch seq_lens),
// make_paged_attention_kernel / make_multi_head_paged_attention_kernel
// (2279-2532: position p in page page_table[p / page_size], slot
// p % page_size) and make_fp16_kv_attention_kernel (2533-2629: half cache,
// fp32 query and output).  A batch entry with no position gives O = 0.
//
// Cache addressing (element offsets, head dim contiguous):
//   contiguous: b * sB + kvh * sH + p * sS
//   paged:      page_table[b * max_pages + p / page_size] * sB + kvh * sH
//               + (p % page_size) * sS          (sB is then the page stride)
//
// MFMA kernel (decode_attn_d<D>_<dt>): fp16 / bf16 cache, head dim 64 or 128,
// up to 16 query heads per KV head.  One wave owns (batch, KV head, a block
// of 16 query heads, a slice of positions) and streams 32-position tiles of K
// and V through a private LDS ring (global -> LDS copies, each position row
// read by consecutive lanes).  Per tile:
//   S^T = K Q^T   v_mfma_f32_16x16x32: A = K rows from LDS, B = Q^T in
//                 registers; lane l holds the scores of query head l % 16
//   O^T += V^T P^T  A = V^T read with ds_read_b64_tr_b16, B = P^T straight
//                 from the S^T accumulators (the position order inside a
//                 32-position MFMA step matches the accumulator layout)
// with an online softmax in the exp2 domain.  A wave writes its slice's
// (max, sum, unnormalised O) to the workspace, or the final O when the
// sequence is one slice; decode_attn_combine merges the slices.
// General kernel (decode_attn_general): any dtype and head dim <= 256, one
// workgroup per (batch, query head), fp32 throughout.
#include "common.h"

struct DecodeParams {
  const void* q;            // [B, Hq, D]
  const uint16_t* k;
  const uint16_t* v;
  void* o;                  // [B, Hq, D]
  float* lse;               // [B, Hq] or null
  const int* seq_lens;      // [B] or null
  const int* page_table;    // [B, max_pages] or null
  float* ws;                // [B, Hq, nsplit, D + 4] partials (nsplit > 1): O, max, sum
  long long sB, sH, sS;     // cache strides (elements)
  int B, Hq, Hkv, D;
  int seq_len;              // length when seq_lens is null; the capacity bound
  int page_size, max_pages;
  int page_shift;           // log2(page_size) when a power of two, else -1
  int nsplit, split_len;    // slices of split_len positions (paged: whole
                            // pages, at most 64 of them)
  float sl2;                // scale * log2(e)
  int q_dt, kv_dt, o_dt;    // TM_DT_* codes
};

// Scratch of tm_decode_attention_noalloc: the per-slice partials (O, max,
// sum) live here instead of in a caller's workspace.  One copy per device,
// allocated when this code object is loaded there and held until the process
// ends; its device address is looked up by name (hipModuleGetGlobal), so it
// has external linkage (a static array would not be in the module's symbol
// table).  Size: TM_DECODE_SCRATCH_BYTES of include/tm_hip.h.
__device__ __align__(256) unsigned char tm_decode_scratch[8u << 20];

namespace {
constexpr float kLn2f = 0.69314718055994530942f;

typedef short s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4_t lds_s4_t;
TM_DEV u2_t tr16(const uint16_t* p) {
  s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(p));
  return __builtin_bit_cast(u2_t, v);
}

// Eight fp32 values as hi + lo pairs of 16-bit operands: hi = round(f),
// lo = round(f - hi) (f - hi is exact in fp32).
template <bool BF16> TM_DEV void split_pack(const float* in, u4_t& hi, u4_t& lo) {
  // fp16: hi saturates at the largest finite half, so lo carries what lies
  // beyond 65504; |x| <= 131008 stays finite (larger values saturate there)
  float f[8], r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f[e] = BF16 ? in[e] : fminf(fmaxf(in[e], -131008.f), 131008.f);
    const float h = BF16 ? f[e] : fminf(fmaxf(f[e], -65504.f), 65504.f);
    r[e] = BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(h)) : f16_bits_to_f32(f32_to_f16_bits(h));
  }
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = BF16 ? pack_bf16x2(r[2 * i], r[2 * i + 1]) : pack_f16x2(r[2 * i], r[2 * i + 1]);
    const float d0 = f[2 * i] - r[2 * i], d1 = f[2 * i + 1] - r[2 * i + 1];
    l[i] = BF16 ? pack_bf16x2(d0, d1) : pack_f16x2(d0, d1);
  }
  hi = u4_t{h[0], h[1], h[2], h[3]};
  lo = u4_t{l[0], l[1], l[2], l[3]};
}

TM_DEV int seq_len_of(const DecodeParams& p, int b) {
  return p.seq_lens ? min(p.seq_lens[b], p.seq_len) : p.seq_len;
}

TM_DEV float ld_any(const void* ptr, long long i, int dt) {
  if (dt == TM_DT_F32) return ((const float*)ptr)[i];
  if (dt == TM_DT_F16) return f16_bits_to_f32(((const uint16_t*)ptr)[i]);
  return bf16_bits_to_f32(((const uint16_t*)ptr)[i]);
}
TM_DEV void st_any(void* ptr, long long i, int dt, float v) {
  if (dt == TM_DT_F32) ((float*)ptr)[i] = v;
  else if (dt == TM_DT_F16) ((uint16_t*)ptr)[i] = f32_to_f16_bits(v);
  else ((uint16_t*)ptr)[i] = f32_to_bf16_bits(v);
}
}  // namespace

// ----------------------------------------------------------------------------
// MFMA kernel.  grid = (nsplit, Hkv * ceil(group / 16), B), block = 64.
// Per-wave LDS ring of NST stages, each [32 positions][D] of K then of V, row
// piece c (16 bytes) of position row r stored at slot c ^ (r & (D / 8 - 1)).
// ----------------------------------------------------------------------------
// SPLIT (a query dtype other than the cache's, e.g. fp32 queries over a
// 16-bit cache as make_fp16_kv_attention_kernel takes them): the query and the
// probabilities each travel as a pair hi + lo of cache-dtype operands,
// hi = round(x), lo = round(x - hi), and every product is two MFMAs.  The
// pair carries 22 (fp16) or 16 (bf16) significant bits, so scores and the
// weighted sum keep fp32-level accuracy against the fp32 computation of the
// reference template instead of one 16-bit rounding of q and P.
// DV < D: a head dim of DV (a multiple of 16 above D / 2) in the LDS layout of
// D: the copies skip the 16-byte pieces at or past DV (masked-off lanes write
// no LDS slot; the K slots are zeroed once, as a k-step may cover them), the
// query's pieces past DV are zero, the k-steps and d tiles wholly past DV are
// skipped, and q, o and the slice partials are addressed with DV.
template <int D, bool BF16, bool SPLIT, int DV = D>
__device__ __forceinline__ void decode_mfma_body(const DecodeParams& p) {
  constexpr int NST = 3;
  constexpr int PR = D / 8;             // 16-byte pieces per row
  constexpr int TB = 32 * D * 2;        // bytes of one K (or V) tile
  constexpr int NCP = TB / 1024;        // 1 KB copies per tile
  constexpr int RPC = 64 / PR;          // rows per copy
  constexpr int KS = (DV + 31) / 32;    // k-steps of S^T = K Q^T
  constexpr int DT = DV / 16;           // 16-row d tiles of O^T
  constexpr int PV = DV / 8;            // pieces of a row below DV
  static_assert(DV % 16 == 0 && DV <= D && 2 * DV > D, "head dim");
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x, l16 = lane & 15, q4 = lane >> 4;
  const int group = p.Hq / p.Hkv, hbn = (group + 15) / 16;
  const int split = blockIdx.x, b = blockIdx.z;
  const int kvh = blockIdx.y / hbn, hb = blockIdx.y - kvh * hbn;
  const int len = seq_len_of(p, b);
  const int p0 = split * p.split_len, p1 = min(len, p0 + p.split_len);
  const int hq = kvh * group + 16 * hb + l16;    // this lane's query head
  const bool hvalid = 16 * hb + l16 < group;

  // Q^T operand: q[b, hq, 32 ks + 8 q4 .. +8] in the cache dtype (SPLIT: its
  // hi and lo parts)
  u4_t qop[KS], qlo[SPLIT ? KS : 1];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qop[ks] = u4_t{0u, 0u, 0u, 0u};
    if constexpr (SPLIT) qlo[ks] = u4_t{0u, 0u, 0u, 0u};
    if (hvalid && (DV == D || 4 * ks + q4 < PV)) {
      const long long qi = ((long long)b * p.Hq + hq) * DV + 32 * ks + 8 * q4;
      if constexpr (!SPLIT) {
        qop[ks] = ldg128((const uint16_t*)p.q + qi);
      } else {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = ld_any(p.q, qi + e, p.q_dt);
        split_pack<BF16>(f, qop[ks], qlo[ks]);
      }
    }
  }

  // ---- copies: lane -> (row r = RPC i + lane / PR, slot lane % PR)
  const long long hoff = (long long)kvh * p.sH;
  const int* pt = p.page_table ? p.page_table + (long long)b * p.max_pages : nullptr;
  const uint32_t lbase = __builtin_amdgcn_readfirstlane(lds_off(lds));
  const int ntile = p1 > p0 ? (p1 - p0 + 31) / 32 : 0;
  // paged: lane i holds the physical page of the slice's i-th page (the slice
  // starts on a page boundary and spans at most 64 pages), fetched below with
  // ds_bpermute so that no table load sits between the copies
  const int fp = pt ? p0 / p.page_size : 0;
  int mypage = 0;
  if (pt && ntile > 0) {
    const int np = (p1 - 1) / p.page_size - fp + 1;
    if (lane < np) mypage = pt[fp + lane];
  }
  auto row_off = [&](int pos) -> long long {  // element offset of cache position pos
    if (pt) {
      const int rel = pos - p0;  // p0 is page aligned
      const int pi = p.page_shift >= 0 ? rel >> p.page_shift : rel / p.page_size;
      const int slot = p.page_shift >= 0 ? rel & (p.page_size - 1) : rel - pi * p.page_size;
      const int page = __builtin_amdgcn_ds_bpermute(4 * pi, mypage);
      return (long long)page * p.sB + hoff + (long long)slot * p.sS;
    }
    return (long long)b * p.sB + hoff + (long long)pos * p.sS;
  };
  // the lane's piece of copy i lies below DV (its slot in the ring is fixed)
  auto piece_in = [&](int i) -> bool {
    if constexpr (DV == D) {
      return true;
    } else {
      const int r = RPC * i + lane / PR, sl = lane % PR;
      return (sl ^ (r & (PR - 1))) < PV;
    }
  };
  if constexpr (DV < D) {
    // the K slots of the pieces past DV in every ring stage: zero once
    for (int sidx = lane; sidx < NST * 32 * (PR - PV); sidx += 64) {
      const int stg = sidx / (32 * (PR - PV)), rem = sidx - stg * 32 * (PR - PV);
      const int r = rem / (PR - PV), c = PV + rem % (PR - PV);
      *(u4_t*)(lds + stg * 2 * TB + 2 * (r * D + 8 * (c ^ (r & (PR - 1))))) =
          u4_t{0u, 0u, 0u, 0u};
    }
  }
  auto issue = [&](int t) {
    const uint32_t st = lbase + (uint32_t)((t % NST) * 2 * TB);
    // all row offsets first (paged: the page fetches overlap), then the copies
    long long e[NCP];
#pragma unroll
    for (int i = 0; i < NCP; ++i) {
      const int r = RPC * i + lane / PR, sl = lane % PR;
      const int pos = min(p0 + 32 * t + r, len - 1);  // rows past the end are masked
      e[i] = row_off(pos) + 8 * (sl ^ (r & (PR - 1)));
    }
    // the cache is read once per call: non-temporal copies (B=8, S=8192:
    // 56.4 -> 52.3 us contiguous, 63.8 -> 61.4 us paged)
#pragma unroll
    for (int i = 0; i < NCP; ++i) {
      if (piece_in(i)) {
        dma16_nt(p.k + e[i], st + 1024 * i);
        dma16_nt(p.v + e[i], st + TB + 1024 * i);
      }
    }
  };
#pragma unroll
  for (int t = 0; t < NST - 1; ++t)
    if (t < ntile) issue(t);

  f4_t oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  for (int t = 0; t < ntile; ++t) {
    const int later = min(NST - 2, ntile - 1 - t);
    if (later >= 1) wait_vm<2 * NCP>();
    else wait_vm<0>();
    asm volatile("" ::: "memory");
    if (t + NST - 1 < ntile) issue(t + NST - 1);
    const uint16_t* ks_ = (const uint16_t*)(lds + (t % NST) * 2 * TB);
    const uint16_t* vs_ = ks_ + TB / 2;
    // S^T = K Q^T for the tile's two 16-position blocks
    f4_t s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f4_t{0.f, 0.f, 0.f, 0.f};
      const int r = 16 * kb + l16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u4_t a = *(const u4_t*)(ks_ + r * D + 8 * ((4 * ks + q4) ^ (r & (PR - 1))));
        s[kb] = mfma16<BF16>(a, qop[ks], s[kb]);
        if constexpr (SPLIT) s[kb] = mfma16<BF16>(a, qlo[ks], s[kb]);
      }
    }
    // positions of this lane's scores: 32 t + 16 kb + 4 q4 + e
    const int pbase = p0 + 32 * t;
    float sc[8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int pos = pbase + 16 * kb + 4 * q4 + e;
        sc[4 * kb + e] = pos < p1 ? s[kb][e] * p.sl2 : -INFINITY;
      }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sc[i]);
    mx = max_swap<32>(max_swap<16>(mx));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    const float mu = m_new == -INFINITY ? 0.0f : m_new;
    float pv[8], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pv[i] = __builtin_amdgcn_exp2f(sc[i] - mu);
      ps += pv[i];
    }
    l_run = l_run * alpha + ps;
    u4_t pop, plo;
    if constexpr (SPLIT) {
      split_pack<BF16>(pv, pop, plo);
    } else {
      pop.x = BF16 ? pack_bf16x2(pv[0], pv[1]) : pack_f16x2(pv[0], pv[1]);
      pop.y = BF16 ? pack_bf16x2(pv[2], pv[3]) : pack_f16x2(pv[2], pv[3]);
      pop.z = BF16 ? pack_bf16x2(pv[4], pv[5]) : pack_f16x2(pv[4], pv[5]);
      pop.w = BF16 ? pack_bf16x2(pv[6], pv[7]) : pack_f16x2(pv[6], pv[7]);
    }
    // O^T += V^T P^T: lane j of 16-lane group q4 addresses row 4 q4 + j / 4
    // (+16 for the second half), d chunk 16 dt + 4 (j % 4)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      oacc[dt] *= alpha;
      const int dd = 16 * dt + 4 * (l16 & 3);
      const int r0 = 4 * q4 + (l16 >> 2), r1 = r0 + 16;
      const u2_t lo = tr16(vs_ + r0 * D + 8 * ((dd >> 3) ^ (r0 & (PR - 1))) + (dd & 7));
      const u2_t hi = tr16(vs_ + r1 * D + 8 * ((dd >> 3) ^ (r1 & (PR - 1))) + (dd & 7));
      u4_t a;
      a.x = lo.x; a.y = lo.y; a.z = hi.x; a.w = hi.y;
      oacc[dt] = mfma16<BF16>(a, pop, oacc[dt]);
      if constexpr (SPLIT) oacc[dt] = mfma16<BF16>(a, plo, oacc[dt]);
    }
  }
  wait_vm<0>();
  l_run = fold_swap<16>(l_run, l_run);
  l_run = fold_swap<32>(l_run, l_run);
  if (!hvalid) return;
  // lane holds O^T[16 dt + 4 q4 + e][head l16]
  if (p.nsplit == 1) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const long long ob = ((long long)b * p.Hq + hq) * DV;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) st_any(p.o, ob + 16 * dt + 4 * q4 + e, p.o_dt, oacc[dt][e] * inv);
    if (p.lse && q4 == 0)
      p.lse[(long long)b * p.Hq + hq] = l_run > 0.0f ? (m_run + __log2f(l_run)) * kLn2f : -INFINITY;
  } else {
    float* w = p.ws + (((long long)b * p.Hq + hq) * p.nsplit + split) * (DV + 4);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *(f4_t*)(w + 16 * dt + 4 * q4) = oacc[dt];
    if (q4 == 0) {
      w[DV] = m_run;
      w[DV + 1] = l_run;
    }
  }
}

#define TM_DECODE(D, DT, BF)                                                                   \
  extern "C" __global__ __launch_bounds__(64) void decode_attn_d##D##_##DT(DecodeParams p) {   \
    decode_mfma_body<D, BF, false>(p);                                                         \
  }                                                                                            \
  extern "C" __global__ __launch_bounds__(64) void decode_attn_d##D##_##DT##_x(DecodeParams p) { \
    decode_mfma_body<D, BF, true>(p);                                                          \
  }
TM_DECODE(128, f16, false)
TM_DECODE(128, bf16, true)
TM_DECODE(64, f16, false)
TM_DECODE(64, bf16, true)
// head dims 48 (in the 64 layout) and 80, 96, 112 (in the 128 layout):
// decode_attn_d<D>v<DV>_<dt>[_x]
#define TM_DECODE_V(D, DV, DT, BF)                                                             \
  extern "C" __global__ __launch_bounds__(64) void decode_attn_d##D##v##DV##_##DT(DecodeParams p) { \
    decode_mfma_body<D, BF, false, DV>(p);                                                     \
  }                                                                                            \
  extern "C" __global__ __launch_bounds__(64) void decode_attn_d##D##v##DV##_##DT##_x(          \
      DecodeParams p) {                                                                        \
    decode_mfma_body<D, BF, true, DV>(p);                                                      \
  }
#define TM_DECODE_VD(D, DV) TM_DECODE_V(D, DV, f16, false) TM_DECODE_V(D, DV, bf16, true)
TM_DECODE_VD(64, 48)
TM_DECODE_VD(128, 80)
TM_DECODE_VD(128, 96)
TM_DECODE_VD(128, 112)

// ----------------------------------------------------------------------------
// fp32 caches and queries (the dtype of the reference's decode templates other
// than make_fp16_kv_attention_kernel): fp32 MFMA v_mfma_f32_16x16x4_f32.
// grid = (nsplit, Hkv * ceil(group / 16), B), block = 64, the same slices,
// partials and combine as the 16-bit kernel.  Per 16-position tile:
//   S^T = K Q^T   A = K rows from LDS (lane l: position l % 16, d 4 s + l / 16),
//                 B = Q^T in registers (query head l % 16): lane l receives
//                 positions 4 (l / 16) + e of its head;
//   O^T += V^T P^T  the MFMA's 4-wide k index bound to positions 4 (l / 16) +
//                 kk at step kk, so P^T is the lane's own score.
// Tiles go global -> registers -> a 2-slot LDS ring ([16][D + 4] floats), the
// next tile's loads in flight while the current one multiplies.
// ----------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void decode_f32_body(const DecodeParams& p) {
  static_assert(D % 16 == 0 && D >= 32 && D <= 128, "head dim");
  constexpr int DS = D + 4;           // LDS row stride (floats)
  constexpr int TILE = 16 * DS;       // floats of one K (or V) tile
  constexpr int PPT = 16 * D / 4 / 64;  // float4 pieces per lane and tile
  constexpr int KS = D / 4;           // k-steps of S^T
  constexpr int DT = D / 16;          // 16-row d tiles of O^T
  extern __shared__ __align__(16) uint8_t lds[];
  float* ring = (float*)lds;          // [2 slots][K tile, V tile]
  const int lane = threadIdx.x, l16 = lane & 15, g = lane >> 4;
  const int group = p.Hq / p.Hkv, hbn = (group + 15) / 16;
  const int split = blockIdx.x, b = blockIdx.z;
  const int kvh = blockIdx.y / hbn, hb = blockIdx.y - kvh * hbn;
  const int len = seq_len_of(p, b);
  const int p0 = split * p.split_len, p1 = min(len, p0 + p.split_len);
  const int hq = kvh * group + 16 * hb + l16;  // this lane's query head
  const bool hvalid = 16 * hb + l16 < group;
  const float* kc = (const float*)p.k;
  const float* vc = (const float*)p.v;

  // Q^T operand: qreg[s] = q[b, hq, 4 s + g]
  float qreg[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qreg[s] = hvalid ? ((const float*)p.q)[((long long)b * p.Hq + hq) * D + 4 * s + g] : 0.0f;

  const long long hoff = (long long)kvh * p.sH;
  const int* pt = p.page_table ? p.page_table + (long long)b * p.max_pages : nullptr;
  const int ntile = p1 > p0 ? (p1 - p0 + 15) / 16 : 0;
  // paged: lane i holds the physical page of the slice's i-th page (the slice
  // starts on a page boundary and spans at most 64 pages)
  const int fp = pt ? p0 / p.page_size : 0;
  int mypage = 0;
  if (pt && ntile > 0) {
    const int np = (p1 - 1) / p.page_size - fp + 1;
    if (lane < np) mypage = pt[fp + lane];
  }
  auto row_off = [&](int pos) -> long long {  // element offset of cache position pos
    if (pt) {
      const int rel = pos - p0;
      const int pi = p.page_shift >= 0 ? rel >> p.page_shift : rel / p.page_size;
      const int slot = p.page_shift >= 0 ? rel & (p.page_size - 1) : rel - pi * p.page_size;
      const int page = __builtin_amdgcn_ds_bpermute(4 * pi, mypage);
      return (long long)page * p.sB + hoff + (long long)slot * p.sS;
    }
    return (long long)b * p.sB + hoff + (long long)pos * p.sS;
  };
  // lane's pieces: row (lane + 64 i) / (D / 4), float4 column (lane + 64 i) % (D / 4)
  f4_t rk[PPT], rv[PPT];
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = lane + 64 * i, r = e / (D / 4), c4 = e - r * (D / 4);
      const long long off = row_off(min(p0 + 16 * t + r, len - 1)) + 4 * c4;
      rk[i] = *(const f4_t*)(kc + off);
      rv[i] = *(const f4_t*)(vc + off);
    }
  };
  auto stash = [&](int slot) {
    float* ks = ring + slot * 2 * TILE;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = lane + 64 * i, r = e / (D / 4), c4 = e - r * (D / 4);
      *(f4_t*)(ks + r * DS + 4 * c4) = rk[i];
      *(f4_t*)(ks + TILE + r * DS + 4 * c4) = rv[i];
    }
  };

  f4_t oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  if (ntile > 0) {
    load(0);
    stash(0);
  }
  for (int t = 0; t < ntile; ++t) {
    const bool more = t + 1 < ntile;
    if (more) load(t + 1);
    const float* ks = ring + (t & 1) * 2 * TILE;
    const float* vs = ks + TILE;
    f4_t st = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
      st = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[l16 * DS + 4 * s + g], qreg[s], st, 0, 0, 0);
    const int pbase = p0 + 16 * t + 4 * g;
    float sc[4], mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc[e] = pbase + e < p1 ? st[e] * p.sl2 : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    mx = max_swap<32>(max_swap<16>(mx));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    const float mu = m_new == -INFINITY ? 0.0f : m_new;
    m_run = m_new;
    float pv[4], ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pv[e] = __builtin_amdgcn_exp2f(sc[e] - mu);
      ps += pv[e];
    }
    l_run = l_run * alpha + ps;  // this lane's positions; the lane groups meet at the end
#pragma unroll
    for (int d = 0; d < DT; ++d) oacc[d] *= alpha;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float* vrow = vs + (4 * g + kk) * DS + l16;
#pragma unroll
      for (int d = 0; d < DT; ++d)
        oacc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * d], pv[kk], oacc[d], 0, 0, 0);
    }
    if (more) stash((t + 1) & 1);
  }
  l_run = fold_swap<16>(l_run, l_run);
  l_run = fold_swap<32>(l_run, l_run);
  if (!hvalid) return;
  // lane holds O^T[16 d + 4 g + e][head l16]
  if (p.nsplit == 1) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const long long ob = ((long long)b * p.Hq + hq) * D;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) st_any(p.o, ob + 16 * d + 4 * g + e, p.o_dt, oacc[d][e] * inv);
    if (p.lse && g == 0)
      p.lse[(long long)b * p.Hq + hq] = l_run > 0.0f ? (m_run + __log2f(l_run)) * kLn2f : -INFINITY;
  } else {
    float* w = p.ws + (((long long)b * p.Hq + hq) * p.nsplit + split) * (D + 4);
#pragma unroll
    for (int d = 0; d < DT; ++d) *(f4_t*)(w + 16 * d + 4 * g) = oacc[d];
    if (g == 0) {
      w[D] = m_run;
      w[D + 1] = l_run;
    }
  }
}

// decode_attn_f32_d<D>, D = 32, 48, ..., 128
#define TM_DECODE_F32(D)                                                                    \
  extern "C" __global__ __launch_bounds__(64) void decode_attn_f32_d##D(DecodeParams p) {   \
    decode_f32_body<D>(p);                                                                  \
  }
TM_DECODE_F32(32)
TM_DECODE_F32(48)
TM_DECODE_F32(64)
TM_DECODE_F32(80)
TM_DECODE_F32(96)
TM_DECODE_F32(112)
TM_DECODE_F32(128)

// ----------------------------------------------------------------------------
// Combine the slices: grid = B * Hq, block = 64 (D <= 256, 4 per lane).  The
// lanes take the slices' maxima in parallel; the weighted sum runs 8 slices
// per step so that their loads are in flight together.
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(64) void decode_attn_combine(DecodeParams p) {
  const int bh = blockIdx.x, lane = threadIdx.x;
  const int D = p.D, ns = p.nsplit, RS = D + 4;
  const float* w = p.ws + (long long)bh * ns * RS;
  if (ns <= 32 && D <= 128) {
    // one round of loads: every slice's (max, sum) (the same address in every
    // lane) and this lane's output elements, then the merge in registers
    constexpr int MS = 32;
    float mj[MS], lj[MS], oj[MS][2];
#pragma unroll
    for (int j = 0; j < MS; ++j) {
      mj[j] = -INFINITY;
      lj[j] = 0.0f;
      oj[j][0] = oj[j][1] = 0.0f;
      if (j < ns) {
        const float* ws = w + j * RS;
        mj[j] = ws[D];
        lj[j] = ws[D + 1];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          if (lane + 64 * i < D) oj[j][i] = ws[lane + 64 * i];
      }
    }
    float Mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < MS; ++j) Mx = fmaxf(Mx, mj[j]);
    const float mu = Mx == -INFINITY ? 0.0f : Mx;
    float L = 0.0f, acc[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MS; ++j) {
      const float f = lj[j] > 0.0f ? __builtin_amdgcn_exp2f(mj[j] - mu) : 0.0f;
      L += lj[j] * f;
      acc[0] += oj[j][0] * f;
      acc[1] += oj[j][1] * f;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int d = lane + 64 * i;
      if (d < D) st_any(p.o, (long long)bh * D + d, p.o_dt, acc[i] * inv);
    }
    if (p.lse && lane == 0) p.lse[bh] = L > 0.0f ? (Mx + __log2f(L)) * kLn2f : -INFINITY;
    return;
  }
  float M = -INFINITY;
  for (int s = lane; s < ns; s += 64) M = fmaxf(M, w[s * RS + D]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  const float mu = M == -INFINITY ? 0.0f : M;
  float L = 0.0f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  int s0 = 0;
  for (; s0 + 8 <= ns; s0 += 8) {
    float f[8], o[8][4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float* ws = w + (s0 + j) * RS;
      const float ls = ws[D + 1];
      f[j] = ls > 0.0f ? __builtin_amdgcn_exp2f(ws[D] - mu) : 0.0f;
      L += ls * f[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[j][i] = lane + 64 * i < D ? ws[lane + 64 * i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += o[j][i] * f[j];
  }
  for (; s0 < ns; ++s0) {
    const float* ws = w + s0 * RS;
    const float ls = ws[D + 1];
    const float f = ls > 0.0f ? __builtin_amdgcn_exp2f(ws[D] - mu) : 0.0f;
    L += ls * f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + 64 * i < D) acc[i] += ws[lane + 64 * i] * f;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) st_any(p.o, (long long)bh * D + d, p.o_dt, acc[i] * inv);
  }
  if (p.lse && lane == 0) p.lse[bh] = L > 0.0f ? (M + __log2f(L)) * kLn2f : -INFINITY;
}

// ----------------------------------------------------------------------------
// General kernel: grid = B * Hq, block = 256, head dim <= 256; fp32 math.
// Positions in chunks of 256 (one per thread): scores, chunk max, running
// rescale, then thread d accumulates sum_p P[p] V[p, d].
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void decode_attn_general(DecodeParams p) {
  __shared__ float qs[256];
  __shared__ float pr[256];
  __shared__ float red[8];
  const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = bh / p.Hq, hq = bh - b * p.Hq;
  const int kvh = hq / (p.Hq / p.Hkv);
  const int D = p.D, len = seq_len_of(p, b);
  const long long hoff = (long long)kvh * p.sH;
  const int* pt = p.page_table ? p.page_table + (long long)b * p.max_pages : nullptr;
  if (tid < D) qs[tid] = ld_any(p.q, (long long)bh * D + tid, p.q_dt);
  __syncthreads();
  float m_run = -INFINITY, l_run = 0.0f, o = 0.0f;
  for (int c0 = 0; c0 < len; c0 += 256) {
    const int pos = c0 + tid;
    float sc = -INFINITY;
    if (pos < len) {
      const long long ro = pt ? (long long)pt[pos / p.page_size] * p.sB + hoff +
                                    (long long)(pos % p.page_size) * p.sS
                              : (long long)b * p.sB + hoff + (long long)pos * p.sS;
      float dot = 0.0f;
      for (int d = 0; d < D; ++d) dot += qs[d] * ld_any(p.k, ro + d, p.kv_dt);
      sc = dot * p.sl2;
    }
    float mx = sc;
    for (int o2 = 32; o2 > 0; o2 >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o2, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first chunk
    const float pe = pos < len ? __builtin_amdgcn_exp2f(sc - m_new) : 0.0f;
    pr[tid] = pe;
    float ps = pe;
    for (int o2 = 32; o2 > 0; o2 >>= 1) ps += __shfl_xor(ps, o2, 64);
    __syncthreads();
    if (lane == 0) red[4 + wave] = ps;
    __syncthreads();
    l_run = l_run * alpha + (red[4] + red[5] + red[6] + red[7]);
    m_run = m_new;
    if (tid < D) {
      float a = 0.0f;
      const int n = min(256, len - c0);
      for (int j = 0; j < n; ++j) {
        const int pj = c0 + j;
        const long long ro = pt ? (long long)pt[pj / p.page_size] * p.sB + hoff +
                                      (long long)(pj % p.page_size) * p.sS
                                : (long long)b * p.sB + hoff + (long long)pj * p.sS;
        a += pr[j] * ld_any(p.v, ro + tid, p.kv_dt);
      }
      o = o * alpha + a;
    }
    __syncthreads();
  }
  if (tid < D) st_any(p.o, (long long)bh * D + tid, p.o_dt, l_run > 0.0f ? o / l_run : 0.0f);
  if (p.lse && tid == 0) p.lse[bh] = l_run > 0.0f ? (m_run + __log2f(l_run)) * kLn2f : -INFINITY;
}
