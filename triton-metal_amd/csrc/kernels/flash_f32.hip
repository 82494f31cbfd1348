// FlashAttention forward in fp32 on the fp32 MFMA (v_mfma_f32_16x16x4_f32):
// the dtype of the reference's own template (make_flash_attention_kernel,
// _msl_templates.py:1568-1767, fp32 Q, K, V and O) and of the @triton.jit
// tests' tensors.  Same semantics as flash_fwd.hip: a score is -inf when
// kv_pos >= seq_len or, if causal, kv_pos > q_pos (1610-1619); O is divided
// by l only when l > 0 (1747-1754); LSE is the natural-log logsumexp.
// Products and sums stay fp32 (the MFMA adds 4 fp32 products per step).
//
// flash_fwd_f32_d<D>_<mask>, D = 32, 48, ..., 128 (multiples of 16) with a
// contiguous head dim and 16-byte aligned rows.  A workgroup of 4 waves owns 64 query rows of one
// (b, h), a wave 16.  Per block of 32 keys:
//   S^T = K Q^T   A = K rows from LDS (lane l: key l % 16, d 4 s + l / 16),
//                 B = Q^T from registers (query l % 16); the result leaves
//                 lane l the scores of query l % 16 against keys 4 (l / 16) + e
//                 of each 16-key tile, so the row max and sum need the two
//                 swaps over lane bits 4 and 5 only;
//   O^T += V^T P^T  with the MFMA's 4-wide k index bound to keys 4 (l / 16) + kk
//                 at step kk, so P^T is the lane's own score e = kk (no
//                 exchange) and V^T is read from LDS in that order.
// K and V tiles go global -> registers -> LDS ([32 keys][D + 4] floats: a
// 16-lane operand read of one column lands on 16 banks, the 4 lane groups 16
// banks apart), the next block's loads in flight while the current one
// multiplies.
#include "common.h"
#include "flash_params.h"

namespace {

constexpr int F32_QW = 16;   // query rows per wave
constexpr int F32_BM = 64;   // query rows per workgroup
constexpr int F32_BN = 32;   // keys per block
constexpr float kLn2f32 = 0.69314718055994530942f;

template <int D, bool CAUSAL>
__device__ __forceinline__ void flash_f32_body(const FlashParams& p) {
  constexpr int DS = D + 4;                  // LDS row stride (floats)
  constexpr int DSTEP = D / 4;               // k-steps of S^T
  constexpr int DT = D / 16;                 // 16-row d tiles of O^T
  constexpr int TILE = F32_BN * DS;          // floats of one K (or V) tile in LDS
  constexpr int NPC = F32_BN * D / 4;          // float4 pieces of one tile
  constexpr int PPT = (NPC + 255) / 256;       // per thread (the last round partial
                                               // unless D % 32 == 0)
  static_assert(D % 16 == 0 && D <= 128, "head dim");
  extern __shared__ __align__(16) float smem[];  // [2][K tile, V tile]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int S = p.S;
  const int nqb = (S + F32_BM - 1) / F32_BM;
  // consecutive workgroups take the query blocks of one head (its K, V stay
  // in L2)
  const int bh = blockIdx.x / nqb, qb = blockIdx.x - bh * nqb;
  const int b = bh / p.H, hh = bh - b * p.H;
  const float* qg = (const float*)p.q + b * p.sqb + hh * p.sqh;
  const float* kg = (const float*)p.k + b * p.skb + hh * p.skh;
  const float* vg = (const float*)p.v + b * p.svb + hh * p.svh;
  float* og = (float*)p.o + b * p.sob + hh * p.soh;
  const int q0 = qb * F32_BM + wave * F32_QW;  // first query row of this wave
  const int qi = q0 + l16;                     // this lane's query row

  // Q^T operand: qreg[s] = Q[qi][4 s + g]
  float qreg[DSTEP];
#pragma unroll
  for (int s = 0; s < DSTEP; ++s) qreg[s] = qi < S ? qg[(long long)qi * p.sqs + 4 * s + g] : 0.f;

  const int kend = CAUSAL ? min(S, qb * F32_BM + F32_BM) : S;
  const int nkb = (kend + F32_BN - 1) / F32_BN;

  f4_t rk[PPT], rv[PPT];
  auto load = [&](int j) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = tid + 256 * i, row = e / (D / 4), c4 = e - row * (D / 4);
      const int key = j * F32_BN + row;
      rk[i] = rv[i] = f4_t{0.f, 0.f, 0.f, 0.f};
      if ((NPC % 256 == 0 || e < NPC) && key < S) {
        rk[i] = *(const f4_t*)(kg + (long long)key * p.sks + 4 * c4);
        rv[i] = *(const f4_t*)(vg + (long long)key * p.svs + 4 * c4);
      }
    }
  };
  auto stash = [&](int buf) {
    float* ks = smem + buf * 2 * TILE;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = tid + 256 * i, row = e / (D / 4), c4 = e - row * (D / 4);
      if (NPC % 256 != 0 && e >= NPC) continue;
      *(f4_t*)(ks + row * DS + 4 * c4) = rk[i];
      *(f4_t*)(ks + TILE + row * DS + 4 * c4) = rv[i];
    }
  };

  f4_t oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float sl2 = p.sl2;

  load(0);
  stash(0);
  __syncthreads();
  for (int j = 0; j < nkb; ++j) {
    const int buf = j & 1;
    const bool more = j + 1 < nkb;
    if (more) load(j + 1);
    const int k0 = j * F32_BN;
    // a wave whose rows all precede this key block has nothing to do
    if (!CAUSAL || k0 <= q0 + F32_QW - 1) {
      const float* ks = smem + buf * 2 * TILE;
      const float* vs = ks + TILE;
      f4_t st[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        st[kt] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < DSTEP; ++s)
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[(16 * kt + l16) * DS + 4 * s + g],
                                                         qreg[s], st[kt], 0, 0, 0);
      }
      // scores of keys k0 + 16 kt + 4 g + e against query qi, log2 domain
      float sc[8];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + 16 * kt + 4 * g + e;
          const bool ok = key < S && (!CAUSAL || key <= qi);
          sc[4 * kt + e] = ok ? st[kt][e] * sl2 : -INFINITY;
          mx = fmaxf(mx, sc[4 * kt + e]);
        }
      mx = max_swap<32>(max_swap<16>(mx));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float mu = m_new == -INFINITY ? 0.0f : m_new;
      m_run = m_new;
      float pv[8], ps = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(sc[i] - mu);
        ps += pv[i];
      }
      l_run = l_run * alpha + ps;  // this lane's keys; the lane groups meet at the end
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
      // O^T[d][q] += V^T[d][key] P^T[key][q], step (kt, kk): key 16 kt + 4 g + kk
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const float* vrow = vs + (16 * kt + 4 * g + kk) * DS + l16;
#pragma unroll
          for (int t = 0; t < DT; ++t)
            oacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * t], pv[4 * kt + kk], oacc[t],
                                                           0, 0, 0);
        }
    }
    if (more) stash(buf ^ 1);
    __syncthreads();
  }

  // O^T[16 t + 4 g + e][qi] in oacc[t][e]; l over the four lane groups
  const float l_half = fold_swap<16>(l_run, l_run);
  const float l_tot = fold_swap<32>(l_half, l_half);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < S) {
    float* orow = og + (long long)qi * p.sos;
#pragma unroll
    for (int t = 0; t < DT; ++t) *(f4_t*)(orow + 16 * t + 4 * g) = oacc[t] * inv;
    if (p.lse && g == 0)
      p.lse[(long long)bh * S + qi] = l_tot > 0.0f ? (m_run + __log2f(l_tot)) * kLn2f32 : -INFINITY;
  }
}

}  // namespace

// grid = ceil(S / 64) * B * H, block = 256, dynamic LDS 2 * 2 * 32 * (D + 4) * 4 bytes
#define TM_FLASH_F32(D, CAUSAL, MASK)                                                         \
  extern "C" __global__ __launch_bounds__(256) void flash_fwd_f32_d##D##_##MASK(FlashParams p) { \
    flash_f32_body<D, CAUSAL>(p);                                                             \
  }
TM_FLASH_F32(32, false, full)
TM_FLASH_F32(32, true, causal)
TM_FLASH_F32(48, false, full)
TM_FLASH_F32(48, true, causal)
TM_FLASH_F32(64, false, full)
TM_FLASH_F32(64, true, causal)
TM_FLASH_F32(80, false, full)
TM_FLASH_F32(80, true, causal)
TM_FLASH_F32(96, false, full)
TM_FLASH_F32(96, true, causal)
TM_FLASH_F32(112, false, full)
TM_FLASH_F32(112, true, causal)
TM_FLASH_F32(128, false, full)
TM_FLASH_F32(128, true, causal)
