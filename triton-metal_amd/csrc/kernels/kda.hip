// KDA (Kimi Delta Attention) chunked gated delta-rule forward for gfx950.
//
// Per head, with state S in R^{Dk x Dv}, per-key-channel log decay g_t and
// write strength beta_t:
//     S <- diag(exp(g_t)) S
//     S <- S + beta_t k_t (v_t - S^T k_t)^T
//     o_t = S^T (scale * q_t)
// The reference has no linear attention; this is the published gated delta
// rule of Kimi Delta Attention in the [B, T, H, D] layout of its chunked
// operator (chunk_kda).
//
// Chunked form (chunk of C = 64 steps, G_t = inclusive cumulative sum of g
// inside the chunk, S0 = state entering the chunk):
//     A[t,s]   = beta_t sum_c k_tc k_sc exp(G_tc - G_sc)      (s < t)
//     Aqk[t,s] = scale sum_c q_tc k_sc exp(G_tc - G_sc)       (s <= t)
//     T = (I + A)^-1
//     [W_k | W_v] = T [beta * k * exp(G) | beta * v]
//     U  = W_v - W_k S0
//     O  = (scale * q * exp(G)) S0 + Aqk U
//     S1 = diag(exp(G_C)) S0 + (k * exp(G_C - G))^T U
//
// kda_intra (one workgroup per (head, chunk), all chunks in parallel) builds
// everything that does not depend on S0 and writes it to a workspace;
// kda_state (one workgroup per (head, 16 value columns)) runs the chunk
// recurrence with bf16 MFMAs and an fp32 state held in registers.
//
// Decay factors.  exp(G_t - G_s) is factored through the first row r of the
// 16-row block holding t: exp(G_t - G_r) * exp(G_r - G_s).  For s < r both
// factors are <= 1 (g <= 0), so nothing overflows and an underflowed factor
// means a negligible product.  Inside the diagonal 16x16 block the second
// factor is >= 1; the fast path is used while every |G_t - G_r| in the chunk
// is <= 80 (factors within [e^-80, e^80], normal fp32/bf16 numbers), else the
// diagonal blocks are recomputed with the exact pairwise exponent.
#include <type_traits>

#include "common.h"

namespace {
constexpr int KC = 64;    // chunk length
constexpr int KD = 128;   // key dim
constexpr int VD = 128;   // value dim
constexpr int GP = KD + 4;             // padded row of the decay tile (bank spread)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kExp2Range = 80.0f * kLog2e;  // |G_t - G_r| <= 80 in natural-log units

// Workspace of one (head, chunk), bytes.  The matrices kda_state reads as
// MFMA operands are stored in fragment order: 1 KB blocks, one per (16-row
// block, 32-column step), in which lane l = 16 q + r of the reading wave finds
// its 16 bytes (row r, columns 8q..8q+7 of the step) at 16 l - so every load
// there is one contiguous 1 KB.
constexpr size_t WS_WK = 0;                    // W_k [64][128]      fragments (16 blocks)
constexpr size_t WS_WV = WS_WK + KC * KD * 2;  // W_v [64/4][128][4] (4 steps of a column together)
constexpr size_t WS_QD = WS_WV + KC * VD * 2;  // scale q exp(G) [64][128] fragments
constexpr size_t WS_KT = WS_QD + KC * KD * 2;  // (k exp(G_C - G))^T [128][64] fragments
constexpr size_t WS_AQ = WS_KT + KD * KC * 2;  // Aqk [64][64]       fragments (8 blocks)
constexpr size_t WS_GC = WS_AQ + KC * KC * 2;  // exp(G_C), fp32 [128]
constexpr size_t WS_CHUNK = WS_GC + KD * 4;
static_assert(WS_CHUNK == 74240, "workspace layout is part of the C ABI");

// Byte offset of (row, 8-column group cg) of a matrix with `steps` 32-column
// steps per row, stored in fragment order.
TM_DEV int frag_off(int row, int cg, int steps) {
  return (((row >> 4) * steps + (cg >> 2)) * 64 + (cg & 3) * 16 + (row & 15)) * 16;
}

TM_DEV u4_t pack8_bf16(const float* x) {
  u4_t r;
  r.x = pack_bf16x2(x[0], x[1]);
  r.y = pack_bf16x2(x[2], x[3]);
  r.z = pack_bf16x2(x[4], x[5]);
  r.w = pack_bf16x2(x[6], x[7]);
  return r;
}
TM_DEV void unpack8_bf16(u4_t v, float* x) {
  x[0] = __uint_as_float(v.x << 16); x[1] = __uint_as_float(v.x & 0xffff0000u);
  x[2] = __uint_as_float(v.y << 16); x[3] = __uint_as_float(v.y & 0xffff0000u);
  x[4] = __uint_as_float(v.z << 16); x[5] = __uint_as_float(v.z & 0xffff0000u);
  x[6] = __uint_as_float(v.w << 16); x[7] = __uint_as_float(v.w & 0xffff0000u);
}
TM_DEV void load8_f32(const float* p, float* x) {
  const f4_t a = *(const f4_t*)p, b = *(const f4_t*)(p + 4);
  x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
  x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
}
// 2^x on the transcendental unit (v_exp_f32).
TM_DEV float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
TM_DEV f4_t mfma_f32_16x16x4(float a, float b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
}  // namespace

struct KdaParams {
  const uint16_t* q;   // [B, T, H, KD] bf16
  const uint16_t* k;   // [B, T, H, KD] bf16
  const uint16_t* v;   // [B, T, H, VD] bf16
  const float* g;      // [B, T, H, KD] fp32
  const void* beta;    // [B, T, H] fp32 or bf16
  const float* s0;     // [B, H, KD, VD] fp32 or null
  uint16_t* o;         // [B, T, H, VD] bf16
  float* st;           // [B, H, KD, VD] fp32 or null
  uint8_t* ws;         // workspace: B*H*NC chunks of WS_CHUNK bytes
  int B, T, H, NC;
  int c0, c1;          // the chunks [c0, c1) of every (batch, head) this launch covers
  float scale;
  int beta_bf16;
};

// ----------------------------------------------------------------------------
// kda_intra: chunk index = bh * NC + chunk; block = 256; any grid (its 78 KB of
// LDS and <= 256 registers per lane let two workgroups share a CU, so the host
// launches two per CU: one wave per SIMD leaves every phase latency-bound, and
// the second workgroup's phases fill those gaps; C5, same box: kda_intra
// 117.5 -> 83.5 us).  Each workgroup takes chunks blockIdx.x, blockIdx.x +
// gridDim.x, ... and loads the next chunk's g, k, v into registers once the
// current ones are staged in LDS, so those loads overlap the current chunk's
// work; q and beta are loaded at the start of their chunk (holding them too
// would exceed 256 registers).  The inputs are read once, non-temporally,
// which leaves the Infinity Cache to the workspace that kda_state reads back
// (221 -> 214 us per call).
// MFMA 16x16x32 bf16 layouts (lane l, q = l/16): A[l%16][8q+e], B[8q+e][l%16],
// D[4q+e][l%16].  MFMA 16x16x4 fp32: A[l%16][l/16], B[l/16][l%16], same D.
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void kda_intra(KdaParams p) {
  // LDS regions; the ones marked "then" are reused after a barrier.
  __shared__ __align__(16) unsigned char lds_g[KC * GP * 4];   // G log2(e), then T fp32 + R
  __shared__ __align__(16) unsigned char lds_k[KC * 136 * 2];  // k, then T bf16
  __shared__ __align__(16) unsigned char lds_v[KC * 136 * 2];  // v, then Aqk bf16
  // scan totals, then A's ten lower-triangular 16x16 blocks: block (tb, sb),
  // sb <= tb, at tb (tb + 1) / 2 + sb
  __shared__ __align__(16) float Ap[10][16][17];
  __shared__ float bet[KC];
  auto Af = [&](int t, int s) -> float& {
    const int tb = t >> 4;
    return Ap[(tb * (tb + 1) >> 1) + (s >> 4)][t & 15][s & 15];
  };

  float(*Gs)[GP] = (float(*)[GP])lds_g;
  float(*Tf)[68] = (float(*)[68])lds_g;                      // 17408 B
  float(*Rs)[16][17] = (float(*)[16][17])(lds_g + KC * 68 * 4);
  uint16_t(*Ks)[136] = (uint16_t(*)[136])lds_k;
  uint16_t(*Tb)[72] = (uint16_t(*)[72])lds_k;
  uint16_t(*Vs)[136] = (uint16_t(*)[136])lds_v;
  uint16_t(*AQs)[72] = (uint16_t(*)[72])lds_v;
  float(*tot)[KD] = (float(*)[KD]) & Ap[0][0][0];            // [8][128]

  // Lane ids are re-derived at the top of every chunk from an opaque copy of
  // the thread index, so that the compiler recomputes the per-lane addresses
  // in each chunk instead of holding them in registers across the loop (two
  // workgroups per CU leave 256 registers per lane).
  int tid, lane, wave, l16, q4, c4, seg, r0, trow;
  auto set_ids = [&] {
    tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    l16 = lane & 15;
    q4 = lane >> 4;
    c4 = tid & 31;     // channels 4 c4 .. 4 c4 + 3
    seg = tid >> 5;    // rows 8 seg .. 8 seg + 7
    r0 = 16 * wave;    // first row of this wave's 16-row block
    trow = r0 + l16;   // A-operand row of this lane
  };
  set_ids();
  const long long rs = (long long)p.H * KD;
  const long long rsv = (long long)p.H * VD;
  const u4_t z4 = {0u, 0u, 0u, 0u};
  const int nsc = p.c1 - p.c0;  // chunks per (batch, head) in this launch
  const int total = p.B * p.H * nsc;

  struct Chunk {
    int gidx;  // workspace chunk index bh * NC + chunk
    int b, h, t0, nt;
    long long base_k, base_v;
  };
  auto locate = [&](int idx) {
    Chunk c;
    const int bh = idx / nsc, chunk = p.c0 + (idx - bh * nsc);
    c.gidx = bh * p.NC + chunk;
    c.b = bh / p.H;
    c.h = bh - c.b * p.H;
    c.t0 = chunk * KC;
    c.nt = min(KC, p.T - c.t0);  // valid steps in this chunk
    c.base_k = ((long long)c.b * p.T + c.t0) * rs + (long long)c.h * KD;
    c.base_v = ((long long)c.b * p.T + c.t0) * rsv + (long long)c.h * VD;
    return c;
  };
  // input registers: g (this thread's 8 rows x 4 channels), k and v pieces,
  // this lane's q row, beta of step tid
  f4_t gv[8];
  u4_t kr[4], vr[4], qr[4];
  float bv = 0.0f;
  auto load_gkv = [&](const Chunk& c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 8 * seg + e;
      gv[e] = t < c.nt ? __builtin_nontemporal_load((const f4_t*)(p.g + c.base_k + t * rs + 4 * c4))
                       : f4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + 256 * j, row = i >> 4, c8 = i & 15;
      kr[j] = row < c.nt ? __builtin_nontemporal_load((const u4_t*)(p.k + c.base_k + row * rs + 8 * c8)) : z4;
      vr[j] = row < c.nt ? __builtin_nontemporal_load((const u4_t*)(p.v + c.base_v + row * rsv + 8 * c8)) : z4;
    }
  };
  auto load_qb = [&](const Chunk& c) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qr[ks] = trow < c.nt ? __builtin_nontemporal_load((const u4_t*)(p.q + c.base_k + trow * rs + 32 * ks + 8 * q4)) : z4;
    bv = 0.0f;
    if (tid < c.nt) {
      const long long bi = ((long long)c.b * p.T + c.t0 + tid) * p.H + c.h;
      bv = p.beta_bf16 ? bf16_bits_to_f32(((const uint16_t*)p.beta)[bi])
                       : ((const float*)p.beta)[bi];
    }
  };

  int idx = blockIdx.x;
  if (idx >= total) return;
  Chunk cur = locate(idx);
  load_gkv(cur);
  for (;;) {
  set_ids();
  load_qb(cur);
  const int nidx = idx + (int)gridDim.x;
  const bool has_next = nidx < total;
  const Chunk nxt = locate(has_next ? nidx : idx);
  const int nt = cur.nt;
  const long long base_k = cur.base_k;
  uint8_t* ws = p.ws + (size_t)cur.gidx * WS_CHUNK;

  // ---- 1. g (cumulative sum), k and v to LDS, beta ---------------------------
  if (tid < KC) bet[tid] = bv;
#pragma unroll
  for (int e = 1; e < 8; ++e) gv[e] += gv[e - 1];
  *(f4_t*)&tot[seg][4 * c4] = gv[7];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j, row = i >> 4, c8 = i & 15;
    *(u4_t*)&Ks[row][8 * c8] = kr[j];
    *(u4_t*)&Vs[row][8 * c8] = vr[j];
  }
  lds_barrier();
  {
    f4_t pre = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < seg; ++j) pre += *(const f4_t*)&tot[j][4 * c4];
#pragma unroll
    for (int e = 0; e < 8; ++e) *(f4_t*)&Gs[8 * seg + e][4 * c4] = (gv[e] + pre) * kLog2e;
  }
  if (has_next) load_gkv(nxt);  // g, k, v are in LDS now
  lds_barrier();

  // ---- 2. t-side operands, Qd, K_end^T, B^T, exp(G_C) ----------------------
  u4_t kt_op[4], qt_op[4];
  bool ok = true;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int c0 = 32 * ks + 8 * q4;
    float gt[8], gr[8], kf[8], qf[8], kt[8], qt[8], qd[8];
    load8_f32(&Gs[trow][c0], gt);
    load8_f32(&Gs[r0][c0], gr);
    unpack8_bf16(*(const u4_t*)&Ks[trow][c0], kf);
    unpack8_bf16(qr[ks], qf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = gt[e] - gr[e];
      ok &= (d >= -kExp2Range) && (d <= kExp2Range);
      const float ex = ex2(d);
      kt[e] = kf[e] * ex;
      qt[e] = p.scale * qf[e] * ex;
      qd[e] = p.scale * qf[e] * ex2(gt[e]);
    }
    kt_op[ks] = pack8_bf16(kt);
    qt_op[ks] = pack8_bf16(qt);
    *(u4_t*)(ws + WS_QD + frag_off(trow, 4 * ks + q4, 4)) = pack8_bf16(qd);
  }
  // B = [beta k e^G | beta v] as the B^T operands of step 5, made by the lanes
  // that multiply them (wave w: B^T rows c = 64 w + 16 cb + l16, steps
  // 8 q4 .. +7 and 32 + 8 q4 .. +7); waves 2 and 3 also write K_end^T (one
  // column c per thread, its 8 step groups) to the workspace, which balances
  // the exponentials between the two halves.
  u4_t bop[4][2];
  if (wave < 2) {
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const int c = 64 * wave + 16 * cb + l16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float bk[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = 32 * h + 8 * q4 + e;
          bk[e] = bet[t] * bf16_bits_to_f32(Ks[t][c]) * ex2(Gs[t][c]);
        }
        bop[cb][h] = pack8_bf16(bk);
      }
      __builtin_amdgcn_sched_barrier(0);  // (keeps each group's LDS reads with it)
    }
  } else {
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const int c = 64 * (wave - 2) + 16 * cb + l16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float bvv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = 32 * h + 8 * q4 + e;
          bvv[e] = bet[t] * bf16_bits_to_f32(Vs[t][c]);
        }
        bop[cb][h] = pack8_bf16(bvv);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    const int c = tid - 128;
    const float gend = Gs[KC - 1][c];
#pragma unroll
    for (int tg = 0; tg < 8; ++tg) {
      float ke[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = 8 * tg + e;
        ke[e] = bf16_bits_to_f32(Ks[t][c]) * ex2(gend - Gs[t][c]);
      }
      *(u4_t*)(ws + WS_KT + frag_off(c, tg, 2)) = pack8_bf16(ke);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (tid < KD) ((float*)(ws + WS_GC))[tid] = ex2(Gs[KC - 1][tid]);
  const int slow = __syncthreads_or(!ok);  // also orders Vs reads before AQs writes

  // ---- 3. A and Aqk: wave w computes rows 16w..16w+15 ----------------------
  for (int sb = 0; sb <= wave; ++sb) {
    const int srow = 16 * sb + l16;
    u4_t ks_op[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c0 = 32 * ks + 8 * q4;
      float gs[8], gr[8], kf[8], x[8];
      load8_f32(&Gs[srow][c0], gs);
      load8_f32(&Gs[r0][c0], gr);
      unpack8_bf16(*(const u4_t*)&Ks[srow][c0], kf);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = kf[e] * ex2(gr[e] - gs[e]);
      ks_op[ks] = pack8_bf16(x);
    }
    f4_t acc_a = {0.f, 0.f, 0.f, 0.f}, acc_q = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      acc_a = mfma16<true>(kt_op[ks], ks_op[ks], acc_a);
      acc_q = mfma16<true>(qt_op[ks], ks_op[ks], acc_q);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = r0 + 4 * q4 + e, s = 16 * sb + l16;
      Af(t, s) = s < t ? bet[t] * acc_a[e] : 0.0f;
      AQs[t][s] = f32_to_bf16_bits(s <= t ? acc_q[e] : 0.0f);
    }
  }
  for (int sb = wave + 1; sb < 4; ++sb)
#pragma unroll
    for (int e = 0; e < 4; ++e) AQs[r0 + 4 * q4 + e][16 * sb + l16] = 0;
  if (slow) {
    // exact pairwise exponent for the diagonal blocks (s <= t, same block)
    lds_barrier();
    for (int i = tid; i < 4 * 256; i += 256) {
      const int blk = i >> 8, tl = (i >> 4) & 15, sl = i & 15;
      if (sl > tl) continue;
      const int t = 16 * blk + tl, s = 16 * blk + sl;
      float a = 0.0f, aq = 0.0f;
      for (int c = 0; c < KD; ++c) {
        const float ex = ex2(Gs[t][c] - Gs[s][c]);
        const float ksv = bf16_bits_to_f32(Ks[s][c]) * ex;
        a += bf16_bits_to_f32(Ks[t][c]) * ksv;
        const float qv = t < nt ? bf16_bits_to_f32(p.q[base_k + t * rs + c]) : 0.0f;
        aq += qv * ksv;
      }
      if (s < t) Af(t, s) = bet[t] * a;
      AQs[t][s] = f32_to_bf16_bits(p.scale * aq);
    }
  }
  lds_barrier();

  // ---- 4. Aqk to the workspace; T = (I + A)^-1 -----------------------------
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    // fragment slot i: block i/64 = (row block, step), lane = 16 q + r
    const int i = tid + 256 * j, blk = i >> 6, ln = i & 63;
    const int row = 16 * (blk >> 1) + (ln & 15), cg = 4 * (blk & 1) + (ln >> 4);
    *(u4_t*)(ws + WS_AQ + 16 * i) = *(const u4_t*)&AQs[row][8 * cg];
  }
  if (wave == 0) {
    // diagonal blocks by forward substitution: lane = (block, column)
    const int base = 16 * q4, j = l16;
    float x[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      float acc = (m == j) ? 1.0f : 0.0f;
#pragma unroll
      for (int n = 0; n < m; ++n) acc -= Af(base + m, base + n) * x[n];
      x[m] = acc;
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) Tf[base + m][base + j] = x[m];
  }
  lds_barrier();
  // off-diagonal blocks, by distance d from the diagonal:
  //   T_ij = -T_ii sum_{m=j}^{i-1} A_im T_mj
  for (int d = 1; d < 4; ++d) {
    if (wave < 4 - d) {
      const int jb = wave, ib = wave + d;
      f4_t r = {0.f, 0.f, 0.f, 0.f};
      for (int mb = jb; mb < ib; ++mb)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          r = mfma_f32_16x16x4(Af(16 * ib + l16, 16 * mb + 4 * kk + q4),
                               Tf[16 * mb + 4 * kk + q4][16 * jb + l16], r);
#pragma unroll
      for (int e = 0; e < 4; ++e) Rs[wave][4 * q4 + e][l16] = r[e];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      f4_t tij = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        tij = mfma_f32_16x16x4(Tf[16 * ib + l16][16 * ib + 4 * kk + q4],
                               Rs[wave][4 * kk + q4][l16], tij);
#pragma unroll
      for (int e = 0; e < 4; ++e) Tf[16 * ib + 4 * q4 + e][16 * jb + l16] = -tij[e];
    }
    lds_barrier();
  }
  {
    // T to bf16 with the upper blocks zeroed
    const int row = tid >> 2, cb = (tid & 3) * 16;
    float x[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = (cb >> 4) <= (row >> 4) ? Tf[row][cb + e] : 0.0f;
    *(u4_t*)&Tb[row][cb] = pack8_bf16(x);
    *(u4_t*)&Tb[row][cb + 8] = pack8_bf16(x + 8);
  }
  lds_barrier();

  // ---- 5. W_k = T B_k, W_v = T B_v: wave w owns columns 64w..64w+63 -------
  // W_k is computed transposed (D = [column][step]) so that each lane holds 4
  // consecutive columns of one step (8 bytes of a fragment); W_v straight
  // (D = [step][column]), 4 consecutive steps of one column.
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const u4_t b0 = bop[cb][0], b1 = bop[cb][1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * i + l16;             // T row this lane reads
      const u4_t t0 = *(const u4_t*)&Tb[t][8 * q4];
      f4_t acc = {0.f, 0.f, 0.f, 0.f};
      if (wave < 2) {
        acc = mfma16<true>(b0, t0, acc);
        if (i >= 2) acc = mfma16<true>(b1, *(const u4_t*)&Tb[t][32 + 8 * q4], acc);
      } else {
        acc = mfma16<true>(t0, b0, acc);
        if (i >= 2) acc = mfma16<true>(*(const u4_t*)&Tb[t][32 + 8 * q4], b1, acc);
      }
      u2_t w;
      w.x = pack_bf16x2(acc[0], acc[1]);
      w.y = pack_bf16x2(acc[2], acc[3]);
      if (wave < 2) {
        // W_k[t][c0 .. c0+3], c0 = 64w + 16cb + 4q4
        const int c0 = 64 * wave + 16 * cb + 4 * q4;
        *(u2_t*)(ws + WS_WK + frag_off(t, c0 >> 3, 4) + 2 * (c0 & 7)) = w;
      } else {
        // W_v[t0 .. t0+3][cv], t0 = 16i + 4q4, cv = 64(w-2) + 16cb + l16
        const int cv = 64 * (wave - 2) + 16 * cb + l16, tq = 4 * i + q4;
        *(u2_t*)(ws + WS_WV + 8 * (tq * VD + cv)) = w;
      }
    }
  }
  if (!has_next) break;
  idx = nidx;
  cur = nxt;
  __syncthreads();  // every wave is done with this chunk's LDS
  }
}

// ----------------------------------------------------------------------------
// kda_state: grid = B*H*(VD/16), block = 256 (4 waves).  The workgroup owns
// value columns v0 .. v0+15 of one head and walks the chunks in order.
// Wave w holds state rows 32w .. 32w+31 (two 16x16 tiles, fp32) and computes
// U / O rows 16w .. 16w+15.  S and U are shared through LDS transposed
// ([column][row], bf16) so that B-operand reads are 16 bytes.  The chunk
// operands are read straight from the fragment-ordered workspace (one
// contiguous 1 KB per load instruction) one chunk ahead, alternating two
// register sets so that no prefetched value is ever copied (a copy would
// wait for the load).  O is computed transposed (D = [column][step]) so that
// each lane stores 4 consecutive columns.  When B*H is a multiple of 8 the 8
// column slices of a head run on one XCD and share its L2.
// ----------------------------------------------------------------------------
namespace {
struct ChunkOps {
  u4_t wk[4], qd[4], aq[2], kt[4];
  f4_t gc[2];
  u2_t wv;  // 4 raw bf16 values of W_v: converted where used
};

// The loads of one chunk in three groups, so that a step can spread them
// over its phases (the per-CU address path, not latency, bounds the step).
TM_DEV void load_chunk_a(const uint8_t* ws, int wave, int lane, ChunkOps& o) {
  const uint8_t* lw = ws + 16 * lane;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) o.wk[ks] = ldg128(lw + WS_WK + 1024 * (4 * wave + ks));
}
TM_DEV void load_chunk_b(const uint8_t* ws, int wave, int lane, int q4, int v0, ChunkOps& o) {
  const uint8_t* lw = ws + 16 * lane;
#pragma unroll
  for (int j = 0; j < 4; ++j) o.kt[j] = ldg128(lw + WS_KT + 1024 * (4 * wave + j));
  const float* gc = (const float*)(ws + WS_GC);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) o.gc[tt] = *(const f4_t*)(gc + 32 * wave + 16 * tt + 4 * q4);
  o.wv = ldg64(ws + WS_WV + 8 * ((4 * wave + q4) * VD + v0 + (lane & 15)));
}
TM_DEV void load_chunk_c(const uint8_t* ws, int wave, int lane, ChunkOps& o) {
  const uint8_t* lw = ws + 16 * lane;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) o.qd[ks] = ldg128(lw + WS_QD + 1024 * (4 * wave + ks));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) o.aq[ks] = ldg128(lw + WS_AQ + 1024 * (2 * wave + ks));
}
TM_DEV void load_chunk(const uint8_t* ws, int wave, int lane, int q4, int v0, ChunkOps& o) {
  load_chunk_a(ws, wave, lane, o);
  load_chunk_b(ws, wave, lane, q4, v0, o);
  load_chunk_c(ws, wave, lane, o);
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void kda_state(KdaParams p) {
  __shared__ __align__(16) uint16_t Sbt[2][16][KD + 8];  // S^T bf16 (double-buffered)
  __shared__ __align__(16) uint16_t Ubt[2][16][KC + 8];  // U^T bf16

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q4 = lane >> 4, l16 = lane & 15;
  constexpr int nvs = VD / 16;
  const int BH = p.B * p.H;
  int bh, vs;
  if ((BH & 7) == 0) {
    const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
    bh = x + 8 * (j >> 3);
    vs = j & 7;
  } else {
    vs = blockIdx.x % nvs;
    bh = blockIdx.x / nvs;
  }
  const int b = bh / p.H, h = bh - b * p.H;
  const int v0 = vs * 16;
  const long long rsv = (long long)p.H * VD;

  // state tiles: rows 32w + 16tt + 4q4 + e, column v0 + l16
  f4_t S[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 32 * wave + 16 * tt + 4 * q4 + e;
      S[tt][e] = p.s0 ? p.s0[((long long)bh * KD + row) * VD + v0 + l16] : 0.0f;
    }

  const uint8_t* wsh = p.ws + (size_t)bh * p.NC * WS_CHUNK;
  // One chunk step: consume `cur` (chunk c) and start loading chunk c+1
  // into `nxt`.
  auto step = [&](const int c, auto bufc, const ChunkOps& cur, ChunkOps& nxt) {
    constexpr int BUF = decltype(bufc)::value;
    const uint8_t* wsn = wsh + (size_t)min(c + 1, p.c1 - 1) * WS_CHUNK;
    load_chunk_a(wsn, wave, lane, nxt);
    asm volatile("" ::: "memory");  // issue points of the next chunk's loads stay spread

    // (a) S -> LDS as S^T bf16
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int row = 32 * wave + 16 * tt + 4 * q4;
      u2_t w;
      w.x = pack_bf16x2(S[tt][0], S[tt][1]);
      w.y = pack_bf16x2(S[tt][2], S[tt][3]);
      *(u2_t*)(&Sbt[BUF][l16][row]) = w;
    }
    lds_barrier();
    load_chunk_b(wsn, wave, lane, q4, v0, nxt);
    asm volatile("" ::: "memory");

    // (b) U rows 16w.. : U = W_v - W_k S; O^T = S^T Qd^T (first part)
    u4_t sb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sb[ks] = *(const u4_t*)(&Sbt[BUF][l16][32 * ks + 8 * q4]);
    f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma16<true>(cur.wk[ks], sb[ks], acc);
    const float wv[4] = {__uint_as_float(cur.wv.x << 16), __uint_as_float(cur.wv.x & 0xffff0000u),
                         __uint_as_float(cur.wv.y << 16), __uint_as_float(cur.wv.y & 0xffff0000u)};
    {
      u2_t w;
      w.x = pack_bf16x2(wv[0] - acc[0], wv[1] - acc[1]);
      w.y = pack_bf16x2(wv[2] - acc[2], wv[3] - acc[3]);
      *(u2_t*)(&Ubt[BUF][l16][16 * wave + 4 * q4]) = w;
    }
    f4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) o = mfma16<true>(sb[ks], cur.qd[ks], o);
    lds_barrier();
    load_chunk_c(wsn, wave, lane, nxt);
    asm volatile("" ::: "memory");

    // (c) O^T += U^T Aqk^T; lane holds O[t][v0 + 4q4 .. +3], t = 64c + 16w + l16
    u4_t ub[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) ub[ks] = *(const u4_t*)(&Ubt[BUF][l16][32 * ks + 8 * q4]);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) o = mfma16<true>(ub[ks], cur.aq[ks], o);
    {
      const int t = c * KC + 16 * wave + l16;
      u2_t w;
      w.x = pack_bf16x2(o[0], o[1]);
      w.y = pack_bf16x2(o[2], o[3]);
      if (t < p.T)
        *(u2_t*)(p.o + ((long long)b * p.T + t) * rsv + (long long)h * VD + v0 + 4 * q4) = w;
    }

    // (d) S = diag(exp(G_C)) S + K_end^T U
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      S[tt] *= cur.gc[tt];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) S[tt] = mfma16<true>(cur.kt[2 * tt + ks], ub[ks], S[tt]);
    }
  };
  ChunkOps ops0, ops1;
  if (p.c1 > p.c0) load_chunk(wsh + (size_t)p.c0 * WS_CHUNK, wave, lane, q4, v0, ops0);
  // pairs of steps with no branch between them, so that each operand set
  // keeps its registers around the loop; an odd last chunk after the loop
  int c = p.c0;
  for (; c + 1 < p.c1; c += 2) {
    step(c, std::integral_constant<int, 0>(), ops0, ops1);
    step(c + 1, std::integral_constant<int, 1>(), ops1, ops0);
  }
  if (c < p.c1) step(c, std::integral_constant<int, 0>(), ops0, ops1);

  if (p.st) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 32 * wave + 16 * tt + 4 * q4 + e;
        p.st[((long long)bh * KD + row) * VD + v0 + l16] = S[tt][e];
      }
  }
}

// ----------------------------------------------------------------------------
// kda_recurrent: the token-by-token form of the same rule (decode: one or a
// few new tokens continuing from a state, e.g. the chunked kernel's final
// state).  grid = B*H*(VD/16), block = 64 (one wave).  The wave owns value
// columns v0 .. v0+15 of one head (64-byte pieces of each state row): lane
// 16 rg + c holds S[32 rg + r][v0 + c] (r < 32) in registers for all steps,
// so both reductions over the key dimension (S^T k and S^T q) are 32 in-lane
// FMAs and two shuffles.  The state is read and written once per call,
// non-temporal: a call streams every state through once, and keeping the
// reads and the write-backs out of the caches halves their interference
// (B=16, H=16, one token: 14.4 -> 11.2 us).
// Per step t:  S <- diag(exp(g_t)) S;  u = beta_t (v_t - S^T k_t);
//              S <- S + k_t u^T;       o_t = S^T (scale q_t).
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(64) void kda_recurrent(KdaParams p) {
  constexpr int CW = 16, RL = KD / (64 / CW);  // columns per wave, rows per lane
  const int lane = threadIdx.x, c = lane & (CW - 1), rg = lane / CW;
  const int vb = blockIdx.x % (VD / CW), bh = blockIdx.x / (VD / CW);
  const int b = bh / p.H, h = bh - b * p.H;
  const int col = CW * vb + c, i0 = RL * rg;
  const size_t sb = (size_t)bh * KD * VD;
  float S[RL];
#pragma unroll
  for (int r = 0; r < RL; ++r)
    S[r] = p.s0 ? __builtin_nontemporal_load(p.s0 + sb + (size_t)(i0 + r) * VD + col) : 0.0f;
  const long long rs = (long long)p.H * KD, rsv = (long long)p.H * VD;
  for (int t = 0; t < p.T; ++t) {
    const long long tk = ((long long)b * p.T + t) * rs + (long long)h * KD + i0;
    const long long tv = ((long long)b * p.T + t) * rsv + (long long)h * VD;
    float kf[RL], qf[RL], gd[RL];
#pragma unroll
    for (int j = 0; j < RL / 8; ++j) {
      unpack8_bf16(ldg128(p.k + tk + 8 * j), kf + 8 * j);
      unpack8_bf16(ldg128(p.q + tk + 8 * j), qf + 8 * j);
      load8_f32(p.g + tk + 8 * j, gd + 8 * j);
    }
    const long long bi = ((long long)b * p.T + t) * p.H + h;
    const float beta = p.beta_bf16 ? bf16_bits_to_f32(((const uint16_t*)p.beta)[bi])
                                   : ((const float*)p.beta)[bi];
    const float vj = bf16_bits_to_f32(p.v[tv + col]);
    float dot = 0.0f;
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      S[r] *= ex2(gd[r] * kLog2e);
      dot = __builtin_fmaf(S[r], kf[r], dot);
    }
#pragma unroll
    for (int o = CW; o < 64; o <<= 1) dot += __shfl_xor(dot, o, 64);
    const float u = beta * (vj - dot);
    float od = 0.0f;
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      S[r] = __builtin_fmaf(kf[r], u, S[r]);
      od = __builtin_fmaf(S[r], qf[r], od);
    }
#pragma unroll
    for (int o = CW; o < 64; o <<= 1) od += __shfl_xor(od, o, 64);
    if (rg == 0) p.o[tv + col] = f32_to_bf16_bits(od * p.scale);
  }
  if (p.st) {
#pragma unroll
    for (int r = 0; r < RL; ++r)
      __builtin_nontemporal_store(S[r], p.st + sb + (size_t)(i0 + r) * VD + col);
  }
}

// kda_recurrent_v4: the same recurrence for 16-byte aligned state buffers.
// A wave owns two 16-column slices (grid = B*H*(VD/32)); lane 4 rg + cq keeps
// S[8 rg + r][v0 + 4 cq + e] (r < 8, e < 4) of each, so every state row piece
// of 16 bytes moves in one access (8 loads and 8 stores per lane and slice
// instead of 32), and the reductions over the key dimension are 8 in-lane
// FMAs per column and four shuffles.  Both slices' state loads are issued
// first, and the first slice is updated and stored while the second is still
// arriving (B=16, H=16, one token, same box: 11.15 -> 10.8 us; four slices
// per wave measured slower).
extern "C" __global__ __launch_bounds__(64) void kda_recurrent_v4(KdaParams p) {
  constexpr int CW = 16, RL = 8, NSL = 2;
  const int lane = threadIdx.x, cq = lane & 3, rg = lane >> 2;
  const int vp = blockIdx.x % (VD / CW / NSL), bh = blockIdx.x / (VD / CW / NSL);
  const int b = bh / p.H, h = bh - b * p.H;
  const int i0 = RL * rg;
  const size_t sb = (size_t)bh * KD * VD;
  f4_t S[NSL][RL];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int col = CW * (NSL * vp + sl) + 4 * cq;
      S[sl][r] = p.s0 ? __builtin_nontemporal_load((const f4_t*)(p.s0 + sb + (size_t)(i0 + r) * VD + col))
                      : f4_t{0.f, 0.f, 0.f, 0.f};
    }
  const long long rs = (long long)p.H * KD, rsv = (long long)p.H * VD;
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    const int col = CW * (NSL * vp + sl) + 4 * cq;
    for (int t = 0; t < p.T; ++t) {
      const long long tk = ((long long)b * p.T + t) * rs + (long long)h * KD + i0;
      const long long tv = ((long long)b * p.T + t) * rsv + (long long)h * VD;
      float kf[RL], qf[RL], gd[RL];
      unpack8_bf16(ldg128(p.k + tk), kf);
      unpack8_bf16(ldg128(p.q + tk), qf);
      load8_f32(p.g + tk, gd);
      const long long bi = ((long long)b * p.T + t) * p.H + h;
      const float beta = p.beta_bf16 ? bf16_bits_to_f32(((const uint16_t*)p.beta)[bi])
                                     : ((const float*)p.beta)[bi];
      const u2_t vw = ldg64(p.v + tv + col);
      const float vj[4] = {bf16_bits_to_f32(vw.x & 0xFFFFu), bf16_bits_to_f32(vw.x >> 16),
                           bf16_bits_to_f32(vw.y & 0xFFFFu), bf16_bits_to_f32(vw.y >> 16)};
      float dot[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < RL; ++r) {
        const float dec = ex2(gd[r] * kLog2e);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          S[sl][r][e] *= dec;
          dot[e] = __builtin_fmaf(S[sl][r][e], kf[r], dot[e]);
        }
      }
#pragma unroll
      for (int o = 4; o < 64; o <<= 1)
#pragma unroll
        for (int e = 0; e < 4; ++e) dot[e] += __shfl_xor(dot[e], o, 64);
      float u[4], od[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) u[e] = beta * (vj[e] - dot[e]);
#pragma unroll
      for (int r = 0; r < RL; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          S[sl][r][e] = __builtin_fmaf(kf[r], u[e], S[sl][r][e]);
          od[e] = __builtin_fmaf(S[sl][r][e], qf[r], od[e]);
        }
#pragma unroll
      for (int o = 4; o < 64; o <<= 1)
#pragma unroll
        for (int e = 0; e < 4; ++e) od[e] += __shfl_xor(od[e], o, 64);
      if (rg == 0)
#pragma unroll
        for (int e = 0; e < 4; ++e) p.o[tv + col + e] = f32_to_bf16_bits(od[e] * p.scale);
    }
    if (p.st)
#pragma unroll
      for (int r = 0; r < RL; ++r)
        __builtin_nontemporal_store(S[sl][r], (f4_t*)(p.st + sb + (size_t)(i0 + r) * VD + col));
  }
}
