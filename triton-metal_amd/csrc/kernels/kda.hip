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
// its 16 bytes at 16 l - so every load there is one contiguous 1 KB.  The 16
// bytes hold row r, columns 4q..4q+3 and 16+4q..16+4q+3 of the step: the
// reduction index of every product kda_state runs is taken in that order, in
// which the rows 4q+e of two vertically adjacent 16x16 MFMA results are
// exactly the 8 reduction positions 8q..8q+7 that lane 16q + n supplies as a
// B operand; so a result feeds the next product from the lane's own
// registers.
constexpr size_t WS_WK = 0;                    // -W_k [64][128]     fragments (16 blocks)
constexpr size_t WS_WV = WS_WK + KC * KD * 2;  // W_v [64/4][128][4] (4 steps of a column together)
constexpr size_t WS_QD = WS_WV + KC * VD * 2;  // scale q exp(G) [64][128] fragments
constexpr size_t WS_KT = WS_QD + KC * KD * 2;  // (k exp(G_C - G))^T [128][64] fragments
constexpr size_t WS_AQ = WS_KT + KD * KC * 2;  // Aqk [64][64]       fragments (8 blocks)
constexpr size_t WS_GC = WS_AQ + KC * KC * 2;  // exp(G_C), fp32 [128]
constexpr size_t WS_CHUNK = WS_GC + KD * 4;
static_assert(WS_CHUNK == 74240, "workspace layout is part of the C ABI");

// Byte offset of (row, 4-column group c4 = columns 4c4..4c4+3) of a matrix
// with `steps` 32-column steps per row, stored in fragment order: in step
// c4/8, group c4%8 = 4h + q goes to lane 16q + row%16, bytes 8h..8h+7.
TM_DEV int frag_off(int row, int c4, int steps) {
  return (((row >> 4) * steps + (c4 >> 3)) * 64 + (c4 & 3) * 16 + (row & 15)) * 16 +
         8 * ((c4 >> 2) & 1);
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
    const u4_t qp = pack8_bf16(qd);
    *(u2_t*)(ws + WS_QD + frag_off(trow, 8 * ks + 2 * q4, 4)) = u2_t{qp.x, qp.y};
    *(u2_t*)(ws + WS_QD + frag_off(trow, 8 * ks + 2 * q4 + 1, 4)) = u2_t{qp.z, qp.w};
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
      const u4_t kp = pack8_bf16(ke);
      *(u2_t*)(ws + WS_KT + frag_off(c, 2 * tg, 2)) = u2_t{kp.x, kp.y};
      *(u2_t*)(ws + WS_KT + frag_off(c, 2 * tg + 1, 2)) = u2_t{kp.z, kp.w};
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
    // fragment slot i: block i/64 = (row block, step), lane = 16 q + r;
    // columns 32 step + 4q .. +3 and 32 step + 16 + 4q .. +3
    const int i = tid + 256 * j, blk = i >> 6, ln = i & 63;
    const int row = 16 * (blk >> 1) + (ln & 15), c = 32 * (blk & 1) + 4 * (ln >> 4);
    const u2_t lo = *(const u2_t*)&AQs[row][c], hi = *(const u2_t*)&AQs[row][c + 16];
    *(u4_t*)(ws + WS_AQ + 16 * i) = u4_t{lo.x, lo.y, hi.x, hi.y};
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
        // -W_k[t][c0 .. c0+3], c0 = 64w + 16cb + 4q4 (sign bits flipped:
        // kda_state accumulates U = W_v + (-W_k) S onto W_v)
        const int c0 = 64 * wave + 16 * cb + 4 * q4;
        *(u2_t*)(ws + WS_WK + frag_off(t, c0 >> 2, 4)) = w ^ 0x80008000u;
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
// kda_state: grid = B*H*(VD/16), block = 192 (3 waves).  The workgroup owns
// value columns v0 .. v0+15 of one head and walks the chunks in order.
//  * Wave 0 runs the recurrence alone, in registers: it holds the whole
//    128 x 16 state S (eight 16x16 fp32 MFMA results) and, per chunk,
//        U = W_v - W_k S        (16 MFMAs: 4 row blocks x 4 steps)
//        S = diag(exp(G_C)) S + K_end^T U     (16 MFMAs: 8 x 2)
//    Because the workspace takes the reduction index in the order of the
//    MFMA result rows (see the layout above), the bf16 B operand of each
//    product is just the previous result packed in the lane's own registers:
//    no LDS round trip and no barrier sits on the recurrence.  U accumulates
//    onto W_v with the workspace's -W_k, and its operands come from LDS: the
//    next chunk's W_k, exp(G_C) and W_v are read into the registers the U
//    products have freed while the state update runs.
//  * Wave 2 copies those operands (W_k, K_end^T, the slice of W_v, exp(G_C):
//    35 copies of 1 KB) global -> LDS three chunks ahead into a ring of four
//    slots, waiting on its own copies only, so that no load of the
//    recurrence's wave waits for memory.
//  * Wave 1 computes the output O = Qd S + Aqk U of the chunk from the
//    packed S and U operands wave 0 leaves in LDS (double-buffered), one
//    chunk behind, on another SIMD; its own operands (Qd, Aqk) load into
//    registers one chunk ahead.  O is computed transposed (D = [column][step])
//    so that each lane stores 4 consecutive columns.
// One barrier per chunk (and one before the first) orders the three: at
// barrier c wave 0 has written chunk c's S and U operands, and wave 2's copies
// of chunk c+2 have landed.  When B*H is a multiple of 8 the 8 column slices
// of a head run on one XCD and share its L2.
// ----------------------------------------------------------------------------
namespace {
// One ring slot: W_k fragments, K_end^T fragments, W_v rows [16 groups of 4
// steps][16 columns][4], exp(G_C) (twice; the second copy is padding).
constexpr int SL_WK = 0, SL_KT = 16384, SL_WV = 32768, SL_GC = 34816, SL_BYTES = 35840;
constexpr int kStateCopies = 35;  // copy instructions per chunk and slot

struct OutOps {
  u4_t qd[16];  // Qd block (row block to, step ks) at 4 to + ks
  u4_t aq[8];   // Aqk block (row block to, step ks) at 2 to + ks
};
TM_DEV void load_out(const uint8_t* ws, int lane, OutOps& o) {
  const uint8_t* lw = ws + 16 * lane;
#pragma unroll
  for (int i = 0; i < 16; ++i) o.qd[i] = ldg128(lw + WS_QD + 1024 * i);
#pragma unroll
  for (int i = 0; i < 8; ++i) o.aq[i] = ldg128(lw + WS_AQ + 1024 * i);
}
// The bf16 B operand of rows 32j .. 32j+31 of a stack of 16x16 results:
// blocks 2j and 2j+1, rows 4q+e of each.
TM_DEV u4_t pack_pair(f4_t a, f4_t b) {
  u4_t r;
  r.x = pack_bf16x2(a[0], a[1]);
  r.y = pack_bf16x2(a[2], a[3]);
  r.z = pack_bf16x2(b[0], b[1]);
  r.w = pack_bf16x2(b[2], b[3]);
  return r;
}
}  // namespace

extern "C" __global__ __launch_bounds__(192) void kda_state(KdaParams p) {
  __shared__ __align__(16) unsigned char ring[4][SL_BYTES];  // wave 0's operands
  __shared__ __align__(16) u4_t Sx[2][4][64];  // packed S operands, by chunk parity
  __shared__ __align__(16) u4_t Ux[2][2][64];  // packed U operands

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  const uint8_t* wsh = p.ws + (size_t)bh * p.NC * WS_CHUNK;
  auto chunk_ws = [&](int c) { return wsh + (size_t)min(c, p.c1 - 1) * WS_CHUNK; };

  if (wave == 0) {
    // ---- the recurrence --------------------------------------------------
    f4_t S[8];  // rows 16 tt + 4 q4 + e, column v0 + l16
#pragma unroll
    for (int tt = 0; tt < 8; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * tt + 4 * q4 + e;
        S[tt][e] = p.s0 ? p.s0[((long long)bh * KD + row) * VD + v0 + l16] : 0.0f;
      }
    lds_barrier();  // the first two chunks' operands have landed
    // this chunk's -W_k, exp(G_C), W_v (read one chunk ahead)
    u4_t wk[16];
    f4_t gc[8];
    u2_t wv[4];
    auto read_ahead = [&](const unsigned char* sl) {
#pragma unroll
      for (int i = 0; i < 16; ++i) wk[i] = *(const u4_t*)(sl + SL_WK + 1024 * i + 16 * lane);
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) gc[tt] = *(const f4_t*)(sl + SL_GC + 4 * (16 * tt + 4 * q4));
#pragma unroll
      for (int tu = 0; tu < 4; ++tu)
        wv[tu] = *(const u2_t*)(sl + SL_WV + 128 * (4 * tu + q4) + 8 * l16);
    };
    if (p.c1 > p.c0) read_ahead(ring[p.c0 & 3]);
    for (int c = p.c0; c < p.c1; ++c) {
      const int par = c & 1;
      const unsigned char* sl = ring[c & 3];
      u4_t sb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) sb[ks] = pack_pair(S[2 * ks], S[2 * ks + 1]);
      f4_t u[4];
#pragma unroll
      for (int tu = 0; tu < 4; ++tu) {
        const u2_t w = wv[tu];
        u[tu] = f4_t{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                     __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int tu = 0; tu < 4; ++tu) u[tu] = mfma16<true>(wk[4 * tu + ks], sb[ks], u[tu]);
      u4_t kt[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) kt[i] = *(const u4_t*)(sl + SL_KT + 1024 * i + 16 * lane);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) Sx[par][ks][lane] = sb[ks];
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) S[tt] *= gc[tt];
      u4_t ub[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ub[ks] = pack_pair(u[2 * ks], u[2 * ks + 1]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) S[tt] = mfma16<true>(kt[2 * tt + ks], ub[ks], S[tt]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) Ux[par][ks][lane] = ub[ks];
      if (c + 1 < p.c1) read_ahead(ring[(c + 1) & 3]);
      lds_barrier();  // chunk c's S and U are in LDS for wave 1
    }
    if (p.st) {
#pragma unroll
      for (int tt = 0; tt < 8; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * tt + 4 * q4 + e;
          p.st[((long long)bh * KD + row) * VD + v0 + l16] = S[tt][e];
        }
    }
  } else if (wave == 2) {
    // ---- wave 0's operands, global -> LDS, two chunks ahead ---------------
    // lane offsets: 1 KB fragment blocks; W_v rows of the slice (16 pieces
    // of 128 B, lane l of copy j takes piece 8j + l/8); exp(G_C) (lanes
    // 32..63 repeat lanes 0..31 into the padding)
    const uint32_t o16 = 16 * lane;
    const uint32_t owv0 = WS_WV + 8 * ((lane >> 3) * VD + v0) + 16 * (lane & 7);
    const uint32_t owv1 = owv0 + 8 * 8 * VD;
    const uint32_t ogc = WS_GC + 16 * (lane & 31);
    auto copy = [&](int c) {
      const uint8_t* src = chunk_ws(c);
      const uint32_t dst = lds_off(ring[c & 3]);
#pragma unroll
      for (int i = 0; i < 16; ++i) dma16s(src, WS_WK + 1024 * i + o16, dst + SL_WK + 1024 * i);
#pragma unroll
      for (int i = 0; i < 16; ++i) dma16s(src, WS_KT + 1024 * i + o16, dst + SL_KT + 1024 * i);
      dma16s(src, owv0, dst + SL_WV);
      dma16s(src, owv1, dst + SL_WV + 1024);
      dma16s(src, ogc, dst + SL_GC);
    };
    if (p.c1 > p.c0) copy(p.c0);
    if (p.c0 + 1 < p.c1) copy(p.c0 + 1);
    if (p.c0 + 2 < p.c1) {
      copy(p.c0 + 2);
      wait_vm<kStateCopies>();  // chunks c0 and c0+1 have landed
    } else {
      wait_vm<0>();
    }
    asm volatile("s_barrier" ::: "memory");
    for (int c = p.c0; c < p.c1; ++c) {
      // slot (c+3) % 4 was last read by wave 0 in chunk c-1, before barrier
      // c-1; wave 0 reads chunk c+2's slot after barrier c
      if (c + 3 < p.c1) {
        copy(c + 3);
        wait_vm<kStateCopies>();  // chunk c+2's copies have landed
      } else {
        wait_vm<0>();
      }
      asm volatile("s_barrier" ::: "memory");
    }
  } else {
    // ---- the output, one chunk behind ------------------------------------
    lds_barrier();
    auto out = [&](const int c, const OutOps& cur, OutOps& nxt) {
      const int par = c & 1;
      load_out(chunk_ws(c + 1), lane, nxt);
      lds_barrier();  // wave 0 has left chunk c's operands
      u4_t sb[4], ub[2];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) sb[ks] = Sx[par][ks][lane];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ub[ks] = Ux[par][ks][lane];
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        f4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) o = mfma16<true>(sb[ks], cur.qd[4 * to + ks], o);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) o = mfma16<true>(ub[ks], cur.aq[2 * to + ks], o);
        // lane holds O[t][v0 + 4 q4 .. +3], t = 64 c + 16 to + l16
        const int t = c * KC + 16 * to + l16;
        u2_t w;
        w.x = pack_bf16x2(o[0], o[1]);
        w.y = pack_bf16x2(o[2], o[3]);
        if (t < p.T)
          *(u2_t*)(p.o + ((long long)b * p.T + t) * rsv + (long long)h * VD + v0 + 4 * q4) = w;
      }
    };
    OutOps ops0, ops1;
    if (p.c1 > p.c0) load_out(chunk_ws(p.c0), lane, ops0);
    int c = p.c0;
    for (; c + 1 < p.c1; c += 2) {
      out(c, ops0, ops1);
      out(c + 1, ops1, ops0);
    }
    if (c < p.c1) out(c, ops0, ops1);
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
    dot = fold_swap<16>(dot, dot);
    dot = fold_swap<32>(dot, dot);
    const float u = beta * (vj - dot);
    float od = 0.0f;
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      S[r] = __builtin_fmaf(kf[r], u, S[r]);
      od = __builtin_fmaf(S[r], qf[r], od);
    }
    od = fold_swap<16>(od, od);
    od = fold_swap<32>(od, od);
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
// FMAs per column and four cross-lane steps (two DPP row rotations, two
// permlane swaps).  Both slices' state loads are issued
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
      for (int e = 0; e < 4; ++e) {
        dot[e] = sum_bits23(dot[e]);
        dot[e] = fold_swap<16>(dot[e], dot[e]);
        dot[e] = fold_swap<32>(dot[e], dot[e]);
      }
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
      // transposed fold of the 4 column sums: lane bit 5 picks columns
      // {0, 1} / {2, 3}, bit 4 one of those, then the sum over bits 2 and 3
      const float oe = sum_bits23(
          fold_swap<16>(fold_swap<32>(od[0], od[2]), fold_swap<32>(od[1], od[3])));
      if ((lane & 12) == 0)
        p.o[tv + col + 2 * ((lane >> 5) & 1) + ((lane >> 4) & 1)] = f32_to_bf16_bits(oe * p.scale);
    }
    if (p.st)
#pragma unroll
      for (int r = 0; r < RL; ++r)
        __builtin_nontemporal_store(S[sl][r], (f4_t*)(p.st + sb + (size_t)(i0 + r) * VD + col));
  }
}
