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
#include "common.h"

namespace {
constexpr int KC = 64;    // chunk length
constexpr int KD = 128;   // key dim
constexpr int VD = 128;   // value dim
constexpr float kExpRange = 80.0f;

// Workspace of one (head, chunk), bytes.
constexpr size_t WS_WK = 0;                    // bf16 [64][128]  W_k
constexpr size_t WS_WV = WS_WK + KC * KD * 2;  // bf16 [64][128]  W_v
constexpr size_t WS_QD = WS_WV + KC * VD * 2;  // bf16 [64][128]  scale q exp(G)
constexpr size_t WS_KT = WS_QD + KC * KD * 2;  // bf16 [128][64]  (k exp(G_C - G))^T
constexpr size_t WS_AQ = WS_KT + KD * KC * 2;  // bf16 [64][64]   Aqk
constexpr size_t WS_GC = WS_AQ + KC * KC * 2;  // fp32 [128]      exp(G_C)
constexpr size_t WS_CHUNK = WS_GC + KD * 4;
static_assert(WS_CHUNK == 74240, "workspace layout is part of the C ABI");

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
  float scale;
  int beta_bf16;
};

// ----------------------------------------------------------------------------
// kda_intra: grid = B*H*NC (block index = bh * NC + chunk), block = 256.
// MFMA 16x16x32 bf16 layouts (lane l, q = l/16): A[l%16][8q+e], B[8q+e][l%16],
// D[4q+e][l%16].  MFMA 16x16x4 fp32: A[l%16][l/16], B[l/16][l%16], same D.
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void kda_intra(KdaParams p) {
  // LDS regions; the ones marked "then" are reused after a barrier.
  __shared__ __align__(16) unsigned char lds_g[KC * KD * 4];   // G, then T fp32 + R
  __shared__ __align__(16) unsigned char lds_k[KC * 136 * 2];  // k, then T bf16
  __shared__ __align__(16) unsigned char lds_v[KC * 136 * 2];  // v, then Aqk bf16
  __shared__ __align__(16) float Af[KC][68];                   // scan totals, then A
  __shared__ __align__(16) uint16_t Bt[KD + VD][72];           // [beta k e^G | beta v]^T
  __shared__ float bet[KC];

  float(*Gs)[KD] = (float(*)[KD])lds_g;
  float(*Tf)[68] = (float(*)[68])lds_g;                      // 17408 B
  float(*Rs)[16][17] = (float(*)[16][17])(lds_g + KC * 68 * 4);
  uint16_t(*Ks)[136] = (uint16_t(*)[136])lds_k;
  uint16_t(*Tb)[72] = (uint16_t(*)[72])lds_k;
  uint16_t(*Vs)[136] = (uint16_t(*)[136])lds_v;
  uint16_t(*AQs)[72] = (uint16_t(*)[72])lds_v;
  float(*tot)[KD] = (float(*)[KD]) & Af[0][0];               // [8][128]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, q4 = lane >> 4;
  const int chunk = blockIdx.x % p.NC, bh = blockIdx.x / p.NC;
  const int b = bh / p.H, h = bh - b * p.H;
  const int t0 = chunk * KC;
  const int nt = min(KC, p.T - t0);  // valid steps in this chunk
  const long long rs = (long long)p.H * KD;
  const long long rsv = (long long)p.H * VD;
  const long long base_k = ((long long)b * p.T + t0) * rs + (long long)h * KD;
  const long long base_v = ((long long)b * p.T + t0) * rsv + (long long)h * VD;
  uint8_t* ws = p.ws + (size_t)blockIdx.x * WS_CHUNK;
  const u4_t z4 = {0u, 0u, 0u, 0u};

  // ---- 1. loads: g (cumulative sum), k and v to LDS, q rows, beta ---------
  const int c4 = tid & 31, seg = tid >> 5;  // channels 4c4.., rows 8seg..8seg+7
  f4_t gv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int t = 8 * seg + e;
    gv[e] = t < nt ? *(const f4_t*)(p.g + base_k + t * rs + 4 * c4) : f4_t{0.f, 0.f, 0.f, 0.f};
  }
  u4_t kr[4], vr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j, row = i >> 4, c8 = i & 15;
    kr[j] = row < nt ? ldg128(p.k + base_k + row * rs + 8 * c8) : z4;
    vr[j] = row < nt ? ldg128(p.v + base_v + row * rsv + 8 * c8) : z4;
  }
  const int r0 = 16 * wave;     // first row of this wave's 16-row block
  const int trow = r0 + l16;    // A-operand row of this lane
  u4_t qr[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qr[ks] = trow < nt ? ldg128(p.q + base_k + trow * rs + 32 * ks + 8 * q4) : z4;
  if (tid < KC) {
    float bv = 0.0f;
    if (tid < nt) {
      const long long bi = ((long long)b * p.T + t0 + tid) * p.H + h;
      bv = p.beta_bf16 ? bf16_bits_to_f32(((const uint16_t*)p.beta)[bi])
                       : ((const float*)p.beta)[bi];
    }
    bet[tid] = bv;
  }
#pragma unroll
  for (int e = 1; e < 8; ++e) gv[e] += gv[e - 1];
  *(f4_t*)&tot[seg][4 * c4] = gv[7];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j, row = i >> 4, c8 = i & 15;
    *(u4_t*)&Ks[row][8 * c8] = kr[j];
    *(u4_t*)&Vs[row][8 * c8] = vr[j];
  }
  __syncthreads();
  {
    f4_t pre = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < seg; ++j) pre += *(const f4_t*)&tot[j][4 * c4];
#pragma unroll
    for (int e = 0; e < 8; ++e) *(f4_t*)&Gs[8 * seg + e][4 * c4] = gv[e] + pre;
  }
  __syncthreads();

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
      ok &= (d >= -kExpRange) && (d <= kExpRange);
      const float ex = __expf(d);
      kt[e] = kf[e] * ex;
      qt[e] = p.scale * qf[e] * ex;
      qd[e] = p.scale * qf[e] * __expf(gt[e]);
    }
    kt_op[ks] = pack8_bf16(kt);
    qt_op[ks] = pack8_bf16(qt);
    *(u4_t*)(ws + WS_QD + 2 * (trow * KD + c0)) = pack8_bf16(qd);
  }
  // (c, 8-step group) tasks: K_end^T to the workspace, B^T to LDS
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j, c = i & 127, tg = i >> 7;
    const float gend = Gs[KC - 1][c];
    float ke[8], bk[8], bvv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 8 * tg + e;
      const float kf = bf16_bits_to_f32(Ks[t][c]);
      const float gtc = Gs[t][c];
      ke[e] = kf * __expf(gend - gtc);
      bk[e] = bet[t] * kf * __expf(gtc);
      bvv[e] = bet[t] * bf16_bits_to_f32(Vs[t][c]);
    }
    *(u4_t*)(ws + WS_KT + 2 * (c * KC + 8 * tg)) = pack8_bf16(ke);
    *(u4_t*)&Bt[c][8 * tg] = pack8_bf16(bk);
    *(u4_t*)&Bt[KD + c][8 * tg] = pack8_bf16(bvv);
  }
  if (tid < KD) ((float*)(ws + WS_GC))[tid] = __expf(Gs[KC - 1][tid]);
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
      for (int e = 0; e < 8; ++e) x[e] = kf[e] * __expf(gr[e] - gs[e]);
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
      Af[t][s] = s < t ? bet[t] * acc_a[e] : 0.0f;
      AQs[t][s] = f32_to_bf16_bits(s <= t ? acc_q[e] : 0.0f);
    }
  }
  for (int sb = wave + 1; sb < 4; ++sb)
#pragma unroll
    for (int e = 0; e < 4; ++e) AQs[r0 + 4 * q4 + e][16 * sb + l16] = 0;
  if (slow) {
    // exact pairwise exponent for the diagonal blocks (s <= t, same block)
    __syncthreads();
    for (int i = tid; i < 4 * 256; i += 256) {
      const int blk = i >> 8, tl = (i >> 4) & 15, sl = i & 15;
      if (sl > tl) continue;
      const int t = 16 * blk + tl, s = 16 * blk + sl;
      float a = 0.0f, aq = 0.0f;
      for (int c = 0; c < KD; ++c) {
        const float ex = __expf(Gs[t][c] - Gs[s][c]);
        const float ksv = bf16_bits_to_f32(Ks[s][c]) * ex;
        a += bf16_bits_to_f32(Ks[t][c]) * ksv;
        const float qv = t < nt ? bf16_bits_to_f32(p.q[base_k + t * rs + c]) : 0.0f;
        aq += qv * ksv;
      }
      if (s < t) Af[t][s] = bet[t] * a;
      AQs[t][s] = f32_to_bf16_bits(p.scale * aq);
    }
  }
  __syncthreads();

  // ---- 4. Aqk to the workspace; T = (I + A)^-1 -----------------------------
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = tid + 256 * j, row = i >> 3, c8 = i & 7;
    *(u4_t*)(ws + WS_AQ + 2 * (row * KC + 8 * c8)) = *(const u4_t*)&AQs[row][8 * c8];
  }
  if (wave == 0) {
    // diagonal blocks by forward substitution: lane = (block, column)
    const int base = 16 * q4, j = l16;
    float x[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      float acc = (m == j) ? 1.0f : 0.0f;
#pragma unroll
      for (int n = 0; n < m; ++n) acc -= Af[base + m][base + n] * x[n];
      x[m] = acc;
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) Tf[base + m][base + j] = x[m];
  }
  __syncthreads();
  // off-diagonal blocks, by distance d from the diagonal:
  //   T_ij = -T_ii sum_{m=j}^{i-1} A_im T_mj
  for (int d = 1; d < 4; ++d) {
    if (wave < 4 - d) {
      const int jb = wave, ib = wave + d;
      f4_t r = {0.f, 0.f, 0.f, 0.f};
      for (int mb = jb; mb < ib; ++mb)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          r = mfma_f32_16x16x4(Af[16 * ib + l16][16 * mb + 4 * kk + q4],
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
    __syncthreads();
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
  __syncthreads();

  // ---- 5. [W_k | W_v]^T = B^T T^T: wave w owns columns 64w..64w+63 --------
  uint16_t* wout = (uint16_t*)(ws + (wave < 2 ? WS_WK : WS_WV));
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const int c = 64 * wave + 16 * cb + l16;
    const u4_t a0 = *(const u4_t*)&Bt[c][8 * q4];
    const u4_t a1 = *(const u4_t*)&Bt[c][32 + 8 * q4];
    const int colg = (64 * wave + 16 * cb + 4 * q4) & 127;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * i + l16;
      f4_t acc = {0.f, 0.f, 0.f, 0.f};
      acc = mfma16<true>(a0, *(const u4_t*)&Tb[t][8 * q4], acc);
      if (i >= 2) acc = mfma16<true>(a1, *(const u4_t*)&Tb[t][32 + 8 * q4], acc);
      u2_t w;
      w.x = pack_bf16x2(acc[0], acc[1]);
      w.y = pack_bf16x2(acc[2], acc[3]);
      *(u2_t*)(wout + t * KD + colg) = w;
    }
  }
}

// ----------------------------------------------------------------------------
// kda_state: grid = B*H*(VD/16), block = 256 (4 waves).  The workgroup owns
// value columns v0 .. v0+15 of one head and walks the chunks in order.
// Wave w holds state rows 32w .. 32w+31 (two 16x16 tiles, fp32) and computes
// U / O rows 16w .. 16w+15.  S and U are shared through LDS transposed
// ([column][row], bf16) so that B-operand reads are 16 bytes.  The operands
// of chunk c+1 are loaded while chunk c is computed.  When B*H is a multiple
// of 8 the 8 column slices of a head run on one XCD and share its L2.
// ----------------------------------------------------------------------------
namespace {
struct ChunkOps {
  u4_t wk[4], qd[4], aq[2], kt[4];
  f4_t gc[2];
  float wv[4];
};
TM_DEV void load_chunk(const uint8_t* ws, int wave, int q4, int l16, int v0, ChunkOps& o) {
  const uint16_t* wk = (const uint16_t*)(ws + WS_WK);
  const uint16_t* wv = (const uint16_t*)(ws + WS_WV);
  const uint16_t* qd = (const uint16_t*)(ws + WS_QD);
  const uint16_t* kt = (const uint16_t*)(ws + WS_KT);
  const uint16_t* aq = (const uint16_t*)(ws + WS_AQ);
  const float* gc = (const float*)(ws + WS_GC);
  const int urow = 16 * wave + l16;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    o.wk[ks] = ldg128(wk + urow * KD + 32 * ks + 8 * q4);
    o.qd[ks] = ldg128(qd + urow * KD + 32 * ks + 8 * q4);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) o.aq[ks] = ldg128(aq + urow * KC + 32 * ks + 8 * q4);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      o.kt[2 * tt + ks] = ldg128(kt + (32 * wave + 16 * tt + l16) * KC + 32 * ks + 8 * q4);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) o.gc[tt] = *(const f4_t*)(gc + 32 * wave + 16 * tt + 4 * q4);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o.wv[e] = bf16_bits_to_f32(wv[(16 * wave + 4 * q4 + e) * VD + v0 + l16]);
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
  ChunkOps cur;
  if (p.NC > 0) load_chunk(wsh, wave, q4, l16, v0, cur);
  for (int c = 0; c < p.NC; ++c) {
    const int buf = c & 1;
    ChunkOps nxt;
    load_chunk(wsh + (size_t)min(c + 1, p.NC - 1) * WS_CHUNK, wave, q4, l16, v0, nxt);

    // (a) S -> LDS as S^T bf16
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int row = 32 * wave + 16 * tt + 4 * q4;
      u2_t w;
      w.x = pack_bf16x2(S[tt][0], S[tt][1]);
      w.y = pack_bf16x2(S[tt][2], S[tt][3]);
      *(u2_t*)(&Sbt[buf][l16][row]) = w;
    }
    __syncthreads();

    // (b) U rows 16w.. : U = W_v - W_k S
    u4_t sb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sb[ks] = *(const u4_t*)(&Sbt[buf][l16][32 * ks + 8 * q4]);
    f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma16<true>(cur.wk[ks], sb[ks], acc);
    f4_t U;
#pragma unroll
    for (int e = 0; e < 4; ++e) U[e] = cur.wv[e] - acc[e];
    {
      u2_t w;
      w.x = pack_bf16x2(U[0], U[1]);
      w.y = pack_bf16x2(U[2], U[3]);
      *(u2_t*)(&Ubt[buf][l16][16 * wave + 4 * q4]) = w;
    }
    // O partial from S while U is shared
    f4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) o = mfma16<true>(cur.qd[ks], sb[ks], o);
    __syncthreads();

    // (c) O rows 16w.. += Aqk U
    u4_t ub[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) ub[ks] = *(const u4_t*)(&Ubt[buf][l16][32 * ks + 8 * q4]);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) o = mfma16<true>(cur.aq[ks], ub[ks], o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = c * KC + 16 * wave + 4 * q4 + e;
      if (t < p.T)
        p.o[((long long)b * p.T + t) * rsv + (long long)h * VD + v0 + l16] =
            f32_to_bf16_bits(o[e]);
    }

    // (d) S = diag(exp(G_C)) S + K_end^T U
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      S[tt] *= cur.gc[tt];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) S[tt] = mfma16<true>(cur.kt[2 * tt + ks], ub[ks], S[tt]);
    }
    cur = nxt;
  }

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
