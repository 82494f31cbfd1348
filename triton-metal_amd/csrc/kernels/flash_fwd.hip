// FlashAttention forward for gfx950.
//
//   O[b,h,i,:] = sum_j softmax_j(scale * Q[b,h,i,:] . K[b,h,j,:]) V[b,h,j,:]
//   LSE[b,h,i] = logsumexp_j(scale * Q[b,h,i,:] . K[b,h,j,:])        (natural log)
//
// Semantics follow make_flash_attention_kernel (_msl_templates.py:1568-1767):
// a score is -inf when kv_pos >= seq_len or, if causal, kv_pos > q_pos
// (1610-1619); the output is divided by l only when l > 0 (1747-1754), so a
// fully masked row is 0.  The layout is the [Z, H, N_CTX, HEAD_DIM] view of
// the @triton.jit kernel (tests/test_flash_attention.py:24-104) with arbitrary
// batch / head / row strides and a contiguous head dimension.
//
// MFMA kernel (flash_fwd_d<D>_<dt>_<mask>): a workgroup of 4 waves owns 128
// query rows of one (b, h); each wave owns 32.  Per key block of 64:
//   S^T = K Q^T with v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q^T from
//         registers), so lane l holds the 32 scores of query column l % 32;
//         the row max needs one exchange with lane l ^ 32 and the rescale of
//         O is uniform per lane;
//   O^T += V^T P^T: P leaves the S^T accumulators directly as the B operand
//         (the key order inside a 16-key MFMA step is chosen to match the
//         accumulator layout, and V^T is read from LDS in that same order).
// K and V tiles stream from global memory straight into LDS
// (global_load_lds_dwordx4, row-major with XOR swizzles, double-buffered); V^T
// operands are read with ds_read_b64_tr_b16.  The next block's copies are in
// flight while the current block computes.  Softmax runs in the exp2 domain with
// scale * log2(e) folded into the scores.  Causal: key blocks past a wave's
// last query are skipped, and a workgroup runs query blocks nqb - 1 - i and i
// so that every workgroup has the same number of key blocks.
//
// General kernel (flash_fwd_general): any head dim <= 128, fp32/fp16/bf16,
// one thread per query row, fp32 throughout.
#include <type_traits>

#include "common.h"
#include "flash_params.h"

namespace {

constexpr float kLn2 = 0.69314718055994530942f;

TM_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

TM_DEV u4_t pack8(const float* v, bool bf16) {
  u4_t r;
  if (bf16) {
    r.x = pack_bf16x2(v[0], v[1]); r.y = pack_bf16x2(v[2], v[3]);
    r.z = pack_bf16x2(v[4], v[5]); r.w = pack_bf16x2(v[6], v[7]);
  } else {
    r.x = pack_f16x2(v[0], v[1]); r.y = pack_f16x2(v[2], v[3]);
    r.z = pack_f16x2(v[4], v[5]); r.w = pack_f16x2(v[6], v[7]);
  }
  return r;
}

}  // namespace

// LDS layouts.  K and V tiles are both stored row-major ([64 keys][D]) and
// written straight from global memory with global_load_lds_dwordx4 (lane l of
// a wave deposits its 16 bytes at LDS base + 16 l, so a 16-byte-granular
// swizzle is applied by choosing each lane's source address):
//   K: chunk c (8 halves) of key row r lives at chunk c ^ ks(r), with
//      ks(r) = (r >> log2(128 / D)) & (D / 8 - 1), so the 16 rows read by
//      one 16-lane MFMA operand fetch land in 16 different bank groups;
//   V: chunk c of key row r lives at chunk c ^ vs(r), vs(r) = 4 (r & 3) for
//      D = 128, 4 ((r >> 1) & 1) for D = 64, 0 for D = 32, which spreads the
//      transposing reads below over all banks.
// The V^T operand of the P V product is read with ds_read_b64_tr_b16: within
// each 16-lane group, lane i's element e is element i % 4 of the 8 bytes
// addressed by lane 4 e + i / 4.  With lane j of group G addressing
// V[k0 + 4 (G / 2) + j / 4][dt*32 + 16 (G % 2) + 4 (j % 4)], lane l receives
// V^T[dt*32 + l % 32][k0 + 4 (l / 32) + e]: the MFMA A operand in the key
// order of the P operand.
template <int D> TM_DEV int k_swz(int r) {
  constexpr int SH = D == 128 ? 0 : D == 64 ? 1 : 2;
  return (r >> SH) & (D / 8 - 1);
}
template <int D> TM_DEV int v_swz(int r) {
  if constexpr (D == 128) return 4 * (r & 3);
  else if constexpr (D == 64) return 4 * ((r >> 1) & 1);
  else return 0;
}

typedef short s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4_t lds_s4_t;

TM_DEV u2_t lds_tr16(const uint16_t* p) {
  s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(p));
  return __builtin_bit_cast(u2_t, v);
}

// DV < D: a head dim of DV (a multiple of 8 above D / 2) in the layout of D.
// The copies skip the 16-byte chunks at or past DV (their lanes are masked
// off, so those LDS slots are never written; the K slots are zeroed once),
// Q's chunks past DV are zero, the contraction steps and O tiles wholly past
// DV are skipped and O's columns past DV are not stored: the MFMA work of a
// DV-wide kernel with D's swizzles and tiling.
template <int D, bool BF16, bool CAUSAL, int DV = D>
__device__ __forceinline__ void flash_fwd_body(const FlashParams& p) {
  constexpr int BM = 128, BN = 64, NW = 4;
  constexpr int DC = D / 16;    // 16-wide contraction steps of Q K^T
  constexpr int DT = D / 32;    // 32-wide d tiles of O^T
  constexpr int CV = DV / 8;    // 16-byte chunks of a row below DV
  constexpr int DCV = (DV + 15) / 16, DTV = (DV + 31) / 32;  // steps / tiles used
  constexpr int NB = BN * D * 2 / 1024;  // 1 KB blocks per tile
  constexpr int BPW = NB / NW;           // blocks per wave
  constexpr int RPB = 512 / D;           // key rows per 1 KB block
  static_assert(D % 32 == 0 && D <= 128 && NB % NW == 0, "head dim");
  static_assert(DV % 8 == 0 && DV <= D && 2 * DV > D, "valid head dim");
  // separate objects per buffer (chosen at compile time below) so that the
  // compiler can tell the reads of one buffer from the DMA into the other
  __shared__ __align__(16) uint16_t Ks0[BN * D], Ks1[BN * D];
  __shared__ __align__(16) uint16_t Vs0[BN * D], Vs1[BN * D];

  // wave index through readfirstlane: known uniform, so what derives from it
  // (copy destinations, row ranges) stays in scalar registers
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h32 = lane >> 5, l32 = lane & 31;
  const int S = p.S;
  const int nqb = (S + BM - 1) / BM;
  const int BH = p.B * p.H;
  // Work order.  Consecutive workgroups go round-robin to the 8 XCDs
  // (blockIdx % 8), each with its own L2; when B*H % 8 == 0 every query block
  // of head bh runs on XCD bh % 8.
  // Causal: a workgroup takes query blocks nqb - 1 - i and i of one head, one
  // after the other (2 (nqb - i) + 2 (i + 1) = 2 nqb + 2 key blocks of 64), so
  // every workgroup has the same work and the grid ends evenly instead of with
  // the long blocks of the last heads on a few CUs.
  // Full: one query block per workgroup; an XCD takes its heads two at a time
  // with their query blocks alternating, so two heads' K and V are live in
  // its L2 at once.
  int bh, qb_first, qb_second, npass;
  if constexpr (CAUSAL) {
    const int npair = (nqb + 1) / 2;
    int pi;
    if ((BH & 7) == 0) {
      const int x = blockIdx.x & 7, sl = blockIdx.x >> 3;
      bh = x + 8 * (sl / npair);
      pi = sl % npair;
    } else {
      bh = blockIdx.x % BH;
      pi = blockIdx.x / BH;
    }
    qb_first = nqb - 1 - pi;                 // the heavier block first
    qb_second = pi;
    npass = (2 * pi + 1 == nqb) ? 1 : 2;     // the middle block of an odd count
  } else {
    int qslot;
    if ((BH & 7) == 0) {
      const int x = blockIdx.x & 7, sl = blockIdx.x >> 3;
      const int hpx = BH >> 3;  // heads per XCD
      const int pair = sl / (2 * nqb), r = sl - pair * (2 * nqb);
      if (2 * pair + 1 < hpx) {
        bh = x + 8 * (2 * pair + (r & 1));
        qslot = r >> 1;
      } else {  // an odd count leaves the last head alone: r < nqb
        bh = x + 8 * (2 * pair);
        qslot = r;
      }
    } else {
      bh = blockIdx.x % BH;
      qslot = blockIdx.x / BH;
    }
    qb_first = qb_second = qslot;
    npass = 1;
  }
  const int b = bh / p.H, hh = bh - b * p.H;
  const uint16_t* qg = (const uint16_t*)p.q + b * p.sqb + hh * p.sqh;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.skb + hh * p.skh;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.svb + hh * p.svh;
  uint16_t* og = (uint16_t*)p.o + b * p.sob + hh * p.soh;

  // ---- K / V tiles: global -> LDS directly ----------------------------------
  // this lane's piece of each 1 KB block: row rb + lane / (D/8), phys chunk
  // lane % (D/8); its source offsets within a key block are fixed, only the
  // block base moves (32-bit offsets; the host checks 64 * stride < 2^31)
  const int prow = lane / (D / 8), pch = lane % (D / 8);
  uint32_t koff[BPW], voff[BPW];  // byte offsets
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int r = (wave * BPW + i) * RPB + prow;
    koff[i] = 2u * (uint32_t)(r * (int)p.sks + 8 * (pch ^ k_swz<D>(r)));
    voff[i] = 2u * (uint32_t)(r * (int)p.svs + 8 * (pch ^ v_swz<D>(r)));
  }
  // the lane's K / V chunk of block i lies below DV
  auto kin = [&](int i) -> bool {
    if constexpr (DV == D) {
      return true;
    } else {
      const int r = (wave * BPW + i) * RPB + prow;
      return (pch ^ k_swz<D>(r)) < CV;
    }
  };
  auto vin = [&](int i) -> bool {
    if constexpr (DV == D) {
      return true;
    } else {
      const int r = (wave * BPW + i) * RPB + prow;
      return (pch ^ v_swz<D>(r)) < CV;
    }
  };
  auto issue_kv = [&](uint16_t* kd, uint16_t* vd, int kv0) {
    const uint16_t* kt = kg + (long long)kv0 * p.sks;
    const uint16_t* vt = vg + (long long)kv0 * p.svs;
    if (kv0 + BN <= S) {
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int blk = wave * BPW + i;
        if (kin(i)) dma16s(kt, koff[i], lds_off(kd) + blk * 1024);
        if (vin(i)) dma16s(vt, voff[i], lds_off(vd) + blk * 1024);
      }
    } else {
      // rows past the end re-read row S - 1 (their scores are masked)
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int blk = wave * BPW + i;
        const int r = blk * RPB + prow;
        const int back = r - min(r, S - 1 - kv0);
        if (kin(i))
          dma16s(kt, koff[i] - 2u * (uint32_t)(back * (int)p.sks), lds_off(kd) + blk * 1024);
        if (vin(i))
          dma16s(vt, voff[i] - 2u * (uint32_t)(back * (int)p.svs), lds_off(vd) + blk * 1024);
      }
    }
  };
  if constexpr (DV < D) {
    // the K slots of the chunks past DV: zero once (no copy writes them)
    constexpr int NPAD = D / 8 - CV;
    for (int sidx = tid; sidx < BN * NPAD; sidx += NW * 64) {
      const int r = sidx / NPAD, c = CV + sidx % NPAD;
      const int off = r * D + 8 * (c ^ k_swz<D>(r));
      *(u4_t*)(Ks0 + off) = u4_t{0u, 0u, 0u, 0u};
      *(u4_t*)(Ks1 + off) = u4_t{0u, 0u, 0u, 0u};
    }
  }

  // ---- LDS read addresses, fixed per lane --------------------------------------
  // K operand rows r = 32 kt + l32 keep their swizzle k_swz(r) = k_swz(l32)
  // for every kt, so the byte offset of chunk 2c + h32 of this lane's row is a
  // per-lane constant kro[c]; the key half (kt) and the buffer are immediates.
  // V^T reads: rows r0 = 16 u + tv_row (+8) keep v_swz(tv_row), which only
  // flips bits 2..3 of the chunk index 4t + cl, so the offset of d tile t is a
  // per-lane constant vro[t]; u and the row half are immediates.
  const int tg = lane >> 4, tj = lane & 15;
  const int tv_row = 4 * (tg >> 1) + (tj >> 2);
  const int tv_d = 16 * (tg & 1) + 4 * (tj & 3);
  uint32_t kro[DC], vro[DT];
  {
    const int ks = k_swz<D>(l32);
#pragma unroll
    for (int c = 0; c < DC; ++c) kro[c] = 2u * (uint32_t)(l32 * D + 8 * ((2 * c + h32) ^ ks));
    const int vsw = v_swz<D>(tv_row);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int cch = (32 * t + tv_d) >> 3, off = (32 * t + tv_d) & 7;
      vro[t] = 2u * (uint32_t)(tv_row * D + 8 * (cch ^ vsw) + off);
    }
  }

  const float sl2 = p.sl2;
  for (int pass = 0; pass < npass; ++pass) {
    const int qb = pass == 0 ? qb_first : qb_second;
    const int q0 = qb * BM + wave * 32;      // first query row of this wave
    const int qi = q0 + l32;                  // this lane's query row
    const int qlast_blk = min(qb * BM + BM - 1, S - 1);
    const int nkb = CAUSAL ? qlast_blk / BN + 1 : (S + BN - 1) / BN;

    // Q^T operands: qreg[c] = Q[qi][16c + 8*h32 .. +8] (zero past DV)
    u4_t qreg[DC];
#pragma unroll
    for (int c = 0; c < DCV; ++c) {
      qreg[c] = u4_t{0u, 0u, 0u, 0u};
      bool qin = qi < S;
      if constexpr (DV < D) qin = qin && 2 * c + h32 < CV;
      if (qin) qreg[c] = ldg128(qg + (long long)qi * p.sqs + 16 * c + 8 * h32);
    }

    f16_t oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] = f16_t{};
    float m_run = -INFINITY, l_run = 0.0f;

    issue_kv(Ks0, Vs0, 0);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();

    // one key block: compute from (ks, vs) while the next block streams into
    // (kn, vn); BUF is the compile-time buffer parity
    auto step = [&](auto bufc, int j) {
      constexpr int BUF = decltype(bufc)::value;
      const char* ks = (const char*)(BUF ? Ks1 : Ks0);
      const char* vs = (const char*)(BUF ? Vs1 : Vs0);
      uint16_t* kn = BUF ? Ks0 : Ks1;
      uint16_t* vn = BUF ? Vs0 : Vs1;
      const int kv0 = j * BN;
      const bool more = j + 1 < nkb;
      if (more) issue_kv(kn, vn, kv0 + BN);

      // a wave whose rows all precede this key block has nothing to do
      const bool active = !CAUSAL || kv0 <= q0 + 31;
      if (active) {
        // raise this wave's issue priority while it feeds the MFMA pipe, so the
        // co-resident wave's softmax fills the gaps instead of competing
        __builtin_amdgcn_s_setprio(1);
        f16_t s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[kt] = f16_t{};
        // The two key halves alternate, so consecutive MFMAs are independent;
        // the K operands of step c + KPD are read while step c multiplies.
        constexpr int KPD = 2;
        u4_t ka[DC][2];
        auto kread = [&](int c) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) ka[c][kt] = *(const u4_t*)(ks + kro[c] + kt * 32 * D * 2);
        };
#pragma unroll
        for (int c = 0; c < KPD; ++c) kread(c);
#pragma unroll
        for (int c = 0; c < DCV; ++c) {
          if (c + KPD < DCV) kread(c + KPD);
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) s[kt] = mfma32<BF16>(ka[c][kt], qreg[c], s[kt]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * KPD, 0);
#pragma unroll
        for (int c = 0; c < DCV; ++c) {
          if (c + KPD < DCV) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        // raw scores sc[16 kt + i] of key kv0 + 32 kt + 8 (i / 4) + 4 h32 + i % 4
        float sc[32];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[16 * kt + i] = s[kt][i];
        if ((kv0 + BN > S) || (CAUSAL && kv0 + BN - 1 > q0)) {
          // keys past the end, or (causal) past this lane's query row
          const int lim = CAUSAL ? min(qi, S - 1) : S - 1;
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            const int kv = kv0 + 32 * (i >> 4) + 8 * ((i >> 2) & 3) + 4 * h32 + (i & 3);
            sc[i] = kv > lim ? -INFINITY : sc[i];
          }
        }
        float mx = sc[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) mx = fmaxf(mx, sc[i]);
        {
          // max with the partner lane l ^ 32 (the other half of this query's keys)
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx),
                                                           __float_as_uint(mx), false, false);
          mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * sl2;
        }
        // Lazy rescale: the running max only moves when a row's max grows by
        // more than 2^8 (log2 domain), so p = exp2(s - m) <= 256 and O is
        // rescaled rarely; l and O always share the same reference m.
        float alpha = 1.0f;
        if (mx > m_run + 8.0f) {
          alpha = fast_exp2(m_run - mx);  // 0 on the first block (m_run = -inf)
          m_run = mx;
        }
        const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
        float lsum = 0.0f;
        u4_t pop[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pv[e] = fast_exp2(__builtin_fmaf(sc[8 * u + e], sl2, -m_use));
            lsum += pv[e];
          }
          pop[u] = pack8(pv, BF16);
        }
        l_run = l_run * alpha + lsum;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // some row's max moved
#pragma unroll
          for (int t = 0; t < DTV; ++t) oacc[t] *= alpha;
        }
        // O^T[d][q] += V^T[d][kv] P^T[kv][q]; MFMA u covers keys
        //   32 (u/2) + 16 (u%2) + 8 (e/4) + 4 h32 + e % 4
        __builtin_amdgcn_s_setprio(1);
        // operand i = DTV u + t; the V^T operands of i + VPD are read while i multiplies
        constexpr int NVO = 4 * DTV, VPD = 2;
        u4_t va[NVO];
        auto vread = [&](int i) {
          const int u = i / DTV, t = i % DTV;
          const u2_t lo = lds_tr16((const uint16_t*)(vs + vro[t] + 16 * u * D * 2));
          const u2_t hi = lds_tr16((const uint16_t*)(vs + vro[t] + (16 * u + 8) * D * 2));
          va[i].x = lo.x; va[i].y = lo.y; va[i].z = hi.x; va[i].w = hi.y;
        };
#pragma unroll
        for (int i = 0; i < VPD; ++i) vread(i);
#pragma unroll
        for (int i = 0; i < NVO; ++i) {
          if (i + VPD < NVO) vread(i + VPD);
          oacc[i % DTV] = mfma32<BF16>(va[i], pop[i / DTV], oacc[i % DTV]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * VPD, 0);
#pragma unroll
        for (int i = 0; i < NVO; ++i) {
          if (i + VPD < NVO) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_s_setprio(0);
      }
      if (more) {
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's tile loads landed
      }
      __syncthreads();
    };
    for (int j = 0; j < nkb; j += 2) {
      step(std::integral_constant<int, 0>{}, j);
      if (j + 1 < nkb) step(std::integral_constant<int, 1>{}, j + 1);
    }

    // ---- epilogue: O = O / l, LSE ----------------------------------------------
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (qi < S) {
      uint16_t* orow = og + (long long)qi * p.sos;
#pragma unroll
      for (int t = 0; t < DTV; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = t * 32 + 8 * g + 4 * h32;
          if constexpr (DV < D) {
            if (d >= DV) continue;
          }
          u2_t w;
          if (BF16) {
            w.x = pack_bf16x2(oacc[t][4 * g] * inv, oacc[t][4 * g + 1] * inv);
            w.y = pack_bf16x2(oacc[t][4 * g + 2] * inv, oacc[t][4 * g + 3] * inv);
          } else {
            w.x = pack_f16x2(oacc[t][4 * g] * inv, oacc[t][4 * g + 1] * inv);
            w.y = pack_f16x2(oacc[t][4 * g + 2] * inv, oacc[t][4 * g + 3] * inv);
          }
          *(u2_t*)(orow + d) = w;
        }
      if (p.lse && h32 == 0)
        p.lse[(long long)bh * S + qi] = l_tot > 0.0f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
    }
  }
}

#define TM_FLASH_INST(D, BF, DT, CAUSAL, MASK)                                              \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void \
      flash_fwd_d##D##_##DT##_##MASK(                                                       \
      FlashParams p) {                                                                      \
    flash_fwd_body<D, BF, CAUSAL>(p);                                                       \
  }
#define TM_FLASH_D(D)                                  \
  TM_FLASH_INST(D, true, bf16, false, full)            \
  TM_FLASH_INST(D, true, bf16, true, causal)           \
  TM_FLASH_INST(D, false, f16, false, full)            \
  TM_FLASH_INST(D, false, f16, true, causal)
TM_FLASH_D(128)
TM_FLASH_D(64)
TM_FLASH_D(32)
// head dims 48 (in the 64 layout) and 80, 96, 112 (in the 128 layout):
// flash_fwd_d<D>v<DV>_<dt>_<mask>
#define TM_FLASH_INST_V(D, DV, BF, DT, CAUSAL, MASK)                                        \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void \
      flash_fwd_d##D##v##DV##_##DT##_##MASK(FlashParams p) {                                \
    flash_fwd_body<D, BF, CAUSAL, DV>(p);                                                   \
  }
#define TM_FLASH_DV(D, DV)                                 \
  TM_FLASH_INST_V(D, DV, true, bf16, false, full)          \
  TM_FLASH_INST_V(D, DV, true, bf16, true, causal)         \
  TM_FLASH_INST_V(D, DV, false, f16, false, full)          \
  TM_FLASH_INST_V(D, DV, false, f16, true, causal)
TM_FLASH_DV(64, 48)
TM_FLASH_DV(128, 80)
TM_FLASH_DV(128, 96)
TM_FLASH_DV(128, 112)

// ----------------------------------------------------------------------------
// General kernel: one thread per query row, keys streamed through LDS in
// fp32, online softmax in fp32.  Any D <= DMAX, any of fp32/fp16/bf16.
// grid = (ceil(S / 64), B * H), block = 64.
// ----------------------------------------------------------------------------
template <int DMAX>
__device__ __forceinline__ void flash_general_body(const FlashParams& p) {
  constexpr int TB = 32;  // keys per LDS tile
  __shared__ float kt[TB][DMAX], vtile[TB][DMAX];
  const int D = p.D, S = p.S, dt = p.dtype;
  const int bh = blockIdx.y, b = bh / p.H, hh = bh - b * p.H;
  const int qi = blockIdx.x * 64 + threadIdx.x;
  const long long qoff = b * p.sqb + hh * p.sqh + (long long)qi * p.sqs;
  float qv[DMAX], ov[DMAX];
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    qv[d] = (qi < S && d < D) ? load_as_f32_rt(p.q, qoff + d, dt) : 0.0f;
    ov[d] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  const int last = p.causal ? min(S, (int)(blockIdx.x * 64 + 64)) : S;
  for (int k0 = 0; k0 < last; k0 += TB) {
    __syncthreads();
    for (int i = threadIdx.x; i < TB * DMAX; i += 64) {
      const int r = i / DMAX, d = i % DMAX;
      const int kv = k0 + r;
      float kx = 0.0f, vx = 0.0f;
      if (kv < S && d < D) {
        kx = load_as_f32_rt(p.k, b * p.skb + hh * p.skh + (long long)kv * p.sks + d, dt);
        vx = load_as_f32_rt(p.v, b * p.svb + hh * p.svh + (long long)kv * p.svs + d, dt);
      }
      kt[r][d] = kx;
      vtile[r][d] = vx;
    }
    __syncthreads();
    for (int r = 0; r < TB; ++r) {
      const int kv = k0 + r;
      if (kv >= S || (p.causal && kv > qi)) continue;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) dot += qv[d] * kt[r][d];
      const float sv = dot * p.sl2;
      const float mn = fmaxf(m, sv);
      const float a = exp2f(m - mn), e = exp2f(sv - mn);
      l = l * a + e;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) ov[d] = ov[d] * a + e * vtile[r][d];
      m = mn;
    }
  }
  if (qi >= S) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const long long ooff = b * p.sob + hh * p.soh + (long long)qi * p.sos;
  for (int d = 0; d < D && d < DMAX; ++d) store_as_f32_rt(p.o, ooff + d, dt, ov[d] * inv);
  if (p.lse) p.lse[(long long)bh * S + qi] = l > 0.0f ? (m + log2f(l)) * kLn2 : -INFINITY;
}

extern "C" __global__ __launch_bounds__(64) void flash_fwd_general_d32(FlashParams p) {
  flash_general_body<32>(p);
}
extern "C" __global__ __launch_bounds__(64) void flash_fwd_general_d64(FlashParams p) {
  flash_general_body<64>(p);
}
extern "C" __global__ __launch_bounds__(64) void flash_fwd_general_d128(FlashParams p) {
  flash_general_body<128>(p);
}
