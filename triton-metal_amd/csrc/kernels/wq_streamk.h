// W-only streaming kernel for long K: int4 (make_int4_matmul_kernel,
// _msl_templates.py:2682-2745; weights [N, K/2] bytes, even k in the low
// nibble) and int8 (make_int8_matmul_kernel, 2630-2679; weights [N, K]),
// 2 <= M <= 64, K > 4096.
//
// The down projections of a model (K = 11008, 14336, 28672, ...) have few
// output columns, so the K <= 4096 streaming kernel's 48- / 64-column
// workgroups would leave most CUs idle (N = 4096: 64 workgroups).  Here a
// workgroup owns NT 16-column tiles (NT = 1 or 2: one workgroup per CU for
// N = 4096 / 8192) and all of K: its nwv waves (at most 8) take the chunks
// c = nwv i + w (i < NCH; int4 chunks are 128 k = one quantisation group,
// int8 chunks 64 k: 64 weight bytes of a row either way), so at any time they
// read adjacent segments of the same rows, and the waves' partial sums meet in
// LDS.  Chunks past the end (the last round when the chunk count is not a
// multiple of nwv) re-read the last chunk and do not count.
//
// Per chunk a wave copies global -> LDS into a 2-slot ring of its own: the
// tiles' weights (16 rows x 64 B each, every 4 consecutive lanes on one
// 64-byte segment) and the chunk's k of the XR activation rows; int4 scales /
// zero-points (one dword per column and chunk) and int8 per-channel ones go to
// its LDS before the first chunk.  Operands are read back in MFMA order
// through XOR swizzles:
//   weight piece p (16 B) of row r at 64 r + 16 (p ^ ((r >> 2) & 3))
//   X piece p of row r at XB r + 16 (p ^ xsw(r))
// Products on v_mfma_f32_16x16x32 (A = the activations, B = exact 16-bit
// operands: int4 OFF + q, int8 q), the row sums of X on the same MFMA against
// an all-ones B.  int4: per chunk y += s (sum x (OFF + q) - (OFF + z) sum x);
// int8: y = s (sum x q - z sum x) at the end.  MULTI (M > 16): passes of 16
// activation rows; the first pass keeps the weight words in registers, the
// later ones stream only X.
// Split-K form (SPLIT): workgroup row blockIdx.y takes the k-slice
// [blockIdx.y K, + K) of rows that are ldk long (X, weights and, int4, the
// group scales / zero-points offset by it) and writes its fp32 sums, scaled
// but without bias, to P[blockIdx.y][M][N]; wq_splitk_reduce adds the slices.
#pragma once
#include "common.h"
#include "wq_common.h"

namespace {
// Copies issued after chunk i's (ring of RS slots; c0 copies per first-pass
// chunk, c1 per later-pass one; the items past the pass end only if another
// pass follows).
constexpr int streamk_ahead(int rs, int nch, int c0, int c1, bool first, int i, bool next) {
  int a = 0;
  for (int d = 1; d < rs; ++d) {
    if (i + d < nch) a += first ? c0 : c1;
    else if (next) a += c1;
  }
  return a;
}
}  // namespace

template <int QB, bool BF16, int ZDT, int NT, int XR, int NCH, bool MULTI, bool SPLIT>
__device__ __forceinline__ void wq_streamk_body(const uint16_t* X, const uint8_t* W,
                                                uint16_t* __restrict__ Y, float* __restrict__ P,
                                                const void* S, const void* Z, int M, int N, int K,
                                                int ldk, const uint16_t* bias) {
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  constexpr int CK = QB == 4 ? 128 : 64;  // k per chunk: 64 weight bytes of a row
  constexpr int NJ = CK / 32;             // MFMA k-steps per chunk
  constexpr int XB = 2 * CK, XPR = XB / 16;
  constexpr int XI = XR * XPR / 64;       // X copies (1 KB each) per chunk
  constexpr int RS = 2;                   // ring slots per wave
  constexpr int SLOT = NT * 1024 + XR * XB;
  constexpr int NQ = NCH / 4;             // int4 scale blocks (4 chunks x 16 columns)
  constexpr int SCB = QB == 4 ? 512 * NT * NQ : 1024;  // per-wave scales / zero-points
  constexpr int WB = RS * SLOT + SCB;
  constexpr int C0 = NT + XI, C1 = XI;    // copies per first- / later-pass chunk
  constexpr int NF = 4 * NT;              // partial sums per lane per pass
  static_assert(NCH % 4 == 0 && NCH >= RS && XI >= 1 && (!MULTI || XR == 16), "streamk shape");
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwv = blockDim.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * (16 * NT);
  const int nchunk = K / CK;
  const int npass = MULTI ? (M + 15) >> 4 : 1;
  // split-K: this workgroup's k-slice (the whole row otherwise, ldk == K)
  const int ks0 = SPLIT ? (int)blockIdx.y * K : 0;
  X += ks0;
  W += QB == 4 ? ks0 >> 1 : ks0;
  const size_t rowbytes = QB == 4 ? (size_t)(ldk >> 1) : (size_t)ldk;
  const size_t srow = (size_t)(ldk / CK);  // int4: groups per row of S / Z
  const size_t g0 = (size_t)(ks0 / CK);
  const uint8_t* const wl = lds + wave * WB;
  const uint8_t* const scl = wl + RS * SLOT;
  const uint32_t wlo = __builtin_amdgcn_readfirstlane(lds_off(wl));
  const uint32_t slo = wlo + RS * SLOT;
  float* const red = (float*)(lds + nwv * WB);  // [nwv][8][64]
  auto chunk_of = [&](int i) { return min(nwv * i + wave, nchunk - 1); };

  // ---- scales / zero-points
  // int4: [qq][t][s, z][64 lanes] dwords; lane (l16, q) holds the dword with
  // chunk 4 qq + q's group of column n0 + 16 t + l16.  int8: dword c holds
  // columns n0 + 2c, 2c + 1 (u8 zero-points: 4c .. 4c + 3).
  if constexpr (QB == 4) {
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const size_t gi = (size_t)min(n0 + 16 * t + l16, N - 1) * srow + g0 + chunk_of(4 * qq + q);
        const uint32_t dst = slo + 512 * (qq * NT + t);
        dma4((const uint16_t*)S + (gi & ~(size_t)1), dst);
        if constexpr (ZDT == 3) dma4((const uint8_t*)Z + (gi & ~(size_t)3), dst + 256);
        else if constexpr (ZDT >= 0) dma4((const uint16_t*)Z + (gi & ~(size_t)1), dst + 256);
      }
    }
  } else {
    const int c2 = min((n0 >> 1) + lane, (N >> 1) - 1);
    dma4((const uint16_t*)S + 2 * c2, slo);
    if constexpr (ZDT == 3) dma4((const uint8_t*)Z + 4 * min((n0 >> 2) + lane, (N >> 2) - 1), slo + 256);
    else if constexpr (ZDT >= 0) dma4((const uint16_t*)Z + 2 * c2, slo + 256);
  }
  // ---- weights: lane l -> row r = l / 4 of the tile, piece (l % 4) ^ ((r >> 2) & 3)
  const uint8_t* wsrc[NT];
  {
    const int r = lane >> 2, pc = (lane & 3) ^ ((r >> 2) & 3);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wsrc[t] = W + (size_t)min(n0 + 16 * t + r, N - 1) * rowbytes + 16 * pc;
  }
  auto xsw = [](int r) { return QB == 4 ? (r & 15) : ((r >> 1) & 7); };
  // ---- X: copy h, lane l -> row h (64 / XPR) + l / XPR, piece (l % XPR) ^ xsw(row)
  auto issue = [&](auto FIRSTC, int p, int i, int slot) {
    const uint32_t sb = wlo + slot * SLOT;
    const int c = chunk_of(i);
    // the slot's previous contents have been read
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (decltype(FIRSTC)::value) {
#pragma unroll
      for (int t = 0; t < NT; ++t) dma16(wsrc[t] + 64 * c, sb + 1024 * t);
    }
#pragma unroll
    for (int h = 0; h < XI; ++h) {
      const int rr = h * (64 / XPR) + lane / XPR;
      const int pc = (lane % XPR) ^ xsw(rr);
      const int m = min(16 * p + rr, M - 1);
      dma16(X + (size_t)m * ldk + CK * c + 8 * pc, sb + NT * 1024 + 1024 * h);
    }
  };
  const std::integral_constant<bool, true> first_c;
  const std::integral_constant<bool, false> later_c;
  static_for<0, RS>([&](auto IC) { issue(first_c, 0, decltype(IC)::value, decltype(IC)::value); });

  // operand offsets in a slot: weight piece q of row l16; X piece of row l16
  // for k-step j (int4 4q + j, int8 2q + j, matching the weight dwords)
  const int woff = 64 * l16 + 16 * (q ^ ((l16 >> 2) & 3));
  const int xrow = l16 & (XR - 1);
  u4_t wv[NT][MULTI ? NCH : 1];

  auto run_pass = [&](auto FIRSTC, int p) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(FIRSTC)::value;
    const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
    const uint32_t s4 = vgpr_const(4u), s8 = vgpr_const(8u), s12 = vgpr_const(12u);
    const bool next = MULTI && p + 1 < npass;
    f4_t y[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) y[t] = f4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t one2 = vgpr_const(BF16 ? 0x3F803F80u : 0x3C003C00u);
    const u4_t ones = {one2, one2, one2, one2};
    f4_t xacc = f4_t{0.f, 0.f, 0.f, 0.f};
    static_for<0, NCH>([&](auto IC) {
      constexpr int i = decltype(IC)::value;
      __builtin_amdgcn_sched_barrier(0);
      if (next) wait_vm<streamk_ahead(RS, NCH, C0, C1, FIRST, i, true)>();
      else wait_vm<streamk_ahead(RS, NCH, C0, C1, FIRST, i, false)>();
      const int slot = MULTI ? (p * NCH + i) % RS : i % RS;
      const uint8_t* sp = wl + slot * SLOT;
      u4_t xo[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int pc = QB == 4 ? 4 * q + j : 2 * q + j;
        xo[j] = *(const u4_t*)(sp + NT * 1024 + xrow * XB + 16 * (pc ^ xsw(xrow)));
      }
      u4_t wcur[NT];
      if constexpr (FIRST) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          wcur[t] = *(const u4_t*)(sp + 1024 * t + woff);
          if constexpr (MULTI) wv[t][i] = wcur[t];
        }
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) wcur[t] = wv[t][MULTI ? i : 0];
      }
      // the slot takes the chunk RS ahead (issued before the MFMAs: nothing
      // is scheduled across)
      if constexpr (i + RS < NCH) issue(FIRSTC, p, i + RS, slot);
      else if (next) issue(later_c, p + 1, i + RS - NCH, slot);
      __builtin_amdgcn_sched_barrier(0);

      const int c = nwv * i + wave;
      const bool live = c < nchunk;  // wave-uniform
      f4_t acc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
      f4_t xr = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const u4_t xop = QB == 4 ? perm_x8(xo[j]) : xo[j];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const u4_t w = wcur[t];
          u4_t wop;
          if constexpr (QB == 4) {
            const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
            wop = w4_operand_v(wj, vmask, vmagic, s4, s8, s12);
          } else {
            // (opaque copies, so that the conversion stays in the pass loop)
            uint32_t w0 = j == 0 ? w.x : w.z, w1 = j == 0 ? w.y : w.w;
            asm volatile("" : "+v"(w0), "+v"(w1));
            wop = w8_operand<BF16>(w0, w1);
          }
          acc[t] = mfma16<BF16>(xop, wop, acc[t]);
        }
        xr = mfma16<BF16>(xop, ones, xr);
      }
      if constexpr (QB == 4) {
        const int cc = live ? c : nchunk - 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          // dword of lane (l16, i % 4) in block (i / 4, t): this chunk's group
          // of column 16 t + l16
          const uint8_t* sp2 = scl + 512 * ((i / 4) * NT + t) + 4 * (16 * (i % 4) + l16);
          const size_t gi = (size_t)min(n0 + 16 * t + l16, N - 1) * srow + g0 + cc;
          float sc = raw_to_f32<SDT>((uint16_t)(*(const uint32_t*)sp2 >> (16 * (gi & 1))));
          sc = live ? sc : 0.0f;
          float zb = w4_offset<BF16>();
          if constexpr (ZDT == 3)
            zb += (float)((*(const uint32_t*)(sp2 + 256) >> (8 * (gi & 3))) & 0xFFu);
          else if constexpr (ZDT >= 0)
            zb += raw_to_f32<ZDT>((uint16_t)(*(const uint32_t*)(sp2 + 256) >> (16 * (gi & 1))));
#pragma unroll
          for (int e = 0; e < 4; ++e) y[t][e] += sc * (acc[t][e] - zb * xr[e]);
        }
      } else if (live) {
        xacc += xr;
#pragma unroll
        for (int t = 0; t < NT; ++t) y[t] += acc[t];
      }
      // (pins the chunk's epilogue here)
#pragma unroll
      for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(y[t]));
    });
    if constexpr (QB == 8) {
      const f4_t xr = xacc;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int c = 16 * t + l16;
        const uint32_t sw = *(const uint32_t*)(scl + 4 * (c >> 1));
        const float sc = raw_to_f32<SDT>((uint16_t)(sw >> (16 * (c & 1))));
        float z = 0.0f;
        if constexpr (ZDT == 3) {
          z = (float)((*(const uint32_t*)(scl + 256 + 4 * (c >> 2)) >> (8 * (c & 3))) & 0xFFu);
        } else if constexpr (ZDT >= 0) {
          const uint32_t zw = *(const uint32_t*)(scl + 256 + 4 * (c >> 1));
          z = raw_to_f32<ZDT>((uint16_t)(zw >> (16 * (c & 1))));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) y[t][e] = sc * (y[t][e] - z * xr[e]);
      }
    }

    // reduce the waves' partial sums, 8 per round: red[wave][f - 8 r][lane]
    static_for<0, (NF + 7) / 8>([&](auto RC) {
      constexpr int r = decltype(RC)::value;
      constexpr int FN = NF - 8 * r < 8 ? NF - 8 * r : 8;
      lds_barrier();  // earlier reads of red are done
#pragma unroll
      for (int f = 0; f < FN; ++f) red[(wave * 8 + f) * 64 + lane] = y[(8 * r + f) >> 2][(8 * r + f) & 3];
      lds_barrier();
      for (int f = wave; f < FN; f += nwv) {
        float v = 0.0f;
        for (int w2 = 0; w2 < nwv; ++w2) v += red[(w2 * 8 + f) * 64 + lane];
        const int F = 8 * r + f, t = F >> 2, e = F & 3;
        const int row = 16 * p + 4 * q + e, col = n0 + 16 * t + l16;
        if (row < M && col < N) {
          if constexpr (SPLIT) P[((size_t)blockIdx.y * M + row) * N + col] = v;
          else store_out(Y, (size_t)row * N + col, v + bias_at(bias, col, BF16), BF16);
        }
      }
    });
  };
  run_pass(first_c, 0);
  if constexpr (MULTI)
    for (int p = 1; p < npass; ++p) run_pass(later_c, p);
}

// wq_streamk_q<QB>_<act>_z<zs>_t<NT>_x<XR><s|m>_c<NCH>; split-K form with the
// suffix _k: (X, W, P, S, Z, M, N, K of a slice, ldk), grid (tiles, slices)
#define TM_STREAMK(QB, BF, ACT, ZS, ZDT, NT, XR, MS, MULTI, NCH)                                   \
  extern "C" __global__ __launch_bounds__(512) void                                                \
      wq_streamk_q##QB##_##ACT##_z##ZS##_t##NT##_x##XR##MS##_c##NCH(                              \
          const uint16_t* X, const uint8_t* W, uint16_t* Y, const void* S, const void* Z, int M,   \
          int N, int K, const uint16_t* bias) {                                                   \
    wq_streamk_body<QB, BF, ZDT, NT, XR, NCH, MULTI, false>(X, W, Y, nullptr, S, Z, M, N, K, K,   \
                                                            bias);                                \
  }
#define TM_STREAMK_SPLIT(QB, BF, ACT, ZS, ZDT, XR, MS, MULTI, NCH)                                 \
  extern "C" __global__ __launch_bounds__(512) void                                                \
      wq_streamk_q##QB##_##ACT##_z##ZS##_t1_x##XR##MS##_c##NCH##_k(                               \
          const uint16_t* X, const uint8_t* W, float* P, const void* S, const void* Z, int M,      \
          int N, int K, int ldk) {                                                                \
    wq_streamk_body<QB, BF, ZDT, 1, XR, NCH, MULTI, true>(X, W, nullptr, P, S, Z, M, N, K, ldk,   \
                                                          nullptr);                               \
  }
#define TM_STREAMK_Z(QB, BF, ACT, NT, XR, MS, MULTI, NCH)                          \
  TM_STREAMK(QB, BF, ACT, n, -1, NT, XR, MS, MULTI, NCH)                           \
  TM_STREAMK(QB, BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), NT, XR, MS, MULTI, NCH) \
  TM_STREAMK(QB, BF, ACT, u, 3, NT, XR, MS, MULTI, NCH)
#define TM_STREAMK_A(QB, NT, XR, MS, MULTI, NCH)        \
  TM_STREAMK_Z(QB, false, f16, NT, XR, MS, MULTI, NCH)  \
  TM_STREAMK_Z(QB, true, bf16, NT, XR, MS, MULTI, NCH)
// single pass (XR = 8 for M <= 8, 16 for M <= 16) and multi-pass (M <= 64,
// NT = 1: the first pass's weight words stay in registers)
#define TM_STREAMK_S(QB, NT, NCH)        \
  TM_STREAMK_A(QB, NT, 8, s, false, NCH) \
  TM_STREAMK_A(QB, NT, 16, s, false, NCH)
#define TM_STREAMK_M(QB, NCH) TM_STREAMK_A(QB, 1, 16, m, true, NCH)
// split-K forms (one 16-column tile per workgroup; the slices supply the
// workgroups): single pass x8 / x16, multi-pass x16
#define TM_STREAMK_SPLIT_Z(QB, BF, ACT, XR, MS, MULTI, NCH)                          \
  TM_STREAMK_SPLIT(QB, BF, ACT, n, -1, XR, MS, MULTI, NCH)                           \
  TM_STREAMK_SPLIT(QB, BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), XR, MS, MULTI, NCH) \
  TM_STREAMK_SPLIT(QB, BF, ACT, u, 3, XR, MS, MULTI, NCH)
#define TM_STREAMK_SPLIT_A(QB, XR, MS, MULTI, NCH)        \
  TM_STREAMK_SPLIT_Z(QB, false, f16, XR, MS, MULTI, NCH)  \
  TM_STREAMK_SPLIT_Z(QB, true, bf16, XR, MS, MULTI, NCH)
#define TM_STREAMK_KS(QB, NCH)                   \
  TM_STREAMK_SPLIT_A(QB, 8, s, false, NCH)       \
  TM_STREAMK_SPLIT_A(QB, 16, s, false, NCH)
#define TM_STREAMK_KM(QB, NCH) TM_STREAMK_SPLIT_A(QB, 16, m, true, NCH)
