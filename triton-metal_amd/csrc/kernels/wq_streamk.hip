// W4A16 streaming kernel for long K: 2 <= M <= XR (8 or 16), G = 128,
// 4096 < K <= 128 NCH nwv (make_int4_matmul_kernel, _msl_templates.py:
// 2682-2745; weights [N, K/2] bytes, even k in the low nibble).
//
// The down projections of a model (K = 11008, 14336, ...) have few output
// columns, so the K <= 4096 streaming kernel's 64-column workgroups would
// leave most CUs idle (N = 4096: 64 workgroups).  Here a workgroup owns NT
// 16-column tiles (NT = 1 or 2: one workgroup per CU for N = 4096 / 8192) and
// all of K: its nwv waves (at most 8) take the 128-k chunks c = nwv i + w
// (i < NCH), so at any time they read adjacent segments of the same rows, and
// the waves' partial sums meet in LDS at the end.  Chunks past K / 128 (the
// last round when K / 128 is not a multiple of nwv) re-read the last chunk and
// count with scale 0.
//
// Per chunk a wave copies global -> LDS into a 2-slot ring of its own: the
// tiles' weights (16 rows x 64 B each, every 4 consecutive lanes on one
// 64-byte segment) and the chunk's 128 k of the XR activation rows (256 B per
// row); its scales / zero-points (one dword per column and chunk) go to its
// LDS before the first chunk.  Operands are read back in MFMA order through
// XOR swizzles:
//   weight piece p (16 B) of row r at 64 r + 16 (p ^ ((r >> 2) & 3))
//   X piece p of row r at 256 r + 16 (p ^ (r & 15))
// Products on v_mfma_f32_16x16x32 (A = the activations, B = the exact halves
// OFF + q), the row sums of X on the same MFMA against an all-ones B, and per
// chunk y += s (sum x (OFF + q) - (OFF + z) sum x) in fp32.
#include "common.h"
#include "wq_common.h"

namespace {
// Copies issued after chunk i's (ring of RS slots, C copies per chunk).
constexpr int streamk_ahead(int rs, int nch, int c, int i) {
  int a = 0;
  for (int d = 1; d < rs; ++d)
    if (i + d < nch) a += c;
  return a;
}
}  // namespace

template <bool BF16, int ZDT, int NT, int XR, int NCH>
__device__ __forceinline__ void wq_streamk_body(const uint16_t* X, const uint8_t* W,
                                                uint16_t* __restrict__ Y, const void* S,
                                                const void* Z, int M, int N, int K,
                                                const uint16_t* bias) {
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  constexpr int CK = 128, NJ = CK / 32, XB = 2 * CK, XPR = XB / 16;
  constexpr int XI = XR * XPR / 64;       // X copies (1 KB each) per chunk
  constexpr int RS = 2;                   // ring slots per wave
  constexpr int SLOT = NT * 1024 + XR * XB;
  constexpr int NQ = NCH / 4;             // scale blocks (4 chunks x 16 columns)
  constexpr int SCB = 512 * NT * NQ;      // per-wave scales / zero-points
  constexpr int WB = RS * SLOT + SCB;
  constexpr int C0 = NT + XI;             // copies per chunk
  constexpr int NF = 4 * NT;              // partial sums per lane
  static_assert(NCH % 4 == 0 && NCH >= RS && XI >= 1, "streamk shape");
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwv = blockDim.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * (16 * NT);
  const int nchunk = K >> 7;
  const size_t rowbytes = (size_t)(K >> 1);
  const uint8_t* const wl = lds + wave * WB;
  const uint8_t* const scl = wl + RS * SLOT;
  const uint32_t wlo = __builtin_amdgcn_readfirstlane(lds_off(wl));
  const uint32_t slo = wlo + RS * SLOT;
  float* const red = (float*)(lds + nwv * WB);  // [nwv][8][64]
  auto chunk_of = [&](int i) { return min(nwv * i + wave, nchunk - 1); };

  // ---- scales / zero-points: [qq][t][s, z][64 lanes] dwords; lane (l16, q)
  // holds the dword with chunk 4 qq + q's group of column n0 + 16 t + l16
#pragma unroll
  for (int qq = 0; qq < NQ; ++qq) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t gi = (size_t)min(n0 + 16 * t + l16, N - 1) * nchunk + chunk_of(4 * qq + q);
      const uint32_t dst = slo + 512 * (qq * NT + t);
      dma4((const uint16_t*)S + (gi & ~(size_t)1), dst);
      if constexpr (ZDT == 3) dma4((const uint8_t*)Z + (gi & ~(size_t)3), dst + 256);
      else if constexpr (ZDT >= 0) dma4((const uint16_t*)Z + (gi & ~(size_t)1), dst + 256);
    }
  }
  // ---- weights: lane l -> row r = l / 4 of the tile, piece (l % 4) ^ ((r >> 2) & 3)
  const uint8_t* wsrc[NT];
  {
    const int r = lane >> 2, pc = (lane & 3) ^ ((r >> 2) & 3);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wsrc[t] = W + (size_t)min(n0 + 16 * t + r, N - 1) * rowbytes + 16 * pc;
  }
  // ---- X: copy h, lane l -> row 4 h + l / 16, piece (l % 16) ^ (row & 15)
  auto issue = [&](int i, int slot) {
    const uint32_t sb = wlo + slot * SLOT;
    const int c = chunk_of(i);
    // the slot's previous contents have been read
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int t = 0; t < NT; ++t) dma16(wsrc[t] + 64 * c, sb + 1024 * t);
#pragma unroll
    for (int h = 0; h < XI; ++h) {
      const int rr = 4 * h + (lane >> 4);
      const int pc = (lane & 15) ^ (rr & 15);
      const int m = min(rr, M - 1);
      dma16(X + (size_t)m * K + CK * c + 8 * pc, sb + NT * 1024 + 1024 * h);
    }
  };
  static_for<0, RS>([&](auto IC) { issue(decltype(IC)::value, decltype(IC)::value); });

  const int woff = 64 * l16 + 16 * (q ^ ((l16 >> 2) & 3));
  const int xrow = l16 & (XR - 1);
  const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
  const uint32_t s4 = vgpr_const(4u), s8 = vgpr_const(8u), s12 = vgpr_const(12u);
  const uint32_t one2 = vgpr_const(BF16 ? 0x3F803F80u : 0x3C003C00u);
  const u4_t ones = {one2, one2, one2, one2};
  f4_t y[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) y[t] = f4_t{0.f, 0.f, 0.f, 0.f};

  static_for<0, NCH>([&](auto IC) {
    constexpr int i = decltype(IC)::value;
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<streamk_ahead(RS, NCH, C0, i)>();
    const int slot = i % RS;
    const uint8_t* sp = wl + slot * SLOT;
    u4_t xo[NJ], wv[NT];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int pc = 4 * q + j;
      xo[j] = *(const u4_t*)(sp + NT * 1024 + xrow * XB + 16 * (pc ^ (xrow & 15)));
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) wv[t] = *(const u4_t*)(sp + 1024 * t + woff);
    // the slot takes the chunk RS ahead (issued before the MFMAs: nothing is
    // scheduled across)
    if constexpr (i + RS < NCH) issue(i + RS, slot);
    __builtin_amdgcn_sched_barrier(0);

    f4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
    f4_t xr = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const u4_t xop = perm_x8(xo[j]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const u4_t w = wv[t];
        const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
        acc[t] = mfma16<BF16>(xop, w4_operand_v(wj, vmask, vmagic, s4, s8, s12), acc[t]);
      }
      xr = mfma16<BF16>(xop, ones, xr);
    }
    const int c = nwv * i + wave;
    const bool live = c < nchunk;
    const int cc = live ? c : nchunk - 1;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // dword of lane (l16, i % 4) in block (i / 4, t): this chunk's group of
      // column 16 t + l16
      const uint8_t* sp2 = scl + 512 * ((i / 4) * NT + t) + 4 * (16 * (i % 4) + l16);
      const size_t gi = (size_t)min(n0 + 16 * t + l16, N - 1) * nchunk + cc;
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
    // (pins the chunk's epilogue here)
#pragma unroll
    for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(y[t]));
  });

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
      const int row = 4 * q + e, col = n0 + 16 * t + l16;
      if (row < M && col < N) store_out(Y, (size_t)row * N + col, v + bias_at(bias, col, BF16), BF16);
    }
  });
}

// wq_streamk_<act>_z<zs>_t<NT>_x<XR>_c<NCH>
#define TM_STREAMK(BF, ACT, ZS, ZDT, NT, XR, NCH)                                                \
  extern "C" __global__ __launch_bounds__(512) void wq_streamk_##ACT##_z##ZS##_t##NT##_x##XR##_c##NCH( \
      const uint16_t* X, const uint8_t* W, uint16_t* Y, const void* S, const void* Z, int M,      \
      int N, int K, const uint16_t* bias) {                                                      \
    wq_streamk_body<BF, ZDT, NT, XR, NCH>(X, W, Y, S, Z, M, N, K, bias);                         \
  }
#define TM_STREAMK_Z(BF, ACT, NT, XR, NCH)                          \
  TM_STREAMK(BF, ACT, n, -1, NT, XR, NCH)                           \
  TM_STREAMK(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), NT, XR, NCH) \
  TM_STREAMK(BF, ACT, u, 3, NT, XR, NCH)
#define TM_STREAMK_A(NT, XR, NCH) TM_STREAMK_Z(false, f16, NT, XR, NCH) TM_STREAMK_Z(true, bf16, NT, XR, NCH)
TM_STREAMK_A(1, 8, 8)
TM_STREAMK_A(1, 8, 16)
TM_STREAMK_A(1, 16, 8)
TM_STREAMK_A(1, 16, 16)
TM_STREAMK_A(2, 8, 8)
TM_STREAMK_A(2, 8, 16)
TM_STREAMK_A(2, 16, 8)
TM_STREAMK_A(2, 16, 16)
