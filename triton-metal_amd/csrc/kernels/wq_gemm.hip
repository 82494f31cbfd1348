// Weight-only quantized matmul for gfx950: W8A16 and W4A16.
//
//   Y[m, n] = sum_k X[m, k] * w(n, k),   w(n, k) = (q(n, k) - z(n, g)) * s(n, g)
//
// Semantics follow the reference templates make_int8_matmul_kernel
// (_msl_templates.py:2630-2679: per-output-channel scale/zero, W int8 [N, K])
// and make_int4_matmul_kernel (_msl_templates.py:2682-2745: W [N, K/2] bytes,
// even k in the low nibble, g = k / group_size, n_groups = ceil(K / G)).
// For int4 the byte layout [N, K/2] is the same bytes as uint32 [N, K/8] with
// nibble i of word j holding k = 8j + i.
//
// Arithmetic.  The reference dequantises in fp32 and accumulates in fp32.
// Rounding each dequantised weight to fp16 before the product (as a plain
// "dequantise then MFMA" kernel would) adds ~2^-12 relative error per weight,
// which at K = 4096 with int8 weights exceeds 2e-2.  These kernels keep the
// MFMA operands exact instead and apply the scale to fp32 partial sums:
//   int4: the MFMA weight operand is the exact half OFF + q, made by ORing
//         the nibble under the exponent of OFF (OFF = 1024 for fp16, 128 for
//         bf16).  For every 128-k chunk c (inside one quantisation group):
//           Y += s * (sum_{k in c} x_k (OFF + q_k)  -  (OFF + z) * sum_{k in c} x_k)
//         which equals sum x (q - z) s for any zero-point value.
//   int8: the operand is the exact value q (|q| <= 128 is exact in both fp16
//         and bf16); at the end  Y = s * (sum x q - z * sum x).
// The per-chunk activation sums sum_{k in c} x_k are computed in fp32 while X
// is staged into LDS.
//
// Kernels
//   wq_gemv4l_*  int4, M = 1, K = 4096 / 8192: GEMV with 1 KB linear weight
//                loads per instruction and VALU dot products.
//   wq_gemv4_*   int4, M <= 8 when K = 8192: GEMV, the whole grid resident,
//                per-chunk MFMAs as the weights land.
//   wq_gemv4x2_* int4, 2 <= M <= 6, K = 4096: the GEMV with two column tiles
//                per workgroup and MFMA row sums.
//   wq_gemv8_*   int8, M = 1, K = 4096: the GEMV layout for int8 weights.
//   wq_stream_*  1 < M <= 64 (int4: 128), K <= 4096: weights and X streamed through LDS
//                rings by global -> LDS copies, K split over the waves.
//   wq_skinny_*  other M <= 8 shapes: the whole X[M, K] is staged once per
//                workgroup in LDS; one workgroup owns 16 output columns, its 4
//                waves split K and are reduced through LDS.
//   wq_tiled_*   larger M: 64 x 64 output tiles, X tiles double-buffered in LDS,
//                each wave unpacks its own 16 weight rows in registers.
//   wq_general   any shape / dtype: fp32 arithmetic exactly as the reference
//                template, one wave per output column.
//   wq_dequant   the dequantised weight tile round((float(q) - z) * s).
// Every matmul kernel takes a trailing bias pointer (NULL: none) in the
// activation dtype: Y[m, n] = round(acc + bias[n]), the fp32 epilogue of the
// nn.Linear form X W^T + b (as make_fused_linear_kernel,
// _msl_templates.py:4013-4135, adds its bias).
#include "common.h"
#include "wq_common.h"

// ----------------------------------------------------------------------------
// Skinny kernel: M <= 8.  grid.x = N / 16, block = 256 (4 waves).
// Preconditions (host-checked): N % 16 == 0; K % (4 * CK) == 0 with CK = 128
// (int4) or 64 (int8); int4: G % 128 == 0; LDS: M * (K + 8) * 2 bytes of X
// plus M * K / 128 * 4 bytes of chunk sums (dynamic).
// ----------------------------------------------------------------------------
template <int QB, bool BF16, int SDT, int ZDT, bool VS>
__device__ __forceinline__ void wq_skinny_body(const uint16_t* __restrict__ X,
                                               const uint8_t* __restrict__ W,
                                               uint16_t* __restrict__ Y,
                                               const void* __restrict__ S,
                                               const void* __restrict__ Z, int M, int N, int K,
                                               int G, const uint16_t* bias) {
  extern __shared__ __align__(16) uint16_t xs[];  // [M][K + 8], then float xsum[M][K/128]
  __shared__ f4_t red[3][64];
  constexpr int CK = (QB == 4) ? 128 : 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ldx = K + 8;
  const int nch = K >> 7;  // 128-k chunks per row
  float* xsum = (float*)(xs + (size_t)M * ldx);
  const int n0 = blockIdx.x * 16;

  const int n = n0 + (lane & 15), q = lane >> 4;
  const int m = min(lane & 15, M - 1);
  const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
  int rows[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) rows[e] = min(4 * q + e, M - 1);
  const int kw = K >> 2;
  const int kbeg = wave * kw;
  const size_t rowbytes = (QB == 4) ? (size_t)(K >> 1) : (size_t)K;
  const uint8_t* wrow = W + (size_t)n * rowbytes;
  const size_t ngroups = (QB == 4) ? (size_t)((K + G - 1) / G) : 1;
  const uint16_t* xrow = xs + m * ldx;

  // Load order: the first X pieces, then the first batch of weights (and
  // int4 scales / zero-points), so that staging X only waits for the X loads
  // and overlaps the weight loads' HBM latency.  Loads are unconditional
  // (indices clamped) so each batch issues without branches.
  constexpr int PF = 8;
  const int nsteps = kw / CK;
  const int ppr = K >> 3;        // 16-byte X pieces per row (a multiple of 64)
  constexpr int XU = 4;          // X pieces per thread per staging round

  // X piece p of row r: k = 8p .. 8p+7.  Staging walks (row, piece) without
  // divisions: round u of thread t covers piece t + 256u of each row.
  auto x_load = [&](int r, int p0, u4_t* v) {
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int p = min(p0 + tid + 256 * u, ppr - 1);
      v[u] = ldg128(X + (size_t)r * K + (size_t)p * 8);
    }
  };
  auto x_store = [&](int r, int p0, const u4_t* v) {
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int p = p0 + tid + 256 * u;  // uniform per 16-lane row since ppr % 16 == 0
      if (p < ppr) {
        const float sm = sum16(sum8<BF16>(v[u]));
        if ((p & 15) == 0) xsum[r * nch + (p >> 4)] = sm;
        u4_t w = v[u];
        if constexpr (QB == 4) w = perm_x8(w);
        *(u4_t*)(xs + r * ldx + p * 8) = w;
      }
    }
  };

  u4_t wv[PF];
  // int4 scales / zero-points of the batch: VS = one vector load of 8
  // consecutive groups (G == 128, batch aligned to 8 groups), else per chunk.
  typename Raw<SDT>::T sraw[PF];
  typename Raw<ZDT>::T zraw[PF];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int kc = kbeg + min(s0 + i, nsteps - 1) * CK;
      const size_t boff = (QB == 4) ? (size_t)(kc >> 1) + 16 * q : (size_t)kc + 16 * q;
      wv[i] = ldg128(wrow + boff);
    }
    if constexpr (QB == 4) {
      if constexpr (VS) {
        const size_t g0 = (size_t)n * ngroups + ((kbeg + s0 * CK) >> 7);
        static_assert(sizeof(typename Raw<SDT>::T) == 2, "vector scales need 16-bit scales");
        const u4_t sv = ldg128((const uint16_t*)S + g0);
        const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int i = 0; i < PF; ++i) sraw[i] = (uint16_t)(sw[i >> 1] >> (16 * (i & 1)));
        if constexpr (ZDT == 3) {
          const u2_t zv = ldg64((const uint8_t*)Z + g0);
#pragma unroll
          for (int i = 0; i < PF; ++i) zraw[i] = (uint8_t)((i < 4 ? zv.x : zv.y) >> (8 * (i & 3)));
        } else if constexpr (ZDT >= 0) {
          const u4_t zv = ldg128((const uint16_t*)Z + g0);
          const uint32_t zw[4] = {zv.x, zv.y, zv.z, zv.w};
#pragma unroll
          for (int i = 0; i < PF; ++i) zraw[i] = (uint16_t)(zw[i >> 1] >> (16 * (i & 1)));
        }
      } else {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
          const int kc = kbeg + min(s0 + i, nsteps - 1) * CK;
          const size_t gi = (size_t)n * ngroups + kc / G;
          sraw[i] = ld_raw<SDT>(S, gi);
          zraw[i] = ld_raw<ZDT>(Z, gi);
        }
      }
    }
  };

  {
    u4_t xv[XU];
    x_load(0, 0, xv);
    load_batch(0);
    x_store(0, 0, xv);
  }
  for (int r = 0; r < M; ++r)
    for (int p0 = (r == 0 ? 256 * XU : 0); p0 < ppr; p0 += 256 * XU) {
      u4_t xv[XU];
      x_load(r, p0, xv);
      x_store(r, p0, xv);
    }
  __syncthreads();

  f4_t y = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsteps; s0 += PF) {
    if (s0 > 0) load_batch(s0);
    if constexpr (QB == 4) {
      // one accumulator per chunk, four chunks at a time: consecutive MFMAs
      // are independent
#pragma unroll
      for (int h = 0; h < PF; h += 4) {
        f4_t a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kl = kbeg + min(s0 + h + i, nsteps - 1) * CK + 32 * q;
            const u4_t w = wv[h + i];
            const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
            a[i] = mfma16<BF16>(*(const u4_t*)(xrow + kl + 8 * j), w4_operand(wj, vmask, vmagic), a[i]);
          }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (s0 + h + i < nsteps) {
            const int ch = (kbeg + (s0 + h + i) * CK) >> 7;
            const float sc = raw_to_f32<SDT>(sraw[h + i]);
            const float zb = w4_offset<BF16>() + raw_to_f32<ZDT>(zraw[h + i]);
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] += sc * (a[i][e] - zb * xsum[rows[e] * nch + ch]);
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        if (s0 + i < nsteps) {
          const int kl = kbeg + (s0 + i) * CK + 16 * q;
          y = mfma16<BF16>(*(const u4_t*)(xrow + kl), w8_operand<BF16>(wv[i].x, wv[i].y), y);
          y = mfma16<BF16>(*(const u4_t*)(xrow + kl + 8), w8_operand<BF16>(wv[i].z, wv[i].w), y);
        }
      }
    }
  }

  if (wave > 0) red[wave - 1][lane] = y;
  __syncthreads();
  if (wave == 0) {
    y += red[0][lane] + red[1][lane] + red[2][lane];
    if constexpr (QB == 8) {
      const float sc = ld_typed<SDT>(S, (size_t)n);
      const float z = ld_typed<ZDT>(Z, (size_t)n);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float xt = 0.0f;
        if constexpr (ZDT >= 0)
          for (int c = 0; c < nch; ++c) xt += xsum[rows[e] * nch + c];
        y[e] = sc * (y[e] - z * xt);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int row = 4 * q + e;
      if (row < M) store_out(Y, (size_t)row * N + n, y[e] + bias_at(bias, n, BF16), BF16);
    }
  }
}

// ----------------------------------------------------------------------------
// GEMV kernel for int4, M <= 8, the exact shape K = NW * PF * 128 with
// group size 128 (the common W4A16 decode case).  grid.x = N / 16,
// block = NW waves; wave w owns k = w*PF*128 .. +PF*128 of the workgroup's
// 16 columns.  Everything is unrolled at compile time: PF 16-byte weight
// loads per lane, one vector load of the PF scales (and zero-points) per
// lane, MFMAs chunk by chunk as the weights arrive.  fp16 activations use the
// 5-instruction operand (w4_operand_h) and a second per-chunk sum, of x * off.
// Dynamic LDS: M * (K + 8) * 2 bytes of X, 2 * (K / 128) * 8 * 4 bytes of
// chunk sums laid out [chunk][row 0..7] (sum x, then sum x * off), then the
// workgroup's scales and zero-points (16 rows x K / 128, 2 bytes each).  S
// (and Z) must be 16-byte aligned.
// ----------------------------------------------------------------------------
template <bool BF16, int ZDT, int NW, int PF>
__device__ __forceinline__ void wq_gemv4_body(const uint16_t* __restrict__ X,
                                              const uint8_t* __restrict__ W,
                                              uint16_t* __restrict__ Y,
                                              const uint16_t* __restrict__ S,
                                              const void* __restrict__ Z, int M, int N, int K,
                                              const uint16_t* bias) {
  constexpr int NT = NW * 64;
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ f4_t red[NW - 1][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ldx = K + 8;
  const int nch = K >> 7;
  float* xsum = (float*)(xs + (size_t)M * ldx);  // [nch][8]
  float* xoff = xsum + nch * 8;                  // fp16: [nch][8] sums of x * off
  uint16_t* sst = (uint16_t*)(xoff + nch * 8);   // scales of the 16 columns [16][nch]
  uint16_t* zst = sst + 16 * nch;                // zero-points [16][nch] (bytes if uint8)
  const int n = blockIdx.x * 16 + (lane & 15), q = lane >> 4;
  const int m = min(lane & 15, M - 1);
  const int kbeg = wave * (PF * 128);
  const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
  const uint32_t vmask_hi = vgpr_const(0x00F000F0u), vmagic_hi = vgpr_const(0x54005400u);

  // 1. first X row pieces (PF / 4 per thread), this workgroup's scales and
  //    zero-points (16 rows x nch, one contiguous block each), 2. weights,
  //    3. stage.  The few small loads go first so that each chunk's MFMAs
  //    can start as soon as that chunk's weights arrive.
  constexpr int XP = PF / 4;  // pieces per thread per row: K / 8 / NT
  u4_t xv[XP];
#pragma unroll
  for (int u = 0; u < XP; ++u) xv[u] = ldg128(X + (size_t)(tid + NT * u) * 8);
  const int sbytes = 32 * nch;
  const int zbytes = ZDT == 3 ? 16 * nch : 32 * nch;
  u4_t sv = {0u, 0u, 0u, 0u}, zv = {0u, 0u, 0u, 0u};
  if (16 * tid < sbytes) sv = ldg128((const uint8_t*)S + (size_t)blockIdx.x * sbytes + 16 * tid);
  if constexpr (ZDT >= 0)
    if (16 * tid < zbytes) zv = ldg128((const uint8_t*)Z + (size_t)blockIdx.x * zbytes + 16 * tid);

  const uint8_t* wrow = W + (size_t)n * (K >> 1) + (kbeg >> 1) + 16 * q;
  u4_t wv[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) wv[i] = ldg128(wrow + 64 * i);

  auto stage = [&](int r, const u4_t* v) {
#pragma unroll
    for (int u = 0; u < XP; ++u) {
      const int p = tid + NT * u;
      const float sm = sum16(sum8<BF16>(v[u]));
      if ((p & 15) == 0) xsum[(p >> 4) * 8 + r] = sm;
      if constexpr (!BF16) {
        const float so = sum16(sumoff8_h(v[u]));
        if ((p & 15) == 0) xoff[(p >> 4) * 8 + r] = so;
      }
      *(u4_t*)(xs + r * ldx + p * 8) = perm_x8(v[u]);
    }
  };
  stage(0, xv);
  if (16 * tid < sbytes) *(u4_t*)((uint8_t*)sst + 16 * tid) = sv;
  if constexpr (ZDT >= 0)
    if (16 * tid < zbytes) *(u4_t*)((uint8_t*)zst + 16 * tid) = zv;
  for (int r = 1; r < M; ++r) {
#pragma unroll
    for (int u = 0; u < XP; ++u) xv[u] = ldg128(X + (size_t)r * K + (size_t)(tid + NT * u) * 8);
    stage(r, xv);
  }
  __syncthreads();

  const uint16_t* xa = xs + m * ldx + kbeg + 32 * q;
  const float* xsr = xsum + (kbeg >> 7) * 8 + 4 * (q & 1);
  // Chunk by chunk: 4 MFMAs into one of two alternating accumulators, then the
  // chunk's scale / zero-point correction folded into y (keeps the register
  // count within 8 waves per SIMD).
  f4_t y = {0.f, 0.f, 0.f, 0.f};
  f4_t a2[2];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    f4_t& a = a2[i & 1];
    a = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u4_t w = wv[i];
      const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
      const u4_t wop = BF16 ? w4_operand(wj, vmask, vmagic)
                            : w4_operand_h(wj, vmask, vmask_hi, vmagic, vmagic_hi);
      a = mfma16<BF16>(*(const u4_t*)(xa + 128 * i + 8 * j), wop, a);
    }
    const int gi = (lane & 15) * nch + (kbeg >> 7) + i;
    const float sc = raw_to_f32<SDT>(sst[gi]);
    float z = 0.0f;
    if constexpr (ZDT == 3) z = (float)((const uint8_t*)zst)[gi];
    else if constexpr (ZDT >= 0) z = raw_to_f32<ZDT>(zst[gi]);
    const f4_t xv4 = *(const f4_t*)(xsr + 8 * i);
    if constexpr (BF16) {
      const float zb = w4_offset<BF16>() + z;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] += sc * (a[e] - zb * xv4[e]);
    } else {
      const f4_t xo4 = *(const f4_t*)(xsr + nch * 8 + 8 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] += sc * (a[e] - xo4[e] - z * xv4[e]);
    }
  }

  if (wave > 0) red[wave - 1][lane] = y;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < NW - 1; ++w) y += red[w][lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      if (row < M) store_out(Y, (size_t)row * N + n, y[e] + bias_at(bias, n, BF16), BF16);
    }
  }
}

// ----------------------------------------------------------------------------
// Linear int4 GEMV, M = 1, K = 2048 * NS, G = 128: wq_gemv4l_<act>_z<zs>_k<NS>.
// grid.x = N / 16, block = 512 (8 waves); the workgroup owns 16 weight rows
// (16 * K / 2 contiguous bytes).  Every weight load instruction reads 1 KB of
// one row (lane l: bytes 1024 h + 16 l): whole 128-byte lines, consecutive
// lines per instruction, non-temporal - the pattern that streams fastest
// (a plain read of the C3 weights this way takes 6.5 us on a box where the
// 16 rows x 64 B pattern of the MFMA GEMV takes 7.4 us).  Wave w takes K
// slice h = w % NS of rows RW * (w / NS) .. +RW (RW = 2 NS), so each lane's
// 32 activations x[2048 h + 32 l .. +32] serve all its rows and its 32 k lie
// in one quantisation group g = 16 h + l / 4.  X comes straight from global
// memory (L2-resident after the first workgroups): staging it (and the scales)
// through LDS behind a workgroup barrier measured slower.
// M = 1 leaves 15 of 16 MFMA rows idle, so the dot products run on the VALU:
// the exact half OFF + q (fp16: a nibble ORed under 0x6400 is 1024 + q, under
// 0x5400 at bits 4..7 it is 64 + q; bf16: under 0x4300 it is 128 + q) times
// pairs of x with v_dot2_f32_{f16,bf16} into fp32, then per row
// s * (sum x (OFF + q) - sum x OFF - z sum x).  The 64 lanes of a row are
// summed with DPP / permlane swaps and the NS slices through LDS.
// ----------------------------------------------------------------------------
template <bool BF16, int ZDT, int NS>
__device__ __forceinline__ void wq_gemv4l_body(const uint16_t* __restrict__ X,
                                               const uint8_t* __restrict__ W,
                                               uint16_t* __restrict__ Y,
                                               const uint16_t* __restrict__ S,
                                               const void* __restrict__ Z, int N,
                                               const uint16_t* bias) {
  constexpr int K = 2048 * NS, RB = K / 2, NG = K / 128, RW = 2 * NS;
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  __shared__ float red[NS][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = wave % NS, r0 = RW * (wave / NS);
  const int n0 = blockIdx.x * 16;
  const int g = 16 * h + (lane >> 2);

  // activations first (short L2 latency, needed before any dot), then the
  // weights, then the scales / zero-points (needed last)
  u4_t xr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xr[j] = ldg128(X + 2048 * h + 32 * lane + 8 * j);
  const uint8_t* wb = W + (size_t)(n0 + r0) * RB + 1024 * h + 16 * lane;
  u4_t wv[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i)
    wv[i] = __builtin_nontemporal_load((const u4_t*)(wb + (size_t)i * RB));
  float sc[RW], zp[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const size_t gi = (size_t)(n0 + r0 + i) * NG + g;
    sc[i] = raw_to_f32<SDT>(S[gi]);
    zp[i] = 0.0f;
    if constexpr (ZDT == 3) zp[i] = (float)((const uint8_t*)Z)[gi];
    else if constexpr (ZDT >= 0) zp[i] = raw_to_f32<ZDT>(((const uint16_t*)Z)[gi]);
  }

  // x as operand pairs (x0, x4) (x1, x5) (x2, x6) (x3, x7) per 8-k word, and
  // its sums
  u4_t xp[4];
  float xsum = 0.0f, xoff = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xp[j] = perm_x8(xr[j]);
    xsum += sum8<BF16>(xr[j]);
    if constexpr (!BF16) xoff += sumoff8_h(xr[j]);
  }
  if constexpr (BF16) xoff = w4_offset<true>() * xsum;

  const uint32_t m_lo = vgpr_const(0x000F000Fu), g_lo = vgpr_const(w4_magic<BF16>());
  const uint32_t m_hi = vgpr_const(0x00F000F0u), g_hi = vgpr_const(0x54005400u);
  float part[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (BF16) {
        // (128 + n0, 128 + n4), ...; the pairs are taken from 8-element
        // vectors (a bit cast of one dword to a bf16 pair is mis-selected by
        // this compiler: every such dot reads the first dword)
        const b8_t op = __builtin_bit_cast(b8_t, w4_operand(wd[j], m_lo, g_lo));
        const b8_t xb = __builtin_bit_cast(b8_t, xp[j]);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(op, op, 0, 1),
                                            __builtin_shufflevector(xb, xb, 0, 1), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(op, op, 2, 3),
                                            __builtin_shufflevector(xb, xb, 2, 3), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(op, op, 4, 5),
                                            __builtin_shufflevector(xb, xb, 4, 5), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(op, op, 6, 7),
                                            __builtin_shufflevector(xb, xb, 6, 7), a, false);
      } else {
        const u4_t op = w4_operand_h(wd[j], m_lo, m_hi, g_lo, g_hi);
        a = __builtin_amdgcn_fdot2(as_h2(op.x), as_h2(xp[j].x), a, false);
        a = __builtin_amdgcn_fdot2(as_h2(op.y), as_h2(xp[j].y), a, false);
        a = __builtin_amdgcn_fdot2(as_h2(op.z), as_h2(xp[j].z), a, false);
        a = __builtin_amdgcn_fdot2(as_h2(op.w), as_h2(xp[j].w), a, false);
      }
    }
    part[i] = sc[i] * (a - xoff - zp[i] * xsum);
  }
  // sum each row's 64 lanes: DPP within rows of 16, then across the 4 rows
#pragma unroll
  for (int i = 0; i < RW; ++i) part[i] = wave_sum(part[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < RW; ++i) red[h][r0 + i] = part[i];
  }
  __syncthreads();
  if (tid < 16) {
    float y = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) y += red[s2][tid];
    const int n = n0 + tid;
    store_out(Y, n, y + bias_at(bias, n, BF16), BF16);
  }
}

// ----------------------------------------------------------------------------
// Linear int8 GEMV, M = 1, K = 4096, fp16 activations, per-channel scales:
// the int4 linear GEMV's layout for int8 weights.  grid.x = N / 16, block =
// 8 waves; wave w owns k = 1024 (w % 4) .. +1024 of the 8 rows 8 (w / 4) ..
// of the workgroup's 16, so each of its 8 weight loads reads 1 KB of one row
// (16 bytes per lane, non-temporal: the weights are read once).  x straight
// from L2 (2 x 16 bytes per lane).  A byte q ^ 0x80 under the exponent byte
// 0x64 is the exact half 1152 + q; pairs of those times pairs of x with
// v_dot2_f32_f16, and per row s * (sum x (1152 + q) - (1152 + z) sum x).
// The 8 rows' lane sums are halved across lanes (permlane swaps over lane
// bits 5, then 4), each lane row's remaining 2 with DPP, the 4 slices through
// LDS.
// ----------------------------------------------------------------------------
template <int ZDT>
__device__ __forceinline__ void wq_gemv8l_body(const uint16_t* __restrict__ X,
                                               const uint8_t* __restrict__ W,
                                               uint16_t* __restrict__ Y,
                                               const uint16_t* __restrict__ S,
                                               const void* __restrict__ Z, int N,
                                               const uint16_t* bias) {
  constexpr int K = 4096, NS = 4, RW = 8;
  __shared__ float red[NS][16];
  __shared__ float xred[NS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = wave % NS, r0 = RW * (wave / NS);
  const int n0 = blockIdx.x * 16;

  const u4_t x0 = ldg128(X + 1024 * h + 16 * lane), x1 = ldg128(X + 1024 * h + 16 * lane + 8);
  const uint8_t* wb = W + (size_t)(n0 + r0) * K + 1024 * h + 16 * lane;
  u4_t wv[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i)
    wv[i] = __builtin_nontemporal_load((const u4_t*)(wb + (size_t)i * K));

  const uint32_t xd[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  const h2_t one = {(half_t)1.0f, (half_t)1.0f};
  float xs = 0.0f;
#pragma unroll
  for (int d = 0; d < 8; ++d) xs = __builtin_amdgcn_fdot2(as_h2(xd[d]), one, xs, false);

  const uint32_t e = vgpr_const(0x64646464u);
  float part[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = wd[j] ^ 0x80808080u;  // q + 128
      a = __builtin_amdgcn_fdot2(as_h2(perm_b32(e, u, 0x04010400u)), as_h2(xd[2 * j]), a, false);
      a = __builtin_amdgcn_fdot2(as_h2(perm_b32(e, u, 0x04030402u)), as_h2(xd[2 * j + 1]), a,
                                 false);
    }
    part[i] = a - 1152.0f * xs;
  }
  // rows 0..3 stay on lanes 0..31, 4..7 on lanes 32..63; then pairs by lane bit 4
  float p4[4], p2[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) p4[i] = fold_swap<32>(part[i], part[i + 4]);
#pragma unroll
  for (int i = 0; i < 2; ++i) p2[i] = fold_swap<16>(p4[i], p4[i + 2]);
  p2[0] = row16_sum(p2[0]);
  p2[1] = row16_sum(p2[1]);
  if ((lane & 15) == 0) {
    const int r = r0 + 4 * (lane >> 5) + 2 * ((lane >> 4) & 1);
    red[h][r] = p2[0];
    red[h][r + 1] = p2[1];
  }
  if constexpr (ZDT >= 0) {
    xs = wave_sum(xs);
    if (wave < NS && lane == 0) xred[h] = xs;
  }
  __syncthreads();
  if (tid < 16) {
    const int n = n0 + tid;
    float y = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) y += red[s2][tid];
    if constexpr (ZDT >= 0)
      y -= ld_typed<ZDT>(Z, (size_t)n) * (xred[0] + xred[1] + xred[2] + xred[3]);
    store_out(Y, n, ld_typed<TM_DT_F16>(S, (size_t)n) * y + bias_at(bias, n, false), false);
  }
}

// ----------------------------------------------------------------------------
// int8 GEMV, M <= 8 (the exact shape K = NW * PF * 64): the int4 GEMV's layout
// for int8 weights.  grid.x = N / 16, block = NW waves; wave w owns
// k = w*PF*64 .. +PF*64 of the workgroup's 16 columns.  Lane (n, q) loads
// 16 bytes at byte 64 i + 16 q of its column's segment (i < PF), so its MFMA
// steps (i, h) cover k = 64 i + 16 q + 8 h + e in natural order - the order in
// which X is staged and read.  Per-channel scale (and zero-point) once at the
// end: Y = s * (sum x q - z * sum x), sum x from MFMAs of the X operands with
// a ones operand.  Dynamic LDS: M * (K + 8) * 2 bytes of X.
// ----------------------------------------------------------------------------
template <bool BF16, int ZDT, int NW, int PF>
__device__ __forceinline__ void wq_gemv8_body(const uint16_t* __restrict__ X,
                                              const uint8_t* __restrict__ W,
                                              uint16_t* __restrict__ Y,
                                              const uint16_t* __restrict__ S,
                                              const void* __restrict__ Z, int M, int N, int K,
                                              const uint16_t* bias) {
  constexpr int NT = NW * 64;
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ f4_t red[NW - 1][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ldx = K + 8;
  const int n = blockIdx.x * 16 + (lane & 15), q = lane >> 4;
  const int m = min(lane & 15, M - 1);
  const int kbeg = wave * (PF * 64);

  // 1. row 0 of X, this lane's channel scale / zero-point, 2. the weights,
  // 3. stage X (later rows one at a time)
  constexpr int XP = PF / 8;  // pieces per thread per row: K / 8 / NT
  u4_t xv[XP];
#pragma unroll
  for (int u = 0; u < XP; ++u) xv[u] = ldg128(X + (size_t)(tid + NT * u) * 8);
  const float sc = ld_typed<SDT>(S, (size_t)n);
  const float z = ld_typed<ZDT>(Z, (size_t)n);
  const uint8_t* wrow = W + (size_t)n * K + kbeg + 16 * q;
  u4_t wv[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) wv[i] = ldg128(wrow + 64 * i);
#pragma unroll
  for (int u = 0; u < XP; ++u) *(u4_t*)(xs + (tid + NT * u) * 8) = xv[u];
  for (int r = 1; r < M; ++r) {
#pragma unroll
    for (int u = 0; u < XP; ++u)
      xv[u] = ldg128(X + (size_t)r * K + (size_t)(tid + NT * u) * 8);
#pragma unroll
    for (int u = 0; u < XP; ++u) *(u4_t*)(xs + r * ldx + (tid + NT * u) * 8) = xv[u];
  }
  __syncthreads();

  const uint16_t* xa = xs + m * ldx + kbeg + 16 * q;
  const uint32_t one2 = vgpr_const(BF16 ? 0x3F803F80u : 0x3C003C00u);
  const u4_t ones = {one2, one2, one2, one2};
  f4_t y = {0.f, 0.f, 0.f, 0.f}, xsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < PF; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u4_t xo = *(const u4_t*)(xa + 64 * i + 8 * h);
      const u4_t w = wv[i];
      y = mfma16<BF16>(xo, w8_operand<BF16>(h ? w.z : w.x, h ? w.w : w.y), y);
      if constexpr (ZDT >= 0) xsum = mfma16<BF16>(xo, ones, xsum);
    }
  }
  if constexpr (ZDT >= 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] -= z * xsum[e];
  }

  if (wave > 0) red[wave - 1][lane] = y;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < NW - 1; ++w) y += red[w][lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      if (row < M)
        store_out(Y, (size_t)row * N + n, sc * y[e] + bias_at(bias, n, BF16), BF16);
    }
  }
}

// ----------------------------------------------------------------------------
// Multi-tile GEMV for 2 <= M <= 8 (int4, the exact shape K = NW * PF * 128,
// G = 128): the GEMV above with NTL 16-column tiles per workgroup, so that the
// M rows of X staged in LDS (M * (K + 8) * 2 bytes) serve NTL tiles and the
// whole grid is resident (N = 14336, NTL = 2: 448 workgroups, two per CU).
// All M rows of X are loaded before any is staged (one round trip, not M),
// and staging is a permute and a store: the per-chunk row sums of the
// zero-point correction (sum x and, for fp16, sum x * offset) come from
// MFMAs of the X operands with constant B operands (ones; the operand's
// offsets 1024 / 64 per position), already in the accumulator layout.
// Wave w owns k = w*PF*128 .. +PF*128 of every tile; the waves' partial sums
// are reduced through the X region of LDS once every wave is past its reads.
// Dynamic LDS: max(M * (K + 8) * 2 bytes of X followed by the scales and
// zero-points of the NTL * 16 columns (NTL * 16 rows x K / 128 each), the
// (NW - 1) * NTL KB of the reduction).  S (and Z) must be 16-byte aligned.
// ----------------------------------------------------------------------------
template <bool BF16, int ZDT, int NW, int PF, int NTL>
__device__ __forceinline__ void wq_gemv4x2_body(const uint16_t* __restrict__ X,
                                                const uint8_t* __restrict__ W,
                                                uint16_t* __restrict__ Y,
                                                const uint16_t* __restrict__ S,
                                                const void* __restrict__ Z, int M, int N, int K,
                                                const uint16_t* bias) {
  constexpr int NT = NW * 64;
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  constexpr int MX = 8;
  extern __shared__ __align__(16) uint16_t xs[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ldx = K + 8;
  const int nch = K >> 7;
  uint16_t* sst = xs + (size_t)M * ldx;          // scales of the columns [16 NTL][nch]
  uint16_t* zst = sst + 16 * NTL * nch;          // zero-points [16 NTL][nch] (bytes if uint8)
  const int nb = blockIdx.x * 16 * NTL, q = lane >> 4;
  const int m = min(lane & 15, M - 1);
  const int kbeg = wave * (PF * 128);
  const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
  const uint32_t vmask_hi = vgpr_const(0x00F000F0u), vmagic_hi = vgpr_const(0x54005400u);

  // 1. every row of X, the scales and zero-points of the columns, 2. the
  //    weights of every tile, 3. stage X.
  constexpr int XP = PF / 4;  // pieces per thread per row: K / 8 / NT
  u4_t xv[MX][XP];
#pragma unroll
  for (int r = 0; r < MX; ++r)
#pragma unroll
    for (int u = 0; u < XP; ++u)
      xv[r][u] = r < M ? ldg128(X + (size_t)r * K + (size_t)(tid + NT * u) * 8)
                       : u4_t{0u, 0u, 0u, 0u};
  // (at most NT * 16 bytes of each: NTL * 32 * nch <= 8 KB)
  const int sbytes = 32 * NTL * nch;
  const int zbytes = ZDT == 3 ? 16 * NTL * nch : 32 * NTL * nch;
  u4_t sv = {0u, 0u, 0u, 0u}, zv = {0u, 0u, 0u, 0u};
  if (16 * tid < sbytes) sv = ldg128((const uint8_t*)S + (size_t)blockIdx.x * sbytes + 16 * tid);
  if constexpr (ZDT >= 0)
    if (16 * tid < zbytes) zv = ldg128((const uint8_t*)Z + (size_t)blockIdx.x * zbytes + 16 * tid);

  u4_t wv[NTL][PF];
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
    const uint8_t* wrow =
        W + (size_t)(nb + 16 * t + (lane & 15)) * (K >> 1) + (kbeg >> 1) + 16 * q;
#pragma unroll
    for (int i = 0; i < PF; ++i) wv[t][i] = ldg128(wrow + 64 * i);
  }

#pragma unroll
  for (int r = 0; r < MX; ++r) {
    if (r < M) {
#pragma unroll
      for (int u = 0; u < XP; ++u) {
        const int p = tid + NT * u;
        *(u4_t*)(xs + r * ldx + p * 8) = perm_x8(xv[r][u]);
      }
    }
  }
  if (16 * tid < sbytes) *(u4_t*)((uint8_t*)sst + 16 * tid) = sv;
  if constexpr (ZDT >= 0)
    if (16 * tid < zbytes) *(u4_t*)((uint8_t*)zst + 16 * tid) = zv;
  __syncthreads();

  const uint16_t* xa = xs + m * ldx + kbeg + 32 * q;
  // constant B operands: ones, and (fp16) the operand's offset per position
  const uint32_t one2 = vgpr_const(BF16 ? 0x3F803F80u : 0x3C003C00u);
  const u4_t ones = {one2, one2, one2, one2};
  const uint32_t o_lo = vgpr_const(0x64006400u), o_hi = vgpr_const(0x54005400u);
  const u4_t offs = {o_lo, o_hi, o_lo, o_hi};
  f4_t y[NTL];
#pragma unroll
  for (int t = 0; t < NTL; ++t) y[t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    u4_t xo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xo[j] = *(const u4_t*)(xa + 128 * i + 8 * j);
    // this chunk's row sums, sum x and (fp16) sum x * offset, for rows 4 q + e
    f4_t xv4 = {0.f, 0.f, 0.f, 0.f}, xo4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv4 = mfma16<BF16>(xo[j], ones, xv4);
      if constexpr (!BF16) xo4 = mfma16<BF16>(xo[j], offs, xo4);
    }
#pragma unroll
    for (int t = 0; t < NTL; ++t) {
      f4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u4_t w = wv[t][i];
        const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
        const u4_t wop = BF16 ? w4_operand(wj, vmask, vmagic)
                              : w4_operand_h(wj, vmask, vmask_hi, vmagic, vmagic_hi);
        a = mfma16<BF16>(xo[j], wop, a);
      }
      const int gi = (16 * t + (lane & 15)) * nch + (kbeg >> 7) + i;
      const float sc = raw_to_f32<SDT>(sst[gi]);
      float z = 0.0f;
      if constexpr (ZDT == 3) z = (float)((const uint8_t*)zst)[gi];
      else if constexpr (ZDT >= 0) z = raw_to_f32<ZDT>(zst[gi]);
      if constexpr (BF16) {
        const float zb = w4_offset<BF16>() + z;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[t][e] += sc * (a[e] - zb * xv4[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[t][e] += sc * (a[e] - xo4[e] - z * xv4[e]);
      }
    }
  }

  // reduction over the waves through the X region ((NW - 1) * NTL KB <= M * ldx * 2)
  __syncthreads();
  f4_t* red = (f4_t*)xs;  // [NW - 1][NTL][64]
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NTL; ++t) red[((wave - 1) * NTL + t) * 64 + lane] = y[t];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < NTL; ++t) {
#pragma unroll
      for (int w = 0; w < NW - 1; ++w) y[t] += red[(w * NTL + t) * 64 + lane];
      const int n = nb + 16 * t + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * q + e;
        if (row < M) store_out(Y, (size_t)row * N + n, y[t][e] + bias_at(bias, n, BF16), BF16);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Streaming kernel: 1 < M <= 128.  A workgroup owns NT 16-column tiles (int4:
// 4, int8: 3) and all M rows; its nwv = K / 512 waves (at most 8) split K and
// are reduced through LDS after each pass of 16 rows.  Wave w takes the chunks
// c = nwv i + w (i = 0, 1, ...), so that at any time the waves of a workgroup
// read adjacent segments of the same weight rows.
// Weights and X reach LDS by global -> LDS copies issued in an order where
// every 4 consecutive lanes read one 64-byte segment: the vector memory path
// serves such groups at about three times the rate of the MFMA operand order,
// in which 4 consecutive lanes touch 4 different rows.  The operands are read
// back in MFMA order through XOR swizzles that keep those reads free of bank
// conflicts.  Each wave streams its chunks (64 weight bytes per row: 128 k for
// int4, 64 k for int8) through a ring of RS slots of its own LDS:
//   slot  [NT][16 rows][64 B] weights, then [XR rows][XB] X
//         weight piece p (16 B) of row r at 64 r + 16 (p ^ ((r >> 2) & 3))
//         X piece p of row r at r XB + 16 (p ^ xsw(r))
// and waits for each with an explicit vmcnt (copies complete in issue order).
// The single-pass kernel (M <= XR) takes each chunk's weights from LDS; the
// multi-pass one keeps the first pass's weight registers for the later passes,
// which stream X only.  Scales and zero-points are copied to each wave's LDS
// ahead of its first chunks (int4: for lane (l16, q) the dword holding the
// value of column 16 t + l16 in group nwv q + wave, the group of the wave's
// chunk q; int8: the per-channel values).
// int4 (group 128 = one chunk):  Y += s * (sum x (OFF + q) - (OFF + z) sum x)
// int8:                          Y  = s * (sum x q - z sum x)
// sum x per chunk comes from v_dot2 on the X operands.
// Dynamic LDS: nwv * (RS * SLOT + SCB) + nwv * 2 KB (reduction), SCB = 2 KB
// (int4) or 1 KB (int8) of scales / zero-points.
// ----------------------------------------------------------------------------
namespace {
// Copies issued after chunk i's (copies per item: c0 in the first pass, c1
// later; rs - 1 items run ahead, the ones past the pass end only if another
// pass follows).
constexpr int stream_ahead(int rs, int nch, int c0, int c1, bool first, int i, bool next) {
  int a = 0;
  for (int d = 1; d < rs; ++d) {
    if (i + d < nch) a += first ? c0 : c1;
    else if (next) a += c1;
  }
  return a;
}
}  // namespace

template <int QB, bool BF16, int SDT, int ZDT, int NT, int XR, bool MULTI>
__device__ __forceinline__ void wq_stream_body(const uint16_t* X, const uint8_t* W,
                                               uint16_t* __restrict__ Y, const void* S,
                                               const void* Z, int M, int N, int K,
                                               const uint16_t* bias) {
  constexpr int KS = 512;                 // k per wave
  constexpr int CK = QB == 4 ? 128 : 64;  // k per chunk: 64 weight bytes of a row
  constexpr int NCH = KS / CK;            // chunks per wave
  constexpr int NJ = CK / 32;             // MFMA k-steps per chunk
  constexpr int XB = 2 * CK;              // X bytes per row per chunk
  constexpr int XPR = XB / 16;            // 16-byte pieces per X row per chunk
  constexpr int XI = XR * XPR / 64;       // X copies (1 KB each) per chunk
  constexpr int RS = QB == 4 ? 2 : 3;     // ring slots per wave
  constexpr int SLOT = NT * 1024 + XR * XB;
  constexpr int SCB = QB == 4 ? 512 * NT : 1024;  // per-wave scales / zero-points
  constexpr int WB = RS * SLOT + SCB;     // per-wave LDS: ring, scales
  constexpr int C0 = NT + XI, C1 = XI;    // copies per first-pass / later-pass chunk
  constexpr int NF = 4 * NT;              // partial sums per lane per pass
  static_assert(XI >= 1 && NCH >= RS && (QB == 8 || NT == 4), "stream kernel shape");
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwv = blockDim.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * (16 * NT);
  const int npass = MULTI ? (M + 15) >> 4 : 1;
  const size_t rowbytes = QB == 4 ? (size_t)(K >> 1) : (size_t)K;
  const uint8_t* const wl = lds + wave * WB;  // this wave's ring
  const uint8_t* const scl = wl + RS * SLOT;  // its scales / zero-points
  const uint32_t wlo = __builtin_amdgcn_readfirstlane(lds_off(wl));
  const uint32_t slo = wlo + RS * SLOT;
  float* const red = (float*)(lds + nwv * WB);  // [nwv][8][64]

  // ---- copies
  // Scales / zero-points.  int4: [t][s, z][64 lanes] dwords, lane (l16, q)
  // holding group g = nwv q + wave of column n0 + 16 t + l16 (its half / byte
  // is fixed by g, as K / 128 is a multiple of 4).  int8: dword c holds
  // columns n0 + 2c, 2c + 1 (u8 zero-points: 4c .. 4c + 3).
  if constexpr (QB == 4) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t gi = (size_t)min(n0 + 16 * t + l16, N - 1) * (K >> 7) + nwv * q + wave;
      dma4((const uint16_t*)S + (gi & ~(size_t)1), slo + 512 * t);
      if constexpr (ZDT == 3) dma4((const uint8_t*)Z + (gi & ~(size_t)3), slo + 512 * t + 256);
      else if constexpr (ZDT >= 0) dma4((const uint16_t*)Z + (gi & ~(size_t)1), slo + 512 * t + 256);
    }
  } else {
    const int c2 = min((n0 >> 1) + lane, (N >> 1) - 1);
    dma4((const uint16_t*)S + 2 * c2, slo);
    if constexpr (ZDT == 3) dma4((const uint8_t*)Z + 4 * min((n0 >> 2) + lane, (N >> 2) - 1), slo + 256);
    else if constexpr (ZDT >= 0) dma4((const uint16_t*)Z + 2 * c2, slo + 256);
  }
  // weights: lane l -> row r = l / 4 of the tile, piece (l % 4) ^ ((r >> 2) & 3)
  // of the 64-byte segment of chunk c = nwv i + wave
  const uint8_t* wsrc[NT];
  {
    const int r = lane >> 2, pc = (lane & 3) ^ ((r >> 2) & 3);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wsrc[t] = W + (size_t)min(n0 + 16 * t + r, N - 1) * rowbytes + 64 * wave + 16 * pc;
  }
  auto xsw = [](int r) { return QB == 4 ? (r & 15) : ((r >> 1) & 7); };
  // X: copy h, lane l -> row h (64 / XPR) + l / XPR, piece (l % XPR) ^ xsw(row)
  auto issue = [&](auto FIRSTC, int p, int i, int slot) {
    const uint32_t sb = wlo + slot * SLOT;
    // the slot's previous contents have been read
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (decltype(FIRSTC)::value) {
#pragma unroll
      for (int t = 0; t < NT; ++t) dma16(wsrc[t] + 64 * nwv * i, sb + 1024 * t);
    }
#pragma unroll
    for (int h = 0; h < XI; ++h) {
      const int rr = h * (64 / XPR) + lane / XPR;
      const int pc = (lane % XPR) ^ xsw(rr);
      const int m = min(16 * p + rr, M - 1);
      dma16(X + (size_t)m * K + CK * (nwv * i + wave) + 8 * pc, sb + NT * 1024 + 1024 * h);
    }
  };
  const std::integral_constant<bool, true> first_c;
  const std::integral_constant<bool, false> later_c;
  static_for<0, RS>([&](auto IC) { issue(first_c, 0, decltype(IC)::value, decltype(IC)::value); });

  // operand offsets in a slot: weight piece q of row l16; X piece of row l16
  // for k-step j (int4 4q + j, int8 2q + j, matching the weight dwords)
  const int woff = 64 * l16 + 16 * (q ^ ((l16 >> 2) & 3));
  const int xrow = l16 & (XR - 1);
  u4_t wv[NT][NCH];

  // One pass: 16 rows of X against the slice's weights.  The first pass is
  // peeled off the loop (it also reads the weights, and its waits count
  // different copies).
  auto run_pass = [&](auto FIRSTC, int p) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(FIRSTC)::value;
    // made per pass (volatile asm) so that the weight conversions below stay
    // in the pass loop
    const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
    const uint32_t s4 = vgpr_const(4u), s8 = vgpr_const(8u), s12 = vgpr_const(12u);
    const bool next = MULTI && p + 1 < npass;
    f4_t y[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) y[t] = f4_t{0.f, 0.f, 0.f, 0.f};
    // row sums of X (element e: row 4 q + e) from MFMAs against an all-ones
    // B operand, already in the accumulator layout: int8 over the pass, int4
    // per chunk
    const uint32_t one2 = vgpr_const(BF16 ? 0x3F803F80u : 0x3C003C00u);
    const u4_t ones = {one2, one2, one2, one2};
    f4_t xacc = f4_t{0.f, 0.f, 0.f, 0.f};
    static_for<0, NCH>([&](auto IC) {
      constexpr int i = decltype(IC)::value;
      __builtin_amdgcn_sched_barrier(0);
      if (next) wait_vm<stream_ahead(RS, NCH, C0, C1, FIRST, i, true)>();
      else wait_vm<stream_ahead(RS, NCH, C0, C1, FIRST, i, false)>();
      const int slot = MULTI ? (p * NCH + i) % RS : i % RS;
      const uint8_t* sp = wl + slot * SLOT;
      u4_t xo[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int pc = QB == 4 ? 4 * q + j : 2 * q + j;
        xo[j] = *(const u4_t*)(sp + NT * 1024 + xrow * XB + 16 * (pc ^ xsw(xrow)));
      }
      if constexpr (FIRST) {
#pragma unroll
        for (int t = 0; t < NT; ++t) wv[t][i] = *(const u4_t*)(sp + 1024 * t + woff);
      }
      // the slot takes the chunk RS ahead (issued before the MFMAs: nothing
      // is scheduled across)
      if constexpr (i + RS < NCH) issue(FIRSTC, p, i + RS, slot);
      else if (next) issue(later_c, p + 1, i + RS - NCH, slot);
      __builtin_amdgcn_sched_barrier(0);

      f4_t acc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const u4_t xop = QB == 4 ? perm_x8(xo[j]) : xo[j];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const u4_t w = wv[t][i];
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
      }
      if constexpr (QB == 4) {
        // the chunk's X row sums (the permutation of k does not change them)
        f4_t xr = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NJ; ++j) xr = mfma16<BF16>(perm_x8(xo[j]), ones, xr);
        const int g = nwv * i + wave;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          // dword of lane (l16, i): group g of column 16 t + l16
          const uint8_t* sp2 = scl + 512 * t + 4 * (16 * i + l16);
          const float sc = raw_to_f32<SDT>((uint16_t)(*(const uint32_t*)sp2 >> (16 * (g & 1))));
          float zb = w4_offset<BF16>();
          if constexpr (ZDT == 3)
            zb += (float)((*(const uint32_t*)(sp2 + 256) >> (8 * (g & 3))) & 0xFFu);
          else if constexpr (ZDT >= 0)
            zb += raw_to_f32<ZDT>((uint16_t)(*(const uint32_t*)(sp2 + 256) >> (16 * (g & 1))));
#pragma unroll
          for (int e = 0; e < 4; ++e) y[t][e] += sc * (acc[t][e] - zb * xr[e]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j) xacc = mfma16<BF16>(xo[j], ones, xacc);
#pragma unroll
        for (int t = 0; t < NT; ++t) y[t] += acc[t];
      }
      // (pins the chunk's epilogue here: the compiler would otherwise sink it
      // and keep every chunk's accumulators live)
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

    // reduce the K-slices, 8 partial sums f = 4 t + e per round:
    // red[wave][f - 8 r][lane]
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
        if (row < M && col < N) store_out(Y, (size_t)row * N + col, v + bias_at(bias, col, BF16), BF16);
      }
    });
  };
  run_pass(first_c, 0);
  if constexpr (MULTI)
    for (int p = 1; p < npass; ++p) run_pass(later_c, p);
}

// ----------------------------------------------------------------------------
// Tiled kernel: any M.  Output tile 64 (m) x 64 (n); block = 256 (4 waves),
// wave w owns columns n0 + 16w .. +15 for all 64 rows (4 m-tiles).
// K steps of KS = 256 with X tiles (and their 128-k chunk sums)
// double-buffered in LDS.
// Preconditions: K % 256 == 0, N % 64 == 0, int4: G % 128 == 0.
// Grid: tiles enumerated so that the row blocks sharing one column block land
// on the same XCD (blockIdx % 8 picks the XCD).
// Split-K form (SPLIT, grid (tiles, slices)): slice blockIdx.y takes k
// blockIdx.y * K .. +K (K here the slice length, a multiple of 256; the last
// slice may be shorter) of rows of length ldk, and writes its fp32 sums,
// scaled but without the bias, to P[slice][M][N] (wq_splitk_reduce adds the
// slices and the bias).
// ----------------------------------------------------------------------------
template <int QB, bool BF16, int SDT, int ZDT, bool SPLIT = false>
__device__ __forceinline__ void wq_tiled_body(const uint16_t* __restrict__ X,
                                              const uint8_t* __restrict__ W,
                                              uint16_t* __restrict__ Y,
                                              const void* __restrict__ S,
                                              const void* __restrict__ Z, int M, int N, int K,
                                              int G, const uint16_t* bias, int ldk = 0,
                                              float* __restrict__ P = nullptr) {
  constexpr int BM = 64, KS = 256, LDX = KS + 8;
  // k range of this workgroup, and the row length of X and W
  const int kbeg = SPLIT ? (int)blockIdx.y * K : 0;
  const int kend = SPLIT ? min(ldk, kbeg + K) : K;
  if constexpr (SPLIT) K = ldk;
  __shared__ __align__(16) uint16_t xs[2][BM * LDX];
  __shared__ __align__(16) float xsm[2][2][BM];  // [buf][chunk][row]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mblocks = (M + BM - 1) / BM;
  const int tiles = mblocks * (N / 64);
  const int nb = gridDim.x;
  int tile = blockIdx.x;
  if ((nb & 7) == 0) tile = (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3);
  if (tile >= tiles) return;
  const int mb = tile % mblocks, nbk = tile / mblocks;
  const int m0 = mb * BM, n0 = nbk * 64;

  const int n = n0 + wave * 16 + (lane & 15), q = lane >> 4;
  const uint32_t vmask = vgpr_const(0x000F000Fu), vmagic = vgpr_const(w4_magic<BF16>());
  const size_t rowbytes = (QB == 4) ? (size_t)(K >> 1) : (size_t)K;
  const uint8_t* wrow = W + (size_t)n * rowbytes;
  const int ngroups = (QB == 4) ? (K + G - 1) / G : 1;

  // X staging: 64 rows x 256 k = 2048 16-byte pieces, 8 per thread; piece p
  // of row r covers k = 8p..8p+7, 16 consecutive pieces form one 128-k chunk.
  // Global loads of step s+1 (X pieces, weights, scales) are issued before
  // the MFMAs of step s; the X pieces go to the other LDS buffer afterwards.
  constexpr int NL = (QB == 4) ? 2 : 4;  // 16-byte weight loads per lane per step
  u4_t xr[8], wv[NL], wn[NL];
  typename Raw<SDT>::T scv[NL], scn[NL];
  typename Raw<ZDT>::T zbv[NL], zbn[NL];
  // rows past M load row M - 1 and are zeroed when stored: zeroing them here
  // would consume each load on the spot (the compiler waits for it), instead
  // of leaving the loads in flight across the current step's MFMAs
  auto load_x = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = tid + 256 * i;
      int r = c >> 5, kc = (c & 31) << 3;
      xr[i] = ldg128(X + (size_t)min(m0 + r, M - 1) * K + k0 + kc);
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = tid + 256 * i;
      int r = c >> 5, kc = (c & 31) << 3;
      u4_t v = m0 + r < M ? xr[i] : u4_t{0u, 0u, 0u, 0u};
      float s = sum16(sum8<BF16>(v));
      if ((c & 15) == 0) xsm[buf][kc >> 7][r] = s;
      if constexpr (QB == 4) v = perm_x8(v);
      *(u4_t*)(&xs[buf][r * LDX + kc]) = v;
    }
  };
  auto load_w = [&](int k0, u4_t* dst, typename Raw<SDT>::T* sc, typename Raw<ZDT>::T* zb) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      int kc = k0 + i * (QB == 4 ? 128 : 64);
      size_t boff = (QB == 4) ? (size_t)(kc >> 1) + 16 * q : (size_t)kc + 16 * q;
      dst[i] = ldg128(wrow + boff);
      if constexpr (QB == 4) {
        const size_t gi = (size_t)n * ngroups + kc / G;
        sc[i] = ld_raw<SDT>(S, gi);
        zb[i] = ld_raw<ZDT>(Z, gi);
      }
    }
  };

  f4_t y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  f4_t xtot[4];  // int8 with zero-points: running row sums of X
#pragma unroll
  for (int t = 0; t < 4; ++t) xtot[t] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int nsteps = (kend - kbeg) / KS;
  load_w(kbeg, wv, scv, zbv);
  load_x(kbeg);
  store_x(0);
  __syncthreads();
  for (int st = 0; st < nsteps; ++st) {
    const int k0 = kbeg + st * KS, buf = st & 1;
    const bool more = st + 1 < nsteps;
    if (more) {
      load_w(k0 + KS, wn, scn, zbn);
      load_x(k0 + KS);
    }
    const uint16_t* xb = xs[buf];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if constexpr (QB == 4) {
        const int kl = i * 128 + 32 * q;
        f4_t a[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] = f4_t{0.f, 0.f, 0.f, 0.f};
        uint32_t ws[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          u4_t b = w4_operand(ws[j], vmask, vmagic);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            a[t] = mfma16<BF16>(*(const u4_t*)(xb + (t * 16 + (lane & 15)) * LDX + kl + 8 * j),
                                b, a[t]);
        }
        const float sc = raw_to_f32<SDT>(scv[i]);
        const float zb = w4_offset<BF16>() + raw_to_f32<ZDT>(zbv[i]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f4_t xv = *(const f4_t*)(&xsm[buf][i][t * 16 + 4 * q]);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[t][e] += sc * (a[t][e] - zb * xv[e]);
        }
      } else {
        const int kl = i * 64 + 16 * q;
        u4_t b0 = w8_operand<BF16>(wv[i].x, wv[i].y);
        u4_t b1 = w8_operand<BF16>(wv[i].z, wv[i].w);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint16_t* xr2 = xb + (t * 16 + (lane & 15)) * LDX + kl;
          y[t] = mfma16<BF16>(*(const u4_t*)xr2, b0, y[t]);
          y[t] = mfma16<BF16>(*(const u4_t*)(xr2 + 8), b1, y[t]);
        }
      }
    }
    if constexpr (QB == 8 && ZDT >= 0) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xtot[t] += *(const f4_t*)(&xsm[buf][0][t * 16 + 4 * q]) +
                   *(const f4_t*)(&xsm[buf][1][t * 16 + 4 * q]);
    }
    if (more) store_x(buf ^ 1);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        wv[i] = wn[i];
        scv[i] = scn[i];
        zbv[i] = zbn[i];
      }
    }
  }

  float sc = 1.0f, z = 0.0f;
  if constexpr (QB == 8) {
    sc = ld_typed<SDT>(S, (size_t)n);
    z = ld_typed<ZDT>(Z, (size_t)n);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int row = m0 + t * 16 + 4 * q + e;
      float v = y[t][e];
      if constexpr (QB == 8) v = sc * (v - z * xtot[t][e]);
      if constexpr (SPLIT) {
        if (row < M) P[((size_t)blockIdx.y * M + row) * N + n] = v;
      } else {
        if (row < M) store_out(Y, (size_t)row * N + n, v + bias_at(bias, n, BF16), BF16);
      }
    }
}

// ----------------------------------------------------------------------------
// Wide kernel: fp16 activations, M > 64; int4 with G = 128 (K % 256 == 0,
// K % 512 == 0 with uint8 zero-points; K <= 4096) or int8 without
// zero-points (K % 128 == 0); N % 128 == 0.
// A workgroup owns 64 rows x 128 columns.  Its 8 waves are 2 column halves
// (64 columns) x 4 K-quarters; each wave accumulates a 64 x 64 block with
// v_mfma_f32_32x32x16_f16 (2 x 2 tiles of 32 x 32), and the four K-quarter
// partials are summed through LDS at the end.
// The weight operand is the dequantised value itself, exactly rounded:
//   int4: round_f16((q - z) * s) - the halves 1024 + q (even k) and 64 + q
//         (odd k) are made by bit operations, then a packed fp16 subtraction
//         of (1024 + z, 64 + z) (exact for integral zero-points: every uint8,
//         and fp16 ones without a fraction) and a packed multiplication by s
//         (one rounding).  A chunk in which some lane's zero-point has a
//         fraction (or exceeds 1000) builds its operands in fp32 instead.
//   int8: q itself; the per-channel scale multiplies the fp32 sums.
// So every product is x * (the dequantised weight tile entry), as in the
// reference's dequantise-then-accumulate formula, with fp32 accumulation.
// Data movement: K advances in stages of 4 CK k; K-quarter kq takes chunk kq
// (CK k) of every stage, so one stage is a contiguous slice of every row:
// X [64 rows][8 CK bytes] and weights [128 rows][128 bytes], copied global ->
// LDS in whole lines into a ring of NS stages.  All 8 waves share the copies;
// one workgroup barrier per stage publishes them.  XOR swizzles keep the MFMA
// operand reads free of bank conflicts:
//   X piece p of tile row r at slot p ^ (r & 15)
//   weight piece p of row r at slot p ^ ((r >> 1) & 7)
// Within a chunk, k-step s of lane half h uses the 8 k of X piece / weight
// group 4 h + s (int4) or 2 h + s (int8), so that one 16-byte read gives a
// lane the weights of all k-steps of the chunk.
// int4 scales / zero-points of the workgroup's 128 rows are copied to LDS once.
// Dynamic LDS: NS * (64 * 8 * CK + 16384) bytes, int4 plus 2 K (scales)
// and 2 K or K (fp16 / uint8 zero-points).
// ----------------------------------------------------------------------------
namespace {
// int4 operand in k order: nibbles n0..n7 of w (k = 8 j + i in nibble i) ->
// fp16 pairs [1024+n0, 64+n1] .. [1024+n6, 64+n7]: byte i of w goes to both
// halves, the low nibble is kept under 0x6400 (ulp 1), the high one under
// 0x5400 (ulp 1/16).  m = 0x00F0000F, g = 0x54006400 (held in VGPRs).
TM_DEV u4_t w4_nat(uint32_t w, uint32_t m, uint32_t g) {
  u4_t r;
  r.x = (perm_b32(w, w, 0x0C000C00u) & m) | g;
  r.y = (perm_b32(w, w, 0x0C010C01u) & m) | g;
  r.z = (perm_b32(w, w, 0x0C020C02u) & m) | g;
  r.w = (perm_b32(w, w, 0x0C030C03u) & m) | g;
  return r;
}
TM_DEV uint32_t hmad_pair(uint32_t v, h2_t zz, h2_t ss) {
  return h2_bits((as_h2(v) + zz) * ss);
}
// round_f16((q - z) * s) for the 8 nibbles of w, in fp32 (any z).
TM_DEV u4_t w4_exact(uint32_t w, float z, float s) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = ((float)((w >> (4 * i)) & 0xFu) - z) * s;
  u4_t r;
  r.x = pack_f16x2(f[0], f[1]);
  r.y = pack_f16x2(f[2], f[3]);
  r.z = pack_f16x2(f[4], f[5]);
  r.w = pack_f16x2(f[6], f[7]);
  return r;
}
}  // namespace

// Split-K form (SPLIT): workgroup row blockIdx.y takes the k-slice
// [blockIdx.y K, + K) of rows ldk long (the last slice ends at ldk, so it may
// be shorter) and writes its fp32 sums (scaled, no bias) to
// P[blockIdx.y][M][N]; the int4 scale / zero-point rows of the slice are
// gathered row by row (ldk / 128 groups apart).
// BF16: bf16 activations, int8 only (q is exact in bf16 and the per-channel
// scale multiplies the fp32 sums; an int4 operand dequantised to bf16 would
// round every weight to 8 bits).
template <int QB, int ZDT, bool SPLIT = false, bool BF16 = false>
__device__ __forceinline__ void wq_wide_body(const uint16_t* __restrict__ X,
                                             const uint8_t* __restrict__ W,
                                             uint16_t* __restrict__ Y, const uint16_t* S,
                                             const void* Z, int M, int N, int K,
                                             const uint16_t* bias, int ldk = 0,
                                             float* __restrict__ P = nullptr) {
  static_assert(!BF16 || QB == 8, "bf16 wide kernel: int8 only");
  constexpr int CK = QB == 4 ? 64 : 32;  // k per chunk and K-quarter
  constexpr int KS = CK / 16;            // MFMA k-steps per chunk
  constexpr int NS = QB == 4 ? 3 : 4;    // ring stages
  constexpr int XRB = 8 * CK;            // X bytes per row per stage (4 quarters)
  constexpr int XPQ = CK / 8;            // X pieces per row per quarter
  constexpr int XT = 64 * XRB;           // X tile bytes
  constexpr int ST = XT + 128 * 128;     // stage: X tile, weight tile [128 rows][128 B]
  constexpr int XLR = 64 / (XRB / 16);   // X rows per 1 KB copy
  constexpr int DX = XT / 8192;          // X copies per wave per stage
  constexpr int D = DX + 2;              // copies per wave per stage
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, kq = wave >> 1;
  const int r32 = lane & 31, h = lane >> 5;

  // workgroup -> (row block, column block): the row blocks of one column block
  // are 8 workgroups apart, i.e. on one XCD, which shares their weights in L2
  const int mtl = (M + 63) >> 6, ntl = N >> 7;
  const int j = blockIdx.x >> 3;
  const int mb = j % mtl, nb = 8 * (j / mtl) + (blockIdx.x & 7);
  if (nb >= ntl) return;
  const int m0 = mb * 64, n0 = nb * 128;
  if constexpr (!SPLIT) ldk = K;
  const int ks0 = SPLIT ? (int)blockIdx.y * K : 0;
  if constexpr (SPLIT) K = min(K, ldk - ks0);  // the last slice may be shorter
  const int NC = K / (4 * CK);  // stages of 4 CK k
  X += ks0;
  W += QB == 4 ? ks0 >> 1 : ks0;
  const size_t wrow = QB == 4 ? (size_t)(ldk >> 1) : (size_t)ldk;
  const int ng = K >> 7;  // int4 groups per row of the slice
  const size_t ngr = (size_t)(ldk >> 7), g0 = (size_t)(ks0 >> 7);  // groups per row of S / Z
  const uint32_t lbase = __builtin_amdgcn_readfirstlane(lds_off(lds));
  const uint32_t sbase = lbase + NS * ST;  // int4 scales, then zero-points
  constexpr int ZRB = ZDT == 3 ? 1 : 2;    // zero-point bytes

  // ---- int4 scales / zero-points of the 128 rows: contiguous blocks (lanes
  // past the end of a block copy nothing: uint8 zero-point blocks are K bytes,
  // a multiple of 512 only)
  if constexpr (QB == 4) {
    const int sb = 128 * ng * 2, zb = 128 * ng * ZRB;
    if constexpr (!SPLIT) {
      for (int o = 1024 * wave; o < sb; o += 8192)
        if (o + 16 * lane < sb) dma16((const uint8_t*)(S + (size_t)n0 * ng) + o + 16 * lane, sbase + o);
      if constexpr (ZDT >= 0)
        for (int o = 1024 * wave; o < zb; o += 8192)
          if (o + 16 * lane < zb)
            dma16((const uint8_t*)Z + (size_t)n0 * ng * ZRB + o + 16 * lane, sbase + sb + o);
    } else {
      // dword d of the [row][group] block: row d / (ng * ZB / 4) (slices of
      // 256 k keep every row of scales and fp16 zero-points a whole number of
      // dwords; uint8 zero-points take slices of 512)
      const int sdw = ng / 2, zdw = ng * ZRB / 4;
      for (int o = 64 * wave; o < 128 * sdw; o += 512) {
        const int d = o + lane, r = d / sdw, j = d - r * sdw;
        if (d < 128 * sdw) dma4(S + (size_t)(n0 + r) * ngr + g0 + 2 * j, sbase + 4 * o);
      }
      if constexpr (ZDT >= 0)
        for (int o = 64 * wave; o < 128 * zdw; o += 512) {
          const int d = o + lane, r = d / zdw, j = d - r * zdw;
          if (d < 128 * zdw)
            dma4((const uint8_t*)Z + ((size_t)(n0 + r) * ngr + g0) * ZRB + 4 * j, sbase + sb + 4 * o);
        }
    }
  }

  // ---- copies of one stage (chunk c of every K-quarter: 4 CK consecutive k).
  // Each copy moves whole lines: X rows of XRB bytes, weight rows of 128 B.
  // X piece p of row r sits at slot p ^ (r & 15); weight piece p of row r at
  // slot p ^ ((r >> 1) & 7).
  const uint8_t* xsrc[DX];
  uint32_t xdst[DX];
#pragma unroll
  for (int i = 0; i < DX; ++i) {
    const int rr = XLR * (DX * wave + i) + lane / (XRB / 16), sl = lane % (XRB / 16);
    xsrc[i] = (const uint8_t*)(X + (size_t)min(m0 + rr, M - 1) * ldk) + 16 * (sl ^ (rr & 15));
    xdst[i] = 1024 * (DX * wave + i);
  }
  const uint8_t* wsrc[2];
  uint32_t wdst[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rr = 8 * (2 * wave + i) + (lane >> 3), sl = lane & 7;
    wsrc[i] = W + (size_t)(n0 + rr) * wrow + 16 * (sl ^ ((rr >> 1) & 7));
    wdst[i] = XT + 1024 * (2 * wave + i);
  }
  auto issue = [&](int c) {
    const uint32_t st = lbase + (uint32_t)(c % NS) * ST;
#pragma unroll
    for (int i = 0; i < DX; ++i) dma16(xsrc[i] + (size_t)c * XRB, st + xdst[i]);
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(wsrc[i] + (size_t)c * 128, st + wdst[i]);
  };
#pragma unroll
  for (int c = 0; c < NS - 1; ++c)
    if (c < NC) issue(c);

  // ---- per-lane operand read offsets within a stage: k-step s of lane half
  // h reads X piece XPQ kq + g and weight group g, g = 4 h + s (int4) or
  // 2 h + s (int8), of this wave's K-quarter
  uint32_t aoff[2][KS];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int row = 32 * mt + r32;
      const int pc = XPQ * kq + (QB == 4 ? 4 * h + s : 2 * h + s);
      aoff[mt][s] = row * XRB + 16 * (pc ^ (row & 15));
    }
  uint32_t boff[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = 64 * wn + 32 * t + r32;
    boff[t] = XT + row * 128 + 16 * ((2 * kq + h) ^ ((row >> 1) & 7));
  }
  const uint32_t vm = vgpr_const(0x00F0000Fu), vg = vgpr_const(0x54006400u);

  f16_t acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[mt][t] = f16_t{};

  for (int c = 0; c < NC; ++c) {
    // this wave's copies of stage c are complete once at most the copies of
    // the later stages already issued are outstanding
    const int later = min(NS - 2, NC - 1 - c);
    if (later >= 2) wait_vm<2 * D>();
    else if (later == 1) wait_vm<D>();
    else wait_vm<0>();
    lds_barrier();  // all waves' copies of stage c, and stage (c - 1) % NS is free
    if (c + NS - 1 < NC) issue(c + NS - 1);
    if constexpr (QB == 4) {
      if (c == 0) {
        // once: the scales / zero-points [row][group] as copied become
        // [group][row], so that the 32 rows a wave reads per chunk are
        // consecutive (read row-major they sit 2 ng bytes apart, all in 4 of
        // the 64 banks).  Through registers: the LDS holds no second copy.
        uint8_t* sl = lds + NS * ST;
        const int ns = 128 * ng;  // entries per block
        u4_t sv = {0u, 0u, 0u, 0u}, zv = {0u, 0u, 0u, 0u};
        const int zper = ZDT == 3 ? 16 : 8;  // zero-points per thread
        const bool hs = 8 * tid < ns, hz = ZDT >= 0 && zper * tid < ns;
        if (hs) sv = *(const u4_t*)(sl + 16 * tid);
        if (hz) zv = *(const u4_t*)(sl + 256 * ng + 16 * tid);
        lds_barrier();
        if (hs) {
          const uint32_t w[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = 8 * tid + e, row = i / ng, g = i - row * ng;
            ((uint16_t*)sl)[g * 128 + row] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
          }
        }
        if (hz) {
          const uint32_t w[4] = {zv.x, zv.y, zv.z, zv.w};
#pragma unroll
          for (int e = 0; e < zper; ++e) {
            const int i = zper * tid + e, row = i / ng, g = i - row * ng;
            if constexpr (ZDT == 3)
              (sl + 256 * ng)[g * 128 + row] = (uint8_t)(w[e >> 2] >> (8 * (e & 3)));
            else
              ((uint16_t*)(sl + 256 * ng))[g * 128 + row] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
          }
        }
        lds_barrier();
      }
    }

    const uint8_t* st = lds + (c % NS) * ST;
    u4_t braw[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) braw[t] = *(const u4_t*)(st + boff[t]);
    // int4: this chunk's group (k = (4 c + kq) CK; every chunk of a wave is
    // in a group of its own); slow: some lane's zero-point has a fraction
    h2_t zz[2], ss[2];
    float zf[2], sf[2];
    bool slow = false;
    if constexpr (QB == 4) {
      const int gg = (4 * c + kq) >> 1;
      const uint8_t* sl = lds + NS * ST;
      bool frac = false;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int gi = gg * 128 + 64 * wn + 32 * t + r32;  // [group][row]
        const uint16_t sbits = ((const uint16_t*)sl)[gi];
        sf[t] = f16_bits_to_f32(sbits);
        zf[t] = 0.0f;
        if constexpr (ZDT == 3) zf[t] = (float)(sl + 256 * ng)[gi];
        else if constexpr (ZDT >= 0) zf[t] = f16_bits_to_f32(((const uint16_t*)(sl + 256 * ng))[gi]);
        if constexpr (ZDT == TM_DT_F16)
          frac = frac || zf[t] != __builtin_rintf(zf[t]) || __builtin_fabsf(zf[t]) > 1000.0f;
        // (1024 + z, 64 + z): exact for integral z, |z| <= 1000
        zz[t] = h2_t{(half_t)(-1024.0f - zf[t]), (half_t)(-64.0f - zf[t])};
        const half_t sh = __builtin_bit_cast(half_t, sbits);
        ss[t] = h2_t{sh, sh};
      }
      if constexpr (ZDT == TM_DT_F16) slow = __builtin_amdgcn_ballot_w64(frac) != 0;
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u4_t a[2], b[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) a[mt] = *(const u4_t*)(st + aoff[mt][s]);
      if constexpr (QB == 4) {
        // one uniform branch per k-step that only chooses how the weight
        // operands are made (the MFMAs below are shared)
        if (slow) {
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const uint32_t wd = s == 0 ? braw[t].x : s == 1 ? braw[t].y : s == 2 ? braw[t].z : braw[t].w;
            b[t] = w4_exact(wd, zf[t], sf[t]);
          }
        } else {
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const uint32_t wd = s == 0 ? braw[t].x : s == 1 ? braw[t].y : s == 2 ? braw[t].z : braw[t].w;
            const u4_t r = w4_nat(wd, vm, vg);
            b[t].x = hmad_pair(r.x, zz[t], ss[t]);
            b[t].y = hmad_pair(r.y, zz[t], ss[t]);
            b[t].z = hmad_pair(r.z, zz[t], ss[t]);
            b[t].w = hmad_pair(r.w, zz[t], ss[t]);
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
          b[t] = s == 0 ? w8_operand<BF16>(braw[t].x, braw[t].y)
                        : w8_operand<BF16>(braw[t].z, braw[t].w);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[mt][t] = mfma32<BF16>(a[mt], b[t], acc[mt][t]);
    }
  }

  // ---- sum the four K-quarters: every wave parks its 4 tiles in LDS, then
  // wave (wn, kq) adds tile kq of the four waves of column half wn
  wait_vm<0>();
  lds_barrier();
  float* red = (float*)lds;  // [wave][tile][e][lane]
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[((wave * 4 + 2 * mt + t) * 16 + e) * 64 + lane] = acc[mt][t][e];
  lds_barrier();
  const int mt = kq >> 1, t = kq & 1;
  float y[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float v = 0.0f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) v += red[(((2 * q4 + wn) * 4 + kq) * 16 + e) * 64 + lane];
    y[e] = v;
  }
  const int col = n0 + 64 * wn + 32 * t + r32;
  float sc = 1.0f;
  if constexpr (QB == 8) sc = BF16 ? bf16_bits_to_f32(S[col]) : f16_bits_to_f32(S[col]);
  const float bv = SPLIT ? 0.0f : bias_at(bias, col, BF16);
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = m0 + 32 * mt + 8 * (e >> 2) + 4 * h + (e & 3);
    if (row < M) {
      if constexpr (SPLIT) P[((size_t)blockIdx.y * M + row) * N + col] = y[e] * sc;
      else store_out(Y, (size_t)row * N + col, y[e] * sc + bv, BF16);
    }
  }
}

// ----------------------------------------------------------------------------
// General kernel: any M, N, K (int4: K even), any dtypes.  One wave per
// column n; fp32 arithmetic exactly as the reference template:
// w = (float(q) - z) * s; acc += x * w.  The lanes take 8 consecutive k at a
// time (one 4-byte int4 / 8-byte int8 load where K % 8 == 0 and the row start
// allows it), and each weight, once dequantised, serves a block of up to 8
// activation rows, so a row of weights is read ceil(M / 8) times, not M.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void st_any(void* p, size_t i, int dt, float v) {
  switch (dt) {
    case TM_DT_F32: ((float*)p)[i] = v; break;
    case TM_DT_F16: ((uint16_t*)p)[i] = f32_to_f16_bits(v); break;
    default: ((uint16_t*)p)[i] = f32_to_bf16_bits(v); break;
  }
}

template <int XDT, int MB>
__device__ __forceinline__ void wq_general_body(const void* __restrict__ X,
                                                const uint8_t* __restrict__ W,
                                                void* __restrict__ Y, const void* __restrict__ S,
                                                const void* __restrict__ Z, int M, int N, int K,
                                                int G, int qbits, int sdt, int zdt,
                                                const void* __restrict__ bias) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int ngroups = (qbits == 4) ? (K + G - 1) / G : 1;
  const uint8_t* wr = W + (size_t)n * (qbits == 4 ? (size_t)(K / 2) : (size_t)K);
  const bool wvec = K % 8 == 0 && ((uintptr_t)wr & (qbits == 4 ? 3u : 7u)) == 0;
  // 8 activations of a row as one 16-byte load (16-bit) or two (fp32)
  const bool xvec = K % 8 == 0 && ((uintptr_t)X & 15u) == 0;
  const bool group8 = qbits == 8 || G % 8 == 0;  // 8 consecutive k share a scale
  for (int m0 = 0; m0 < M; m0 += MB) {
    float acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = 0.0f;
    // one row: several steps' loads in flight at once
    constexpr int KU = MB == 1 ? 4 : 1;
#pragma unroll KU
    for (int k0 = 8 * lane; k0 < K; k0 += 512) {
      // loads first: weights, scale / zero-point, the block's activations
      uint32_t wlo = 0, whi = 0;
      if (wvec) {
        if (qbits == 4) {
          wlo = *(const uint32_t*)(wr + k0 / 2);
        } else {
          const uint2 v = *(const uint2*)(wr + k0);
          wlo = v.x;
          whi = v.y;
        }
      }
      float sc = 0.0f, zp = 0.0f;
      if (group8) {
        const size_t si = qbits == 4 ? (size_t)n * ngroups + k0 / G : (size_t)n;
        sc = ld_scalar(S, si, sdt);
        zp = ld_scalar(Z, si, zdt);
      }
      float xv[MB][8];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
        if (m0 + i >= M) continue;
        const size_t xo = (size_t)(m0 + i) * K + k0;
        if (xvec) {
          if constexpr (XDT == TM_DT_F32) {
            const f4_t lo = *(const f4_t*)((const float*)X + xo);
            const f4_t hi = *(const f4_t*)((const float*)X + xo + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              xv[i][e] = lo[e];
              xv[i][4 + e] = hi[e];
            }
          } else {
            const u4_t v = *(const u4_t*)((const uint16_t*)X + xo);
            const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t hbits = (wd[e / 2] >> (16 * (e & 1))) & 0xFFFFu;
              xv[i][e] = XDT == TM_DT_F16 ? f16_bits_to_f32((uint16_t)hbits)
                                          : bf16_bits_to_f32((uint16_t)hbits);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k0 + e < K) xv[i][e] = ld_typed<XDT>(X, xo + e);
        }
      }
      float w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = k0 + e;
        w[e] = 0.0f;
        if (k < K) {
          float qv;
          if (qbits == 4) {
            const uint32_t b = wvec ? wlo >> (4 * e) : (uint32_t)wr[k / 2] >> (4 * (k & 1));
            qv = (float)(b & 0xF);
          } else {
            const uint32_t b = wvec ? (e < 4 ? wlo : whi) >> (8 * (e & 3)) : (uint32_t)wr[k];
            qv = (float)(int8_t)(b & 0xFF);
          }
          if (!group8) {
            const size_t si = (size_t)n * ngroups + k / G;
            sc = ld_scalar(S, si, sdt);
            zp = ld_scalar(Z, si, zdt);
          }
          w[e] = (qv - zp) * sc;
        }
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i] += xv[i][e] * w[e];
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (m0 + i < M) {
        const float sum = wave_sum(acc[i]);
        if (lane == 0)
          st_any(Y, (size_t)(m0 + i) * N + n, XDT,
                 sum + (bias ? ld_typed<XDT>(bias, n) : 0.0f));
      }
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void wq_general(
    const void* __restrict__ X, const uint8_t* __restrict__ W, void* __restrict__ Y,
    const void* __restrict__ S, const void* __restrict__ Z, int M, int N, int K, int G, int qbits,
    int xdt, int sdt, int zdt, const void* __restrict__ bias) {
  // a pass serves 8 activation rows (1 when there is one)
#define TM_WQ_GENERAL_MB(XDT)                                                         \
  if (M == 1) wq_general_body<XDT, 1>(X, W, Y, S, Z, M, N, K, G, qbits, sdt, zdt, bias); \
  else wq_general_body<XDT, 8>(X, W, Y, S, Z, M, N, K, G, qbits, sdt, zdt, bias);
  if (xdt == TM_DT_F32) {
    TM_WQ_GENERAL_MB(TM_DT_F32)
  } else if (xdt == TM_DT_F16) {
    TM_WQ_GENERAL_MB(TM_DT_F16)
  } else {
    TM_WQ_GENERAL_MB(TM_DT_BF16)
  }
#undef TM_WQ_GENERAL_MB
}

// ----------------------------------------------------------------------------
// Dequantised weight tile: Wd[n, k] = round_out((float(q) - z) * s).
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void wq_dequant(
    const uint8_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ Z,
    void* __restrict__ Wd, int N, int K, int G, int qbits, int sdt, int zdt, int odt) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)N * K) return;
  int n = (int)(i / K), k = (int)(i - (size_t)n * K);
  float qv;
  size_t si;
  if (qbits == 4) {
    uint8_t byte = W[(size_t)n * (K / 2) + k / 2];
    qv = (float)((k & 1) ? ((byte >> 4) & 0xF) : (byte & 0xF));
    si = (size_t)n * ((K + G - 1) / G) + k / G;
  } else {
    qv = (float)(int8_t)W[(size_t)n * K + k];
    si = (size_t)n;
  }
  st_any(Wd, i, odt, (qv - ld_scalar(Z, si, zdt)) * ld_scalar(S, si, sdt));
}

// ----------------------------------------------------------------------------
// Named instantiations: wq_{skinny,tiled}_q{4,8}_{f16,bf16}_z{n,s,u}
// Scales have the activation dtype; zero-points: n = none, s = scale dtype,
// u = uint8.
// ----------------------------------------------------------------------------
// skinny: int8 at 4 waves per SIMD (<= 128 VGPRs); int4 (more operand
// registers per weight word) at 3 (<= 168 VGPRs), free of scratch spills.
#define TM_WQ_ATTR_skinny(QB) __attribute__((amdgpu_waves_per_eu(QB == 4 ? 3 : 4)))
#define TM_WQ_ATTR_tiled(QB)
#define TM_WQ_INST(KIND, QB, BF, ACT, ZS, ZDT, SUF, ...)                                        \
  extern "C" __global__ __launch_bounds__(256) TM_WQ_ATTR_##KIND(QB) void                       \
      wq_##KIND##_q##QB##_##ACT##_z##ZS##SUF(const uint16_t* X, const uint8_t* W, uint16_t* Y,   \
                                             const void* S, const void* Z, int M, int N, int K,  \
                                             int G, const uint16_t* bias) {                       \
    wq_##KIND##_body<QB, BF, (BF ? TM_DT_BF16 : TM_DT_F16), ZDT __VA_ARGS__>(X, W, Y, S, Z, M,   \
                                                                              N, K, G, bias);     \
  }
// skinny: _v = vector scale loads (G == 128, K % 4096 == 0)
#define TM_WQ_Z(KIND, QB, BF, ACT, SUF, ...)                                          \
  TM_WQ_INST(KIND, QB, BF, ACT, n, -1, SUF, __VA_ARGS__)                              \
  TM_WQ_INST(KIND, QB, BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), SUF, __VA_ARGS__)   \
  TM_WQ_INST(KIND, QB, BF, ACT, u, 3, SUF, __VA_ARGS__)

TM_WQ_Z(skinny, 4, false, f16, , , false)
TM_WQ_Z(skinny, 4, true, bf16, , , false)
TM_WQ_Z(skinny, 4, false, f16, _v, , true)
TM_WQ_Z(skinny, 4, true, bf16, _v, , true)
TM_WQ_Z(skinny, 8, false, f16, , , false)
TM_WQ_Z(skinny, 8, true, bf16, , , false)
TM_WQ_Z(tiled, 4, false, f16, , )
TM_WQ_Z(tiled, 4, true, bf16, , )
// tiled split-K forms: (X, W, P, S, Z, M, N, K of a slice, ldk, G), grid
// (tiles, slices)
#define TM_TILED_K(QB, BF, ACT, ZS, ZDT)                                                      \
  extern "C" __global__ __launch_bounds__(256) void wq_tiled_q##QB##_##ACT##_z##ZS##_k(       \
      const uint16_t* X, const uint8_t* W, float* P, const void* S, const void* Z, int M,     \
      int N, int K, int ldk, int G) {                                                         \
    wq_tiled_body<QB, BF, (BF ? TM_DT_BF16 : TM_DT_F16), ZDT, true>(X, W, nullptr, S, Z, M, N, \
                                                                   K, G, nullptr, ldk, P);    \
  }
#define TM_TILED_K_Z(QB, BF, ACT)                            \
  TM_TILED_K(QB, BF, ACT, n, -1)                             \
  TM_TILED_K(QB, BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16))  \
  TM_TILED_K(QB, BF, ACT, u, 3)
TM_TILED_K_Z(4, false, f16)
TM_TILED_K_Z(4, true, bf16)
TM_TILED_K_Z(8, false, f16)
TM_TILED_K_Z(8, true, bf16)
TM_WQ_Z(tiled, 8, false, f16, , )
TM_WQ_Z(tiled, 8, true, bf16, , )

// Wide kernels (fp16 activations): wq_wide_q4_f16_z{n,s,u}, wq_wide_q8_f16_zn
#define TM_WIDE(QB, BF, ACT, ZS, ZDT)                                                        \
  extern "C" __global__ __launch_bounds__(512) void wq_wide_q##QB##_##ACT##_z##ZS(             \
      const uint16_t* X, const uint8_t* W, uint16_t* Y, const uint16_t* S, const void* Z,    \
      int M, int N, int K, const uint16_t* bias) {                                            \
    wq_wide_body<QB, ZDT, false, BF>(X, W, Y, S, Z, M, N, K, bias);                           \
  }
// split-K forms: (X, W, P, S, Z, M, N, K of a slice, ldk), grid (tiles, slices)
#define TM_WIDE_K(QB, BF, ACT, ZS, ZDT)                                                         \
  extern "C" __global__ __launch_bounds__(512) void wq_wide_q##QB##_##ACT##_z##ZS##_k(          \
      const uint16_t* X, const uint8_t* W, float* P, const uint16_t* S, const void* Z, int M,   \
      int N, int K, int ldk) {                                                                  \
    wq_wide_body<QB, ZDT, true, BF>(X, W, nullptr, S, Z, M, N, K, nullptr, ldk, P);             \
  }
// fp16: int4 every zero-point form, int8 without zero-points; bf16: int8
#define TM_WIDE_ALL(M_)                                       \
  M_(4, false, f16, n, -1) M_(4, false, f16, s, TM_DT_F16)    \
  M_(4, false, f16, u, 3) M_(8, false, f16, n, -1)            \
  M_(8, true, bf16, n, -1)
TM_WIDE_ALL(TM_WIDE)
TM_WIDE_ALL(TM_WIDE_K)

// Streaming kernels: wq_stream_q<QB>_<act>_z<zs>_x<XR><s|m> (s: single pass,
// M <= XR; m: multi-pass, M <= 128).  Scales are of the activation dtype.
#define TM_STREAM(QB, BF, ACT, ZS, ZDT, NT, XR, MS, MULTI)                                     \
  extern "C" __global__ __launch_bounds__(512) void wq_stream_q##QB##_##ACT##_z##ZS##_x##XR##MS( \
      const uint16_t* X, const uint8_t* W, uint16_t* Y, const void* S, const void* Z, int M,    \
      int N, int K, const uint16_t* bias) {                                                    \
    wq_stream_body<QB, BF, (BF ? TM_DT_BF16 : TM_DT_F16), ZDT, NT, XR, MULTI>(X, W, Y, S, Z, M, \
                                                                              N, K, bias);     \
  }
#define TM_STREAM_V(QB, BF, ACT, ZS, ZDT, NT) \
  TM_STREAM(QB, BF, ACT, ZS, ZDT, NT, 8, s, false) \
  TM_STREAM(QB, BF, ACT, ZS, ZDT, NT, 16, s, false) \
  TM_STREAM(QB, BF, ACT, ZS, ZDT, NT, 16, m, true)
#define TM_STREAM_Z(QB, BF, ACT, NT)                          \
  TM_STREAM_V(QB, BF, ACT, n, -1, NT)                         \
  TM_STREAM_V(QB, BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), NT) \
  TM_STREAM_V(QB, BF, ACT, u, 3, NT)
TM_STREAM_Z(4, false, f16, 4)
TM_STREAM_Z(4, true, bf16, 4)
TM_STREAM_Z(8, false, f16, 3)
TM_STREAM_Z(8, true, bf16, 3)

// GEMV (int4, exact K = NW * PF * 128, G = 128): wq_gemv4_<act>_z<zs>_w<NW>p<PF>.
// Instantiated for K = 8192 (2 <= M <= 8); at K = 4096 the two-tile GEMV and
// the streaming kernel cover the same rows.
#define TM_GEMV4(BF, ACT, ZS, ZDT, NW, PF)                                                     \
  extern "C" __global__ __launch_bounds__(NW * 64)                                              \
  void wq_gemv4_##ACT##_z##ZS##_w##NW##p##PF(                                                   \
      const uint16_t* X, const uint8_t* W, uint16_t* Y, const uint16_t* S, const void* Z, int M, \
      int N, int K, const uint16_t* bias) {                                                     \
    wq_gemv4_body<BF, ZDT, NW, PF>(X, W, Y, S, Z, M, N, K, bias);                               \
  }
#define TM_GEMV4_Z(BF, ACT, NW, PF)                                   \
  TM_GEMV4(BF, ACT, n, -1, NW, PF)                                    \
  TM_GEMV4(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), NW, PF)         \
  TM_GEMV4(BF, ACT, u, 3, NW, PF)
TM_GEMV4_Z(false, f16, 8, 8)
TM_GEMV4_Z(true, bf16, 8, 8)

// Linear GEMV (int4, M = 1, K = 2048 * NS, G = 128): wq_gemv4l_<act>_z<zs>_k<NS>
// K = 4096: 8 waves per SIMD (<= 64 VGPRs); K = 8192 holds twice the rows per
// wave and runs at 4 (<= 128 VGPRs), which keeps it free of scratch spills.
#define TM_GEMV4L(BF, ACT, ZS, ZDT, NS)                                                         \
  extern "C" __global__ __launch_bounds__(512)                                                  \
  __attribute__((amdgpu_waves_per_eu(NS == 4 ? 4 : 8))) void                                    \
      wq_gemv4l_##ACT##_z##ZS##_k##NS(const uint16_t* X, const uint8_t* W, uint16_t* Y,         \
                                      const uint16_t* S, const void* Z, int M, int N, int K,    \
                                      const uint16_t* bias) {                                   \
    wq_gemv4l_body<BF, ZDT, NS>(X, W, Y, S, Z, N, bias);                                        \
  }
#define TM_GEMV4L_Z(BF, ACT, NS)                                 \
  TM_GEMV4L(BF, ACT, n, -1, NS)                                  \
  TM_GEMV4L(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), NS)       \
  TM_GEMV4L(BF, ACT, u, 3, NS)
TM_GEMV4L_Z(false, f16, 2)
TM_GEMV4L_Z(true, bf16, 2)
TM_GEMV4L_Z(false, f16, 4)
TM_GEMV4L_Z(true, bf16, 4)

// Two-tile GEMV (2 <= M <= 8, K = 4096, G = 128): wq_gemv4x2_<act>_z<zs>_w8p4,
// 8 waves, two workgroups per CU (<= 128 VGPRs).
#define TM_GEMV4XN(BF, ACT, ZS, ZDT, NTL, WPE)                                                  \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPE))) void   \
      wq_gemv4x##NTL##_##ACT##_z##ZS##_w8p4(const uint16_t* X, const uint8_t* W, uint16_t* Y,   \
                                            const uint16_t* S, const void* Z, int M, int N,     \
                                            int K, const uint16_t* bias) {                      \
    wq_gemv4x2_body<BF, ZDT, 8, 4, NTL>(X, W, Y, S, Z, M, N, K, bias);                          \
  }
#define TM_GEMV4XN_Z(BF, ACT, NTL, WPE)                              \
  TM_GEMV4XN(BF, ACT, n, -1, NTL, WPE)                               \
  TM_GEMV4XN(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), NTL, WPE)    \
  TM_GEMV4XN(BF, ACT, u, 3, NTL, WPE)
TM_GEMV4XN_Z(false, f16, 2, 4)
TM_GEMV4XN_Z(true, bf16, 2, 4)

// int8 GEMV (K = 4096, bf16 activations; fp16 runs on the linear int8 GEMV):
// wq_gemv8_<act>_z<zs>_w8p8; 8 waves per SIMD (<= 64 VGPRs), so the whole
// grid is resident.
#define TM_GEMV8(BF, ACT, ZS, ZDT)                                                              \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(8))) void     \
      wq_gemv8_##ACT##_z##ZS##_w8p8(const uint16_t* X, const uint8_t* W, uint16_t* Y,           \
                                    const uint16_t* S, const void* Z, int M, int N, int K,      \
                                    const uint16_t* bias) {                                     \
    wq_gemv8_body<BF, ZDT, 8, 8>(X, W, Y, S, Z, M, N, K, bias);                                 \
  }
#define TM_GEMV8_Z(BF, ACT)                              \
  TM_GEMV8(BF, ACT, n, -1)                               \
  TM_GEMV8(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16))    \
  TM_GEMV8(BF, ACT, u, 3)
TM_GEMV8_Z(true, bf16)

// Linear int8 GEMV (M = 1, K = 4096, fp16): wq_gemv8l_f16_z<zs>
#define TM_GEMV8L(ZS, ZDT)                                                                     \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(8))) void     \
      wq_gemv8l_f16_z##ZS(const uint16_t* X, const uint8_t* W, uint16_t* Y, const uint16_t* S,  \
                          const void* Z, int M, int N, int K, const uint16_t* bias) {           \
    wq_gemv8l_body<ZDT>(X, W, Y, S, Z, N, bias);                                                \
  }
TM_GEMV8L(n, -1)
TM_GEMV8L(s, TM_DT_F16)
TM_GEMV8L(u, 3)
