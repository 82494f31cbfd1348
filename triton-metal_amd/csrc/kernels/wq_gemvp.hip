// Persistent W4A16 GEMV for M = 1, K = 4096, group 128 (make_int4_matmul_kernel,
// _msl_templates.py:2682-2745; weight format as in wq_gemm.hip: [N, K/2] bytes,
// even k in the low nibble).
//
// One workgroup per CU owns 4 RW consecutive weight rows (RW = 14 at N = 14336
// on 256 CUs, so every CU streams the same number of bytes).  Wave w takes rows
// RW (w % 4) .. + RW - 1 of them and the K half h = w / 4: 1 KB of each row, read
// by one non-temporal 16-byte load per lane (whole 128-byte lines, consecutive
// lines per instruction).  X (the lane's 32 k, from L2) and the scales /
// zero-points go first; then the first RW / 2 + 1 rows, the rest once the
// wave has multiplied two rows (measured: this beats issuing all rows up front,
// and sliding windows of 3-10 rows, by 3-7%).
//
// Dot products on the MFMA units: v_mfma_f32_4x4x4_16b multiplies 16
// independent 4x4 blocks, block b taking A's rows and B's columns from lanes
// 4 b .. 4 b + 3.  With the lane's 4 x values as A row l % 4 and its 4 weight
// operands as B column l % 4, the diagonal entry D_b[l % 4][l % 4] (lane l,
// element l % 4) accumulates exactly lane l's own dot product; two such MFMAs
// per 8-k word, so only the operand building stays on the VALU.
//
// Arithmetic (exact operands, fp32 corrections, as the other W-only kernels):
// the operand is the exact half OFF + q (fp16: OFF = 1024 for even k, 64 for
// odd k, 5 instructions per 8 nibbles; bf16: OFF = 128), and per row and
// quantisation group y += s (sum x (OFF + q) - sum x OFF - z sum x).
// The lane partials are folded across lanes in a transposed butterfly (each
// exchange halves the rows a lane holds): first over the 4 lanes of a group,
// so each lane then scales only 4 rows (4 scale and 4 zero-point loads instead
// of RW each), then over the groups; the two K halves meet in LDS.
#include "common.h"
#include "wq_common.h"

namespace {

// The lane folds run on the VALU's own cross-lane paths (DPP and the permlane
// swaps), with no LDS round trip between stages (with __shfl_xor, six
// dependent ds_bpermute stages: 7.31 -> 7.11 us per step).
// One transposed-butterfly stage over lane bit O = 1 or 2 (quad DPP): R rows
// per lane -> R / 2, a lane keeping the upper half when its bit O is set.
template <int O, int R> TM_DEV void fold_dpp(float (&v)[16], int lane) {
  const bool up = lane & O;
  static_for<0, R / 2>([&](auto IC) {
    constexpr int i = decltype(IC)::value;
    const float keep = up ? v[i + R / 2] : v[i], send = up ? v[i] : v[i + R / 2];
    const int got =
        __builtin_amdgcn_mov_dpp(__float_as_int(send), O == 1 ? 0xB1 : 0x4E, 0xF, 0xF, false);
    v[i] = keep + __int_as_float(got);
  });
}
// Sum over lane bits 0 and 1 (a quad), every lane receiving it.
TM_DEV float sum_bits01(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
  return v;
}

}  // namespace

// RW rows per wave (4 <= RW <= 16); the row's K in KS segments of 2048 k (1 KB
// of weights: one 16-byte load per lane), the last one partial when K <
// 2048 KS; RG groups of RW rows; KS x RG waves.  Wave w takes segment
// s = w / RG of rows RW (w % RG) .. + RW - 1 (for K = 4096: the two K halves
// of 4 row groups, 512 threads).  Preconditions (host-checked): K % 128 == 0,
// 2048 (KS - 1) < K <= 2048 KS, G = 128, 64 KS RG threads, gridDim.x =
// ceil(N / (RG RW)), N >= RG RW; X, W 16-byte aligned.  The last workgroup is
// shifted back to end at row N: it recomputes rows of its neighbour and writes
// the same values.  EXACT: K == 2048 KS as a compile-time constant.
template <bool BF16, int ZDT, int RW, int KS, int RG, bool EXACT>
__device__ __forceinline__ void wq_gemv4p_body(const uint16_t* __restrict__ X,
                                               const uint8_t* __restrict__ W,
                                               uint16_t* __restrict__ Y,
                                               const uint16_t* __restrict__ S,
                                               const void* __restrict__ Z, int N, int Kr,
                                               const uint16_t* bias) {
  static_assert(RW >= 4 && RW <= 16, "rows per wave");
  static_assert(KS * RG <= 16, "at most 16 waves");
  const int K = EXACT ? 2048 * KS : Kr;
  const int RB = K / 2, NG = K / 128;
  constexpr int SDT = BF16 ? TM_DT_BF16 : TM_DT_F16;
  constexpr int R1 = RW / 2 + 1;  // rows issued before the first dot products
  constexpr int NR = RG * RW;     // rows per workgroup
  __shared__ float red[KS][NR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = wave / RG, ws = wave % RG;
  const int n0 = min((int)blockIdx.x * NR, N - NR), r0 = n0 + RW * ws;
  const int g = 16 * h + (lane >> 2);  // the quantisation group of the lane's 32 k
  // lanes past the end of a partial last segment hold no k (whole groups:
  // K % 128 == 0); they read nothing and contribute zeros
  const bool live = EXACT || h < KS - 1 || 2048 * h + 32 * lane < K;

  // X first (L2), then the scales / zero-points, then the weights (HBM)
  u4_t xr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xr[j] = u4_t{0u, 0u, 0u, 0u};
    if (live) xr[j] = ldg128(X + 2048 * h + 32 * lane + 8 * j);
  }
  // scales / zero-points of the 4 rows this lane scales after the first two
  // fold stages: rows 8 b0 + 4 b1 + m (b0, b1 = lane bits 0, 1), group g
  const int rq = 8 * (lane & 1) + 4 * ((lane >> 1) & 1);
  typename Raw<SDT>::T sraw[4];
  typename Raw<ZDT>::T zraw[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    sraw[m] = 0;
    zraw[m] = 0;
    if (live) {
      const size_t gi = (size_t)(r0 + min(rq + m, RW - 1)) * NG + g;
      sraw[m] = ld_raw<SDT>(S, gi);
      zraw[m] = ld_raw<ZDT>(Z, gi);
    }
  }
  const uint8_t* wb = W + (size_t)r0 * RB + 1024 * h + 16 * lane;
  u4_t wv[RW];
#pragma unroll
  for (int i = 0; i < R1; ++i) {
    wv[i] = u4_t{0u, 0u, 0u, 0u};
    if (live) wv[i] = __builtin_nontemporal_load((const u4_t*)(wb + (size_t)i * RB));
  }
  __builtin_amdgcn_sched_barrier(0);

  // x in the operand element order n0 n4 n1 n5 n2 n6 n3 n7 of each 8-k word,
  // and the lane's sums sum x, sum x OFF
  u4_t xp[4];
  float xsum = 0.0f, xoff = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xp[j] = perm_x8(xr[j]);
    xsum += xsum8(xr[j], BF16);
    if constexpr (!BF16) xoff += sumoff8_h(xr[j]);
  }

  const uint32_t m_lo = vgpr_const(0x000F000Fu), g_lo = vgpr_const(w4_magic<BF16>());
  const uint32_t m_hi = vgpr_const(0x00F000F0u), g_hi = vgpr_const(0x54005400u);
  const uint32_t s4 = vgpr_const(4u), s8 = vgpr_const(8u), s12 = vgpr_const(12u);
  f4_t acc[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    if (i == 2) {  // the remaining rows
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i2 = R1; i2 < RW; ++i2) {
        wv[i2] = u4_t{0u, 0u, 0u, 0u};
        if (live) wv[i2] = __builtin_nontemporal_load((const u4_t*)(wb + (size_t)i2 * RB));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
    f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u4_t op = BF16 ? w4_operand_v(wd[j], m_lo, g_lo, s4, s8, s12)
                           : w4_operand_h(wd[j], m_lo, m_hi, g_lo, g_hi);
      c = mfma4x4<BF16>(u2_t{xp[j].x, xp[j].y}, u2_t{op.x, op.y}, c);
      c = mfma4x4<BF16>(u2_t{xp[j].z, xp[j].w}, u2_t{op.z, op.w}, c);
    }
    acc[i] = c;
  }
  // the lane's own dot products (diagonal element lane % 4), folded over the
  // 4 lanes of its quantisation group: rows 8 b0 + 4 b1 + m stay on the lane
  const int e = lane & 3;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i < RW) v[i] = e == 0 ? acc[i][0] : e == 1 ? acc[i][1] : e == 2 ? acc[i][2] : acc[i][3];
    else v[i] = 0.0f;
  }
  fold_dpp<1, 16>(v, lane);
  fold_dpp<2, 8>(v, lane);
  // the group's sum x and sum x OFF
  xsum = sum_bits01(xsum);
  xoff = BF16 ? w4_offset<true>() * xsum : sum_bits01(xoff);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float zp = 0.0f;
    if constexpr (ZDT >= 0) zp = raw_to_f32<ZDT>(zraw[m]);
    const float p = raw_to_f32<SDT>(sraw[m]) * (v[m] - xoff - zp * xsum);
    v[m] = (live && rq + m < RW) ? p : 0.0f;
  }
  // rows rq + m -> over lane bits 4 and 5 -> row rq + 2 b4 + b5; then the sum
  // over bits 2 and 3 (the remaining groups)
  const float u0 = fold_swap<16>(v[0], v[2]), u1 = fold_swap<16>(v[1], v[3]);
  const float rs = sum_bits23(fold_swap<32>(u0, u1));
  const int r = rq + 2 * ((lane >> 4) & 1) + ((lane >> 5) & 1);
  if ((lane & 12) == 0 && r < RW) red[h][RW * ws + r] = rs;
  lds_barrier();
  if (tid < NR) {
    const int n = n0 + tid;
    float y = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) y += red[s2][tid];
    store_out(Y, n, y + bias_at(bias, n, BF16), BF16);
  }
}

// K = 4096 (the headline): wq_gemv4p_<act>_z<zs>_r<RW>, 2 segments x 4 row
// groups, K a compile-time constant.
#define TM_GEMV4P(BF, ACT, ZS, ZDT, RW)                                                         \
  extern "C" __global__ __launch_bounds__(512) void wq_gemv4p_##ACT##_z##ZS##_r##RW(            \
      const uint16_t* X, const uint8_t* W, uint16_t* Y, const uint16_t* S, const void* Z, int M, \
      int N, int K, const uint16_t* bias) {                                                     \
    wq_gemv4p_body<BF, ZDT, RW, 2, 4, true>(X, W, Y, S, Z, N, K, bias);                         \
  }
#define TM_GEMV4P_Z(BF, ACT, RW)                               \
  TM_GEMV4P(BF, ACT, n, -1, RW)                                \
  TM_GEMV4P(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), RW)     \
  TM_GEMV4P(BF, ACT, u, 3, RW)
#define TM_GEMV4P_RW(RW) TM_GEMV4P_Z(false, f16, RW) TM_GEMV4P_Z(true, bf16, RW)
TM_GEMV4P_RW(4)
TM_GEMV4P_RW(7)
TM_GEMV4P_RW(8)
TM_GEMV4P_RW(11)
TM_GEMV4P_RW(12)
TM_GEMV4P_RW(14)
TM_GEMV4P_RW(16)

// Other K (K % 128 == 0, K <= 16384): wq_gemv4k_<act>_z<zs>_s<KS>_g<RG>_r<RW>,
// KS segments of 2048 k (the last one partial when K < 2048 KS) x RG row
// groups of RW rows, K at run time.  Row-group shapes (RG, RW): (1, 8),
// (1, 16), (2, 16), (4, 16) where KS RG <= 16.  Few, long waves stream best
// here (K = 14336, N = 4096, one box: 7 waves x 16 rows 8.97 us, 14 waves x
// 8 rows 10.34, 14 x 4 in two workgroups per CU 13.87; K = 8192: 4 waves x 16
// rows 6.88, 8 x 8 7.58, 16 x 4 8.11).
#define TM_GEMV4K(BF, ACT, ZS, ZDT, KS, RG, RW)                                                 \
  extern "C" __global__ __launch_bounds__(64 * KS * RG) void                                    \
      wq_gemv4k_##ACT##_z##ZS##_s##KS##_g##RG##_r##RW(                                         \
          const uint16_t* X, const uint8_t* W, uint16_t* Y, const uint16_t* S, const void* Z,   \
          int M, int N, int K, const uint16_t* bias) {                                          \
    wq_gemv4p_body<BF, ZDT, RW, KS, RG, false>(X, W, Y, S, Z, N, K, bias);                      \
  }
#define TM_GEMV4K_Z(BF, ACT, KS, RG, RW)                               \
  TM_GEMV4K(BF, ACT, n, -1, KS, RG, RW)                                \
  TM_GEMV4K(BF, ACT, s, (BF ? TM_DT_BF16 : TM_DT_F16), KS, RG, RW)     \
  TM_GEMV4K(BF, ACT, u, 3, KS, RG, RW)
#define TM_GEMV4K_A(KS, RG, RW) TM_GEMV4K_Z(false, f16, KS, RG, RW) TM_GEMV4K_Z(true, bf16, KS, RG, RW)
#define TM_GEMV4K_KS3(KS) TM_GEMV4K_A(KS, 1, 8) TM_GEMV4K_A(KS, 1, 16) TM_GEMV4K_A(KS, 2, 16)
#define TM_GEMV4K_KS4(KS) TM_GEMV4K_KS3(KS) TM_GEMV4K_A(KS, 4, 16)
TM_GEMV4K_KS4(1)
TM_GEMV4K_KS4(2)
TM_GEMV4K_KS4(3)
TM_GEMV4K_KS4(4)
TM_GEMV4K_KS3(5)
TM_GEMV4K_KS3(6)
TM_GEMV4K_KS3(7)
TM_GEMV4K_KS3(8)

// ----------------------------------------------------------------------------
// Pure-read twin of wq_gemv4p (a measurement kernel, not part of any matmul):
// the same grid, the same rows per workgroup and the same weight loads (1 KB
// of one row per instruction, non-temporal, RW / 2 + 1 rows first and the rest
// after two rows), plus (SZ) the workgroup's scale and zero-point rows read
// contiguously, 16 bytes per lane.  The words read are XOR-reduced and
// written only if the reduction equals a fixed value, so the reads cannot be
// dropped and nothing is written for any ordinary data.  Its time per call
// is the floor that streaming these bytes with this grid sets under the GEMV.
// Arguments: W [N, 2048] bytes, S and Z [N, 32] 16-bit, sink uint32 [grid].
// ----------------------------------------------------------------------------
template <int RW, bool SZ>
__device__ __forceinline__ void wq_read_twin_body(const uint8_t* __restrict__ W,
                                                  const uint16_t* __restrict__ S,
                                                  const uint16_t* __restrict__ Z,
                                                  uint32_t* __restrict__ sink, int N) {
  constexpr int K = 4096, RB = K / 2, NG = K / 128;
  constexpr int R1 = RW / 2 + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = wave >> 2, ws = wave & 3;
  const int n0 = min((int)blockIdx.x * 4 * RW, N - 4 * RW), r0 = n0 + RW * ws;
  uint32_t acc = 0;
  if constexpr (SZ) {
    // 4 RW rows x 64 B of scales and of zero-points
    if (tid < 16 * RW) {
      const u4_t a = ldg128(S + (size_t)n0 * NG + 8 * tid);
      const u4_t b = ldg128(Z + (size_t)n0 * NG + 8 * tid);
      acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    }
  }
  const uint8_t* wb = W + (size_t)r0 * RB + 1024 * h + 16 * lane;
  u4_t wv[RW];
#pragma unroll
  for (int i = 0; i < R1; ++i) wv[i] = __builtin_nontemporal_load((const u4_t*)(wb + (size_t)i * RB));
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    if (i == 2) {
#pragma unroll
      for (int i2 = R1; i2 < RW; ++i2)
        wv[i2] = __builtin_nontemporal_load((const u4_t*)(wb + (size_t)i2 * RB));
    }
    acc ^= wv[i].x ^ wv[i].y ^ wv[i].z ^ wv[i].w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}
// wq_read_twin_r<RW> (weights, scales, zero-points), wq_read_twin_w_r<RW>
// (weights only)
#define TM_READ_TWIN(RW)                                                                        \
  extern "C" __global__ __launch_bounds__(512) void wq_read_twin_r##RW(                         \
      const uint8_t* W, const uint16_t* S, const uint16_t* Z, uint32_t* sink, int N) {          \
    wq_read_twin_body<RW, true>(W, S, Z, sink, N);                                              \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(512) void wq_read_twin_w_r##RW(                       \
      const uint8_t* W, const uint16_t* S, const uint16_t* Z, uint32_t* sink, int N) {          \
    wq_read_twin_body<RW, false>(W, S, Z, sink, N);                                             \
  }
TM_READ_TWIN(14)
