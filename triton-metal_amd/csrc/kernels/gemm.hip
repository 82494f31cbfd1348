// Dense fp16/bf16 GEMM for gfx950 with fp32 accumulation.
//
//   C[M, N] = A[M, K] @ B[K, N]          (B_T = false; the tl.dot / matmul
//                                          template layout, all row-major)
//   C[M, N] = A[M, K] @ W[N, K]^T (+ bias[N])   (B_T = true; nn.Linear layout)
//
// Reference semantics: make_matmul_kernel (_msl_templates.py:447-585: fp32
// accumulate, output in the input dtype, bounds-checked tiles),
// make_simdgroup_matmul_kernel (_msl_templates.py:3501-3667: fp16 inputs,
// fp32 accumulate, fp32 output) and make_fused_linear_kernel
// (_msl_templates.py:4013-4135: input @ weight^T + bias).
//
// Design: BM x BN output tile per workgroup, WM x WN waves, K stepped by BK
// through two LDS buffers (the next tile is fetched to registers while the
// MFMAs consume the current one; one barrier per step).  Both operands live
// in LDS k-contiguous ([rows][BK + 8] halves, the +8 pad staggers banks); a
// row-major B [K, N] is transposed on the way in: each thread loads an 8 (k)
// x 8 (n) block and transposes it in registers with byte permutes, so every
// LDS access is 16 bytes wide.
#include "common.h"

namespace {

template <int ODT> TM_DEV void store_c(void* C, size_t i, float v) { store_from_f32<ODT>(C, i, v); }

// Transpose an 8x8 block of 16-bit values held as 8 rows x 4 dwords.
TM_DEV void transpose8x8(const u4_t in[8], u4_t out[8]) {
  // out[c] holds column c: halves in[0][c], in[1][c], ..., in[7][c].
  uint32_t r[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) { r[i][0] = in[i].x; r[i][1] = in[i].y; r[i][2] = in[i].z; r[i][3] = in[i].w; }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int d = c >> 1;
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;  // high or low half of each source
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) o[p] = perm_b32(r[2 * p + 1][d], r[2 * p][d], sel);
    out[c] = u4_t{o[0], o[1], o[2], o[3]};
  }
}

}  // namespace

template <int BM, int BN, int BK, int WM, int WN, bool BT, bool BF16, int ODT, bool BIAS>
__device__ __forceinline__ void gemm_body(const uint16_t* __restrict__ A,
                                          const uint16_t* __restrict__ B, void* __restrict__ C,
                                          const uint16_t* __restrict__ bias, int M, int N, int K,
                                          int lda, int ldb, int ldc) {
  constexpr int NT = WM * WN * 64;
  constexpr int LDS = BK + 8;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16x16 tiles per wave
  static_assert(TM >= 1 && TN >= 1, "wave tile");
  __shared__ __align__(16) uint16_t As[2][BM * LDS];
  __shared__ __align__(16) uint16_t Bs[2][BN * LDS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_n = (N + BN - 1) / BN;
  const int m0 = (blockIdx.x / tiles_n) * BM, n0 = (blockIdx.x % tiles_n) * BN;

  // ---- global -> register loaders ------------------------------------------
  constexpr int A_CH = BM * BK / 8;                 // 16-byte chunks of the A tile
  constexpr int A_PT = (A_CH + NT - 1) / NT;
  constexpr int B_CH = BT ? BN * BK / 8 : BN * BK / 64;  // chunks or 8x8 blocks
  constexpr int B_PT = (B_CH + NT - 1) / NT;
  constexpr int B_RL = BT ? 1 : 8;                   // 16-byte loads per B item
  u4_t ra[A_PT], rb[B_PT][B_RL];

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      int c = tid + NT * i;
      ra[i] = u4_t{0u, 0u, 0u, 0u};
      if (c < A_CH) {
        int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        int gr = m0 + r, gk = k0 + kc;
        if (gr < M && gk < K) ra[i] = ldg128(A + (size_t)gr * lda + gk);
      }
    }
  };
  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      int c = tid + NT * i;
      if constexpr (BT) {
        rb[i][0] = u4_t{0u, 0u, 0u, 0u};
        if (c < B_CH) {
          int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
          int gn = n0 + r, gk = k0 + kc;
          if (gn < N && gk < K) rb[i][0] = ldg128(B + (size_t)gn * ldb + gk);
        }
      } else {
        // 8x8 block: k rows kb..kb+7, n columns nb..nb+7; consecutive
        // threads take consecutive n so each row load is coalesced.
        int nb = (c % (BN / 8)) * 8, kb = (c / (BN / 8)) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          rb[i][j] = u4_t{0u, 0u, 0u, 0u};
          int gk = k0 + kb + j, gn = n0 + nb;
          if (c < B_CH && gk < K && gn < N) rb[i][j] = ldg128(B + (size_t)gk * ldb + gn);
        }
      }
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      int c = tid + NT * i;
      if (c < A_CH) {
        int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        *(u4_t*)(&As[buf][r * LDS + kc]) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      int c = tid + NT * i;
      if (c < B_CH) {
        if constexpr (BT) {
          int r = c / (BK / 8), kc = (c % (BK / 8)) * 8;
          *(u4_t*)(&Bs[buf][r * LDS + kc]) = rb[i][0];
        } else {
          int nb = (c % (BN / 8)) * 8, kb = (c / (BN / 8)) * 8;
          u4_t t[8];
          transpose8x8(rb[i], t);
#pragma unroll
          for (int j = 0; j < 8; ++j) *(u4_t*)(&Bs[buf][(nb + j) * LDS + kb]) = t[j];
        }
      }
    }
  };

  f4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + BK - 1) / BK;
  load_a(0);
  load_b(0);
  store_tiles(0);
  __syncthreads();
  const int q = lane >> 4, r16 = lane & 15;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
    const uint16_t* as = As[buf];
    const uint16_t* bs = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      u4_t af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *(const u4_t*)(as + (wm * TM * 16 + i * 16 + r16) * LDS + kk + 8 * q);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *(const u4_t*)(bs + (wn * TN * 16 + j * 16 + r16) * LDS + kk + 8 * q);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16<BF16>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) store_tiles(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      int col = n0 + wn * TN * 16 + j * 16 + r16;
      if (col >= N) continue;
      float bv = 0.0f;
      if constexpr (BIAS) bv = BF16 ? bf16_bits_to_f32(bias[col]) : f16_bits_to_f32(bias[col]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int row = m0 + wm * TM * 16 + i * 16 + 4 * q + e;
        if (row < M) store_c<ODT>(C, (size_t)row * ldc + col, acc[i][j][e] + bv);
      }
    }
}

// General fallback: one thread per output, fp32 accumulation (any shape,
// any alignment); the reference template's arithmetic.
extern "C" __global__ __launch_bounds__(256) void gemm_general(
    const void* __restrict__ A, const void* __restrict__ B, void* __restrict__ C,
    const void* __restrict__ bias, int M, int N, int K, int lda, int ldb, int ldc, int bt,
    int idt, int odt) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * N) return;
  int m = (int)(i / N), n = (int)(i - (size_t)m * N);
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    size_t ai = (size_t)m * lda + k;
    size_t bi = bt ? (size_t)n * ldb + k : (size_t)k * ldb + n;
    float a, b;
    if (idt == TM_DT_F32) { a = ((const float*)A)[ai]; b = ((const float*)B)[bi]; }
    else if (idt == TM_DT_F16) { a = (float)((const half_t*)A)[ai]; b = (float)((const half_t*)B)[bi]; }
    else { a = bf16_bits_to_f32(((const uint16_t*)A)[ai]); b = bf16_bits_to_f32(((const uint16_t*)B)[bi]); }
    acc += a * b;
  }
  if (bias) {
    if (idt == TM_DT_F32) acc += ((const float*)bias)[n];
    else if (idt == TM_DT_F16) acc += (float)((const half_t*)bias)[n];
    else acc += bf16_bits_to_f32(((const uint16_t*)bias)[n]);
  }
  size_t ci = (size_t)m * ldc + n;
  if (odt == TM_DT_F32) ((float*)C)[ci] = acc;
  else if (odt == TM_DT_F16) ((uint16_t*)C)[ci] = f32_to_f16_bits(acc);
  else ((uint16_t*)C)[ci] = f32_to_bf16_bits(acc);
}

// Named instantiations: gemm_<tile>_<bt>_<in>_<out>[_bias]
#define TM_GEMM_INST(NAME, BM, BN, BK, WM, WN, BT, BF, ODT, BIAS)                               \
  extern "C" __global__ __launch_bounds__(WM * WN * 64) void NAME(                              \
      const uint16_t* A, const uint16_t* B, void* C, const uint16_t* bias, int M, int N, int K, \
      int lda, int ldb, int ldc) {                                                               \
    gemm_body<BM, BN, BK, WM, WN, BT, BF, ODT, BIAS>(A, B, C, bias, M, N, K, lda, ldb, ldc);    \
  }

// t32k: 32 x 32 tiles with the whole K <= 512 staged at once - for small
// problems the K loop of t32 is a chain of exposed load latencies
#define TM_GEMM_TILES(BT, BTN, BF, IN, ODT, OUT, BIAS, BN_)                               \
  TM_GEMM_INST(gemm_t128_##BTN##_##IN##_##OUT##BN_, 128, 128, 64, 2, 2, BT, BF, ODT, BIAS) \
  TM_GEMM_INST(gemm_t64_##BTN##_##IN##_##OUT##BN_, 64, 64, 64, 2, 2, BT, BF, ODT, BIAS)    \
  TM_GEMM_INST(gemm_t32_##BTN##_##IN##_##OUT##BN_, 32, 32, 64, 2, 2, BT, BF, ODT, BIAS)    \
  TM_GEMM_INST(gemm_t32k_##BTN##_##IN##_##OUT##BN_, 32, 32, 512, 2, 2, BT, BF, ODT, BIAS)

#define TM_GEMM_OUTS(BT, BTN, BF, IN, BIAS, BN_)                      \
  TM_GEMM_TILES(BT, BTN, BF, IN, (BF ? TM_DT_BF16 : TM_DT_F16), same, BIAS, BN_) \
  TM_GEMM_TILES(BT, BTN, BF, IN, TM_DT_F32, f32, BIAS, BN_)

TM_GEMM_OUTS(false, nn, false, f16, false, )
TM_GEMM_OUTS(false, nn, true, bf16, false, )
TM_GEMM_OUTS(true, nt, false, f16, false, )
TM_GEMM_OUTS(true, nt, true, bf16, false, )
TM_GEMM_OUTS(true, nt, false, f16, true, _bias)
TM_GEMM_OUTS(true, nt, true, bf16, true, _bias)
