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

// ----------------------------------------------------------------------------
// Small problems, K = 4 KW with KW = 64 or 128, M % 32 == 0, N % 32 == 0 (C1,
// 512^3: one workgroup per CU).  A workgroup owns a 32 x 32 output tile and
// its 4 waves split K: wave w copies its own A slice [32][KW] and B slice
// (nn: [KW][32], nt: [32][KW]) global -> LDS (2 KW / 16 copies of 1 KB) and
// waits on those copies only, so nothing but the final sum needs a barrier;
// then KW / 16 v_mfma_f32_32x32x16 in two accumulator chains, the row-major B
// read with ds_read_b64_tr_b16 (lane l: column l % 32, k = 8 (l / 32) + e).
// The four K partials meet in LDS (each wave parks its own in its own region)
// and every thread sums 4 consecutive columns of one row and stores them in
// one access.  A rows (and nt B rows) keep piece p at slot p ^ (r & 7).
// Same box against the 32 x 32 whole-K tile it replaces there: 512^3
// 4.24 -> 2.75 us, 1024 x 1024 x 512 10.8 -> 5.6 us.
// ----------------------------------------------------------------------------
namespace {
typedef short gs_s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) gs_s4_t gs_lds_s4_t;
TM_DEV u2_t gs_tr16(const uint16_t* p) {
  gs_s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gs_lds_s4_t*)(p));
  return __builtin_bit_cast(u2_t, v);
}
}  // namespace

template <int KW, bool BT, bool BF16, int ODT, bool BIAS>
__device__ __forceinline__ void gemm_s32_body(const uint16_t* __restrict__ A,
                                              const uint16_t* __restrict__ B,
                                              void* __restrict__ C,
                                              const uint16_t* __restrict__ bias, int N, int lda,
                                              int ldb, int ldc) {
  static_assert(KW == 64 || KW == 128, "k per wave");
  constexpr int NCP = KW / 16;           // 1 KB copies per operand and wave
  constexpr int WREG = 2 * 32 * KW * 2;  // LDS bytes per wave: A slice, B slice
  __shared__ __align__(16) uint8_t lds[4 * WREG];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_n = N >> 5;
  const int m0 = (blockIdx.x / tiles_n) * 32, n0 = (blockIdx.x % tiles_n) * 32;
  const int k0 = wave * KW;
  uint8_t* wa = lds + wave * WREG;
  uint8_t* wb = wa + 32 * KW * 2;
  // copy i, lane l fills bytes 1024 i + 16 l of the slice: row r, slot sl
#pragma unroll
  for (int i = 0; i < NCP; ++i) {
    const int o = 1024 * i + 16 * lane, r = o / (2 * KW), sl = (o % (2 * KW)) / 16;
    dma16(A + (size_t)(m0 + r) * lda + k0 + 8 * (sl ^ (r & 7)), lds_off(wa) + 1024 * i);
  }
#pragma unroll
  for (int i = 0; i < NCP; ++i) {
    if constexpr (BT) {
      const int o = 1024 * i + 16 * lane, r = o / (2 * KW), sl = (o % (2 * KW)) / 16;
      dma16(B + (size_t)(n0 + r) * ldb + k0 + 8 * (sl ^ (r & 7)), lds_off(wb) + 1024 * i);
    } else {
      const int kr = 16 * i + (lane >> 2), pc = lane & 3;  // [KW][32]: 64-byte rows
      dma16(B + (size_t)(k0 + kr) * ldb + n0 + 8 * pc, lds_off(wb) + 1024 * i);
    }
  }
  wait_vm<0>();
  const int l32 = lane & 31, h32 = lane >> 5;
  const int tg = lane >> 4, tj = lane & 15;
  const int tr_k = 8 * (tg >> 1) + (tj >> 2), tr_c = 16 * (tg & 1) + 4 * (tj & 3);
  f16_t acc[2] = {f16_t{}, f16_t{}};
#pragma unroll
  for (int s = 0; s < KW / 16; ++s) {
    const int p = 2 * s + h32;
    const u4_t a = *(const u4_t*)(wa + l32 * (2 * KW) + 16 * (p ^ (l32 & 7)));
    u4_t b;
    if constexpr (BT) {
      b = *(const u4_t*)(wb + l32 * (2 * KW) + 16 * (p ^ (l32 & 7)));
    } else {
      const int ka = 16 * s + tr_k;
      const u2_t lo = gs_tr16((const uint16_t*)(wb + ka * 64) + tr_c);
      const u2_t hi = gs_tr16((const uint16_t*)(wb + (ka + 4) * 64) + tr_c);
      b = u4_t{lo.x, lo.y, hi.x, hi.y};
    }
    acc[s & 1] = mfma32<BF16>(a, b, acc[s & 1]);
  }
  // this wave's partial [e][lane] into its own region (its operand reads are
  // done: the MFMAs consumed them); then the sum over the four waves
  float* red = (float*)wa;
#pragma unroll
  for (int e = 0; e < 16; ++e) red[e * 64 + lane] = acc[0][e] + acc[1][e];
  __syncthreads();
  const int row = tid >> 3, c4 = 4 * (tid & 7);
  // D layout: row 8 (e / 4) + 4 h + e % 4, column l32 (lane l32 + 32 h)
  const int e = 4 * (row >> 3) + (row & 3), hh = (row >> 2) & 1;
  f4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < 4; ++w) v += *(const f4_t*)(lds + w * WREG + 4 * (e * 64 + 32 * hh + c4));
  if constexpr (BIAS) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      v[c] += BF16 ? bf16_bits_to_f32(bias[n0 + c4 + c]) : f16_bits_to_f32(bias[n0 + c4 + c]);
  }
  const size_t ci = (size_t)(m0 + row) * ldc + n0 + c4;
  if constexpr (ODT == TM_DT_F32) {
    *(f4_t*)((float*)C + ci) = v;
  } else {
    u2_t w;
    if constexpr (ODT == TM_DT_BF16) {
      w.x = pack_bf16x2(v[0], v[1]);
      w.y = pack_bf16x2(v[2], v[3]);
    } else {
      w.x = pack_f16x2(v[0], v[1]);
      w.y = pack_f16x2(v[2], v[3]);
    }
    *(u2_t*)((uint16_t*)C + ci) = w;
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

// gemm_s32k<KW>_<bt>_<in>_<out>[_bias]
#define TM_GEMM_S32(KW, BT, BTN, BF, IN, ODT, OUT, BIAS, BN_)                                     \
  extern "C" __global__ __launch_bounds__(256) void gemm_s32k##KW##_##BTN##_##IN##_##OUT##BN_(   \
      const uint16_t* A, const uint16_t* B, void* C, const uint16_t* bias, int M, int N, int K,   \
      int lda, int ldb, int ldc) {                                                                \
    gemm_s32_body<KW, BT, BF, ODT, BIAS>(A, B, C, bias, N, lda, ldb, ldc);                        \
  }
#define TM_GEMM_S32_OUTS(KW, BT, BTN, BF, IN, BIAS, BN_)                             \
  TM_GEMM_S32(KW, BT, BTN, BF, IN, (BF ? TM_DT_BF16 : TM_DT_F16), same, BIAS, BN_) \
  TM_GEMM_S32(KW, BT, BTN, BF, IN, TM_DT_F32, f32, BIAS, BN_)
#define TM_GEMM_S32_ALL(KW)                                   \
  TM_GEMM_S32_OUTS(KW, false, nn, false, f16, false, )        \
  TM_GEMM_S32_OUTS(KW, false, nn, true, bf16, false, )        \
  TM_GEMM_S32_OUTS(KW, true, nt, false, f16, false, )         \
  TM_GEMM_S32_OUTS(KW, true, nt, true, bf16, false, )         \
  TM_GEMM_S32_OUTS(KW, true, nt, false, f16, true, _bias)     \
  TM_GEMM_S32_OUTS(KW, true, nt, true, bf16, true, _bias)
TM_GEMM_S32_ALL(64)
TM_GEMM_S32_ALL(128)

// ----------------------------------------------------------------------------
// Matmul with its sizes in device memory: C[M, N] = A[M, K] @ B[K, N], all
// row-major with leading dimensions K, N, N (make_matmul_2d_kernel,
// _msl_templates.py:588-679, and make_matmul_swizzled_kernel, 682-781, which
// read M, N, K from `device const uint*` buffers).  The grid covers a
// host-known capacity (max_m x max_n); workgroups whose tile lies past the
// sizes read on the device return at once, so one launch (or one captured
// graph node) serves any M <= max_m, N <= max_n (M, N beyond are clamped to
// it).  The buffers' element counts come with the launch: sizes on the device
// whose M K, K N or M N exceed them make the launch do nothing.
//
// 64 x 64 output tile per 256-thread workgroup, K in steps of 16 through LDS
// ([k][row] fp32, so each thread's 4 x 4 outputs take 8 LDS reads per k),
// fp32 accumulation, inputs fp32 / fp16 / bf16.  Tile order: group_m = 0 is
// the 2-D grid (blockIdx.x -> tile column, blockIdx.y -> tile row);
// group_m > 0 is the grouped order of the swizzled template on a 1-D grid -
// runs of group_m tile rows, the tiles of one run taken column by column, so
// that consecutive workgroups share B's columns.
// ----------------------------------------------------------------------------
template <int IDT, int ODT>
__device__ __forceinline__ void gemm_dd_body(const void* __restrict__ A,
                                             const void* __restrict__ B, void* __restrict__ C,
                                             const unsigned* __restrict__ Mp,
                                             const unsigned* __restrict__ Np,
                                             const unsigned* __restrict__ Kp, int max_m,
                                             int max_n, unsigned long long a_elems,
                                             unsigned long long b_elems,
                                             unsigned long long c_elems, int group_m) {
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const int M = (int)min(Mp[0], (unsigned)max_m), N = (int)min(Np[0], (unsigned)max_n);
  const int K = (int)min(Kp[0], 0x7fffffffu);
  // sizes the buffers cannot hold produce nothing (no read or write past them)
  if ((unsigned long long)M * K > a_elems || (unsigned long long)K * N > b_elems ||
      (unsigned long long)M * N > c_elems)
    return;
  const int ntr = (M + 63) / 64, ntc = (N + 63) / 64;
  int tr, tc;
  if (group_m <= 0) {
    tc = blockIdx.x;
    tr = blockIdx.y;
  } else {
    const long long pid = blockIdx.x;
    if (pid >= (long long)ntr * ntc) return;
    const long long per_group = (long long)group_m * ntc;
    const int gid = (int)(pid / per_group);
    const int first = gid * group_m;
    const int rows = min(ntr - first, group_m);
    const int in_group = (int)(pid - (long long)gid * per_group);
    tr = first + in_group % rows;
    tc = in_group / rows;
  }
  if (tr >= ntr || tc >= ntc) return;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = tr * 64, n0 = tc * 64;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i;
      const int r = e >> 4, kk = e & 15, gm = m0 + r, gk = k0 + kk;
      As[kk][r] = (gm < M && gk < K) ? load_as_f32<IDT>(A, (size_t)gm * K + gk) : 0.0f;
      const int kb = e >> 6, c = e & 63, gn = n0 + c, gkb = k0 + kb;
      Bs[kb][c] = (gkb < K && gn < N) ? load_as_f32<IDT>(B, (size_t)gkb * N + gn) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + ty + 16 * i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + tx + 16 * j;
      if (gn < N) store_from_f32<ODT>(C, (size_t)gm * N + gn, acc[i][j]);
    }
  }
}

// gemm_dd_<in>_<out>: out "same" (the input dtype, as the templates) or f32
#define TM_GEMM_DD(IN, IDT, OUT, ODT)                                                           \
  extern "C" __global__ __launch_bounds__(256) void gemm_dd_##IN##_##OUT(                       \
      const void* A, const void* B, void* C, const unsigned* Mp, const unsigned* Np,            \
      const unsigned* Kp, int max_m, int max_n, unsigned long long a_elems,                     \
      unsigned long long b_elems, unsigned long long c_elems, int group_m) {                    \
    gemm_dd_body<IDT, ODT>(A, B, C, Mp, Np, Kp, max_m, max_n, a_elems, b_elems, c_elems,       \
                           group_m);                                                            \
  }
TM_GEMM_DD(f32, TM_DT_F32, same, TM_DT_F32)
TM_GEMM_DD(f16, TM_DT_F16, same, TM_DT_F16)
TM_GEMM_DD(f16, TM_DT_F16, f32, TM_DT_F32)
TM_GEMM_DD(bf16, TM_DT_BF16, same, TM_DT_BF16)
TM_GEMM_DD(bf16, TM_DT_BF16, f32, TM_DT_F32)
