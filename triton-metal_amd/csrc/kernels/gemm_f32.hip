// Dense fp32 matmul on the fp32 MFMA (v_mfma_f32_16x16x4_f32): the
// reference's default dtype (make_matmul_kernel(dtype="fp32"),
// _msl_templates.py:447-585; make_fused_linear_kernel in fp32, 4013-4135).
//
//   C[M, N] = A[M, K] @ B[K, N]              (nn)
//   C[M, N] = A[M, K] @ W[N, K]^T (+ bias)   (nt, the nn.Linear layout)
//
// Products and sums stay fp32, as in the reference: the MFMA multiplies in
// fp32 and adds 4 products per step into the fp32 accumulator.
//
// 64 x 64 output tile per 256-thread workgroup: 2 x 2 waves of 32 x 32, each
// 2 x 2 MFMA tiles of 16 x 16 (A[l % 16][l / 16], B[l / 16][l % 16],
// D[4 (l / 16) + e][l % 16]).  K in steps of 16 through two LDS buffers; the
// next step's global loads are in flight in registers while the current step
// multiplies.  Both operands sit in LDS k-major, [16 k][64 (+16 pad) m or n],
// so a 16-lane operand read is 16 consecutive floats and the four k rows of
// one read land 16 banks apart.  Rows and k past the matrix count as zero.
//
// gemm_f32t64_* (A and B 16-byte aligned, leading dimensions multiples of 4):
// each thread's piece of 4 floats per operand and step is one unconditional
// 16-byte load.  A piece starts at a multiple of 4 of an aligned row; one
// past the matrix is moved to the last piece holding an element of it (row
// at most rows - 1, k or n at most its extent - 1), so every load reads an
// aligned chunk holding a valid element (never a page the matrix does not
// touch), and the elements past the matrix are zeroed when the piece is
// stored to LDS.  A load whose registers another branch also wrote would
// make the compiler wait for it on the spot, which is what the unconditional
// form avoids: the next step's loads stay in flight across the MFMAs.
// gemm_f32t64u_*: any alignment, element loads each bounds-checked.
#include "common.h"

namespace {

constexpr int FB = 64;         // output tile edge
constexpr int FK = 16;         // k per LDS step
constexpr int FS = FB + 16;    // LDS row stride (floats)

template <int ODT> TM_DEV void f32_store(void* C, size_t i, float v) {
  if constexpr (ODT == TM_DT_F32) ((float*)C)[i] = v;
  else if constexpr (ODT == TM_DT_F16) ((uint16_t*)C)[i] = f32_to_f16_bits(v);
  else ((uint16_t*)C)[i] = f32_to_bf16_bits(v);
}

// 4 consecutive floats of row r at k .. k+3, element by element (zero past
// rows / k)
TM_DEV f4_t f32_row4(const float* __restrict__ P, long ld, int r, int rows, int k, int K) {
  f4_t v = f4_t{0.f, 0.f, 0.f, 0.f};
  if (r >= rows) return v;
  const float* p = P + (size_t)r * ld + k;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (k + j < K) v[j] = p[j];
  return v;
}

// The 16-byte piece of row r at k .. k+3 (k a multiple of 4, rows >= 1,
// K >= 1), moved back into the matrix when past it; its elements past the
// matrix are zeroed by f32_keep.
TM_DEV f4_t f32_piece(const float* __restrict__ P, long ld, int r, int rows, int k, int K) {
  return *(const f4_t*)(P + (size_t)min(r, rows - 1) * ld + min(k, (K - 1) & ~3));
}
TM_DEV f4_t f32_keep(f4_t v, int r, int rows, int k, int K) {
  const int n = r < rows ? max(0, min(K - k, 4)) : 0;
  if (n < 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = j < n ? v[j] : 0.f;
  }
  return v;
}

template <bool BT, int ODT, bool BIAS, bool VEC>
__device__ __forceinline__ void gemm_f32_body(const float* __restrict__ A,
                                              const float* __restrict__ B, void* __restrict__ C,
                                              const float* __restrict__ bias, int M, int N, int K,
                                              int lda, int ldb, int ldc) {
  __shared__ __align__(16) float As[2][FK * FS], Bs[2][FK * FS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = (N + FB - 1) / FB;
  const int m0 = (int)(blockIdx.x / ntn) * FB, n0 = (int)(blockIdx.x % ntn) * FB;
  // global -> registers: A (and W of nt) as row r = tid / 4, k piece 4 (tid % 4);
  // B of nn as k row tid / 16, n piece 4 (tid % 16)
  const int ar = tid >> 2, ak = 4 * (tid & 3);
  const int bk = tid >> 4, bn = 4 * (tid & 15);
  f4_t ra, rb;
  auto load = [&](int k0) {
    if constexpr (VEC) {
      ra = f32_piece(A, lda, m0 + ar, M, k0 + ak, K);
      if constexpr (BT) rb = f32_piece(B, ldb, n0 + ar, N, k0 + ak, K);
      else rb = f32_piece(B, ldb, k0 + bk, K, n0 + bn, N);
    } else {
      ra = f32_row4(A, lda, m0 + ar, M, k0 + ak, K);
      if constexpr (BT) rb = f32_row4(B, ldb, n0 + ar, N, k0 + ak, K);
      else rb = f32_row4(B, ldb, k0 + bk, K, n0 + bn, N);
    }
  };
  // the pieces loaded at k0 into LDS buffer buf
  auto stash = [&](int buf, int k0) {
    if constexpr (VEC) {
      ra = f32_keep(ra, m0 + ar, M, k0 + ak, K);
      if constexpr (BT) rb = f32_keep(rb, n0 + ar, N, k0 + ak, K);
      else rb = f32_keep(rb, k0 + bk, K, n0 + bn, N);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) As[buf][(ak + j) * FS + ar] = ra[j];
    if constexpr (BT) {
#pragma unroll
      for (int j = 0; j < 4; ++j) Bs[buf][(ak + j) * FS + ar] = rb[j];
    } else {
      *(f4_t*)&Bs[buf][bk * FS + bn] = rb;
    }
  };

  f4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int l16 = lane & 15, q = lane >> 4;
  const int nst = (K + FK - 1) / FK;
  load(0);
  stash(0, 0);
  __syncthreads();
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1;
    if (s + 1 < nst) load((s + 1) * FK);
    const float* as = As[buf];
    const float* bs = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < FK / 4; ++kk) {
      const int kr = (4 * kk + q) * FS;
      float a[2], b[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        a[t] = as[kr + 32 * wm + 16 * t + l16];
        b[t] = bs[kr + 32 * wn + 16 * t + l16];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nst) stash(buf ^ 1, (s + 1) * FK);
    __syncthreads();
  }
  // D[4 q + e][l16] of tile (i, j)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + 32 * wn + 16 * j + l16;
    if (col >= N) continue;
    const float bv = BIAS ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + 32 * wm + 16 * i + 4 * q + e;
        if (row < M) f32_store<ODT>(C, (size_t)row * ldc + col, acc[i][j][e] + bv);
      }
  }
}

}  // namespace

// gemm_f32t64{,u}_<nn|nt>_<out>[_bias]: out f32 / f16 / bf16; grid =
// ceil(M / 64) * ceil(N / 64), block = 256
#define TM_GEMM_F32_V(KN, VEC, BTN, BT, OUT, ODT, BIAS, SUF)                                     \
  extern "C" __global__ __launch_bounds__(256) void KN##_##BTN##_##OUT##SUF(                    \
      const float* A, const float* B, void* C, const float* bias, int M, int N, int K, int lda, \
      int ldb, int ldc) {                                                                       \
    gemm_f32_body<BT, ODT, BIAS, VEC>(A, B, C, bias, M, N, K, lda, ldb, ldc);                   \
  }
#define TM_GEMM_F32(BTN, BT, OUT, ODT, BIAS, SUF)                 \
  TM_GEMM_F32_V(gemm_f32t64, true, BTN, BT, OUT, ODT, BIAS, SUF)  \
  TM_GEMM_F32_V(gemm_f32t64u, false, BTN, BT, OUT, ODT, BIAS, SUF)
#define TM_GEMM_F32_OUT(OUT, ODT)                 \
  TM_GEMM_F32(nn, false, OUT, ODT, false, )       \
  TM_GEMM_F32(nt, true, OUT, ODT, false, )        \
  TM_GEMM_F32(nt, true, OUT, ODT, true, _bias)
TM_GEMM_F32_OUT(f32, TM_DT_F32)
TM_GEMM_F32_OUT(f16, TM_DT_F16)
TM_GEMM_F32_OUT(bf16, TM_DT_BF16)
