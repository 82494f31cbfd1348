// On-disk int4 checkpoint formats -> the int4 layout of the W4A16 kernels
// (weight [N, K/2] bytes = uint32 [N, K/8] with nibble i of word j holding
// k = 8 j + i; scales / zero-points [N, K/G]), the layout of
// make_int4_matmul_kernel (_msl_templates.py:2687-2697).
//
//   GPTQ: qweight int32 [K/8, N]: nibble i of word (j, n) is q[n, 8 j + i] -
//         the same 8-nibble words as the target, transposed; qzeros int32
//         [K/G, N/8]: nibble i of word (g, b) is z[8 b + i, g] - zero_offset.
//   AWQ:  qweight int32 [K, N/8]: nibble p of word (k, b) is
//         q[8 b + ORDER[p], k], ORDER = (0, 2, 4, 6, 1, 3, 5, 7); qzeros
//         [K/G, N/8] in the same order.
//   scales fp16 [K/G, N] in both: transposed.
//
// One-time conversions at load time; tiles go through LDS so that the global
// reads and writes are both row-contiguous.
#include "common.h"

namespace {
// nibble position of column i (of 8) in an AWQ word: the inverse of ORDER
TM_DEV int awq_pos(int i) { return ((i & 1) << 2) | (i >> 1); }
}  // namespace

// weights: grid (ceil(N / 64), ceil(K / 8 / 64)), block 256.  Output word
// (n, j) of a 64 x 64 tile.
extern "C" __global__ __launch_bounds__(256) void wq_repack_gptq_weight(
    const uint32_t* __restrict__ qw, uint32_t* __restrict__ out, int N, int K) {
  __shared__ uint32_t tile[64][65];
  const int KW = K >> 3;
  const int n0 = blockIdx.x * 64, j0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  // read rows j of qweight (contiguous along n)
  for (int i = tid; i < 64 * 64; i += 256) {
    const int jj = i >> 6, nn = i & 63;
    const int j = j0 + jj, n = n0 + nn;
    tile[jj][nn] = (j < KW && n < N) ? qw[(size_t)j * N + n] : 0u;
  }
  __syncthreads();
  // write rows n of the output (contiguous along j)
  for (int i = tid; i < 64 * 64; i += 256) {
    const int nn = i >> 6, jj = i & 63;
    const int j = j0 + jj, n = n0 + nn;
    if (j < KW && n < N) out[(size_t)n * KW + j] = tile[jj][nn];
  }
}

// grid (ceil(N / 64), ceil(K / 8 / 64)), block 256.  The tile needs qweight
// rows 8 j0 .. 8 j0 + 511 and words n0 / 8 .. n0 / 8 + 7 of each.
extern "C" __global__ __launch_bounds__(256) void wq_repack_awq_weight(
    const uint32_t* __restrict__ qw, uint32_t* __restrict__ out, int N, int K) {
  __shared__ uint32_t tile[512][9];
  const int KW = K >> 3, NB = N >> 3;
  const int n0 = blockIdx.x * 64, j0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  for (int i = tid; i < 512 * 8; i += 256) {
    const int kk = i >> 3, bb = i & 7;
    const int k = 8 * j0 + kk, b = (n0 >> 3) + bb;
    tile[kk][bb] = (k < K && b < NB) ? qw[(size_t)k * NB + b] : 0u;
  }
  __syncthreads();
  for (int i = tid; i < 64 * 64; i += 256) {
    const int nn = i >> 6, jj = i & 63;
    const int j = j0 + jj, n = n0 + nn;
    if (j >= KW || n >= N) continue;
    const int sh = 4 * awq_pos(nn & 7);
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) w |= ((tile[8 * jj + e][nn >> 3] >> sh) & 0xFu) << (4 * e);
    out[(size_t)n * KW + j] = w;
  }
}

// zero-points: out[n, g] = nibble of qzeros[g, n / 8] + offset (uint8).
// grid ceil(N * ng / 256), block 256.
extern "C" __global__ __launch_bounds__(256) void wq_repack_zeros(
    const uint32_t* __restrict__ qz, uint8_t* __restrict__ out, int N, int ng, int awq,
    int offset) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)N * ng) return;
  const int n = (int)(i / ng), g = (int)(i - (long long)n * ng);
  const int pos = awq ? awq_pos(n & 7) : (n & 7);
  const uint32_t w = qz[(size_t)g * (N >> 3) + (n >> 3)];
  out[i] = (uint8_t)(((w >> (4 * pos)) & 0xFu) + offset);
}

// 16-bit transpose: out[c, r] = in[r, c] for in [R, C].  grid (ceil(C / 64),
// ceil(R / 64)), block 256.
extern "C" __global__ __launch_bounds__(256) void wq_transpose16(
    const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int R, int C) {
  __shared__ uint16_t tile[64][66];
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  for (int i = tid; i < 64 * 64; i += 256) {
    const int rr = i >> 6, cc = i & 63;
    const int r = r0 + rr, c = c0 + cc;
    tile[rr][cc] = (r < R && c < C) ? in[(size_t)r * C + c] : (uint16_t)0;
  }
  __syncthreads();
  for (int i = tid; i < 64 * 64; i += 256) {
    const int cc = i >> 6, rr = i & 63;
    const int r = r0 + rr, c = c0 + cc;
    if (r < R && c < C) out[(size_t)c * R + r] = tile[rr][cc];
  }
}
