// Split-K reduction of the W-only kernels' slice sums (the split-K forms of
// wq_streamk and wq_wide write fp32 P[S][M][N], scaled, without bias):
//   Y[m, n] = round(sum_s P[s][m][n] + bias[n])
// in the activation dtype, the bias added to the fp32 sum before the output
// rounding as in the single-launch kernels.  Four consecutive outputs per
// thread (N % 4 == 0), one 8-byte store where the output allows it;
// grid = ceil(M N / 1024) workgroups of 256.
#include "common.h"
#include "wq_common.h"

template <bool BF16>
__device__ __forceinline__ void wq_splitk_reduce_body(const float* __restrict__ P,
                                                      uint16_t* __restrict__ Y,
                                                      const uint16_t* __restrict__ bias, int M,
                                                      int N, int S) {
  const size_t MN = (size_t)M * N;
  const size_t i = 4 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= MN) return;
  f4_t v = *(const f4_t*)(P + i);
  for (int s = 1; s < S; ++s) v += *(const f4_t*)(P + (size_t)s * MN + i);
  const int n = (int)(i % (size_t)N);
  if (bias) {
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] += bias_at(bias, n + c, BF16);
  }
  if (((uintptr_t)(Y + i) & 7u) != 0) {  // an output view not 8-byte aligned
#pragma unroll
    for (int c = 0; c < 4; ++c) store_out(Y, i + c, v[c], BF16);
    return;
  }
  u2_t w;
  if constexpr (BF16) {
    w.x = pack_bf16x2(v[0], v[1]);
    w.y = pack_bf16x2(v[2], v[3]);
  } else {
    w.x = pack_f16x2(v[0], v[1]);
    w.y = pack_f16x2(v[2], v[3]);
  }
  *(u2_t*)(Y + i) = w;
}

extern "C" __global__ __launch_bounds__(256) void wq_splitk_reduce_f16(
    const float* P, uint16_t* Y, const uint16_t* bias, int M, int N, int S) {
  wq_splitk_reduce_body<false>(P, Y, bias, M, N, S);
}
extern "C" __global__ __launch_bounds__(256) void wq_splitk_reduce_bf16(
    const float* P, uint16_t* Y, const uint16_t* bias, int M, int N, int S) {
  wq_splitk_reduce_body<true>(P, Y, bias, M, N, S);
}
