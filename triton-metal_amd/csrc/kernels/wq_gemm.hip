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
//   wq_skinny_*  M <= 8: the whole X[M, K] is staged once per workgroup in LDS;
//                one workgroup owns 16 output columns, its 4 waves split K and
//                are reduced through LDS.  Weights stream with 128-bit loads.
//   wq_tiled_*   larger M: 64 x 64 output tiles, X tiles double-buffered in LDS,
//                each wave unpacks its own 16 weight rows in registers.
//   wq_general   any shape / dtype: fp32 arithmetic exactly as the reference
//                template, one wave per output column.
//   wq_dequant   the dequantised weight tile round((float(q) - z) * s).
#include "common.h"

namespace {

// Scalar of a runtime dtype (scales / zero-points); dt < 0 means absent (0).
TM_DEV float ld_scalar(const void* p, size_t i, int dt) {
  switch (dt) {
    case TM_DT_F32: return ((const float*)p)[i];
    case TM_DT_F16: return (float)((const half_t*)p)[i];
    case TM_DT_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case 3: return (float)((const uint8_t*)p)[i];
    default: return 0.0f;
  }
}

// int4: one word (8 nibbles) -> one 8 x 16-bit MFMA operand of OFF + q in
// element order [n0, n4, n1, n5, n2, n6, n3, n7].
template <bool BF16> TM_DEV u4_t w4_operand(uint32_t w) {
  constexpr uint32_t MAGIC = BF16 ? 0x43004300u : 0x64006400u;  // 128.0 / 1024.0
  u4_t r;
  r.x = (w & 0x000F000Fu) | MAGIC;
  r.y = ((w >> 4) & 0x000F000Fu) | MAGIC;
  r.z = ((w >> 8) & 0x000F000Fu) | MAGIC;
  r.w = ((w >> 12) & 0x000F000Fu) | MAGIC;
  return r;
}
template <bool BF16> constexpr float w4_offset() { return BF16 ? 128.0f : 1024.0f; }

// int8: two words (8 signed bytes) -> exact q in natural element order.
template <bool BF16> TM_DEV u4_t w8_operand(uint32_t w0, uint32_t w1) {
  uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;  // q + 128
  u4_t r;
  if constexpr (!BF16) {
    const uint32_t e = 0x64646464u;                       // halves 1152 + q
    const h2_t off = h2_t{(half_t)1152.0f, (half_t)1152.0f};
    r.x = h2_bits(as_h2(perm_b32(e, u0, 0x04010400u)) - off);
    r.y = h2_bits(as_h2(perm_b32(e, u0, 0x04030402u)) - off);
    r.z = h2_bits(as_h2(perm_b32(e, u1, 0x04010400u)) - off);
    r.w = h2_bits(as_h2(perm_b32(e, u1, 0x04030402u)) - off);
  } else {
    // exact fp32 of q, whose low 16 bits are zero -> high half is exact bf16
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = (float)((u0 >> (8 * i)) & 0xFFu) - 128.0f;
      f[4 + i] = (float)((u1 >> (8 * i)) & 0xFFu) - 128.0f;
    }
    r.x = perm_b32(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u);
    r.y = perm_b32(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u);
    r.z = perm_b32(__float_as_uint(f[5]), __float_as_uint(f[4]), 0x07060302u);
    r.w = perm_b32(__float_as_uint(f[7]), __float_as_uint(f[6]), 0x07060302u);
  }
  return r;
}

// Permute 8 halves [x0..x7] into [x0,x4,x1,x5,x2,x6,x3,x7] (the int4 operand order).
TM_DEV u4_t perm_x8(u4_t x) {
  u4_t r;
  r.x = perm_b32(x.z, x.x, 0x05040100u);
  r.y = perm_b32(x.z, x.x, 0x07060302u);
  r.z = perm_b32(x.w, x.y, 0x05040100u);
  r.w = perm_b32(x.w, x.y, 0x07060302u);
  return r;
}

template <bool BF16> TM_DEV float sum8(u4_t v) {
  uint32_t d[4] = {v.x, v.y, v.z, v.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (BF16) {
      s += __uint_as_float(d[i] << 16) + __uint_as_float(d[i] & 0xFFFF0000u);
    } else {
      h2_t h = as_h2(d[i]);
      s += (float)h.x + (float)h.y;
    }
  }
  return s;
}

// Sum over aligned groups of 16 lanes.
TM_DEV float sum16(float v) {
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 1, 64);
  return v;
}

TM_DEV void store_out(uint16_t* Y, size_t i, float v, bool bf16) {
  Y[i] = bf16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

}  // namespace

// ----------------------------------------------------------------------------
// Skinny kernel: M <= 8.  grid.x = N / 16, block = 256 (4 waves).
// Preconditions (host-checked): N % 16 == 0; K % (4 * CK) == 0 with CK = 128
// (int4) or 64 (int8); int4: G % 128 == 0; LDS: M * (K + 8) * 2 bytes of X
// plus M * K / 128 * 4 bytes of chunk sums (dynamic).
// ----------------------------------------------------------------------------
template <int QB, bool BF16>
__device__ __forceinline__ void wq_skinny_body(const uint16_t* __restrict__ X,
                                               const uint8_t* __restrict__ W,
                                               uint16_t* __restrict__ Y,
                                               const void* __restrict__ S,
                                               const void* __restrict__ Z, int M, int N, int K,
                                               int G, int sdt, int zdt) {
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
  int rows[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) rows[e] = min(4 * q + e, M - 1);
  const int kw = K >> 2;
  const int kbeg = wave * kw;
  const size_t rowbytes = (QB == 4) ? (size_t)(K >> 1) : (size_t)K;
  const uint8_t* wrow = W + (size_t)n * rowbytes;
  const size_t ngroups = (QB == 4) ? (size_t)((K + G - 1) / G) : 1;
  const uint16_t* xrow = xs + m * ldx;

  // Weight (and int4 scale / zero-point) loads of a batch of PF chunks;
  // the first batch is issued before X is staged so its latency overlaps.
  constexpr int PF = 8;
  const int nsteps = kw / CK;
  u4_t wv[PF];
  float scv[PF], zbv[PF];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if (s0 + i < nsteps) {
        int kc = kbeg + (s0 + i) * CK;
        size_t boff = (QB == 4) ? (size_t)(kc >> 1) + 16 * q : (size_t)kc + 16 * q;
        wv[i] = ldg128(wrow + boff);
        if constexpr (QB == 4) {
          const size_t gi = (size_t)n * ngroups + kc / G;
          scv[i] = ld_scalar(S, gi, sdt);
          zbv[i] = w4_offset<BF16>() + ld_scalar(Z, gi, zdt);
        }
      }
    }
  };
  load_batch(0);

  // Stage X (16-byte pieces) and the per-128-k-chunk row sums.
  const int pieces = M * (K >> 3);
  for (int c = tid; c < pieces; c += 256) {
    int r = c / (K >> 3), kc = (c - r * (K >> 3)) << 3;
    u4_t v = ldg128(X + (size_t)r * K + kc);
    float s = sum16(sum8<BF16>(v));
    if ((c & 15) == 0) xsum[r * nch + (kc >> 7)] = s;
    if constexpr (QB == 4) v = perm_x8(v);
    *(u4_t*)(xs + r * ldx + kc) = v;
  }
  __syncthreads();

  f4_t y = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsteps; s0 += PF) {
    if (s0 > 0) load_batch(s0);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if (s0 + i < nsteps) {
        int kc = kbeg + (s0 + i) * CK;
        if constexpr (QB == 4) {
          const int kl = kc + 32 * q;
          f4_t a = {0.f, 0.f, 0.f, 0.f};
          uint32_t ws[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            a = mfma16<BF16>(*(const u4_t*)(xrow + kl + 8 * j), w4_operand<BF16>(ws[j]), a);
          const int ch = kc >> 7;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            y[e] += scv[i] * (a[e] - zbv[i] * xsum[rows[e] * nch + ch]);
        } else {
          const int kl = kc + 16 * q;
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
      const float sc = ld_scalar(S, (size_t)n, sdt);
      const float z = ld_scalar(Z, (size_t)n, zdt);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float xt = 0.0f;
        if (zdt >= 0)
          for (int c = 0; c < nch; ++c) xt += xsum[rows[e] * nch + c];
        y[e] = sc * (y[e] - z * xt);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int row = 4 * q + e;
      if (row < M) store_out(Y, (size_t)row * N + n, y[e], BF16);
    }
  }
}

// ----------------------------------------------------------------------------
// Tiled kernel: any M.  Output tile 64 (m) x 64 (n); block = 256 (4 waves),
// wave w owns columns n0 + 16w .. +15 for all 64 rows (4 m-tiles).
// K steps of KS = 256 with X tiles (and their 128-k chunk sums)
// double-buffered in LDS.
// Preconditions: K % 256 == 0, N % 64 == 0, int4: G % 128 == 0.
// Grid: tiles enumerated so that the row blocks sharing one column block land
// on the same XCD (blockIdx % 8 picks the XCD).
// ----------------------------------------------------------------------------
template <int QB, bool BF16>
__device__ __forceinline__ void wq_tiled_body(const uint16_t* __restrict__ X,
                                              const uint8_t* __restrict__ W,
                                              uint16_t* __restrict__ Y,
                                              const void* __restrict__ S,
                                              const void* __restrict__ Z, int M, int N, int K,
                                              int G, int sdt, int zdt) {
  constexpr int BM = 64, KS = 256, LDX = KS + 8;
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
  const size_t rowbytes = (QB == 4) ? (size_t)(K >> 1) : (size_t)K;
  const uint8_t* wrow = W + (size_t)n * rowbytes;
  const int ngroups = (QB == 4) ? (K + G - 1) / G : 1;

  // X staging: 64 rows x 256 k = 2048 16-byte pieces, 8 per thread; piece p
  // of row r covers k = 8p..8p+7, 16 consecutive pieces form one 128-k chunk.
  // Global loads of step s+1 (X pieces, weights, scales) are issued before
  // the MFMAs of step s; the X pieces go to the other LDS buffer afterwards.
  constexpr int NL = (QB == 4) ? 2 : 4;  // 16-byte weight loads per lane per step
  u4_t xr[8], wv[NL], wn[NL];
  float scv[NL], zbv[NL], scn[NL], zbn[NL];
  auto load_x = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = tid + 256 * i;
      int r = c >> 5, kc = (c & 31) << 3;
      int gr = m0 + r;
      xr[i] = u4_t{0u, 0u, 0u, 0u};
      if (gr < M) xr[i] = ldg128(X + (size_t)gr * K + k0 + kc);
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = tid + 256 * i;
      int r = c >> 5, kc = (c & 31) << 3;
      u4_t v = xr[i];
      float s = sum16(sum8<BF16>(v));
      if ((c & 15) == 0) xsm[buf][kc >> 7][r] = s;
      if constexpr (QB == 4) v = perm_x8(v);
      *(u4_t*)(&xs[buf][r * LDX + kc]) = v;
    }
  };
  auto load_w = [&](int k0, u4_t* dst, float* sc, float* zb) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      int kc = k0 + i * (QB == 4 ? 128 : 64);
      size_t boff = (QB == 4) ? (size_t)(kc >> 1) + 16 * q : (size_t)kc + 16 * q;
      dst[i] = ldg128(wrow + boff);
      if constexpr (QB == 4) {
        const size_t gi = (size_t)n * ngroups + kc / G;
        sc[i] = ld_scalar(S, gi, sdt);
        zb[i] = w4_offset<BF16>() + ld_scalar(Z, gi, zdt);
      }
    }
  };

  f4_t y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  f4_t xtot[4];  // int8 with zero-points: running row sums of X
#pragma unroll
  for (int t = 0; t < 4; ++t) xtot[t] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int nsteps = K / KS;
  load_w(0, wv, scv, zbv);
  load_x(0);
  store_x(0);
  __syncthreads();
  for (int st = 0; st < nsteps; ++st) {
    const int k0 = st * KS, buf = st & 1;
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
          u4_t b = w4_operand<BF16>(ws[j]);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            a[t] = mfma16<BF16>(*(const u4_t*)(xb + (t * 16 + (lane & 15)) * LDX + kl + 8 * j),
                                b, a[t]);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f4_t xv = *(const f4_t*)(&xsm[buf][i][t * 16 + 4 * q]);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[t][e] += scv[i] * (a[t][e] - zbv[i] * xv[e]);
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
    if constexpr (QB == 8) {
      if (zdt >= 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          xtot[t] += *(const f4_t*)(&xsm[buf][0][t * 16 + 4 * q]) +
                     *(const f4_t*)(&xsm[buf][1][t * 16 + 4 * q]);
      }
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
    sc = ld_scalar(S, (size_t)n, sdt);
    z = ld_scalar(Z, (size_t)n, zdt);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int row = m0 + t * 16 + 4 * q + e;
      float v = y[t][e];
      if constexpr (QB == 8) v = sc * (v - z * xtot[t][e]);
      if (row < M) store_out(Y, (size_t)row * N + n, v, BF16);
    }
}

// ----------------------------------------------------------------------------
// General kernel: any M, N, K (int4: K even), any dtypes.  One wave per
// column n; lanes stride over k; fp32 arithmetic exactly as the reference
// template: w = (float(q) - z) * s; acc += x * w.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void st_any(void* p, size_t i, int dt, float v) {
  switch (dt) {
    case TM_DT_F32: ((float*)p)[i] = v; break;
    case TM_DT_F16: ((uint16_t*)p)[i] = f32_to_f16_bits(v); break;
    default: ((uint16_t*)p)[i] = f32_to_bf16_bits(v); break;
  }
}

extern "C" __global__ __launch_bounds__(256) void wq_general(
    const void* __restrict__ X, const uint8_t* __restrict__ W, void* __restrict__ Y,
    const void* __restrict__ S, const void* __restrict__ Z, int M, int N, int K, int G, int qbits,
    int xdt, int sdt, int zdt) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int ngroups = (qbits == 4) ? (K + G - 1) / G : 1;
  for (int m = 0; m < M; ++m) {
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) {
      float qv;
      size_t si;
      if (qbits == 4) {
        uint8_t byte = W[(size_t)n * (K / 2) + k / 2];
        qv = (float)((k & 1) ? ((byte >> 4) & 0xF) : (byte & 0xF));
        si = (size_t)n * ngroups + k / G;
      } else {
        qv = (float)(int8_t)W[(size_t)n * K + k];
        si = (size_t)n;
      }
      float w = (qv - ld_scalar(Z, si, zdt)) * ld_scalar(S, si, sdt);
      acc += ld_scalar(X, (size_t)m * K + k, xdt) * w;
    }
    acc = wave_sum(acc);
    if (lane == 0) st_any(Y, (size_t)m * N + n, xdt, acc);
  }
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
// Named instantiations: wq_{skinny,tiled}_q{4,8}_{f16,bf16}
// ----------------------------------------------------------------------------
#define TM_WQ_INST(KIND, QB, BF, ACT)                                                           \
  extern "C" __global__ __launch_bounds__(256) void wq_##KIND##_q##QB##_##ACT(                   \
      const uint16_t* X, const uint8_t* W, uint16_t* Y, const void* S, const void* Z, int M,     \
      int N, int K, int G, int sdt, int zdt) {                                                   \
    wq_##KIND##_body<QB, BF>(X, W, Y, S, Z, M, N, K, G, sdt, zdt);                               \
  }

TM_WQ_INST(skinny, 4, false, f16)
TM_WQ_INST(skinny, 4, true, bf16)
TM_WQ_INST(skinny, 8, false, f16)
TM_WQ_INST(skinny, 8, true, bf16)
TM_WQ_INST(tiled, 4, false, f16)
TM_WQ_INST(tiled, 4, true, bf16)
TM_WQ_INST(tiled, 8, false, f16)
TM_WQ_INST(tiled, 8, true, bf16)
