// tl.dot in general form for gfx950: arbitrary element strides per operand,
// a batch dimension, fp16 / bf16 / fp32 / FP8 inputs and the epilogues of the
// reference's strided dot template.
//
//   C[b, m, n] = epi( sum_k A[b, m, k] B[b, k, n] )
//   epi: none | add-matrix (+ Z[b, m, n]) | add-rows (+ Z[b, m, 0]) |
//        add-cols (+ Z[b, 0, n]) | softmax over n | chain-dot (P @ W, W [N, L])
//
// Semantics: _lower_dot_via_prebuilt_template (_lowerer_templates.py:
// 1116-1540): strided operand access (1291-1380), the 3-D batched dot
// (1151-1160, 1453-1470), accumulators initialised from the bias of the
// add-* epilogues (1395-1438), softmax and chain-dot from the unrounded fp32
// product (1488-1522); FP8 operands decoded to float as msl_builtins.py's
// converters do (FP8 output is fp32 there, _msl_templates.py:475-476).
//
// dot_tile: MFMA kernel for 16-bit and FP8 inputs with the none / add-*
// epilogues.  64 x 64 output tile per 256-thread workgroup (2 x 2 waves of
// 32 x 32, v_mfma_f32_16x16x32), K in steps of 32 through two LDS buffers,
// operands stored k-contiguous in LDS whatever their layout in memory.  Each
// operand is fetched in one of three modes chosen by the host from its
// strides: k-contiguous (16-byte row pieces), row-contiguous (a transposed
// view: 16-byte pieces of 8 rows at one k, scattered into LDS) or scalar
// (any strides).  FP8 codes are decoded to fp16 through a 256-entry table in
// LDS: every FP8 value of the five formats is exactly an fp16 value, so the
// fp16 MFMA forms the same products the reference forms in fp32.
//
// dot_tile_f32: the same tiling for fp32 inputs on the fp32 MFMA (the
// reference computes fp32 dots in fp32), K in steps of 16.
//
// dot_rows: one workgroup per (batch, row), fp32 FMA, any dtype and strides,
// every epilogue.  The softmax and chain-dot epilogues need the whole row of
// the product, which the workgroup keeps in LDS (N <= 8192); it also serves
// K = 0 and a bias read in place across rows.
#include "common.h"

enum { EPI_NONE = 0, EPI_ADD_MATRIX = 1, EPI_ADD_ROWS = 2, EPI_ADD_COLS = 3, EPI_SOFTMAX = 4,
       EPI_CHAIN = 5 };
// FP8 dtype codes (include/tm_hip.h)
enum { DT_FP8_E4M3 = 4, DT_FP8_E5M2 = 5, DT_FP8_E4M3B15 = 6, DT_FP8_E4M3B8 = 7,
       DT_FP8_E5M2B16 = 8 };
// operand fetch modes of dot_tile
enum { MODE_KC = 0, MODE_RC = 1, MODE_SCALAR = 2 };

struct DotParams {
  const void* A;
  const void* B;
  void* C;
  const void* Z;
  const void* W;
  long long sa_b, sa_m, sa_k;
  long long sb_b, sb_k, sb_n;
  long long sc_b, sc_m, sc_n;
  long long sz_b, sz_m, sz_n;
  long long sw_n, sw_l;
  int batch, M, N, K, L;
  int epi;
  int in_dt, out_dt, z_dt, w_dt;
  int a_mode, b_mode;
};

namespace {

TM_DEV bool is_fp8(int dt) { return dt >= DT_FP8_E4M3 && dt <= DT_FP8_E5M2B16; }

// One FP8 code as float, by the format's bit fields: exponent field 0 is
// subnormal, the all-ones exponent is NaN for mantissa all ones (4-bit
// exponent formats) or inf / NaN (5-bit formats).
TM_DEV float fp8_to_f32(uint32_t c, int dt) {
  int eb = 4, mb = 3, bias = 7;
  bool has_inf = false;
  if (dt == DT_FP8_E5M2) { eb = 5; mb = 2; bias = 15; has_inf = true; }
  else if (dt == DT_FP8_E4M3B15) { bias = 15; }
  else if (dt == DT_FP8_E4M3B8) { bias = 8; }
  else if (dt == DT_FP8_E5M2B16) { eb = 5; mb = 2; bias = 16; has_inf = true; }
  const uint32_t e = (c >> mb) & ((1u << eb) - 1), m = c & ((1u << mb) - 1);
  const uint32_t emax = (1u << eb) - 1;
  float v;
  if (e == emax && has_inf) v = m == 0 ? __builtin_inff() : __builtin_nanf("");
  else if (e == emax && m == (1u << mb) - 1) v = __builtin_nanf("");
  else if (e == 0) v = __builtin_ldexpf((float)m, 1 - bias - mb);
  else v = __builtin_ldexpf((float)((1u << mb) + m), (int)e - bias - mb);
  return (c & 0x80u) ? -v : v;
}

// Any input element as float (dot_rows).
TM_DEV float load_elem(const void* p, long long i, int dt) {
  if (dt == TM_DT_F32) return ((const float*)p)[i];
  if (dt == TM_DT_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  if (dt == TM_DT_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  return fp8_to_f32(((const uint8_t*)p)[i], dt);
}

TM_DEV void store_elem(void* p, long long i, int dt, float v) { store_as_f32_rt(p, i, dt, v); }

}  // namespace

// ----------------------------------------------------------------------------
// dot_tile: grid (tiles_m * tiles_n, batch), block 256.
// ----------------------------------------------------------------------------
template <bool BF16>
__device__ __forceinline__ void dot_tile_body(const DotParams& p) {
  constexpr int BM = 64, BN = 64, BK = 32, LDK = BK + 8;
  __shared__ __align__(16) uint16_t As[2][BM * LDK];
  __shared__ __align__(16) uint16_t Bs[2][BN * LDK];
  __shared__ uint16_t lut[256];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int m0 = (blockIdx.x / tiles_n) * BM, n0 = (blockIdx.x % tiles_n) * BN;
  const int b = blockIdx.y;
  const bool fp8 = is_fp8(p.in_dt);
  const int esz = fp8 ? 1 : 2;
  if (fp8) {
    lut[tid] = f32_to_f16_bits(fp8_to_f32((uint32_t)tid, p.in_dt));
    __syncthreads();
  }
  const uint8_t* Ab = (const uint8_t*)p.A + (long long)b * p.sa_b * esz;
  const uint8_t* Bb = (const uint8_t*)p.B + (long long)b * p.sb_b * esz;

  // A raw element (16-bit bits or an FP8 code) of operand X at element offset i
  auto raw = [&](const uint8_t* X, long long i) -> uint32_t {
    return fp8 ? (uint32_t)X[i] : (uint32_t)((const uint16_t*)X)[i];
  };
  // Fetch of one operand tile [64 rows][32 k] (rows m or n): 8 raw values per
  // thread.  KC / SCALAR: row r = tid / 4, k = 8 (tid % 4) + e.  RC: rows
  // 8 (tid % 8) + e, k = tid / 8.
  struct Frag { uint32_t v[8]; };
  auto fetch = [&](const uint8_t* X, int mode, int rows, int r0, long long s_r, long long s_k,
                   int k0, Frag& f) {
    if (mode == MODE_RC) {
      const int rc = 8 * (tid & 7), kk = k0 + (tid >> 3);
      const long long base = (long long)(r0 + rc) * s_r + (long long)kk * s_k;
      if (kk < p.K && r0 + rc + 8 <= rows) {
        if (fp8) {
          const u2_t w = *(const u2_t*)(X + base);
#pragma unroll
          for (int e = 0; e < 8; ++e) f.v[e] = ((e < 4 ? w.x : w.y) >> (8 * (e & 3))) & 0xFFu;
        } else {
          const u4_t w = ldg128(X + 2 * base);
          const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) f.v[e] = (d[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          f.v[e] = (kk < p.K && r0 + rc + e < rows) ? raw(X, base + (long long)e * s_r) : 0u;
      }
      return;
    }
    const int r = tid >> 2, kc = k0 + 8 * (tid & 3);
    const long long base = (long long)(r0 + r) * s_r + (long long)kc * s_k;
    if (mode == MODE_KC && r0 + r < rows && kc + 8 <= p.K) {
      if (fp8) {
        const u2_t w = *(const u2_t*)(X + base);
#pragma unroll
        for (int e = 0; e < 8; ++e) f.v[e] = ((e < 4 ? w.x : w.y) >> (8 * (e & 3))) & 0xFFu;
      } else {
        const u4_t w = ldg128(X + 2 * base);
        const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) f.v[e] = (d[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        f.v[e] = (r0 + r < rows && kc + e < p.K) ? raw(X, base + (long long)e * s_k) : 0u;
    }
  };
  auto cvt = [&](uint32_t x) -> uint32_t { return fp8 ? (uint32_t)lut[x] : x; };
  auto put = [&](uint16_t* Xs, int mode, const Frag& f) {
    if (mode == MODE_RC) {
      const int rc = 8 * (tid & 7), kk = tid >> 3;
#pragma unroll
      for (int e = 0; e < 8; ++e) Xs[(rc + e) * LDK + kk] = (uint16_t)cvt(f.v[e]);
    } else {
      const int r = tid >> 2, kc = 8 * (tid & 3);
      u4_t w;
      w.x = cvt(f.v[0]) | (cvt(f.v[1]) << 16);
      w.y = cvt(f.v[2]) | (cvt(f.v[3]) << 16);
      w.z = cvt(f.v[4]) | (cvt(f.v[5]) << 16);
      w.w = cvt(f.v[6]) | (cvt(f.v[7]) << 16);
      *(u4_t*)&Xs[r * LDK + kc] = w;
    }
  };

  f4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  Frag fa, fb;
  const int nk = (p.K + BK - 1) / BK;
  fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, 0, fa);
  fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, 0, fb);
  put(As[0], p.a_mode, fa);
  put(Bs[0], p.b_mode, fb);
  __syncthreads();
  const int q = lane >> 4, r16 = lane & 15;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, (kt + 1) * BK, fa);
      fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, (kt + 1) * BK, fb);
    }
    u4_t af[2], bfr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      af[i] = *(const u4_t*)&As[buf][(32 * wm + 16 * i + r16) * LDK + 8 * q];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      bfr[j] = *(const u4_t*)&Bs[buf][(32 * wn + 16 * j + r16) * LDK + 8 * q];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma16<BF16>(af[i], bfr[j], acc[i][j]);
    if (kt + 1 < nk) {
      put(As[buf ^ 1], p.a_mode, fa);
      put(Bs[buf ^ 1], p.b_mode, fb);
    }
    __syncthreads();
  }

  // epilogue: lane holds rows 32 wm + 16 i + 4 q + e, column 32 wn + 16 j + r16
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 32 * wn + 16 * j + r16;
      if (col >= p.N) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + 32 * wm + 16 * i + 4 * q + e;
        if (row >= p.M) continue;
        float v = acc[i][j][e];
        const long long zb = (long long)b * p.sz_b;
        if (p.epi == EPI_ADD_MATRIX)
          v += load_elem(p.Z, zb + (long long)row * p.sz_m + (long long)col * p.sz_n, p.z_dt);
        else if (p.epi == EPI_ADD_ROWS)
          v += load_elem(p.Z, zb + (long long)row * p.sz_m, p.z_dt);
        else if (p.epi == EPI_ADD_COLS)
          v += load_elem(p.Z, zb + (long long)col * p.sz_n, p.z_dt);
        store_elem(p.C, (long long)b * p.sc_b + (long long)row * p.sc_m + (long long)col * p.sc_n,
                   p.out_dt, v);
      }
    }
}

extern "C" __global__ __launch_bounds__(256) void dot_tile_f16(DotParams p) {
  dot_tile_body<false>(p);
}
extern "C" __global__ __launch_bounds__(256) void dot_tile_bf16(DotParams p) {
  dot_tile_body<true>(p);
}

// ----------------------------------------------------------------------------
// dot_tile_f32: fp32 inputs with the none / add-* epilogues on the fp32 MFMA
// (v_mfma_f32_16x16x4_f32: fp32 products, 4 added per step into the fp32
// accumulator).  Grid (tiles_m * tiles_n, batch), block 256: a 64 x 64 output
// tile, 2 x 2 waves of 32 x 32, each 2 x 2 MFMA tiles of 16 x 16
// (A[l % 16][l / 16], B[l / 16][l % 16], D[4 (l / 16) + e][l % 16]).  K in
// steps of 16 through two LDS buffers, both operands k-major there
// ([16 k][64 + 16 pad] floats: a 16-lane operand read is 16 consecutive
// floats, the four k rows of one read 16 banks apart).  Fetch modes of an
// operand [64 rows][16 k]: KC  row tid / 4, 4 k from 4 (tid % 4), one
// 16-byte load; RC  k tid / 16, 4 rows from 4 (tid % 16), one 16-byte load
// stored as one 16-byte LDS write; SCALAR  the KC mapping element by element.
// Rows and k past the operand read as zero.
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void dot_tile_f32(DotParams p) {
  constexpr int TB = 64, TK = 16, TS = TB + 16;
  __shared__ __align__(16) float As[2][TK * TS], Bs[2][TK * TS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + TB - 1) / TB;
  const int m0 = (blockIdx.x / tiles_n) * TB, n0 = (blockIdx.x % tiles_n) * TB;
  const int b = blockIdx.y;
  const float* Ab = (const float*)p.A + (long long)b * p.sa_b;
  const float* Bb = (const float*)p.B + (long long)b * p.sb_b;

  auto fetch = [&](const float* X, int mode, int rows, int r0, long long s_r, long long s_k,
                   int k0) -> f4_t {
    f4_t v = f4_t{0.f, 0.f, 0.f, 0.f};
    if (mode == MODE_RC) {  // s_r == 1
      const int kk = k0 + (tid >> 4), rc = r0 + 4 * (tid & 15);
      if (kk < p.K) {
        const float* q = X + rc + (long long)kk * s_k;
        if (rc + 3 < rows) {
          v = *(const f4_t*)q;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (rc + j < rows) v[j] = q[j];
        }
      }
      return v;
    }
    const int r = r0 + (tid >> 2), kc = k0 + 4 * (tid & 3);
    if (r < rows) {
      const float* q = X + (long long)r * s_r + (long long)kc * s_k;
      if (mode == MODE_KC && kc + 3 < p.K) {
        v = *(const f4_t*)q;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kc + j < p.K) v[j] = q[(long long)j * s_k];
      }
    }
    return v;
  };
  auto put = [&](float* Xs, int mode, f4_t v) {
    if (mode == MODE_RC) {
      *(f4_t*)&Xs[(tid >> 4) * TS + 4 * (tid & 15)] = v;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) Xs[(4 * (tid & 3) + j) * TS + (tid >> 2)] = v[j];
    }
  };

  f4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int nk = (p.K + TK - 1) / TK;
  f4_t fa = fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, 0);
  f4_t fb = fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, 0);
  put(As[0], p.a_mode, fa);
  put(Bs[0], p.b_mode, fb);
  __syncthreads();
  const int q = lane >> 4, r16 = lane & 15;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      fa = fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, (kt + 1) * TK);
      fb = fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, (kt + 1) * TK);
    }
    const float* as = As[buf];
    const float* bs = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < TK / 4; ++kk) {
      const int kr = (4 * kk + q) * TS;
      float a[2], bv[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        a[t] = as[kr + 32 * wm + 16 * t + r16];
        bv[t] = bs[kr + 32 * wn + 16 * t + r16];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      put(As[buf ^ 1], p.a_mode, fa);
      put(Bs[buf ^ 1], p.b_mode, fb);
    }
    __syncthreads();
  }

  // epilogue: lane holds rows 32 wm + 16 i + 4 q + e, column 32 wn + 16 j + r16
  const long long zb = (long long)b * p.sz_b;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 32 * wn + 16 * j + r16;
      if (col >= p.N) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + 32 * wm + 16 * i + 4 * q + e;
        if (row >= p.M) continue;
        float v = acc[i][j][e];
        if (p.epi == EPI_ADD_MATRIX)
          v += load_elem(p.Z, zb + (long long)row * p.sz_m + (long long)col * p.sz_n, p.z_dt);
        else if (p.epi == EPI_ADD_ROWS)
          v += load_elem(p.Z, zb + (long long)row * p.sz_m, p.z_dt);
        else if (p.epi == EPI_ADD_COLS)
          v += load_elem(p.Z, zb + (long long)col * p.sz_n, p.z_dt);
        store_elem(p.C, (long long)b * p.sc_b + (long long)row * p.sc_m + (long long)col * p.sc_n,
                   p.out_dt, v);
      }
    }
}

// ----------------------------------------------------------------------------
// dot_rows: grid batch * M, block 256.  Columns in groups of 1024 (4 per
// thread); A's row staged through LDS in pieces of 2048; for softmax and
// chain-dot the product row stays in LDS (N <= 8192).
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void dot_rows(DotParams p) {
  constexpr int KCH = 2048, NPT = 4, NMAX = 8192;
  __shared__ float arow[KCH];
  __shared__ float prow[NMAX];
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int b = blockIdx.x / p.M, m = blockIdx.x - b * p.M;
  const long long ab = (long long)b * p.sa_b + (long long)m * p.sa_m;
  const long long bb = (long long)b * p.sb_b;
  const long long zb = (long long)b * p.sz_b;
  const long long cb = (long long)b * p.sc_b + (long long)m * p.sc_m;
  const bool keep = p.epi == EPI_SOFTMAX || p.epi == EPI_CHAIN;
  // the row bias is read before any store of this row (in place: Z may be C)
  const float rbias = p.epi == EPI_ADD_ROWS ? load_elem(p.Z, zb + (long long)m * p.sz_m, p.z_dt)
                                            : 0.0f;
  __syncthreads();
  for (int n0 = 0; n0 < p.N; n0 += 256 * NPT) {
    float acc[NPT];
#pragma unroll
    for (int j = 0; j < NPT; ++j) acc[j] = 0.0f;
    for (int k0 = 0; k0 < p.K; k0 += KCH) {
      const int kn = min(KCH, p.K - k0);
      for (int k = tid; k < kn; k += 256)
        arow[k] = load_elem(p.A, ab + (long long)(k0 + k) * p.sa_k, p.in_dt);
      __syncthreads();
      for (int k = 0; k < kn; ++k) {
        const float a = arow[k];
        const long long kb = bb + (long long)(k0 + k) * p.sb_k;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
          const int n = n0 + tid + 256 * j;
          if (n < p.N) acc[j] = __builtin_fmaf(a, load_elem(p.B, kb + (long long)n * p.sb_n, p.in_dt), acc[j]);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int n = n0 + tid + 256 * j;
      if (n >= p.N) continue;
      float v = acc[j];
      if (keep) {
        prow[n] = v;
        continue;
      }
      if (p.epi == EPI_ADD_MATRIX)
        v += load_elem(p.Z, zb + (long long)m * p.sz_m + (long long)n * p.sz_n, p.z_dt);
      else if (p.epi == EPI_ADD_ROWS)
        v += rbias;
      else if (p.epi == EPI_ADD_COLS)
        v += load_elem(p.Z, zb + (long long)n * p.sz_n, p.z_dt);
      store_elem(p.C, cb + (long long)n * p.sc_n, p.out_dt, v);
    }
  }
  if (!keep) return;
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  if (p.epi == EPI_SOFTMAX) {
    float mx = -__builtin_inff();
    for (int n = tid; n < p.N; n += 256) mx = fmaxf(mx, prow[n]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
    for (int n = tid; n < p.N; n += 256) s += expf(prow[n] - mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    s = red[0] + red[1] + red[2] + red[3];
    for (int n = tid; n < p.N; n += 256)
      store_elem(p.C, cb + (long long)n * p.sc_n, p.out_dt, expf(prow[n] - mx) / s);
    return;
  }
  // chain-dot: C[b, m, l] = sum_n P[n] W[n, l]
  for (int l = tid; l < p.L; l += 256) {
    float v = 0.0f;
    for (int n = 0; n < p.N; ++n)
      v = __builtin_fmaf(prow[n], load_elem(p.W, (long long)n * p.sw_n + (long long)l * p.sw_l, p.w_dt), v);
    store_elem(p.C, cb + (long long)l * p.sc_n, p.out_dt, v);
  }
}
