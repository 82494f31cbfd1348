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
// epilogues.  64 x 64 output tile (dot_tile128: 128 x 128, for problems with
// enough tiles to fill the chip) per 256-thread workgroup (2 x 2 waves,
// v_mfma_f32_16x16x32), K in steps of 64 (32 for the 128 tile) through two
// LDS buffers.  Each operand is fetched in one of three modes chosen by the
// host from its strides: k-contiguous (16-byte row pieces, kept [row][k] in
// LDS), row-contiguous (a transposed view: 16-byte pieces of 8 rows at one k,
// kept [k][row] in LDS and read back through the transposing LDS read) or
// scalar (any strides, element loads, the 64 tile only).  FP8 codes are decoded to fp16 through a 256-entry table in
// LDS: every FP8 value of the five formats is exactly an fp16 value, so the
// fp16 MFMA forms the same products the reference forms in fp32.
//
// dot_tile_f32: the same tiling for fp32 inputs on the fp32 MFMA (the
// reference computes fp32 dots in fp32), K in steps of 16.
//
// dot_rows: one workgroup per (batch, row), fp32 FMA, any dtype and strides,
// every epilogue.  The softmax and chain-dot epilogues need the whole row of
// the product, which the workgroup keeps in LDS (N <= 8192); it also serves
// K = 0 and a bias read in place across rows.  With an fp32 output the
// softmax takes the tile kernels and dot_softmax_rows instead, with another
// output and N <= 2048 dot_softmax16, and chain-dot with C apart from its
// operands the fused dot_chain kernels.
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

// The element at byte `byte` (0..3) of an aligned 4-byte word, as float.
TM_DEV float word_elem(uint32_t w, int byte, int dt) {
  if (dt == TM_DT_F32) return __uint_as_float(w);
  const uint16_t h = (uint16_t)(w >> (8 * (byte & 2)));
  if (dt == TM_DT_F16) return f16_bits_to_f32(h);
  if (dt == TM_DT_BF16) return bf16_bits_to_f32(h);
  return fp8_to_f32((w >> (8 * byte)) & 0xFFu, dt);
}

}  // namespace

// Keep the first n elements of a piece (the rest zero): 16-bit elements in 4
// dwords, or FP8 codes in the low 2.
template <bool FP8> TM_DEV u4_t piece_keep(u4_t w, int n) {
  const int bits = (FP8 ? 8 : 16) * n;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int lo = 32 * d;
    w[d] = bits >= lo + 32 ? w[d] : bits <= lo ? 0u : w[d] & ((1u << (bits - lo)) - 1u);
  }
  return w;
}

// Epilogue of the tile kernels: lane holds rows wt wm + 16 i + 4 q + e,
// column wt wn + 16 j + r16 of the workgroup's tile; the add-* bias in fp32,
// then one store in the output dtype.  The element loop stays rolled:
// unrolled, the runtime-dtype loads and stores of 4 x 4 tiles outgrow the
// unroller and the accumulators go to scratch.
template <int FT>
TM_DEV void tile_epilogue(const DotParams& p, const f4_t (&acc)[FT][FT], int m0, int n0, int b,
                          int wt, int wm, int wn, int q, int r16) {
  const long long zb = (long long)b * p.sz_b;
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int j = 0; j < FT; ++j) {
      const int col = n0 + wt * wn + 16 * j + r16;
      const f4_t a4 = acc[i][j];
      if (col >= p.N) continue;
#pragma unroll 1
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wt * wm + 16 * i + 4 * q + e;
        if (row >= p.M) continue;
        float v = a4[e];
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
// dot_tile{,128}_<f16|bf16|fp8>: both operands KC or RC, grid (tiles, batch),
// block 256.  Output tile BT x BT (64 or 128), 2 x 2 waves of BT/2 x BT/2,
// each (BT/32)^2 MFMA tiles of 16 x 16 (v_mfma_f32_16x16x32: lane l supplies
// row l % 16, k 8 (l / 16) .. +7 of each operand and holds
// D[4 (l / 16) + e][l % 16]).  K in steps of BK (64; 32 for the 128 tile, to
// keep two waves per SIMD).  An operand's [BT rows][BK k] step is
// BT BK / 2048 pieces of 8 elements per thread (piece h: rows + 64 (h %
// (BT / 64)), k + 32 (h / (BT / 64))), each one 16-byte (FP8: 8-byte) load:
//   KC  row tid / 4, k 8 (tid % 4) .. +7
//   RC  rows 8 (tid % 8) .. +7, k tid / 8
// kept packed in registers.  Loads run two steps ahead (two register sets):
// step kt + 2 is loaded while step kt multiplies from LDS and step kt + 1
// goes from registers to the other LDS buffer.  Every load is
// unconditional: a piece starts at a multiple of 8 elements of an aligned
// row, and one past the operand is moved to the last piece holding an
// element of it (row at most rows - 1, k at most K - 1), so each load reads
// an aligned chunk holding a valid element (never a page the operand does
// not touch) and nothing writes its registers before the LDS store that
// consumes it; that store zeroes the elements past the operand.
// LDS, KC operands: [row][BK k + 8 pad] halves, the 16-byte k chunk c of
// row r at c ^ ((r / 16) % 4), so the 16 rows of one MFMA operand read touch
// every bank once.  RC operands: [k][BT rows + 16 pad] halves, each piece
// stored whole at its k; an operand is read with two ds_read_b64_tr_b16 per
// lane (rows r0 + 4 (j % 4) .. +3, j = lane % 16), which hand each lane the
// 4 k values of one row.
// Workgroups are taken in XCD order (dispatch i runs on XCD i % 8): when the
// tile count is a multiple of 8, XCD x takes tiles x T / 8 .. (x + 1) T / 8 - 1,
// rows of tiles that share their A rows in one L2.
// ----------------------------------------------------------------------------
typedef short dot_s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) dot_s4_t dot_lds_s4_t;
TM_DEV u2_t dot_tr16(const uint16_t* p) {
  dot_s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((dot_lds_s4_t*)(p));
  return __builtin_bit_cast(u2_t, v);
}

TM_DEV int tile_lds(int row, int k, int ldk) {
  return row * ldk + ((((k >> 3) ^ (row >> 4)) & 3) | (k >> 3 & ~3)) * 8 + (k & 7);
}

template <bool BF16, bool FP8, int BT, bool ARC, bool BRC>
__device__ __forceinline__ void dot_tile_vec_body(const DotParams& p) {
  constexpr int BK = BT == 64 ? 64 : 32, LDK = BK + 8;
  constexpr int LDT = BT + 16;  // RC operands: [k][BT rows + 16 pad]
  constexpr int WT = BT / 2;   // wave tile edge
  constexpr int FT = WT / 16;  // MFMA tiles per wave tile edge
  constexpr int RP = BT / 64;  // row blocks of 64 per operand step
  constexpr int NP = RP * BK / 32;  // pieces per thread and operand step
  constexpr int esz = FP8 ? 1 : 2;
  constexpr int ASZ = ARC ? BK * LDT : BT * LDK, BSZ = BRC ? BK * LDT : BT * LDK;
  __shared__ __align__(16) uint16_t As[2][ASZ];
  __shared__ __align__(16) uint16_t Bs[2][BSZ];
  __shared__ uint16_t lut[256];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + BT - 1) / BT;
  const int ntiles = gridDim.x;
  const int t = (ntiles & 7) ? (int)blockIdx.x
                             : (int)(blockIdx.x & 7) * (ntiles >> 3) + (int)(blockIdx.x >> 3);
  const int m0 = (t / tiles_n) * BT, n0 = (t % tiles_n) * BT;
  const int b = blockIdx.y;
  if constexpr (FP8) {
    lut[tid] = f32_to_f16_bits(fp8_to_f32((uint32_t)tid, p.in_dt));
  }
  const uint8_t* Ab = (const uint8_t*)p.A + (long long)b * p.sa_b * esz;
  const uint8_t* Bb = (const uint8_t*)p.B + (long long)b * p.sb_b * esz;

  auto vload = [&](const uint8_t* X, long long i) -> u4_t {
    if constexpr (FP8) {
      const u2_t w = *(const u2_t*)(X + i);
      return u4_t{w.x, w.y, 0u, 0u};
    } else {
      return ldg128(X + 2 * i);
    }
  };
  // piece h of operand X [rows][K] (rows from r0) at k0
  auto fetch = [&](const uint8_t* X, int mode, int rows, int r0, long long s_r, long long s_k,
                   int k0, int h) -> u4_t {
    const int rs = 64 * (h % RP), ks = 32 * (h / RP);
    long long off;
    if (mode == MODE_RC) {  // s_r == 1
      const int rc = r0 + rs + 8 * (tid & 7), kk = k0 + ks + (tid >> 3);
      off = (long long)min(rc, (rows - 1) & ~7) + (long long)min(kk, p.K - 1) * s_k;
    } else {                // s_k == 1
      const int r = r0 + rs + (tid >> 2), kc = k0 + ks + 8 * (tid & 3);
      off = (long long)min(r, rows - 1) * s_r + (long long)min(kc, (p.K - 1) & ~7);
    }
    return vload(X, off);
  };
  auto elem = [&](const u4_t& w, int e) -> uint32_t {
    if constexpr (FP8) return (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
    else return (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
  };
  auto cvt = [&](uint32_t x) -> uint32_t {
    if constexpr (FP8) return (uint32_t)lut[x];
    else return x;
  };
  // piece h (fetched at k0) into LDS buffer Xs, elements past the operand
  // zeroed: KC pieces into [row][k] (swizzled), RC pieces (8 rows at one k)
  // as they are into [k][rows]
  auto put = [&](auto rcc, uint16_t* Xs, u4_t w, int rows, int r0, int k0, int h) {
    constexpr bool RC = decltype(rcc)::value;
    const int rs = 64 * (h % RP), ks = 32 * (h / RP);
    int n, off;
    if constexpr (RC) {
      const int rc = rs + 8 * (tid & 7), kk = ks + (tid >> 3);
      n = k0 + kk < p.K ? max(0, min(rows - r0 - rc, 8)) : 0;
      off = kk * LDT + rc;
    } else {
      const int r = rs + (tid >> 2), kc = ks + 8 * (tid & 3);
      n = r0 + r < rows ? max(0, min(p.K - k0 - kc, 8)) : 0;
      off = tile_lds(r, kc, LDK);
    }
    if (n < 8) w = piece_keep<FP8>(w, n);
    u4_t o = w;
    if constexpr (FP8) {
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] = cvt(elem(w, 2 * d)) | (cvt(elem(w, 2 * d + 1)) << 16);
    }
    *(u4_t*)(Xs + off) = o;
  };
  // MFMA operand of rows r0 .. r0 + 15 at k kb .. kb + 31: lane l supplies row
  // l % 16, k kb + 8 (l / 16) .. +7.  KC: one 16-byte read.  RC: two
  // transposing reads (ds_read_b64_tr_b16: lane i of a 16-lane group gets
  // element i % 4 of the 8 bytes lane 4 e + i / 4 addresses, for e = 0..3),
  // lane j addressing rows r0 + 4 (j % 4) .. +3 at k kb + 8 (l / 16) + j / 4
  // (+ 4 for the second read)
  const std::integral_constant<bool, true> rc_c;
  const std::integral_constant<bool, false> kc_c;
  auto frag = [&](auto rcc, const uint16_t* Xs, int r0, int kb) -> u4_t {
    if constexpr (decltype(rcc)::value) {
      const int j = lane & 15;
      const uint16_t* a = Xs + (kb + 8 * (lane >> 4) + (j >> 2)) * LDT + r0 + 4 * (j & 3);
      const u2_t lo = dot_tr16(a), hi = dot_tr16(a + 4 * LDT);
      return u4_t{lo.x, lo.y, hi.x, hi.y};
    } else {
      return *(const u4_t*)(Xs + tile_lds(r0 + (lane & 15), kb + 8 * (lane >> 4), LDK));
    }
  };

  f4_t acc[FT][FT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int j = 0; j < FT; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (p.K + BK - 1) / BK;
  u4_t ra0[NP], rb0[NP], ra1[NP], rb1[NP];
  constexpr int AM = ARC ? MODE_RC : MODE_KC, BM = BRC ? MODE_RC : MODE_KC;
  auto load_step = [&](u4_t* ra, u4_t* rb, int kt) {
#pragma unroll
    for (int h = 0; h < NP; ++h) {
      ra[h] = fetch(Ab, AM, p.M, m0, p.sa_m, p.sa_k, kt * BK, h);
      rb[h] = fetch(Bb, BM, p.N, n0, p.sb_n, p.sb_k, kt * BK, h);
    }
  };
  auto put_step = [&](int buf, const u4_t* ra, const u4_t* rb, int kt) {
#pragma unroll
    for (int h = 0; h < NP; ++h) {
      if constexpr (ARC) put(rc_c, As[buf], ra[h], p.M, m0, kt * BK, h);
      else put(kc_c, As[buf], ra[h], p.M, m0, kt * BK, h);
      if constexpr (BRC) put(rc_c, Bs[buf], rb[h], p.N, n0, kt * BK, h);
      else put(kc_c, Bs[buf], rb[h], p.N, n0, kt * BK, h);
    }
  };
  const int q = lane >> 4, r16 = lane & 15;
  auto compute = [&](int buf) {
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      u4_t af[FT], bfr[FT];
#pragma unroll
      for (int i = 0; i < FT; ++i) {
        if constexpr (ARC) af[i] = frag(rc_c, As[buf], WT * wm + 16 * i, 32 * s);
        else af[i] = frag(kc_c, As[buf], WT * wm + 16 * i, 32 * s);
      }
#pragma unroll
      for (int j = 0; j < FT; ++j) {
        if constexpr (BRC) bfr[j] = frag(rc_c, Bs[buf], WT * wn + 16 * j, 32 * s);
        else bfr[j] = frag(kc_c, Bs[buf], WT * wn + 16 * j, 32 * s);
      }
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int j = 0; j < FT; ++j) acc[i][j] = mfma16<BF16>(af[i], bfr[j], acc[i][j]);
    }
  };
  // step kt: its operands are in LDS buffer kt & 1, step kt + 1's in the
  // registers (rn), and the other set (rf) is free for step kt + 2
  auto step = [&](int kt, u4_t* rfa, u4_t* rfb, const u4_t* rna, const u4_t* rnb) {
    if (kt + 2 < nk) load_step(rfa, rfb, kt + 2);
    compute(kt & 1);
    if (kt + 1 < nk) put_step((kt + 1) & 1, rna, rnb, kt + 1);
    __syncthreads();
  };

  load_step(ra0, rb0, 0);
  if (nk > 1) load_step(ra1, rb1, 1);
  if constexpr (FP8) __syncthreads();  // the table before the first store
  put_step(0, ra0, rb0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, ra0, rb0, ra1, rb1);
    if (kt + 1 < nk) step(kt + 1, ra1, rb1, ra0, rb0);
  }

  tile_epilogue<FT>(p, acc, m0, n0, b, WT, wm, wn, q, r16);
}

// ----------------------------------------------------------------------------
// dot_tile_s_<f16|bf16|fp8>: some operand with neither k nor its rows
// contiguous (or unaligned), grid (tiles_m * tiles_n, batch), block 256.
// 64 x 64 output tile, 2 x 2 waves of 32 x 32, each 2 x 2 MFMA tiles of
// 16 x 16 (v_mfma_f32_16x16x32: lane l supplies row l % 16, k 8 (l / 16) ..
// +7 of each operand and holds D[4 (l / 16) + e][l % 16]); K in steps of 32
// through two LDS buffers ([row][32 k + 8 pad]).  Each thread fetches 8
// elements per operand and step, one load each:
//   KC / SCALAR  row tid / 4, k 8 (tid % 4) .. +7
//   RC           rows 8 (tid % 8) .. +7, k tid / 8
// at addresses clamped into the operand (row at most rows - 1, k at most
// K - 1), unconditional and into registers of their own, so that the next
// step's loads stay in flight across the MFMAs; the LDS store zeroes the
// elements past the operand and packs them (8 halves, or FP8 codes decoded
// to halves).
// ----------------------------------------------------------------------------
template <bool BF16, bool FP8>
__device__ __forceinline__ void dot_tile_s_body(const DotParams& p) {
  constexpr int BT = 64, BK = 32, LDK = BK + 8;
  constexpr int esz = FP8 ? 1 : 2;
  __shared__ __align__(16) uint16_t As[2][BT * LDK];
  __shared__ __align__(16) uint16_t Bs[2][BT * LDK];
  __shared__ uint16_t lut[256];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + BT - 1) / BT;
  const int m0 = (blockIdx.x / tiles_n) * BT, n0 = (blockIdx.x % tiles_n) * BT;
  const int b = blockIdx.y;
  if constexpr (FP8) {
    lut[tid] = f32_to_f16_bits(fp8_to_f32((uint32_t)tid, p.in_dt));
    __syncthreads();
  }
  const uint8_t* Ab = (const uint8_t*)p.A + (long long)b * p.sa_b * esz;
  const uint8_t* Bb = (const uint8_t*)p.B + (long long)b * p.sb_b * esz;

  auto raw = [&](const uint8_t* X, long long i) -> uint32_t {
    if constexpr (FP8) return (uint32_t)X[i];
    else return (uint32_t)((const uint16_t*)X)[i];
  };
  struct Raw8 { uint32_t v[8]; };
  // the thread's 8 elements of operand X [rows][K] (rows from r0) at k0
  auto fetch = [&](const uint8_t* X, int mode, int rows, int r0, long long s_r, long long s_k,
                   int k0) -> Raw8 {
    Raw8 f;
    if (mode == MODE_RC) {
      const int rc = r0 + 8 * (tid & 7), kk = min(k0 + (tid >> 3), p.K - 1);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        f.v[e] = raw(X, (long long)min(rc + e, rows - 1) * s_r + (long long)kk * s_k);
      return f;
    }
    const int r = min(r0 + (tid >> 2), rows - 1), kc = k0 + 8 * (tid & 3);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      f.v[e] = raw(X, (long long)r * s_r + (long long)min(kc + e, p.K - 1) * s_k);
    return f;
  };
  auto cvt = [&](uint32_t x) -> uint32_t {
    if constexpr (FP8) return (uint32_t)lut[x];
    else return x;
  };
  // the elements fetched for rows from r0 at k0 into LDS buffer Xs, those
  // past the operand zeroed
  auto put = [&](uint16_t* Xs, int mode, const Raw8& f, int rows, int r0, int k0) {
    if (mode == MODE_RC) {
      const int rc = 8 * (tid & 7), kk = tid >> 3;
      const bool kok = k0 + kk < p.K;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        Xs[(rc + e) * LDK + kk] = kok && r0 + rc + e < rows ? (uint16_t)cvt(f.v[e]) : (uint16_t)0;
      return;
    }
    const int r = tid >> 2, kc = 8 * (tid & 3);
    const bool rok = r0 + r < rows;
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = rok && k0 + kc + e < p.K ? cvt(f.v[e]) : 0u;
    u4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = h[2 * d] | (h[2 * d + 1] << 16);
    *(u4_t*)&Xs[r * LDK + kc] = o;
  };

  f4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (p.K + BK - 1) / BK;
  Raw8 fa = fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, 0);
  Raw8 fb = fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, 0);
  put(As[0], p.a_mode, fa, p.M, m0, 0);
  put(Bs[0], p.b_mode, fb, p.N, n0, 0);
  __syncthreads();
  const int q = lane >> 4, r16 = lane & 15;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      fa = fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, (kt + 1) * BK);
      fb = fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, (kt + 1) * BK);
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
      put(As[buf ^ 1], p.a_mode, fa, p.M, m0, (kt + 1) * BK);
      put(Bs[buf ^ 1], p.b_mode, fb, p.N, n0, (kt + 1) * BK);
    }
    __syncthreads();
  }
  tile_epilogue<2>(p, acc, m0, n0, b, 32, wm, wn, q, r16);
}

// dot_tile{,128}_<f16|bf16|fp8> and dot_tile_s_<f16|bf16|fp8>: fp8 covers
// the five FP8 formats (in_dt), decoded to fp16 through the table
#define TM_DOT_TILE_M(NAME, BF16, FP8, BT, ARC, BRC)                                \
  extern "C" __global__ __launch_bounds__(256) void NAME(DotParams p) {             \
    dot_tile_vec_body<BF16, FP8, BT, ARC, BRC>(p);                                  \
  }
// _<a><b>: each operand k-contiguous (k) or row-contiguous (r)
#define TM_DOT_TILE(NAME, BF16, FP8, BT)                         \
  TM_DOT_TILE_M(NAME##_kk, BF16, FP8, BT, false, false)          \
  TM_DOT_TILE_M(NAME##_kr, BF16, FP8, BT, false, true)           \
  TM_DOT_TILE_M(NAME##_rk, BF16, FP8, BT, true, false)           \
  TM_DOT_TILE_M(NAME##_rr, BF16, FP8, BT, true, true)
#define TM_DOT_TILE_S(NAME, BF16, FP8)                                              \
  extern "C" __global__ __launch_bounds__(256) void NAME(DotParams p) {             \
    dot_tile_s_body<BF16, FP8>(p);                                                  \
  }
TM_DOT_TILE(dot_tile_f16, false, false, 64)
TM_DOT_TILE(dot_tile_bf16, true, false, 64)
TM_DOT_TILE(dot_tile_fp8, false, true, 64)
TM_DOT_TILE(dot_tile128_f16, false, false, 128)
TM_DOT_TILE(dot_tile128_bf16, true, false, 128)
TM_DOT_TILE(dot_tile128_fp8, false, true, 128)
TM_DOT_TILE_S(dot_tile_s_f16, false, false)
TM_DOT_TILE_S(dot_tile_s_bf16, true, false)
TM_DOT_TILE_S(dot_tile_s_fp8, false, true)

// ----------------------------------------------------------------------------
// dot_tile_f32: fp32 inputs with the none / add-* epilogues on the fp32 MFMA
// (v_mfma_f32_16x16x4_f32: fp32 products, 4 added per step into the fp32
// accumulator).  Grid (tiles_m * tiles_n, batch), block 256: a 64 x 64 output
// tile, 2 x 2 waves of 32 x 32, each 2 x 2 MFMA tiles of 16 x 16
// (A[l % 16][l / 16], B[l / 16][l % 16], D[4 (l / 16) + e][l % 16]).  K in
// steps of 16 through two LDS buffers, both operands k-major there
// ([16 k][64 + 16 pad] floats: a 16-lane operand read is 16 consecutive
// floats, the four k rows of one read 16 banks apart).  Pieces of 4 floats
// per thread and operand: KC / SCALAR  row tid / 4, k 4 (tid % 4) .. +3;
// RC  k tid / 16, rows 4 (tid % 16) .. +3 (stored as one 16-byte LDS write).
// VEC (both operands KC or RC): one unconditional 16-byte load per piece,
// moved back to the last piece holding a valid element when past the
// operand, and the elements past it zeroed at the LDS store, as in dot_tile;
// dot_tile_s_f32: element loads, each bounds-checked.
// ----------------------------------------------------------------------------
template <bool VEC>
__device__ __forceinline__ void dot_tile_f32_body(const DotParams& p) {
  constexpr int TB = 64, TK = 16, TS = TB + 16;
  __shared__ __align__(16) float As[2][TK * TS], Bs[2][TK * TS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + TB - 1) / TB;
  const int m0 = (blockIdx.x / tiles_n) * TB, n0 = (blockIdx.x % tiles_n) * TB;
  const int b = blockIdx.y;
  const float* Ab = (const float*)p.A + (long long)b * p.sa_b;
  const float* Bb = (const float*)p.B + (long long)b * p.sb_b;

  // piece of operand X [rows][K] (rows from r0) at k0; n = its count of valid
  // elements (VEC: applied when the piece is stored)
  auto fetch = [&](const float* X, int mode, int rows, int r0, long long s_r, long long s_k,
                   int k0, int& n) -> f4_t {
    if constexpr (VEC) {
      long long off;
      if (mode == MODE_RC) {  // s_r == 1
        const int rc = r0 + 4 * (tid & 15), kk = k0 + (tid >> 4);
        off = (long long)min(rc, (rows - 1) & ~3) + (long long)min(kk, p.K - 1) * s_k;
        n = kk < p.K ? max(0, min(rows - rc, 4)) : 0;
      } else {                // s_k == 1
        const int r = r0 + (tid >> 2), kc = k0 + 4 * (tid & 3);
        off = (long long)min(r, rows - 1) * s_r + (long long)min(kc, (p.K - 1) & ~3);
        n = r < rows ? max(0, min(p.K - kc, 4)) : 0;
      }
      return *(const f4_t*)(X + off);
    } else {
      n = 4;
      f4_t v = f4_t{0.f, 0.f, 0.f, 0.f};
      if (mode == MODE_RC) {
        const int rc = r0 + 4 * (tid & 15), kk = k0 + (tid >> 4);
        if (kk < p.K) {
          const float* q = X + (long long)rc * s_r + (long long)kk * s_k;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (rc + j < rows) v[j] = q[(long long)j * s_r];
        }
        return v;
      }
      const int r = r0 + (tid >> 2), kc = k0 + 4 * (tid & 3);
      if (r < rows) {
        const float* q = X + (long long)r * s_r + (long long)kc * s_k;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kc + j < p.K) v[j] = q[(long long)j * s_k];
      }
      return v;
    }
  };
  auto put = [&](float* Xs, int mode, f4_t v, int n) {
    if constexpr (VEC) {
      if (n < 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = j < n ? v[j] : 0.f;
      }
    }
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
  int xa, xb;
  f4_t fa = fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, 0, xa);
  f4_t fb = fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, 0, xb);
  put(As[0], p.a_mode, fa, xa);
  put(Bs[0], p.b_mode, fb, xb);
  __syncthreads();
  const int q = lane >> 4, r16 = lane & 15;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      fa = fetch(Ab, p.a_mode, p.M, m0, p.sa_m, p.sa_k, (kt + 1) * TK, xa);
      fb = fetch(Bb, p.b_mode, p.N, n0, p.sb_n, p.sb_k, (kt + 1) * TK, xb);
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
      put(As[buf ^ 1], p.a_mode, fa, xa);
      put(Bs[buf ^ 1], p.b_mode, fb, xb);
    }
    __syncthreads();
  }

  tile_epilogue<2>(p, acc, m0, n0, b, 32, wm, wn, q, r16);
}

extern "C" __global__ __launch_bounds__(256) void dot_tile_f32(DotParams p) {
  dot_tile_f32_body<true>(p);
}
extern "C" __global__ __launch_bounds__(256) void dot_tile_s_f32(DotParams p) {
  dot_tile_f32_body<false>(p);
}

// ----------------------------------------------------------------------------
// dot_softmax_rows: grid batch * M, block 256.  The softmax epilogue with an
// fp32 output after the tile kernels have written the unrounded fp32 product
// into C: each workgroup replaces its row by exp(x - max) / sum, with the
// arithmetic of dot_rows' softmax (N <= 8192).
// ----------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void dot_softmax_rows(DotParams p) {
  constexpr int NMAX = 8192;
  __shared__ float prow[NMAX];
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x / p.M, m = blockIdx.x - b * p.M;
  float* crow = (float*)p.C + (long long)b * p.sc_b + (long long)m * p.sc_m;
  for (int n = tid; n < p.N; n += 256) prow[n] = crow[(long long)n * p.sc_n];
  __syncthreads();
  float mx = -__builtin_inff();
  for (int n = tid; n < p.N; n += 256) mx = fmaxf(mx, prow[n]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sm = 0.0f;
  for (int n = tid; n < p.N; n += 256) sm += expf(prow[n] - mx);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sm += __shfl_xor(sm, o, 64);
  if (lane == 0) red[wave] = sm;
  __syncthreads();
  sm = red[0] + red[1] + red[2] + red[3];
  for (int n = tid; n < p.N; n += 256) crow[(long long)n * p.sc_n] = expf(prow[n] - mx) / sm;
}

// ----------------------------------------------------------------------------
// dot_chain{16,32}_<f16|bf16|fp8|f32>: the chain-dot epilogue fused,
//   C[b, m, l] = sum_n P[b, m, n] W[n, l],  P = A @ B in fp32, never rounded,
// at any strides.  Grid (ceil(M / BM) * ceil(L / 64), batch), block 256:
// each workgroup owns a BM x 64 tile of C and walks N in chunks of 64.  For
// each chunk the P tile [BM][64] is formed over K in steps of 64 (wave w:
// columns 16 w .. +15 of the chunk, BM / 16 tiles of 16 rows) on
// v_mfma_f32_16x16x32 (FP8 decoded exactly to fp16 through the LDS table, as
// in dot_tile) or, for fp32 inputs, v_mfma_f32_16x16x4_f32; written to LDS as
// fp32 and multiplied into the C tile on v_mfma_f32_16x16x4_f32 (wave w:
// columns 16 w .. +15 of the C tile) against the chunk's W [64][64] (any
// input dtype, as fp32).  Every operand is read by element loads whose lane
// order follows its smaller stride (the _vb forms: a 16-bit B row-contiguous
// in aligned pieces by 16-byte loads, as dot_tile's RC operands), at addresses clamped into the operand
// (W: the aligned 4-byte word holding the element, decoded at the LDS
// store); the LDS store zeroes the elements past the operand.  Loads run two
// steps ahead in two register sets, since a step holds few MFMAs; every step
// issues the same loads (its chunk's W included, stored to LDS with the
// chunk's last k step; the last step's loads again at the end), since a load
// under a branch makes the compiler wait for every load at the next use of an
// older one, and the stores mask with integer ANDs rather than selects, which
// the compiler turns into branches.
// LDS: A [BM][64 k + 8], B [64 n][64 k + 8] halves (16-byte operand reads at
// a 144-byte row pitch: the 16 rows of one read start on distinct 4-bank
// groups; fp32 inputs: + 4 floats, the 16 rows x 4 k of one read on 64
// distinct banks); floats: P [BM][64 + 4] (the 16 rows x 4 k of one
// read on 64 distinct banks), W [2 chunks][64 n][64 + 16].
// ----------------------------------------------------------------------------
namespace {
template <bool BF16, bool FP8, int BM, bool F32 = false, bool SMX = false, bool VB = false>
__device__ __forceinline__ void dot_chain_body(const DotParams& p) {
  // VB: 16-bit B row-contiguous (n) in aligned 16-byte pieces of 8 n at one k,
  // two per thread and step (piece h: k (tid + 256 h) / 8, n 8 (tid % 8) .. +7),
  // kept in rb[4 h .. 4 h + 3]
  static_assert(!VB || (!FP8 && !F32), "B pieces of 8 halves");
  // SMX: the softmax epilogue instead of chain-dot; P keeps whole rows of up
  // to SMX_NMAX columns and no W is read
  constexpr int SMX_NMAX = 2048;
  constexpr int BN = 64, BK = 64, BL = 64, LDK = BK + (F32 ? 4 : 8);
  constexpr int LDP = (SMX ? SMX_NMAX : BN) + 4, LDW = BL + 16;
  constexpr int RI = BM / 16;        // MFMA row tiles per wave
  constexpr int AE = BM * BK / 256;  // A elements per thread and step
  constexpr int BE = BN * BK / 256;  // B elements per thread and step
  constexpr int WE = BN * BL / 256;  // W elements per thread and chunk
  using lds_t = typename std::conditional<F32, uint32_t, uint16_t>::type;
  __shared__ __align__(16) lds_t As[BM * LDK];
  __shared__ __align__(16) lds_t Bs[BN * LDK];
  __shared__ __align__(16) float Ps[BM * LDP];
  __shared__ __align__(16) float Ws[2][SMX ? 4 : BN * LDW];
  __shared__ uint16_t lut[256];
  using raw_t = typename std::conditional<F32, uint32_t,
                typename std::conditional<FP8, uint8_t, uint16_t>::type>::type;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  const int tiles_l = SMX ? 1 : (p.L + BL - 1) / BL;
  const int m0 = (int)(blockIdx.x / tiles_l) * BM, l0 = (int)(blockIdx.x % tiles_l) * BL;
  const int b = blockIdx.y;
  if constexpr (FP8) lut[tid] = f32_to_f16_bits(fp8_to_f32((uint32_t)tid, p.in_dt));
  const raw_t* Ab = (const raw_t*)p.A + (long long)b * p.sa_b;
  const raw_t* Bb = (const raw_t*)p.B + (long long)b * p.sb_b;

  // element e of a thread: A (row, k), B (n, k), W (n, l), the lanes along
  // the operand's smaller stride
  const bool a_kf = p.sa_k <= p.sa_m, b_kf = p.sb_k <= p.sb_n, w_lf = p.sw_l <= p.sw_n;
  auto a_at = [&](int e, int& r, int& k) {
    const int i = tid + 256 * e;
    if (a_kf) { r = i / BK; k = i % BK; } else { r = i % BM; k = i / BM; }
  };
  auto b_at = [&](int e, int& n, int& k) {
    const int i = tid + 256 * e;
    if (b_kf) { n = i / BK; k = i % BK; } else { n = i % BN; k = i / BN; }
  };
  auto w_at = [&](int e, int& n, int& l) {
    const int i = tid + 256 * e;
    if (w_lf) { n = i / BL; l = i % BL; } else { n = i % BN; l = i / BN; }
  };

  const int ksteps = (p.K + BK - 1) / BK, nchunks = (p.N + BN - 1) / BN;
  const int nsteps = ksteps * nchunks;
  // step s: k step s % ksteps of chunk s / ksteps
  auto is_last = [&](int s) { return s % ksteps == ksteps - 1; };
  // W element (n, l) of chunk c: its byte address.  The aligned 4-byte word
  // holding it is loaded (no dtype branch between a load and its use, which
  // would wait for the load there) and decoded when stored to LDS.
  const int wsz = p.w_dt == TM_DT_F32 ? 4 : p.w_dt == TM_DT_F16 || p.w_dt == TM_DT_BF16 ? 2 : 1;
  auto w_addr = [&](int c, int n, int l) -> uintptr_t {
    return (uintptr_t)p.W + (uintptr_t)(((long long)min(c * BN + n, p.N - 1) * p.sw_n +
                                         (long long)min(l0 + l, p.L - 1) * p.sw_l) * wsz);
  };
  // its offset in the 4-byte word (the address's low bits, in 32 bits)
  auto w_byte = [&](int c, int n, int l) -> int {
    const uint32_t i = (uint32_t)min(c * BN + n, p.N - 1) * (uint32_t)p.sw_n +
                       (uint32_t)min(l0 + l, p.L - 1) * (uint32_t)p.sw_l;
    return (int)((i * (uint32_t)wsz + (uint32_t)(uintptr_t)p.W) & 3u);
  };
  auto load_step = [&](uint32_t* ra, uint32_t* rb, uint32_t* rw, int s) {
    const int c = s / ksteps, k0 = (s - c * ksteps) * BK, n0 = c * BN;
#pragma unroll
    for (int e = 0; e < AE; ++e) {
      int r, k;
      a_at(e, r, k);
      ra[e] = Ab[(long long)min(m0 + r, p.M - 1) * p.sa_m + (long long)min(k0 + k, p.K - 1) * p.sa_k];
    }
    if constexpr (VB) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int pc = tid + 256 * h, k = pc >> 3, n8 = 8 * (pc & 7);
        const u4_t w = ldg128(Bb + (long long)min(n0 + n8, (p.N - 1) & ~7) +
                              (long long)min(k0 + k, p.K - 1) * p.sb_k);
        rb[4 * h] = w.x; rb[4 * h + 1] = w.y; rb[4 * h + 2] = w.z; rb[4 * h + 3] = w.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < BE; ++e) {
        int n, k;
        b_at(e, n, k);
        rb[e] = Bb[(long long)min(n0 + n, p.N - 1) * p.sb_n + (long long)min(k0 + k, p.K - 1) * p.sb_k];
      }
    }
    if constexpr (!SMX) {
#pragma unroll
      for (int e = 0; e < WE; ++e) {
        int n, l;
        w_at(e, n, l);
        rw[e] = *(const uint32_t*)(w_addr(c, n, l) & ~(uintptr_t)3);
      }
    }
  };
  auto put_step = [&](const uint32_t* ra, const uint32_t* rb, const uint32_t* rw, int s) {
    const int c = s / ksteps, k0 = (s - c * ksteps) * BK, n0 = c * BN;
#pragma unroll
    for (int e = 0; e < AE; ++e) {
      int r, k;
      a_at(e, r, k);
      const uint32_t v = FP8 ? (uint32_t)lut[ra[e]] : ra[e];
      As[r * LDK + k] = (lds_t)(v & (0u - (uint32_t)(m0 + r < p.M && k0 + k < p.K)));
    }
    if constexpr (VB) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int pc = tid + 256 * h, k = pc >> 3, n8 = 8 * (pc & 7);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t v = rb[4 * h + (e >> 1)] >> (16 * (e & 1));
          Bs[(n8 + e) * LDK + k] =
              (lds_t)(v & (0u - (uint32_t)(n0 + n8 + e < p.N && k0 + k < p.K)));
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < BE; ++e) {
        int n, k;
        b_at(e, n, k);
        const uint32_t v = FP8 ? (uint32_t)lut[rb[e]] : rb[e];
        Bs[n * LDK + k] = (lds_t)(v & (0u - (uint32_t)(n0 + n < p.N && k0 + k < p.K)));
      }
    }
    if (!SMX && is_last(s)) {
      float* ws = Ws[c & 1];
      // one dtype branch around the whole chunk, so the loop is straight-line
      auto put_w = [&](auto dtc) {
        constexpr int DT = decltype(dtc)::value;
#pragma unroll
        for (int e = 0; e < WE; ++e) {
          int n, l;
          w_at(e, n, l);
          const int byte = w_byte(c, n, l);
          float v;
          if constexpr (DT == TM_DT_F32) v = __uint_as_float(rw[e]);
          else if constexpr (DT == TM_DT_F16) v = f16_bits_to_f32((uint16_t)(rw[e] >> (8 * (byte & 2))));
          else if constexpr (DT == TM_DT_BF16) v = bf16_bits_to_f32((uint16_t)(rw[e] >> (8 * (byte & 2))));
          else v = word_elem(rw[e], byte, p.w_dt);
          const uint32_t keep = 0u - (uint32_t)(n0 + n < p.N && l0 + l < p.L);
          ws[n * LDW + l] = __uint_as_float(__float_as_uint(v) & keep);
        }
      };
      if (p.w_dt == TM_DT_F16) put_w(std::integral_constant<int, TM_DT_F16>());
      else if (p.w_dt == TM_DT_BF16) put_w(std::integral_constant<int, TM_DT_BF16>());
      else if (p.w_dt == TM_DT_F32) put_w(std::integral_constant<int, TM_DT_F32>());
      else put_w(std::integral_constant<int, -1>());
    }
  };

  f4_t accp[RI], accc[RI];
#pragma unroll
  for (int i = 0; i < RI; ++i) {
    accp[i] = f4_t{0.f, 0.f, 0.f, 0.f};
    accc[i] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
  // step s multiplies from LDS while step s + 1 goes from registers to LDS
  // (after the barrier) and step s + 2 is loaded into the registers step s
  // came through.  P goes to LDS after the chunk's last k step; W has two
  // LDS buffers, as chunk c + 1's is stored before chunk c's is read.
  auto step = [&](int s, uint32_t* ra_n, uint32_t* rb_n, uint32_t* rw_n, const uint32_t* ra_p,
                  const uint32_t* rb_p, const uint32_t* rw_p) {
    const bool last = is_last(s);
    load_step(ra_n, rb_n, rw_n, min(s + 2, nsteps - 1));
    if (s >= nsteps) return;  // the loop's second step past the end: loads only
    if constexpr (F32) {
      // fp32 operands: v_mfma_f32_16x16x4_f32, lane l row l % 16, k kk + l / 16
#pragma unroll
      for (int kk = 0; kk < BK; kk += 4) {
        const float bv = __uint_as_float(Bs[(16 * wave + r16) * LDK + kk + q]);
#pragma unroll
        for (int i = 0; i < RI; ++i)
          accp[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(
              __uint_as_float(As[(16 * i + r16) * LDK + kk + q]), bv, accp[i], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < BK; kb += 32) {
        const u4_t bv = *(const u4_t*)(Bs + (16 * wave + r16) * LDK + kb + 8 * q);
#pragma unroll
        for (int i = 0; i < RI; ++i) {
          const u4_t av = *(const u4_t*)(As + (16 * i + r16) * LDK + kb + 8 * q);
          accp[i] = mfma16<BF16 && !FP8>(av, bv, accp[i]);
        }
      }
    }
    __syncthreads();
    if (s + 1 < nsteps) put_step(ra_p, rb_p, rw_p, s + 1);
    if (last) {
#pragma unroll
      for (int i = 0; i < RI; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          Ps[(16 * i + 4 * q + e) * LDP + (SMX ? (s / ksteps) * BN : 0) + 16 * wave + r16] =
              accp[i][e];
        accp[i] = f4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
    __syncthreads();
    if (!SMX && last) {
      const float* ws = Ws[(s / ksteps) & 1];
#pragma unroll 4
      for (int kk = 0; kk < BN; kk += 4) {
        const float wv = ws[(kk + q) * LDW + 16 * wave + r16];
#pragma unroll
        for (int i = 0; i < RI; ++i)
          accc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(Ps[(16 * i + r16) * LDP + kk + q], wv,
                                                        accc[i], 0, 0, 0);
      }
    }
  };
  uint32_t ra0[AE], rb0[BE], rw0[WE], ra1[AE], rb1[BE], rw1[WE];
  if constexpr (FP8) __syncthreads();  // the decode table
  load_step(ra0, rb0, rw0, 0);
  load_step(ra1, rb1, rw1, min(1, nsteps - 1));
  put_step(ra0, rb0, rw0, 0);
  __syncthreads();
  for (int s = 0; s < nsteps; s += 2) {
    step(s, ra0, rb0, rw0, ra1, rb1, rw1);
    step(s + 1, ra1, rb1, rw1, ra0, rb0, rw0);
  }

  const long long cb = (long long)b * p.sc_b;
  if constexpr (SMX) {
    // softmax of each row, the arithmetic of dot_rows: exp(x - max) / sum;
    // wave w takes rows w, w + 4, ..  (the last step's barrier ordered P)
    for (int r = wave; r < BM; r += 4) {
      const int m = m0 + r;
      if (m >= p.M) break;
      const float* pr = Ps + r * LDP;
      float mx = -__builtin_inff();
      for (int n = lane; n < p.N; n += 64) mx = fmaxf(mx, pr[n]);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      float sm = 0.0f;
      for (int n = lane; n < p.N; n += 64) sm += expf(pr[n] - mx);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sm += __shfl_xor(sm, o, 64);
      const long long rb = cb + (long long)m * p.sc_m;
      for (int n = lane; n < p.N; n += 64)
        store_elem(p.C, rb + (long long)n * p.sc_n, p.out_dt, expf(pr[n] - mx) / sm);
    }
    return;
  }
  const int l = l0 + 16 * wave + r16;
  if (l >= p.L) return;
#pragma unroll
  for (int i = 0; i < RI; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 16 * i + 4 * q + e;
      if (m < p.M) store_elem(p.C, cb + (long long)m * p.sc_m + (long long)l * p.sc_n, p.out_dt, accc[i][e]);
    }
}
}  // namespace

#define TM_DOT_CHAIN(NAME, BF, F8, BM, F32)                                       \
  extern "C" __global__ __launch_bounds__(256) void NAME(DotParams p) {         \
    dot_chain_body<BF, F8, BM, F32>(p);                                         \
  }
// _vb: 16-bit B row-contiguous in aligned 16-byte pieces
#define TM_DOT_CHAIN_VB(NAME, BF, BM, SMX)                                       \
  extern "C" __global__ __launch_bounds__(256) void NAME(DotParams p) {         \
    dot_chain_body<BF, false, BM, false, SMX, true>(p);                         \
  }
TM_DOT_CHAIN_VB(dot_chain16_f16_vb, false, 16, false)
TM_DOT_CHAIN_VB(dot_chain16_bf16_vb, true, 16, false)
TM_DOT_CHAIN_VB(dot_chain32_f16_vb, false, 32, false)
TM_DOT_CHAIN_VB(dot_chain32_bf16_vb, true, 32, false)
TM_DOT_CHAIN_VB(dot_softmax16_f16_vb, false, 16, true)
TM_DOT_CHAIN_VB(dot_softmax16_bf16_vb, true, 16, true)
TM_DOT_CHAIN(dot_chain16_f16, false, false, 16, false)
TM_DOT_CHAIN(dot_chain16_bf16, true, false, 16, false)
TM_DOT_CHAIN(dot_chain16_fp8, false, true, 16, false)
TM_DOT_CHAIN(dot_chain16_f32, false, false, 16, true)
TM_DOT_CHAIN(dot_chain32_f16, false, false, 32, false)
TM_DOT_CHAIN(dot_chain32_bf16, true, false, 32, false)
TM_DOT_CHAIN(dot_chain32_fp8, false, true, 32, false)
TM_DOT_CHAIN(dot_chain32_f32, false, false, 32, true)

// dot_softmax16_<f16|bf16|fp8|f32>: the softmax epilogue for rows of N <=
// 2048 on the same P pipeline (16-row blocks, grid (ceil(M / 16), batch)):
// whole fp32 P rows in LDS, then each row's softmax into C in any dtype.
#define TM_DOT_SOFTMAX(NAME, BF, F8, F32)                                        \
  extern "C" __global__ __launch_bounds__(256) void NAME(DotParams p) {         \
    dot_chain_body<BF, F8, 16, F32, true>(p);                                   \
  }
TM_DOT_SOFTMAX(dot_softmax16_f16, false, false, false)
TM_DOT_SOFTMAX(dot_softmax16_bf16, true, false, false)
TM_DOT_SOFTMAX(dot_softmax16_fp8, false, true, false)
TM_DOT_SOFTMAX(dot_softmax16_f32, false, false, true)

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
