// Typed entry point for tl.dot in general form (strided / transposed
// operands, a batch dimension, FP8 inputs, epilogues): the dot_tile kernels
// (MFMA, the none / add-* epilogues, and the product before dot_softmax_rows),
// dot_softmax16 (softmax into other outputs, N <= 2048), dot_chain
// (chain-dot) or dot_rows (every epilogue, any case the others do not take).
// Also the FP8 path of tm_matmul.
#include <cstring>

#include "runtime.h"

using namespace tmhip;

namespace {

// Kernel argument block; must match struct DotParams in dot.hip.
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

enum { MODE_KC = 0, MODE_RC = 1, MODE_SCALAR = 2 };

bool is_fp8(int dt) { return dt >= TM_DT_FP8_E4M3 && dt <= TM_DT_FP8_E5M2B16; }
int elem_size(int dt) { return dt == TM_DT_F32 ? 4 : is_fp8(dt) ? 1 : 2; }
bool is_input(int dt) { return is_float(dt) || is_fp8(dt); }

// Fetch mode of a [rows, K] operand with strides (s_b, s_r, s_k): pieces of
// 8 elements (fp32: 4; 16 bytes, FP8 8 bytes) along k or along the rows when
// that dimension is contiguous and every piece starts aligned, else element
// by element.
int fetch_mode(const void* X, long long s_b, long long s_r, long long s_k, int batch, int esz) {
  const int piece = esz == 4 ? 4 : 8;
  const uintptr_t align = (uintptr_t)piece * (uintptr_t)esz;
  const bool base_ok = ((uintptr_t)X % align) == 0 && (batch <= 1 || s_b % piece == 0);
  if (base_ok && s_k == 1 && s_r % piece == 0) return MODE_KC;
  if (base_ok && s_r == 1 && s_k % piece == 0) return MODE_RC;
  return MODE_SCALAR;
}

// Byte extent [lo, hi) of a strided 3-D view (non-negative strides).
void extent(const void* p, int esz, long long d0, long long d1, long long d2, long long s0,
            long long s1, long long s2, uintptr_t* lo, uintptr_t* hi) {
  const long long last = (d0 - 1) * s0 + (d1 - 1) * s1 + (d2 - 1) * s2;
  *lo = (uintptr_t)p;
  *hi = (uintptr_t)p + (uintptr_t)((last + 1) * esz);
}

}  // namespace

namespace tmhip {

int dot_impl(const char* op, const void* A, const void* B, void* C, const void* Z, const void* W,
             int batch, int M, int N, int K, int L, const long long* st, int epilogue,
             int in_dtype, int out_dtype, int z_dtype, int w_dtype, void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0)
    return fail(TM_ERR_INVALID_ARG, "%s: batch=%d M=%d N=%d K=%d", op, batch, M, N, K);
  if (epilogue < TM_EPI_NONE || epilogue > TM_EPI_CHAIN_DOT)
    return fail(TM_ERR_INVALID_ARG, "%s: epilogue %d", op, epilogue);
  if (!is_input(in_dtype) || !is_float(out_dtype))
    return fail(TM_ERR_INVALID_ARG, "%s: dtypes %d -> %d", op, in_dtype, out_dtype);
  const bool chain = epilogue == TM_EPI_CHAIN_DOT;
  const bool add = epilogue >= TM_EPI_ADD_MATRIX && epilogue <= TM_EPI_ADD_COLS;
  if (chain && L < 0) return fail(TM_ERR_INVALID_ARG, "%s: L=%d", op, L);
  const int NC = chain ? L : N;  // columns of C
  if (batch == 0 || M == 0 || NC == 0) return 0;
  if (!A || !B || !C || !st) return fail(TM_ERR_INVALID_ARG, "%s: null buffer or strides", op);
  if (add && (!Z || !is_input(z_dtype)))
    return fail(TM_ERR_INVALID_ARG, "%s: the add epilogues need Z and its dtype", op);
  if (chain && (!W || !is_input(w_dtype)))
    return fail(TM_ERR_INVALID_ARG, "%s: chain-dot needs W and its dtype", op);
  for (int i = 0; i < 14; ++i)
    if (st[i] < 0) return fail(TM_ERR_INVALID_ARG, "%s: negative stride %d", op, i);
  if ((epilogue == TM_EPI_SOFTMAX || chain) && N > 8192)
    return fail(TM_ERR_UNSUPPORTED, "%s: softmax / chain-dot rows of N=%d > 8192", op, N);
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();

  DotParams p;
  memset(&p, 0, sizeof p);
  p.A = A; p.B = B; p.C = C; p.Z = Z; p.W = W;
  p.sa_b = st[0]; p.sa_m = st[1]; p.sa_k = st[2];
  p.sb_b = st[3]; p.sb_k = st[4]; p.sb_n = st[5];
  p.sc_b = st[6]; p.sc_m = st[7]; p.sc_n = st[8];
  p.sz_b = st[9]; p.sz_m = st[10]; p.sz_n = st[11];
  p.sw_n = st[12]; p.sw_l = st[13];
  p.batch = batch; p.M = M; p.N = N; p.K = K; p.L = L;
  p.epi = epilogue;
  p.in_dt = in_dtype; p.out_dt = out_dtype; p.z_dt = z_dtype; p.w_dt = w_dtype;

  // A bias read in place from the output (Z overlapping C), as the
  // reference's test kernels do: add-matrix reads and writes each element in
  // one thread, which is only race-free when Z is C element for element (same
  // base, dtype and strides); add-rows reads its row's element in the row's
  // own workgroup (dot_rows) before any store; add-cols across rows would race.
  bool rows_kernel = epilogue == TM_EPI_SOFTMAX || chain || K == 0;
  if (add) {
    uintptr_t zl, zh, cl, ch;
    extent(Z, elem_size(z_dtype), batch, M, N, st[9], st[10], st[11], &zl, &zh);
    extent(C, elem_size(out_dtype), batch, M, NC, st[6], st[7], st[8], &cl, &ch);
    const bool overlap = zl < ch && cl < zh;
    if (overlap && epilogue == TM_EPI_ADD_MATRIX) {
      const bool same_b = st[9] == st[6] || batch == 1;
      if (Z != C || z_dtype != out_dtype || !same_b || st[10] != st[7] || st[11] != st[8])
        return fail(TM_ERR_INVALID_ARG,
                    "%s: add-matrix with Z overlapping C needs Z to be C itself (same "
                    "dtype and strides)", op);
    } else if (overlap) {
      if (epilogue == TM_EPI_ADD_COLS && (long long)batch * M > 1)
        return fail(TM_ERR_INVALID_ARG,
                    "%s: add-cols with Z overlapping C is only defined for one row", op);
      rows_kernel = true;
    }
  }
  if (!rows_kernel && batch > 65535) rows_kernel = true;
  // softmax with an fp32 output that shares no memory with A or B: the
  // product (unrounded fp32) through the tile kernels into C, then each row
  // replaced by its softmax (dot_rows re-reads all of B for every row)
  if (epilogue == TM_EPI_SOFTMAX && out_dtype == TM_DT_F32 && K > 0 && batch <= 65535) {
    uintptr_t al, ah, bl, bh, cl, chh;
    const int isz = elem_size(in_dtype);
    extent(A, isz, batch, M, K, st[0], st[1], st[2], &al, &ah);
    extent(B, isz, batch, K, N, st[3], st[4], st[5], &bl, &bh);
    extent(C, 4, batch, M, N, st[6], st[7], st[8], &cl, &chh);
    if (!(cl < ah && al < chh) && !(cl < bh && bl < chh)) {
      int rc = dot_impl(op, A, B, C, nullptr, nullptr, batch, M, N, K, 0, st, TM_EPI_NONE,
                        in_dtype, TM_DT_F32, TM_DT_NONE, TM_DT_NONE, stream);
      if (rc) return rc;
      static Kernel ksm("dot_softmax_rows");
      return launch(ksm, dim3((unsigned)((long long)batch * M)), dim3(256), 0, stream, p);
    }
  }
  // dot_softmax16 / dot_chain read a 16-bit B that is row-contiguous in
  // aligned 16-byte pieces (n contiguous) with 16-byte loads (the _vb forms)
  const auto vec_b = [&]() {
    return is_half(in_dtype) && fetch_mode(B, st[3], st[5], st[4], batch, 2) == MODE_RC;
  };
  // softmax into any other C (a 16-bit one: the product must not be rounded
  // first) with rows of N <= 2048 and C sharing no memory with A or B:
  // dot_softmax16 keeps 16 whole product rows on chip
  if (epilogue == TM_EPI_SOFTMAX && K > 0 && N <= 2048 && batch <= 65535) {
    uintptr_t al, ah, bl, bh, cl, chh;
    const int isz = elem_size(in_dtype);
    extent(A, isz, batch, M, K, st[0], st[1], st[2], &al, &ah);
    extent(B, isz, batch, K, N, st[3], st[4], st[5], &bl, &bh);
    extent(C, elem_size(out_dtype), batch, M, N, st[6], st[7], st[8], &cl, &chh);
    if (!(cl < ah && al < chh) && !(cl < bh && bl < chh)) {
      char name[40];
      snprintf(name, sizeof name, "dot_softmax16_%s%s",
               is_fp8(in_dtype) ? "fp8" : in_dtype == TM_DT_BF16 ? "bf16"
               : in_dtype == TM_DT_F32 ? "f32" : "f16", vec_b() ? "_vb" : "");
      return launch(kernel_named(name), dim3((unsigned)((M + 15) / 16), (unsigned)batch),
                    dim3(256), 0, stream, p);
    }
  }
  // chain-dot with C sharing no memory with A, B or W:
  // dot_chain keeps each P tile on chip and multiplies it into C at once
  // (dot_rows re-reads all of B for every row).  32-row C tiles when they
  // already make a workgroup per CU, else 16-row ones for twice as many.
  if (chain && K > 0 && N > 0 && batch <= 65535) {
    uintptr_t al, ah, bl, bh, wl, wh, cl, chh;
    const int isz = elem_size(in_dtype);
    extent(A, isz, batch, M, K, st[0], st[1], st[2], &al, &ah);
    extent(B, isz, batch, K, N, st[3], st[4], st[5], &bl, &bh);
    extent(W, elem_size(w_dtype), 1, N, L, 0, st[12], st[13], &wl, &wh);
    extent(C, elem_size(out_dtype), batch, M, L, st[6], st[7], st[8], &cl, &chh);
    const auto apart = [&](uintptr_t lo, uintptr_t hi) { return !(cl < hi && lo < chh); };
    const long long tl = (L + 63) / 64;
    const bool b32 = (long long)((M + 31) / 32) * tl * batch >= cu_count();
    const long long groups = (long long)((M + (b32 ? 31 : 15)) / (b32 ? 32 : 16)) * tl;
    if (apart(al, ah) && apart(bl, bh) && apart(wl, wh) && groups <= 0x7fffffffLL) {
      char name[40];
      snprintf(name, sizeof name, "dot_chain%d_%s%s", b32 ? 32 : 16,
               is_fp8(in_dtype) ? "fp8" : in_dtype == TM_DT_BF16 ? "bf16"
               : in_dtype == TM_DT_F32 ? "f32" : "f16", vec_b() ? "_vb" : "");
      return launch(kernel_named(name), dim3((unsigned)groups, (unsigned)batch), dim3(256), 0,
                    stream, p);
    }
  }
  // fp32 without an epilogue, one batch, k- and n-contiguous rows (B as [K, N]
  // or [N, K]): the fp32-MFMA dense kernel
  const auto fits = [](long long v) { return v >= 0 && v <= 0x7fffffffLL; };
  if (in_dtype == TM_DT_F32 && epilogue == TM_EPI_NONE && batch == 1 && K > 0 && st[2] == 1 &&
      st[8] == 1 && (st[5] == 1 || st[4] == 1) && fits(st[1]) && fits(st[4]) && fits(st[5]) &&
      fits(st[7])) {
    const bool bt = st[5] != 1;  // B [N, K]: row n at stride sb_n, k contiguous
    const long long ldb = bt ? st[5] : st[4];
    if (st[1] >= K && st[7] >= N && ldb >= (bt ? K : N))
      return dense_f32((const float*)A, (const float*)B, C, M, N, K, (int)st[1], (int)ldb,
                       (int)st[7], bt, out_dtype, stream);
  }
  // 16-bit, no epilogue, one batch, k- and n-contiguous rows, output in the
  // input dtype or fp32: the dense selection's MFMA tile kernels, when it has
  // one for these sizes and alignments
  if (is_half(in_dtype) && (out_dtype == in_dtype || out_dtype == TM_DT_F32) &&
      epilogue == TM_EPI_NONE && batch == 1 && K > 0 && st[2] == 1 && st[8] == 1 &&
      (st[5] == 1 || st[4] == 1) && fits(st[1]) && fits(st[4]) && fits(st[5]) && fits(st[7])) {
    const bool bt = st[5] != 1;
    const long long ldb = bt ? st[5] : st[4];
    if (st[1] >= K && st[7] >= N && ldb >= (bt ? K : N)) {
      bool used = false;
      const int rc = dense_mfma(A, B, C, M, N, K, (int)st[1], (int)ldb, (int)st[7], bt, in_dtype,
                                out_dtype, stream, &used);
      if (used || rc) return rc;
    }
  }
  if (rows_kernel) {
    static Kernel kr("dot_rows");
    return launch(kr, dim3((unsigned)((long long)batch * M)), dim3(256), 0, stream, p);
  }
  const int esz = elem_size(in_dtype);
  p.a_mode = fetch_mode(A, p.sa_b, p.sa_m, p.sa_k, batch, esz);
  p.b_mode = fetch_mode(B, p.sb_b, p.sb_n, p.sb_k, batch, esz);
  // [f16, bf16, fp8, f32]: both operands in 16-byte pieces (KC / RC) ->
  // dot_tile (16-bit and FP8: 128 x 128 tiles from 1.5 of them per CU, else
  // 64 x 64: two 128-tile workgroups fit a CU, four 64-tile ones, and at one
  // 128 tile per CU the 64 tiles measured faster: fp16 2048^3 81 -> 57 us,
  // 4 x 1024^3 46 -> 33 us, while 2560 x 2560 x 4096 (400 tiles of 128) kept
  // the 128 tiles, 167 against 189 us), else the element-load form dot_tile_s
  static Kernel* ks[4] = {new Kernel("dot_tile_s_f16"), new Kernel("dot_tile_s_bf16"),
                          new Kernel("dot_tile_s_fp8"), new Kernel("dot_tile_s_f32")};
  static Kernel* k32 = new Kernel("dot_tile_f32");
  const int kind = in_dtype == TM_DT_F32 ? 3 : is_fp8(in_dtype) ? 2 : in_dtype == TM_DT_BF16 ? 1 : 0;
  const bool vec = p.a_mode != MODE_SCALAR && p.b_mode != MODE_SCALAR;
  const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128);
  const bool big = vec && kind != 3 && 2 * t128 * batch >= 3LL * cu_count();
  const int edge = big ? 128 : 64;
  const long long tiles = (long long)((M + edge - 1) / edge) * ((N + edge - 1) / edge);
  if (tiles > 0x7fffffffLL) return fail(TM_ERR_UNSUPPORTED, "%s: too many tiles", op);
  Kernel* kp = vec ? k32 : ks[kind];
  if (vec && kind != 3) {
    // dot_tile{,128}_<dt>_<a><b>: each operand k- (k) or row-contiguous (r)
    static const char* dts[3] = {"f16", "bf16", "fp8"};
    char name[64];
    snprintf(name, sizeof name, "dot_tile%s_%s_%c%c", big ? "128" : "", dts[kind],
             p.a_mode == MODE_RC ? 'r' : 'k', p.b_mode == MODE_RC ? 'r' : 'k');
    kp = &kernel_named(name);
  }
  Kernel& kt = *kp;
  return launch(kt, dim3((unsigned)tiles, (unsigned)batch), dim3(256), 0, stream, p);
}

}  // namespace tmhip

extern "C" int tm_dot(const void* A, const void* B, void* C, const void* Z, const void* W,
                      int batch, int M, int N, int K, int L, const long long* strides,
                      int epilogue, int in_dtype, int out_dtype, int z_dtype, int w_dtype,
                      void* stream) {
  return dot_impl("tm_dot", A, B, C, Z, W, batch, M, N, K, L, strides, epilogue, in_dtype,
                  out_dtype, z_dtype, w_dtype, stream);
}
