// Typed entry points for the matmul family: W8A16 / W4A16 weight-only
// matmul, the dequantised weight tile, dense matmul and fused linear.
// Each validates its arguments, picks a kernel variant from the shape and
// dtypes and launches it asynchronously on the caller's stream.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>

#include "runtime.h"

using namespace tmhip;

namespace {

const char* dt_name(int dt) {
  switch (dt) {
    case TM_DT_F32: return "f32";
    case TM_DT_F16: return "f16";
    case TM_DT_BF16: return "bf16";
    case TM_DT_U8: return "u8";
    case TM_DT_NONE: return "none";
    default: return "?";
  }
}

Kernel& kernel(const std::string& name) { return tmhip::kernel_named(name); }

// ---- W-only kernel selection ------------------------------------------------
// A pure function of the problem (sizes, dtypes, pointer alignment, the
// device's CU count and LDS limit): the launch path and tm_wq_plan share it.
// Split-K plans (split_ok: the caller supplies a workspace) run the split-K
// form of a kernel over `splits` k-slices, grid (grid, splits), writing fp32
// [splits][M][N] into the workspace, then wq_splitk_reduce_<act>.
enum { WQ_ARGS_STD = 0, WQ_ARGS_G = 1, WQ_ARGS_GENERAL = 2, WQ_ARGS_SPLIT = 3,
       WQ_ARGS_SPLIT_G = 4 };
struct WqPlan {
  char name[64];
  unsigned grid, block, lds;
  int form;       // argument list: WQ_ARGS_*
  int splits;     // k-slices (1: no split)
  int kslice;     // k per slice (the last may be shorter: WQ_ARGS_SPLIT_G)
  size_t ws;      // workspace bytes (split-K plans)
};

void wq_plan(int qbits, int M, int N, int K, int G, int adt, int sdt, int zdt, unsigned align,
             int cus, size_t max_lds, bool split_ok, WqPlan* pl) {
  pl->splits = 1;
  pl->kslice = K;
  pl->ws = 0;
  auto set = [&](unsigned grid, unsigned block, size_t lds, int form) {
    pl->grid = grid;
    pl->block = block;
    pl->lds = (unsigned)lds;
    pl->form = form;
  };
  const bool a16 = align & TM_WQ_ALIGN_XW16, s16 = align & TM_WQ_ALIGN_S16,
             z16 = align & TM_WQ_ALIGN_Z16, sz4 = align & TM_WQ_ALIGN_SZ4;
  const int CK = qbits == 4 ? 128 : 64;
  const bool fast = is_half(adt) && sdt == adt &&
                    (zdt == TM_DT_NONE || zdt == sdt || zdt == TM_DT_U8) &&
                    (qbits == 8 || G % 128 == 0) && N % 16 == 0 && K > 0 && a16;
  const char* act = adt == TM_DT_BF16 ? "bf16" : "f16";
  const char zc = zdt == TM_DT_NONE ? 'n' : (zdt == TM_DT_U8 ? 'u' : 's');
  // wide kernel: M > 64, 64 x 128 output blocks (int4: fp16 activations;
  // int8: fp16 or bf16).  With a workspace, split-K over S k-slices when its
  // tiles would fill less than half the CUs, or when int4 K exceeds the 4096
  // whose scales fit in LDS
  // (int4: K % 512 == 0 with uint8 zero-points, whose per-row bytes the
  // split form gathers as dwords; K % 256 == 0 otherwise.  Where no equal
  // slicing fits, slices of whole units with a shorter last one.)
  const bool w4k = qbits == 4 && (K % 512 == 0 || (K % 256 == 0 && zdt != TM_DT_U8));
  if (fast && M > 64 && N % 128 == 0 && s16 && z16 &&
      ((w4k && adt == TM_DT_F16 && G == 128) ||
       (qbits == 8 && zdt == TM_DT_NONE && K % 128 == 0))) {
    const int ns = qbits == 4 ? 3 : 4, ck = qbits == 4 ? 64 : 32;
    const int unit = qbits == 4 ? (K % 512 == 0 ? 512 : 256) : 128;  // slice granularity
    const int mtl = (M + 63) / 64, ntl = N / 128;
    const long tiles = (long)mtl * ntl;
    int S = 1, Ks = K;
    if (split_ok && (tiles < cus / 2 || (qbits == 4 && K > 4096))) {
      S = 0;
      // the largest valid slice count up to the one that fills the CUs, else
      // the smallest above it (int4: at least K / 4096 slices)
      const int smin = qbits == 4 ? (K + 4095) / 4096 : 1;
      const int want = (int)std::min<long>(std::max<long>((cus + tiles - 1) / tiles, smin), 16);
      auto ok = [&](int s2) { return K % (s2 * unit) == 0 && (qbits == 8 || K / s2 <= 4096); };
      for (int s2 = want; s2 >= std::max(smin, 2) && !S; --s2)
        if (ok(s2)) S = s2;
      for (int s2 = want + 1; s2 <= 16 && !S; ++s2)
        if (ok(s2)) S = s2;
      if (S) {
        Ks = K / S;
      } else if (qbits == 4 && K > 4096) {
        // slices of whole units, the last one shorter
        const int units = K / unit, per = (units + want - 1) / want;
        if ((long)per * unit <= 4096) {
          S = (units + per - 1) / per;
          Ks = per * unit;
        }
      } else {
        S = 1;
      }
    }
    if (S && (qbits == 8 || Ks <= 4096)) {
      size_t wl = (size_t)ns * 4 * (64 * 2 * ck + 4096);  // ring stages
      if (qbits == 4)  // scales and zero-points of the 128 columns
        wl += (size_t)2 * Ks +
              (zdt == TM_DT_NONE ? 0 : zdt == TM_DT_U8 ? (size_t)Ks : (size_t)2 * Ks);
      if (wl <= max_lds) {
        snprintf(pl->name, sizeof pl->name, "wq_wide_q%d_%s_z%c%s", qbits, act, zc,
                 S > 1 ? "_k" : "");
        set(8 * mtl * ((ntl + 7) / 8), 512, wl, S > 1 ? WQ_ARGS_SPLIT : WQ_ARGS_STD);
        pl->splits = S;
        pl->kslice = Ks;
        pl->ws = S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
        return;
      }
    }
  }
  // two-tile int4 GEMV: 2 <= M <= 6 at K = 4096 (from M = 7 on the streaming
  // kernel is as fast or faster), 32 columns per workgroup
  if (fast && qbits == 4 && M >= 2 && M <= 6 && G == 128 && K == 4096 && N % 32 == 0 && s16 &&
      z16) {
    // X, then the scales and zero-points of 32 columns; at least the
    // reduction's 7 waves x 2 tiles x 1 KB
    size_t glds = (size_t)M * (K + 8) * 2 + (size_t)4 * 32 * (K / 128);
    glds = std::max(glds, (size_t)7 * 2 * 1024);
    if (glds <= max_lds) {
      snprintf(pl->name, sizeof pl->name, "wq_gemv4x2_%s_z%c_w8p4", act, zc);
      return set(N / 32, 512, glds, WQ_ARGS_STD);
    }
  }
  // streaming kernel: 1 < M <= 64 (int4: 128), K-slices of 512 per wave (at
  // most 8); past 64 rows the int8 tiled kernel is the faster one
  if (fast && M > 1 && M <= (qbits == 4 ? 128 : 64) && K % 512 == 0 && K <= 4096 && sz4 &&
      (qbits == 8 || G == 128)) {
    const int nwv = K / 512;
    const int nt = qbits == 4 ? 4 : 3;           // 16-column tiles per workgroup
    const int xr = M <= 8 ? 8 : 16;              // X rows staged per chunk
    const int rs = qbits == 4 ? 2 : 3;           // ring slots per wave
    const int slot = nt * 1024 + xr * (qbits == 4 ? 256 : 128);
    // per wave: ring, scales / zero-points (int4 2 KB, int8 1 KB); reduction
    const size_t slds = (size_t)nwv * (rs * slot + (qbits == 4 ? 2048 : 1024)) +
                        (size_t)nwv * 8 * 64 * sizeof(float);
    if (slds <= max_lds) {
      snprintf(pl->name, sizeof pl->name, "wq_stream_q%d_%s_z%c_x%d%c", qbits, act, zc, xr,
               M <= 16 ? 's' : 'm');
      const int tiles = N / 16;
      return set((tiles + nt - 1) / nt, 64 * nwv, slds, WQ_ARGS_STD);
    }
  }
  // persistent int4 GEMV: M = 1, K = 4096, G = 128; one workgroup per CU owns
  // 4 RW rows, RW the smallest instantiated count that keeps the grid within
  // the CUs (a second round of workgroups would double the time)
  if (fast && qbits == 4 && M == 1 && G == 128 && K == 4096) {
    static const int kRW[] = {4, 7, 8, 11, 12, 14, 16};
    for (int rw : kRW) {
      const int grid = (N + 4 * rw - 1) / (4 * rw);
      if (N >= 4 * rw && grid <= cus) {
        snprintf(pl->name, sizeof pl->name, "wq_gemv4p_%s_z%c_r%d", act, zc, rw);
        return set(grid, 512, 0, WQ_ARGS_STD);
      }
    }
  }
  // persistent int4 GEMV for other K (K % 128 == 0, K <= 16384): KS segments
  // of 2048 k x RG row groups of RW rows, the first shape (fewest rows per
  // workgroup) that keeps the grid within the CUs
  if (fast && qbits == 4 && M == 1 && G == 128 && K != 4096 && K % 128 == 0 && K <= 16384) {
    const int ks = (K + 2047) / 2048;
    static const int kShape[][2] = {{1, 8}, {1, 16}, {2, 16}, {4, 16}};  // (RG, RW)
    for (const auto& sh : kShape) {
      const int rg = sh[0], rw = sh[1];
      if (ks * rg > 16 || (ks > 4 && rg > 2)) continue;
      const int rows = rg * rw, grid = (N + rows - 1) / rows;
      if (N >= rows && grid <= cus) {
        snprintf(pl->name, sizeof pl->name, "wq_gemv4k_%s_z%c_s%d_g%d_r%d", act, zc, ks, rg, rw);
        return set(grid, 64 * ks * rg, 0, WQ_ARGS_STD);
      }
    }
  }
  // linear int4 GEMV: M = 1, G = 128, K = 4096 or 8192 with N past the
  // persistent kernels' reach (VALU dot products, 1 KB of one row per load)
  if (fast && qbits == 4 && M == 1 && G == 128 && (K == 4096 || K == 8192)) {
    snprintf(pl->name, sizeof pl->name, "wq_gemv4l_%s_z%c_k%d", act, zc, K / 2048);
    return set(N / 16, 512, 0, WQ_ARGS_STD);
  }
  // exact-shape int4 GEMV: K = 8 waves x 8 chunks x 128 = 8192, G = 128,
  // 2 <= M <= 8 (M = 1 took the linear GEMV above)
  if (fast && qbits == 4 && M <= 8 && G == 128 && K == 8192 && s16 && z16) {
    // X, two [chunk][8] float sums (sum x, sum x * offset), scales + zero-points
    size_t glds = (size_t)M * (K + 8) * 2 + 2 * (size_t)(K / 128) * 8 * 4 + (size_t)(K / 128) * 64;
    if (glds <= max_lds) {
      snprintf(pl->name, sizeof pl->name, "wq_gemv4_%s_z%c_w8p8", act, zc);
      return set(N / 16, 512, glds, WQ_ARGS_STD);
    }
  }
  // long-K streaming kernel: M <= 64, K > 4096 in chunks of 64 weight bytes
  // per row (int4 128 k = one group, int8 64 k), NCH chunks per wave over at
  // most 8 waves (int4 K <= 32768, int8 K <= 16384); NT = 1 or 2 16-column
  // tiles per workgroup (one workgroup per CU for the N of a down projection;
  // NT = 2 only where its LDS fits); M > 16 in passes of 16 rows (NT = 1;
  // int4 K <= 16384, as the first pass's weights stay in registers).  Past
  // those K, with a workspace: split-K over the fewest slices that fit.
  if (fast && M <= 64 && K > 4096 && K % CK == 0 && sz4 && (qbits == 8 || G == 128)) {
    const bool multi = M > 16;
    const int kmax = qbits == 4 ? (multi ? 16384 : 32768) : 16384;
    int S = K <= kmax ? 1 : 0;
    if (!S && split_ok)
      for (int s2 = 2; s2 <= 64 && !S; ++s2)
        if (K % (s2 * CK) == 0 && K / s2 <= kmax) S = s2;
    const int Ks = S ? K / S : K;
    const int nchunk = Ks / CK;
    // split-K forms: int4 multi-pass 16 chunks per wave, the others 32
    const int nch = S > 1 ? (qbits == 4 && multi ? 16 : 32)
                          : (nchunk <= 64 && qbits == 4 ? 8 : nchunk <= 128 ? 16 : 32);
    const int nwv = (nchunk + nch - 1) / nch;
    const int tiles = N / 16;
    const int xr = M <= 8 ? 8 : 16;
    for (int nt = S == 1 && tiles > cus && !multi ? 2 : 1; S && nt >= 1; --nt) {
      const size_t slot = (size_t)nt * 1024 + (size_t)xr * 2 * CK;
      const size_t scb = qbits == 4 ? (size_t)512 * nt * (nch / 4) : 1024;
      const size_t slds = (size_t)nwv * (2 * slot + scb + 8 * 64 * sizeof(float));
      if (slds <= max_lds) {
        snprintf(pl->name, sizeof pl->name, "wq_streamk_q%d_%s_z%c_t%d_x%d%c_c%d%s", qbits, act,
                 zc, nt, xr, multi ? 'm' : 's', nch, S > 1 ? "_k" : "");
        set((tiles + nt - 1) / nt, 64 * nwv, slds, S > 1 ? WQ_ARGS_SPLIT : WQ_ARGS_STD);
        pl->splits = S;
        pl->kslice = K / S;
        pl->ws = S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
        return;
      }
    }
  }
  // linear int8 GEMV: M = 1, K = 4096, fp16 (VALU dot products, 1 KB of one
  // row per load instruction)
  if (fast && qbits == 8 && M == 1 && K == 4096 && adt == TM_DT_F16) {
    snprintf(pl->name, sizeof pl->name, "wq_gemv8l_f16_z%c", zc);
    return set(N / 16, 512, 0, WQ_ARGS_STD);
  }
  // int8 GEMV: M = 1, K = 4096, bf16 (8 waves x 8 loads of 16 bytes per lane)
  if (fast && qbits == 8 && M == 1 && K == 4096 && adt == TM_DT_BF16) {
    snprintf(pl->name, sizeof pl->name, "wq_gemv8_%s_z%c_w8p8", act, zc);
    return set(N / 16, 512, (size_t)(K + 8) * 2, WQ_ARGS_STD);
  }
  const size_t lds = (size_t)M * (K + 8) * 2 + (size_t)M * (K / 128) * 4;
  if (fast && M <= 8 && K % (4 * CK) == 0 && lds <= max_lds) {
    const bool vs = qbits == 4 && G == 128 && K % 4096 == 0;
    snprintf(pl->name, sizeof pl->name, "wq_skinny_q%d_%s_z%c%s", qbits, act, zc, vs ? "_v" : "");
    return set(N / 16, 256, lds, WQ_ARGS_G);
  }
  // tiled kernel: 64 x 64 output tiles walking K in steps of 256.  With a
  // workspace and fewer tiles than CUs: split-K over slices of whole steps
  // (the last one shorter), about two workgroups per CU, at most 16 slices
  if (fast && K % 256 == 0 && N % 64 == 0) {
    const int tiles = ((M + 63) / 64) * (N / 64), steps = K / 256;
    int S = 1, per = steps;
    if (split_ok && tiles < cus && steps > 1) {
      const int want = std::min(std::min(16, (2 * cus + tiles - 1) / tiles), steps);
      per = (steps + want - 1) / want;
      S = (steps + per - 1) / per;
    }
    snprintf(pl->name, sizeof pl->name, "wq_tiled_q%d_%s_z%c%s", qbits, act, zc,
             S > 1 ? "_k" : "");
    set((tiles + 7) / 8 * 8, 256, 0, S > 1 ? WQ_ARGS_SPLIT_G : WQ_ARGS_G);
    pl->splits = S;
    pl->kslice = per * 256;
    pl->ws = S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
    return;
  }
  snprintf(pl->name, sizeof pl->name, "wq_general");
  set((N + 3) / 4, 256, 0, WQ_ARGS_GENERAL);
}

unsigned wq_align(const void* X, const void* W, const void* S, const void* Z) {
  unsigned align = 0;
  if (aligned16(X) && aligned16(W)) align |= TM_WQ_ALIGN_XW16;
  if (aligned16(S)) align |= TM_WQ_ALIGN_S16;
  if (!Z || aligned16(Z)) align |= TM_WQ_ALIGN_Z16;
  if (((uintptr_t)S & 3u) == 0 && (!Z || ((uintptr_t)Z & 3u) == 0)) align |= TM_WQ_ALIGN_SZ4;
  return align;
}

int wq_matmul(int qbits, const void* X, const void* W, void* Y, const void* S, const void* Z,
              int M, int N, int K, int G, int adt, int sdt, int zdt, const void* bias,
              void* workspace, size_t workspace_bytes, void* stream) {
  const char* op = bias ? (qbits == 4 ? "tm_int4_linear" : "tm_int8_linear")
                        : (qbits == 4 ? "tm_int4_matmul" : "tm_int8_matmul");
  if (M < 0 || N < 0 || K < 0) return fail(TM_ERR_INVALID_ARG, "%s: negative size", op);
  if (M == 0 || N == 0) return 0;
  if (!X || !W || !Y || !S) return fail(TM_ERR_INVALID_ARG, "%s: null buffer", op);
  if (qbits == 4 && (K % 2 != 0))
    return fail(TM_ERR_INVALID_ARG, "%s: K=%d must be even (two nibbles per byte)", op, K);
  if (qbits == 4 && G <= 0) return fail(TM_ERR_INVALID_ARG, "%s: group_size=%d", op, G);
  if (!is_float(adt) || !is_float(sdt))
    return fail(TM_ERR_INVALID_ARG, "%s: act dtype %s / scale dtype %s", op, dt_name(adt),
                dt_name(sdt));
  if (!(zdt == TM_DT_NONE || is_float(zdt) || zdt == TM_DT_U8))
    return fail(TM_ERR_INVALID_ARG, "%s: zero dtype %d", op, zdt);
  if (zdt != TM_DT_NONE && !Z) return fail(TM_ERR_INVALID_ARG, "%s: zeros is NULL", op);
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();

  if (workspace && !aligned16(workspace))
    return fail(TM_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", op);
  const unsigned align = wq_align(X, W, S, Z);
  WqPlan pl;
  wq_plan(qbits, M, N, K, G, adt, sdt, zdt, align, cu_count(), (size_t)max_dynamic_lds(),
          workspace != nullptr, &pl);
  if (pl.splits > 1 && workspace_bytes < pl.ws)
    return fail(TM_ERR_INVALID_ARG, "%s: workspace of %zu bytes, this call needs %zu", op,
                workspace_bytes, pl.ws);
  Kernel& k = kernel(pl.name);
  const dim3 grid(pl.grid), block(pl.block);
  switch (pl.form) {
    case WQ_ARGS_SPLIT:
    case WQ_ARGS_SPLIT_G: {
      float* P = (float*)workspace;
      int rc = pl.form == WQ_ARGS_SPLIT
                   ? launch(k, dim3(pl.grid, (unsigned)pl.splits), block, pl.lds, stream, X, W, P,
                            S, Z, M, N, pl.kslice, K)
                   : launch(k, dim3(pl.grid, (unsigned)pl.splits), block, pl.lds, stream, X, W, P,
                            S, Z, M, N, pl.kslice, K, G);
      if (rc) return rc;
      const size_t quads = (size_t)M * N / 4;
      return launch(kernel(adt == TM_DT_BF16 ? "wq_splitk_reduce_bf16" : "wq_splitk_reduce_f16"),
                    dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, (const float*)P,
                    Y, bias, M, N, pl.splits);
    }
    case WQ_ARGS_G:
      return launch(k, grid, block, pl.lds, stream, X, W, Y, S, Z, M, N, K, G, bias);
    case WQ_ARGS_GENERAL:
      return launch(k, grid, block, pl.lds, stream, X, (const uint8_t*)W, Y, S, Z, M, N, K,
                    qbits == 4 ? G : 1, qbits, adt, sdt, zdt, bias);
    default:
      return launch(k, grid, block, pl.lds, stream, X, W, Y, S, Z, M, N, K, bias);
  }
}

// ---- dense kernel selection ---------------------------------------------------
// A pure function of the call (sizes, leading dimensions, dtypes, whether B is
// the transposed nn.Linear weight and a bias is given, pointer alignment): the
// launch path and tm_gemm_plan share it.  FP8 inputs are not planned here (they
// run the general dot); fp32 inputs take gemm_f32t64, 16-bit inputs the MFMA
// tile kernels where sizes and alignment allow, else the strided dot's tile
// kernels ("tm_dot": grid and block are the dot's own choice, reported as 0),
// and K = 0 gemm_general.
struct GemmPlan {
  char name[96];
  unsigned grid, block;
  bool general;  // not a dense tile kernel: tm_dot, or gemm_general (K = 0)
};

void gemm_plan(int M, int N, int K, int lda, int ldb, int ldc, bool bt, bool bias, int idt,
               int odt, bool ab16, bool c16, GemmPlan* pl) {
  pl->general = false;
  if (idt == TM_DT_F32) {
    // fp32 inputs (the reference's default dtype): 64 x 64 tiles on the fp32
    // MFMA (gemm_f32.hip); 16-byte operand pieces when A and B are 16-byte
    // aligned with leading dimensions multiples of 4 (gemm_f32t64), else
    // element loads (gemm_f32t64u)
    const bool vec = ab16 && lda % 4 == 0 && ldb % 4 == 0;
    snprintf(pl->name, sizeof pl->name, "gemm_f32t64%s_%s_%s%s", vec ? "" : "u", bt ? "nt" : "nn",
             odt == TM_DT_F32 ? "f32" : odt == TM_DT_F16 ? "f16" : "bf16",
             (bt && bias) ? "_bias" : "");
    pl->grid = (unsigned)(((M + 63) / 64) * ((N + 63) / 64));
    pl->block = 256;
    return;
  }
  const char* dt = idt == TM_DT_BF16 ? "bf16" : "f16";
  const char* od = odt == TM_DT_F32 ? "f32" : "same";
  const char* bs = (bt && bias) ? "_bias" : "";
  const bool mfma = is_half(idt) && (odt == idt || odt == TM_DT_F32) && K % 8 == 0 &&
                    lda % 8 == 0 && ldb % 8 == 0 && ab16 && (bt || N % 8 == 0);
  if (mfma) {
    // 256 x 256 tiles (gemm_big.hip) for aligned problems from 32 tiles on:
    // one such workgroup per CU beats four 128 x 128 ones over the same
    // outputs even when most CUs stay idle (one box, fp16, K = 4096: 2048 x
    // 3072 78 against 125 us, 2560 x 4096 84 against 241; at 16 tiles the
    // smaller tiles win, 140 against 147 us); the 32-bit copy offsets of a
    // tile (up to 256 rows of A / B^T, 64 rows of B) must fit
    const long t256 = (M % 256 == 0 && N % 256 == 0) ? (long)(M / 256) * (N / 256) : 0;
    if (t256 >= 32 && K % 64 == 0 && 256LL * lda * 2 < (1LL << 32) &&
        (bt ? 256LL : 64LL) * ldb * 2 < (1LL << 32)) {
      snprintf(pl->name, sizeof pl->name, "gemm_t256_%s_%s_%s%s", bt ? "nt" : "nn", dt, od, bs);
      pl->grid = (unsigned)t256;
      pl->block = 512;
      return;
    }
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    // small aligned problems with K = 256 or 512 (C1): 32 x 32 tiles, K split
    // over the workgroup's 4 waves, 16-byte copies and 8 / 16-byte stores
    if (t128 < 256 && M % 32 == 0 && N % 32 == 0 && (K == 256 || K == 512) && c16 &&
        ldc % 4 == 0) {
      snprintf(pl->name, sizeof pl->name, "gemm_s32k%d_%s_%s_%s%s", K / 4, bt ? "nt" : "nn", dt,
               od, bs);
      pl->grid = (unsigned)((M / 32) * (N / 32));
      pl->block = 256;
      return;
    }
    const char* tile;
    const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    int bm;
    if (t128 >= 256) { tile = "t128"; bm = 128; }
    else if (t64 >= 192) { tile = "t64"; bm = 64; }
    else if (K <= 512) { tile = "t32k"; bm = 32; }  // one load stage
    else { tile = "t32"; bm = 32; }
    snprintf(pl->name, sizeof pl->name, "gemm_%s_%s_%s_%s%s", tile, bt ? "nt" : "nn", dt, od, bs);
    pl->grid = (unsigned)(((M + bm - 1) / bm) * ((N + bm - 1) / bm));
    pl->block = 256;
    return;
  }
  pl->general = true;
  if (K > 0) {
    snprintf(pl->name, sizeof pl->name, "tm_dot");
    pl->grid = pl->block = 0;
    return;
  }
  snprintf(pl->name, sizeof pl->name, "gemm_general");
  pl->grid = (unsigned)(((size_t)M * N + 255) / 256);
  pl->block = 256;
}

int dense(const void* A, const void* B, void* C, const void* bias, int M, int N, int K, int lda,
          int ldb, int ldc, bool bt, int idt, int odt, void* stream) {
  const char* op = bt ? "tm_linear" : "tm_matmul";
  if (!bt && idt >= TM_DT_FP8_E4M3 && idt <= TM_DT_FP8_E5M2B16) {
    // FP8 inputs: the general dot on row-major operands
    if (lda < K || ldb < N || ldc < N)
      return fail(TM_ERR_INVALID_ARG, "%s: leading dimension too small", op);
    const long long st[14] = {0, lda, 1, 0, ldb, 1, 0, ldc, 1, 0, 0, 0, 0, 0};
    return dot_impl(op, A, B, C, nullptr, nullptr, 1, M, N, K, 0, st, TM_EPI_NONE, idt, odt,
                    TM_DT_NONE, TM_DT_NONE, stream);
  }
  if (M < 0 || N < 0 || K < 0) return fail(TM_ERR_INVALID_ARG, "%s: negative size", op);
  if (M == 0 || N == 0) return 0;
  if (!A || !B || !C) return fail(TM_ERR_INVALID_ARG, "%s: null buffer", op);
  if (!is_float(idt) || !is_float(odt))
    return fail(TM_ERR_INVALID_ARG, "%s: dtypes %s -> %s", op, dt_name(idt), dt_name(odt));
  if (lda < K || ldc < N || (bt ? ldb < K : ldb < N))
    return fail(TM_ERR_INVALID_ARG, "%s: leading dimension too small", op);
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  GemmPlan pl;
  gemm_plan(M, N, K, lda, ldb, ldc, bt, bias != nullptr, idt, odt, aligned16(A) && aligned16(B),
            aligned16(C), &pl);
  if (pl.general) {
    // 16-bit operands the tile kernels cannot take (K or a leading dimension
    // not a multiple of 8, unaligned A / B): the strided dot's MFMA tile
    // kernels, the bias as its add-cols epilogue; K = 0 (a product of zeros)
    // on the one-thread-per-output kernel
    if (K > 0) {
      const long long st[14] = {0, lda, 1, 0, bt ? 1 : ldb, bt ? ldb : 1, 0, ldc, 1, 0, 0, 1,
                                0, 0};
      return dot_impl(op, A, B, C, bias, nullptr, 1, M, N, K, 0, st,
                      bias ? TM_EPI_ADD_COLS : TM_EPI_NONE, idt, odt, bias ? idt : TM_DT_NONE,
                      TM_DT_NONE, stream);
    }
    return launch(kernel(pl.name), dim3(pl.grid), dim3(pl.block), 0, stream, A, B, C, bias, M, N,
                  K, lda, ldb, ldc, bt ? 1 : 0, idt, odt);
  }
  return launch(kernel(pl.name), dim3(pl.grid), dim3(pl.block), 0, stream, A, B, C, bias, M, N,
                K, lda, ldb, ldc);
}

}  // namespace

int tmhip::dense_f32(const float* A, const float* B, void* C, int M, int N, int K, int lda,
                     int ldb, int ldc, bool bt, int out_dtype, void* stream) {
  GemmPlan pl;
  gemm_plan(M, N, K, lda, ldb, ldc, bt, false, TM_DT_F32, out_dtype, aligned16(A) && aligned16(B),
            aligned16(C), &pl);
  return launch(kernel(pl.name), dim3(pl.grid), dim3(pl.block), 0, stream, A, B, C,
                (const float*)nullptr, M, N, K, lda, ldb, ldc);
}

int tmhip::dense_mfma(const void* A, const void* B, void* C, int M, int N, int K, int lda,
                      int ldb, int ldc, bool bt, int in_dtype, int out_dtype, void* stream,
                      bool* used) {
  *used = false;
  if (!is_half(in_dtype)) return 0;
  GemmPlan pl;
  gemm_plan(M, N, K, lda, ldb, ldc, bt, false, in_dtype, out_dtype, aligned16(A) && aligned16(B),
            aligned16(C), &pl);
  if (pl.general) return 0;
  *used = true;
  return launch(kernel(pl.name), dim3(pl.grid), dim3(pl.block), 0, stream, A, B, C,
                (const void*)nullptr, M, N, K, lda, ldb, ldc);
}

extern "C" {

int tm_int8_matmul(const void* input, const void* weight, void* output, const void* scales,
                   const void* zeros, int M, int N, int K, int act_dtype, int scale_dtype,
                   int zero_dtype, void* stream) {
  return wq_matmul(8, input, weight, output, scales, zeros, M, N, K, 1, act_dtype, scale_dtype,
                   zero_dtype, nullptr, nullptr, 0, stream);
}

int tm_int4_matmul(const void* input, const void* weight, void* output, const void* scales,
                   const void* zeros, int M, int N, int K, int group_size, int act_dtype,
                   int scale_dtype, int zero_dtype, void* stream) {
  return wq_matmul(4, input, weight, output, scales, zeros, M, N, K, group_size, act_dtype,
                   scale_dtype, zero_dtype, nullptr, nullptr, 0, stream);
}

int tm_int8_linear(const void* input, const void* weight, const void* bias, void* output,
                   const void* scales, const void* zeros, int M, int N, int K, int act_dtype,
                   int scale_dtype, int zero_dtype, void* stream) {
  return wq_matmul(8, input, weight, output, scales, zeros, M, N, K, 1, act_dtype, scale_dtype,
                   zero_dtype, bias, nullptr, 0, stream);
}

int tm_int4_linear(const void* input, const void* weight, const void* bias, void* output,
                   const void* scales, const void* zeros, int M, int N, int K, int group_size,
                   int act_dtype, int scale_dtype, int zero_dtype, void* stream) {
  return wq_matmul(4, input, weight, output, scales, zeros, M, N, K, group_size, act_dtype,
                   scale_dtype, zero_dtype, bias, nullptr, 0, stream);
}

int tm_wq_matmul_ws(int qbits, const void* input, const void* weight, const void* bias,
                    void* output, const void* scales, const void* zeros, int M, int N, int K,
                    int group_size, int act_dtype, int scale_dtype, int zero_dtype,
                    void* workspace, size_t workspace_bytes, void* stream) {
  if (qbits != 4 && qbits != 8)
    return fail(TM_ERR_INVALID_ARG, "tm_wq_matmul_ws: qbits=%d (4 or 8)", qbits);
  return wq_matmul(qbits, input, weight, output, scales, zeros, M, N, K,
                   qbits == 4 ? group_size : 1, act_dtype, scale_dtype, zero_dtype, bias,
                   workspace, workspace_bytes, stream);
}

size_t tm_wq_workspace_bytes(int qbits, const void* input, const void* weight,
                             const void* scales, const void* zeros, int M, int N, int K,
                             int group_size, int act_dtype, int scale_dtype, int zero_dtype) {
  if ((qbits != 4 && qbits != 8) || M <= 0 || N <= 0 || K <= 0 || (qbits == 4 && group_size <= 0))
    return 0;
  if (!api()) return 0;
  WqPlan pl;
  wq_plan(qbits, M, N, K, qbits == 4 ? group_size : 1, act_dtype, scale_dtype, zero_dtype,
          wq_align(input, weight, scales, zeros), cu_count(), (size_t)max_dynamic_lds(), true,
          &pl);
  return pl.ws;
}


int tm_wq_plan(int qbits, int M, int N, int K, int group_size, int act_dtype, int scale_dtype,
               int zero_dtype, unsigned align_flags, int cu_count, size_t max_lds,
               int with_workspace, char* name, size_t name_len, unsigned* grid, unsigned* block,
               unsigned* lds_bytes, unsigned* splits, size_t* workspace_bytes) {
  if ((qbits != 4 && qbits != 8) || M <= 0 || N <= 0 || K <= 0 || cu_count <= 0 ||
      (qbits == 4 && group_size <= 0))
    return fail(TM_ERR_INVALID_ARG, "tm_wq_plan: qbits=%d M=%d N=%d K=%d G=%d cus=%d", qbits, M,
                N, K, group_size, cu_count);
  clear_error();
  WqPlan pl;
  wq_plan(qbits, M, N, K, qbits == 4 ? group_size : 1, act_dtype, scale_dtype, zero_dtype,
          align_flags, cu_count, max_lds, with_workspace != 0, &pl);
  if (name && name_len) snprintf(name, name_len, "%s", pl.name);
  if (grid) *grid = pl.grid;
  if (block) *block = pl.block;
  if (lds_bytes) *lds_bytes = pl.lds;
  if (splits) *splits = (unsigned)pl.splits;
  if (workspace_bytes) *workspace_bytes = pl.ws;
  return 0;
}

int tm_gemm_plan(int M, int N, int K, int lda, int ldb, int ldc, int trans_b, int has_bias,
                 int in_dtype, int out_dtype, unsigned align_flags, char* name, size_t name_len,
                 unsigned* grid, unsigned* block) {
  const bool bt = trans_b != 0;
  if (M <= 0 || N <= 0 || K <= 0 || lda < K || ldc < N || (bt ? ldb < K : ldb < N))
    return fail(TM_ERR_INVALID_ARG, "tm_gemm_plan: M=%d N=%d K=%d lda=%d ldb=%d ldc=%d", M, N, K,
                lda, ldb, ldc);
  if (!is_float(in_dtype) || !is_float(out_dtype))
    return fail(in_dtype >= TM_DT_FP8_E4M3 && in_dtype <= TM_DT_FP8_E5M2B16 ? TM_ERR_UNSUPPORTED
                                                                            : TM_ERR_INVALID_ARG,
                "tm_gemm_plan: dtypes %d -> %d (FP8 inputs run the general dot)", in_dtype,
                out_dtype);
  clear_error();
  GemmPlan pl;
  gemm_plan(M, N, K, lda, ldb, ldc, bt, bt && has_bias != 0, in_dtype, out_dtype,
            (align_flags & TM_GEMM_ALIGN_AB16) != 0, (align_flags & TM_GEMM_ALIGN_C16) != 0, &pl);
  if (name && name_len) snprintf(name, name_len, "%s", pl.name);
  if (grid) *grid = pl.grid;
  if (block) *block = pl.block;
  return 0;
}

namespace {
// GPTQ / AWQ int4 checkpoints -> the int4 layout of tm_int4_matmul.
int repack(bool awq, const void* qweight, const void* qzeros, const void* scales, int N, int K,
           int group_size, int zero_offset, void* weight_out, void* scales_out, void* zeros_out,
           void* stream) {
  const char* op = awq ? "tm_wq_repack_awq" : "tm_wq_repack_gptq";
  if (N < 0 || K < 0 || group_size <= 0 || K % 8 || N % 8)
    return fail(TM_ERR_INVALID_ARG, "%s: N=%d K=%d group_size=%d (N, K multiples of 8)", op, N,
                K, group_size);
  if (!qweight || !weight_out) return fail(TM_ERR_INVALID_ARG, "%s: null weight buffer", op);
  if ((qzeros != nullptr) != (zeros_out != nullptr) ||
      (scales != nullptr) != (scales_out != nullptr))
    return fail(TM_ERR_INVALID_ARG, "%s: zeros / scales given without their output", op);
  if (zero_offset < 0 || zero_offset > 240)
    return fail(TM_ERR_INVALID_ARG, "%s: zero_offset=%d", op, zero_offset);
  if (N == 0 || K == 0) return 0;
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  static Kernel kg("wq_repack_gptq_weight"), ka("wq_repack_awq_weight"), kz("wq_repack_zeros"),
      kt("wq_transpose16");
  const int ng = (K + group_size - 1) / group_size;
  int rc = launch(awq ? ka : kg, dim3((N + 63) / 64, (K / 8 + 63) / 64), dim3(256), 0, stream,
                  qweight, weight_out, N, K);
  if (rc) return rc;
  if (qzeros) {
    const long long total = (long long)N * ng;
    rc = launch(kz, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, qzeros,
                zeros_out, N, ng, awq ? 1 : 0, zero_offset);
    if (rc) return rc;
  }
  if (scales)
    rc = launch(kt, dim3((N + 63) / 64, (ng + 63) / 64), dim3(256), 0, stream, scales, scales_out,
                ng, N);
  return rc;
}
}  // namespace

int tm_wq_repack_gptq(const void* qweight, const void* qzeros, const void* scales, int N, int K,
                      int group_size, int zero_offset, void* weight_out, void* scales_out,
                      void* zeros_out, void* stream) {
  return repack(false, qweight, qzeros, scales, N, K, group_size, zero_offset, weight_out,
                scales_out, zeros_out, stream);
}

int tm_wq_repack_awq(const void* qweight, const void* qzeros, const void* scales, int N, int K,
                     int group_size, void* weight_out, void* scales_out, void* zeros_out,
                     void* stream) {
  return repack(true, qweight, qzeros, scales, N, K, group_size, 0, weight_out, scales_out,
                zeros_out, stream);
}

int tm_wq_dequant(const void* weight, const void* scales, const void* zeros, void* out, int N,
                  int K, int group_size, int qbits, int scale_dtype, int zero_dtype,
                  int out_dtype, void* stream) {
  if (!weight || !scales || !out) return fail(TM_ERR_INVALID_ARG, "tm_wq_dequant: null buffer");
  if (qbits != 4 && qbits != 8) return fail(TM_ERR_INVALID_ARG, "tm_wq_dequant: qbits=%d", qbits);
  if (N < 0 || K < 0 || (qbits == 4 && (K % 2 || group_size <= 0)))
    return fail(TM_ERR_INVALID_ARG, "tm_wq_dequant: N=%d K=%d G=%d", N, K, group_size);
  if (!is_float(scale_dtype) || !is_float(out_dtype) ||
      !(zero_dtype == TM_DT_NONE || is_float(zero_dtype) || zero_dtype == TM_DT_U8))
    return fail(TM_ERR_INVALID_ARG, "tm_wq_dequant: dtype");
  if (zero_dtype != TM_DT_NONE && !zeros)
    return fail(TM_ERR_INVALID_ARG, "tm_wq_dequant: zeros is NULL");
  size_t total = (size_t)N * K;
  if (total == 0) return 0;
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  int G = qbits == 4 ? group_size : 1;
  return launch(kernel("wq_dequant"), dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                stream, (const uint8_t*)weight, scales, zeros, out, N, K, G, qbits, scale_dtype,
                zero_dtype, out_dtype);
}

namespace {
int matmul_dd(const char* op, const void* A, const void* B, void* C, const unsigned* Mp,
              const unsigned* Np, const unsigned* Kp, int max_m, int max_n, size_t a_elems,
              size_t b_elems, size_t c_elems, int group_m, int idt, int odt, void* stream) {
  if (max_m < 0 || max_n < 0 || group_m < 0)
    return fail(TM_ERR_INVALID_ARG, "%s: max_m=%d max_n=%d group=%d", op, max_m, max_n, group_m);
  if (max_m == 0 || max_n == 0) return 0;
  if (!A || !B || !C || !Mp || !Np || !Kp)
    return fail(TM_ERR_INVALID_ARG, "%s: null buffer", op);
  if (!is_float(idt) || !(odt == idt || odt == TM_DT_F32))
    return fail(TM_ERR_INVALID_ARG, "%s: dtypes %s -> %s", op, dt_name(idt), dt_name(odt));
  const long long ntr = (max_m + 63) / 64, ntc = (max_n + 63) / 64;
  if (group_m == 0 ? ntr > 65535 : ntr * ntc > 0x7fffffffLL)
    return fail(TM_ERR_UNSUPPORTED, "%s: capacity %d x %d", op, max_m, max_n);
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  char name[64];
  snprintf(name, sizeof name, "gemm_dd_%s_%s", dt_name(idt),
           odt == idt ? "same" : "f32");
  const dim3 grid = group_m == 0 ? dim3((unsigned)ntc, (unsigned)ntr)
                                 : dim3((unsigned)(ntr * ntc));
  const unsigned long long ae = a_elems, be = b_elems, ce = c_elems;
  return launch(kernel(name), grid, dim3(256), 0, stream, A, B, C, Mp, Np, Kp, max_m, max_n, ae,
                be, ce, group_m);
}
}  // namespace

int tm_matmul_2d(const void* A, const void* B, void* C, const unsigned* M, const unsigned* N,
                 const unsigned* K, int max_m, int max_n, size_t a_elems, size_t b_elems,
                 size_t c_elems, int in_dtype, int out_dtype, void* stream) {
  return matmul_dd("tm_matmul_2d", A, B, C, M, N, K, max_m, max_n, a_elems, b_elems, c_elems, 0,
                   in_dtype, out_dtype, stream);
}

int tm_matmul_swizzled(const void* A, const void* B, void* C, const unsigned* M,
                       const unsigned* N, const unsigned* K, int max_m, int max_n,
                       size_t a_elems, size_t b_elems, size_t c_elems, int group_size,
                       int in_dtype, int out_dtype, void* stream) {
  if (group_size <= 0)
    return fail(TM_ERR_INVALID_ARG, "tm_matmul_swizzled: group_size=%d", group_size);
  return matmul_dd("tm_matmul_swizzled", A, B, C, M, N, K, max_m, max_n, a_elems, b_elems,
                   c_elems, group_size, in_dtype, out_dtype, stream);
}

int tm_matmul(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb,
              int ldc, int in_dtype, int out_dtype, void* stream) {
  return dense(A, B, C, nullptr, M, N, K, lda, ldb, ldc, false, in_dtype, out_dtype, stream);
}

int tm_linear(const void* input, const void* weight, const void* bias, void* output, int M,
              int N, int K, int in_dtype, int out_dtype, void* stream) {
  return dense(input, weight, output, bias, M, N, K, K, K, N, true, in_dtype, out_dtype, stream);
}

}  // extern "C"

// Kernel registry keyed by name (names are compile-time constants of the
// instantiations in the .hip sources).
Kernel& tmhip::kernel_named(const std::string& name) {
  static std::mutex mu;
  static std::map<std::string, Kernel*> table;
  std::lock_guard<std::mutex> lk(mu);
  auto it = table.find(name);
  if (it != table.end()) return *it->second;
  char* stored = strdup(name.c_str());
  Kernel* k = new Kernel(stored);
  table[name] = k;
  return *k;
}
