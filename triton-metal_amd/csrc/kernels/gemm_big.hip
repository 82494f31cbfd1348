// Large-tile dense fp16/bf16 GEMM for gfx950 (fp32 accumulation):
//
//   C[M, N] = A[M, K] @ B[K, N]              (nn: the tl.dot / matmul layout)
//   C[M, N] = A[M, K] @ W[N, K]^T (+ bias[N])  (nt: the nn.Linear layout)
//
// for M % 256 == 0, N % 256 == 0, K % 64 == 0 (the host picks it for large
// aligned problems; the other shapes run in gemm.hip).  Reference semantics as
// gemm.hip: make_matmul_kernel / make_simdgroup_matmul_kernel /
// make_fused_linear_kernel (_msl_templates.py:447-585, 3501-3667, 4013-4135).
//
// A workgroup of 8 waves owns a 256 x 256 output tile; wave (wm, wn) = (w / 4,
// w % 4) owns rows 128 wm .. +127 and columns 64 wn .. +63 as 4 x 2 tiles of
// v_mfma_f32_32x32x16 (128 accumulator registers).  K advances in steps of
// 64 through two LDS stages of 64 KB; every step's A and B tiles stream from
// global memory straight into LDS (global_load_lds_dwordx4 issued in asm, one
// 1 KB block per instruction, 8 per wave per step), one step ahead of the
// MFMAs, with one barrier per step.
// LDS layouts (16-byte pieces, XOR-swizzled so the operand reads spread over
// the banks):
//   A, and B of nt:  [256 rows][64 k], row = 8 pieces (128 bytes, so the
//                    64 banks hold two rows), piece p of row r at
//                    p ^ ((r >> 1) & 7): the 16 rows of one 16-lane read phase
//                    land in 16 different 16-byte bank groups; operands by
//                    ds_read_b128 (row l % 32, k = 8 (l / 32) + e);
//   B of nn:         [64 k][256 n], row = 32 pieces, piece p of row k at
//                    p ^ 4 (k & 3); operands by two ds_read_b64_tr_b16 (lane
//                    l: column l % 32, rows k = 8 (l / 32) + e), the order of
//                    the A operand.
#include "common.h"

namespace {

constexpr int GB_BM = 256, GB_BN = 256, GB_BK = 64;

typedef short gb_s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) gb_s4_t gb_lds_s4_t;

// XOR swizzle of the 128-byte rows of the A (and nt B) tiles
TM_DEV int gb_sw(int r) { return (r >> 1) & 7; }

TM_DEV u2_t gb_tr16(const uint16_t* p) {
  gb_s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gb_lds_s4_t*)(p));
  return __builtin_bit_cast(u2_t, v);
}

template <int ODT> TM_DEV void gb_store(void* C, size_t i, float v) { store_from_f32<ODT>(C, i, v); }

}  // namespace

template <bool BT, bool BF16, int ODT, bool BIAS>
__device__ __forceinline__ void gemm_big_body(const uint16_t* __restrict__ A,
                                              const uint16_t* __restrict__ B,
                                              void* __restrict__ C,
                                              const uint16_t* __restrict__ bias, int M, int N,
                                              int K, int lda, int ldb, int ldc) {
  // separate objects per stage, chosen at compile time, so the compiler can
  // tell the reads of one stage from the copies into the other
  __shared__ __align__(16) uint16_t As0[GB_BM * GB_BK], As1[GB_BM * GB_BK];
  __shared__ __align__(16) uint16_t Bs0[GB_BN * GB_BK], Bs1[GB_BN * GB_BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, h32 = lane >> 5;
  const int tiles_n = N / GB_BN;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const int m0 = tm * GB_BM, n0 = tn * GB_BN;

  // ---- copies: this lane's byte offsets of its 4 A and 4 B pieces per step,
  // relative to a per-step scalar base.  Instruction i of wave w fills the 1 KB
  // block 4 w + i of a tile.
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = 4 * wave + i;
    const int r = 8 * blk + (lane >> 3), ph = lane & 7;  // row-major [256][64] tile
    aoff[i] = 2u * (uint32_t)(r * lda + 8 * (ph ^ gb_sw(r)));
    if constexpr (BT) {
      boff[i] = 2u * (uint32_t)(r * ldb + 8 * (ph ^ gb_sw(r)));
    } else {
      const int kr = 2 * blk + (lane >> 5), pc = lane & 31;  // [64][256] tile
      boff[i] = 2u * (uint32_t)(kr * ldb + 8 * (pc ^ (4 * (kr & 3))));
    }
  }
  const uint16_t* a_row0 = A + (size_t)m0 * lda;
  const uint16_t* b_row0 = BT ? B + (size_t)n0 * ldb : B + n0;
  auto issue = [&](uint16_t* as, uint16_t* bs, int k0) {
    const uint16_t* ab = a_row0 + k0;
    const uint16_t* bb = BT ? b_row0 + k0 : b_row0 + (size_t)k0 * ldb;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16s(ab, aoff[i], lds_off(as) + 1024 * (4 * wave + i));
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16s(bb, boff[i], lds_off(bs) + 1024 * (4 * wave + i));
  };

  f16_t acc[4][2];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = f16_t{};

  // per-lane constants of the nn B reads: 16-lane group G, lane j in it
  const int tg = lane >> 4, tj = lane & 15;
  const int tr_k = 8 * (tg >> 1) + (tj >> 2);        // + 16 kk (+ 4 for elements 4..7)
  const int tr_c = 16 * (tg & 1) + 4 * (tj & 3);     // + 64 wn + 32 ct

  // operands of one 16-k substep: 4 A row tiles, 2 B column tiles
  auto read_ops = [&](const uint16_t* as, const uint16_t* bs, int kk, u4_t* ao, u4_t* bo) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int r = 128 * wm + 32 * rt + l32, p = 2 * kk + h32;
      ao[rt] = *(const u4_t*)(as + r * GB_BK + 8 * (p ^ gb_sw(r)));
    }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      if constexpr (BT) {
        const int r = 64 * wn + 32 * ct + l32, p = 2 * kk + h32;
        bo[ct] = *(const u4_t*)(bs + r * GB_BK + 8 * (p ^ gb_sw(r)));
      } else {
        const int c = 64 * wn + 32 * ct + tr_c, pc = c >> 3, co = c & 7;
        const int k0 = 16 * kk + tr_k, k1 = k0 + 4;
        const u2_t lo = gb_tr16(bs + k0 * GB_BN + 8 * (pc ^ (4 * (k0 & 3))) + co);
        const u2_t hi = gb_tr16(bs + k1 * GB_BN + 8 * (pc ^ (4 * (k1 & 3))) + co);
        bo[ct] = u4_t{lo.x, lo.y, hi.x, hi.y};
      }
    }
  };
  // the operands of substep kk + 1 are read while substep kk multiplies
  constexpr int NRD = BT ? 6 : 8;  // LDS reads per substep
  auto compute = [&](const uint16_t* as, const uint16_t* bs) {
    u4_t ao[2][4], bo[2][2];
    read_ops(as, bs, 0, ao[0], bo[0]);
#pragma unroll
    for (int kk = 0; kk < GB_BK / 16; ++kk) {
      if (kk + 1 < GB_BK / 16) read_ops(as, bs, kk + 1, ao[(kk + 1) & 1], bo[(kk + 1) & 1]);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
          acc[rt][ct] = mfma32<BF16>(ao[kk & 1][rt], bo[kk & 1][ct], acc[rt][ct]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);
#pragma unroll
    for (int kk = 0; kk < GB_BK / 16; ++kk) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (kk + 1 < GB_BK / 16 && j < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
  };

  const int nk = K / GB_BK;
  issue(As0, Bs0, 0);
  wait_vm<0>();
  __syncthreads();
  auto step = [&](auto bufc, int kt) {
    constexpr int BUF = decltype(bufc)::value;
    const bool more = kt + 1 < nk;
    if (more) issue(BUF ? As0 : As1, BUF ? Bs0 : Bs1, (kt + 1) * GB_BK);
    compute(BUF ? As1 : As0, BUF ? Bs1 : Bs0);
    if (more) wait_vm<0>();  // this wave's copies of step kt + 1 landed
    __syncthreads();
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
  }

  // ---- epilogue: D layout row 8 (e / 4) + 4 h32 + e % 4, column l32
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int col = n0 + 64 * wn + 32 * ct + l32;
    float bv = 0.0f;
    if constexpr (BIAS) bv = BF16 ? bf16_bits_to_f32(bias[col]) : f16_bits_to_f32(bias[col]);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + 128 * wm + 32 * rt + 8 * (e >> 2) + 4 * h32 + (e & 3);
        gb_store<ODT>(C, (size_t)row * ldc + col, acc[rt][ct][e] + bv);
      }
  }
}

// gemm_t256_<bt>_<in>_<out>[_bias]
#define TM_GEMM_BIG(NAME, BT, BF, ODT, BIAS)                                                    \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void     \
      NAME(const uint16_t* A, const uint16_t* B, void* C, const uint16_t* bias, int M, int N,   \
           int K, int lda, int ldb, int ldc) {                                                  \
    gemm_big_body<BT, BF, ODT, BIAS>(A, B, C, bias, M, N, K, lda, ldb, ldc);                    \
  }
TM_GEMM_BIG(gemm_t256_nn_f16_same, false, false, TM_DT_F16, false)
TM_GEMM_BIG(gemm_t256_nn_f16_f32, false, false, TM_DT_F32, false)
TM_GEMM_BIG(gemm_t256_nn_bf16_same, false, true, TM_DT_BF16, false)
TM_GEMM_BIG(gemm_t256_nn_bf16_f32, false, true, TM_DT_F32, false)
TM_GEMM_BIG(gemm_t256_nt_f16_same, true, false, TM_DT_F16, false)
TM_GEMM_BIG(gemm_t256_nt_f16_f32, true, false, TM_DT_F32, false)
TM_GEMM_BIG(gemm_t256_nt_bf16_same, true, true, TM_DT_BF16, false)
TM_GEMM_BIG(gemm_t256_nt_bf16_f32, true, true, TM_DT_F32, false)
TM_GEMM_BIG(gemm_t256_nt_f16_same_bias, true, false, TM_DT_F16, true)
TM_GEMM_BIG(gemm_t256_nt_f16_f32_bias, true, false, TM_DT_F32, true)
TM_GEMM_BIG(gemm_t256_nt_bf16_same_bias, true, true, TM_DT_BF16, true)
TM_GEMM_BIG(gemm_t256_nt_bf16_f32_bias, true, true, TM_DT_F32, true)
