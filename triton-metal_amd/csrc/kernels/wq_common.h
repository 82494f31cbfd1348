// Helpers shared by the weight-only matmul kernels (wq_gemm.hip, wq_xreg.hip):
// scale / zero-point loads of a compile-time or runtime dtype, and the exact
// 16-bit MFMA / dot operands built from int4 and int8 weights.
#pragma once
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

// Scalar of a compile-time dtype (ZDT < 0: absent, reads as 0).
template <int DT> TM_DEV float ld_typed(const void* p, size_t i) {
  if constexpr (DT < 0) return 0.0f;
  else if constexpr (DT == TM_DT_F32) return ((const float*)p)[i];
  else if constexpr (DT == TM_DT_F16) return (float)((const half_t*)p)[i];
  else if constexpr (DT == TM_DT_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else return (float)((const uint8_t*)p)[i];
}

// Raw storage type of a scale / zero-point dtype, loaded without conversion so
// the load can stay in flight until the value is used.
template <int DT> struct Raw { using T = uint16_t; };
template <> struct Raw<TM_DT_F32> { using T = float; };
template <> struct Raw<3> { using T = uint8_t; };
template <> struct Raw<-1> { using T = uint8_t; };
template <int DT> TM_DEV typename Raw<DT>::T ld_raw(const void* p, size_t i) {
  if constexpr (DT < 0) return 0;
  else return ((const typename Raw<DT>::T*)p)[i];
}
template <int DT> TM_DEV float raw_to_f32(typename Raw<DT>::T v) {
  if constexpr (DT < 0) return 0.0f;
  else if constexpr (DT == TM_DT_F32) return v;
  else if constexpr (DT == TM_DT_F16) return (float)__builtin_bit_cast(half_t, v);
  else if constexpr (DT == TM_DT_BF16) return bf16_bits_to_f32(v);
  else return (float)v;
}

// int4: one word (8 nibbles) -> one 8 x 16-bit MFMA operand of OFF + q in
// element order [n0, n4, n1, n5, n2, n6, n3, n7].
// `mask` = 0x000F000F and `magic` = the OFF exponent pattern, both held in
// VGPRs (vgpr_const) so each half-pair costs one v_and_or_b32.
// Same with the shift amounts held in registers (vgpr_const inside a loop
// keeps the whole conversion inside that loop).
TM_DEV u4_t w4_operand_v(uint32_t w, uint32_t mask, uint32_t magic, uint32_t s4, uint32_t s8,
                         uint32_t s12) {
  u4_t r;
  r.x = (w & mask) | magic;
  r.y = ((w >> s4) & mask) | magic;
  r.z = ((w >> s8) & mask) | magic;
  r.w = ((w >> s12) & mask) | magic;
  return r;
}
TM_DEV u4_t w4_operand(uint32_t w, uint32_t mask, uint32_t magic) {
  u4_t r;
  r.x = (w & mask) | magic;
  r.y = ((w >> 4) & mask) | magic;
  r.z = ((w >> 8) & mask) | magic;
  r.w = ((w >> 12) & mask) | magic;
  return r;
}
template <bool BF16> constexpr uint32_t w4_magic() { return BF16 ? 0x43004300u : 0x64006400u; }
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

// fp16 int4 operand in 5 instructions: a nibble at bits 0-3 of a half ORed
// under 0x6400 (1024) is 1024 + q; one at bits 4-7 ORed under 0x5400 (64,
// whose ulp is 1/16) is 64 + q.  The halves come out in w4_operand's order
// [n0 n4] [n1 n5] [n2 n6] [n3 n7]: nibble j (k = 8 w + j) carries the offset
// 1024 for even j, 64 for odd j.
TM_DEV u4_t w4_operand_h(uint32_t w, uint32_t m_lo, uint32_t m_hi, uint32_t g_lo,
                         uint32_t g_hi) {
  const uint32_t t = w >> 8;
  u4_t r;
  r.x = (w & m_lo) | g_lo;
  r.y = (w & m_hi) | g_hi;
  r.z = (t & m_lo) | g_lo;
  r.w = (t & m_hi) | g_hi;
  return r;
}
// sum of x_k * off_k over 8 fp16 values in k order (off: 1024 even k, 64 odd k)
TM_DEV float sumoff8_h(u4_t v) {
  const h2_t off = {(half_t)1024.0f, (half_t)64.0f};
  float a = 0.0f;
  a = __builtin_amdgcn_fdot2(as_h2(v.x), off, a, false);
  a = __builtin_amdgcn_fdot2(as_h2(v.y), off, a, false);
  a = __builtin_amdgcn_fdot2(as_h2(v.z), off, a, false);
  a = __builtin_amdgcn_fdot2(as_h2(v.w), off, a, false);
  return a;
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
TM_DEV float sum16(float v) { return row16_sum(v); }

// bias[n] in the activation dtype (fp16 / bf16), 0 without a bias
TM_DEV float bias_at(const uint16_t* bias, int n, bool bf16) {
  if (!bias) return 0.0f;
  return bf16 ? bf16_bits_to_f32(bias[n]) : f16_bits_to_f32(bias[n]);
}

TM_DEV void store_out(uint16_t* Y, size_t i, float v, bool bf16) {
  Y[i] = bf16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// (The dwords go through by-value helpers: __builtin_bit_cast applied directly
// to a vector element such as v.y reads element 0 in this compiler.)
TM_DEV bf2_t as_bf2(uint32_t u) { return __builtin_bit_cast(bf2_t, u); }
TM_DEV float xsum8(u4_t v, bool bf16) {
  float a = 0.0f;
  if (bf16) {
    const bf2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(v.x), one, a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(v.y), one, a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(v.z), one, a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(v.w), one, a, false);
  } else {
    const h2_t one = {(half_t)1.0f, (half_t)1.0f};
    a = __builtin_amdgcn_fdot2(as_h2(v.x), one, a, false);
    a = __builtin_amdgcn_fdot2(as_h2(v.y), one, a, false);
    a = __builtin_amdgcn_fdot2(as_h2(v.z), one, a, false);
    a = __builtin_amdgcn_fdot2(as_h2(v.w), one, a, false);
  }
  return a;
}
}  // namespace
