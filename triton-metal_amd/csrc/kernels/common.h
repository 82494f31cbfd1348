// Shared device-side helpers for the gfx950 (CDNA4) kernels of this library.
//
// Everything here is written for 64-lane wavefronts and the gfx950 MFMA
// shapes v_mfma_f32_16x16x32_{f16,bf16} and v_mfma_f32_32x32x16_{f16,bf16}.
//
// MFMA operand layouts used throughout (lane l of a 64-lane wave):
//   16x16x32:  A: row l%16, k = 8*(l/16)+e (e<8)     B: col l%16, same k
//              D: col l%16, row 4*(l/16)+e (e<4)
//   32x32x16:  A: row l%32, k = 8*(l/32)+e (e<8)     B: col l%32, same k
//              D: col l%32, row 8*(e/4)+4*(l/32)+(e%4) (e<16)
// A GEMM only needs A and B to agree on the k <-> (lane, element) mapping, so
// kernels are free to feed any fixed permutation of k to both operands.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

typedef _Float16 half_t;
typedef __bf16 bf16_t;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

#define TM_DEV __device__ __forceinline__

// dtype codes shared with the C-ABI (include/tm_hip.h).
enum { TM_DT_F32 = 0, TM_DT_F16 = 1, TM_DT_BF16 = 2 };

// ---- scalar conversions -----------------------------------------------------
TM_DEV float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

typedef float f2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 / fp16 with round to nearest even (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32 on gfx950).
TM_DEV uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
TM_DEV uint16_t f32_to_f16_bits(float f) {
  half_t h = (half_t)f;
  return __builtin_bit_cast(uint16_t, h);
}
TM_DEV float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(half_t, b); }

// Two fp32 -> packed 16-bit pair (lo in bits 0..15), one instruction.
TM_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{lo, hi}, bf2_t));
}
TM_DEV uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{lo, hi}, h2_t));
}

template <int DT> TM_DEV float load_as_f32(const void* p, size_t i) {
  if constexpr (DT == TM_DT_F32) return ((const float*)p)[i];
  else if constexpr (DT == TM_DT_F16) return (float)((const half_t*)p)[i];
  else return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
template <int DT> TM_DEV void store_from_f32(void* p, size_t i, float v) {
  if constexpr (DT == TM_DT_F32) ((float*)p)[i] = v;
  else if constexpr (DT == TM_DT_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}

// Runtime-dtype element access (general / fallback kernels only).
TM_DEV float load_as_f32_rt(const void* p, long long i, int dt) {
  if (dt == TM_DT_F32) return ((const float*)p)[i];
  if (dt == TM_DT_F16) return (float)((const half_t*)p)[i];
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
TM_DEV void store_as_f32_rt(void* p, long long i, int dt, float v) {
  if (dt == TM_DT_F32) ((float*)p)[i] = v;
  else if (dt == TM_DT_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}

// ---- MFMA wrappers ------------------------------------------------------------
// The 8 x 16-bit operand of a 16x16x32 / 32x32x16 MFMA travels as 4 dwords.
template <bool BF16> TM_DEV f4_t mfma16(u4_t a, u4_t b, f4_t c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a),
                                                   __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a),
                                                  __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}
template <bool BF16> TM_DEV f16_t mfma32(u4_t a, u4_t b, f16_t c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8_t, a),
                                                   __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, a),
                                                  __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// v_mfma_f32_4x4x4_16b: 16 independent 4x4x4 blocks; block b = l / 4 takes A's
// row l % 4 and B's column l % 4 (4 x 16-bit values each) from lane l, and
// lane l receives D_b[e][l % 4] in element e.
template <bool BF16> TM_DEV f4_t mfma4x4(u2_t a, u2_t b, f4_t c) {
  typedef short s4_t __attribute__((ext_vector_type(4)));
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s4_t, a),
                                                  __builtin_bit_cast(s4_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, a),
                                              __builtin_bit_cast(h4_t, b), c, 0, 0, 0);
}

// ---- packed 16-bit helpers ---------------------------------------------------
// Byte permute: result byte i = byte sel_i of the 8-byte value {hi:lo}.
TM_DEV uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
TM_DEV h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
TM_DEV uint32_t h2_bits(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Buffer-free 16-byte global load that the compiler keeps as one dwordx4.
TM_DEV u4_t ldg128(const void* p) { return *(const u4_t*)p; }

typedef __attribute__((address_space(3))) void lds_void_t;

// Workgroup barrier for data exchanged through LDS alone: waits for this
// wave's LDS operations (lgkmcnt) and meets the other waves, without draining
// outstanding global loads, stores or global -> LDS copies as the fence of
// __syncthreads() does.  The asm's memory clobber keeps the compiler from
// moving memory accesses across it; LDS filled by global -> LDS copies needs
// the copying waves' own wait_vm before the barrier.
TM_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Byte offset of an LDS location (the address a global -> LDS copy takes).
TM_DEV uint32_t lds_off(const void* p) { return (uint32_t)(uintptr_t)(lds_void_t*)p; }

// Global -> LDS copies (global_load_lds_dwordx4 / _dword) issued in asm: lane
// l deposits its 16 (4) bytes at LDS byte offset lds + 16 l (4 l); lds must be
// wave-uniform.  The copies count in vmcnt like loads.  The compiler does not
// see them, so it adds no waits for them (with the global_load_lds builtin in
// a function, every LDS read there waits for all earlier LDS reads,
// lgkmcnt(0), instead of only for its own).  The caller waits with
// wait_vm<N>() - N = copies (and other vector memory operations) issued after
// the awaited one - before reading the data, and must not overwrite LDS that
// a copy still targets.  m0 is written here and declared clobbered, so the
// compiler keeps none of its own values in m0 across a copy.  A global load into LDS needs one wait
// state after the write of m0 it reads (an s_nop 0 between the two).
TM_DEV void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
// The same copy, non-temporal: for data read once (a weight or KV-cache
// stream), so that it does not displace what is reused from the caches.
TM_DEV void dma16_nt(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
// The same copy from a wave-uniform base plus a 32-bit byte offset per lane
// (one VGPR per copy instead of a 64-bit address pair).
TM_DEV void dma16s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
TM_DEV void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
// Wait until at most N vector memory operations of this wave are outstanding
// (they complete in issue order).
template <int N> TM_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// f(std::integral_constant<int, I>) for I = B .. E-1, unrolled with I usable
// in constant expressions.
template <int B, int E, typename F> TM_DEV void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}
TM_DEV u2_t ldg64(const void* p) { return *(const u2_t*)p; }

// A 32-bit constant the compiler must keep in a VGPR (it cannot see its value).
// With the masks of an (a & m) | o held this way, instruction selection emits a
// single v_and_or_b32 (a VOP3 form that cannot encode literals on gfx9)
// instead of separate v_and / v_or with literals.  Only a v_mov is hidden in
// the asm; every instruction that consumes the value is compiler-generated, so
// hazard tracking (e.g. VALU -> MFMA operand) stays with the compiler.
TM_DEV uint32_t vgpr_const(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

// Sum over each row of 16 lanes with DPP (all 16 lanes receive the sum).
TM_DEV float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

// A transposed butterfly step over lane bit 4 (O = 16) or 5 (O = 32) for two
// values: the lanes with the bit clear return lo summed with their partner
// lane's lo, the others hi summed with their partner's hi.  One permlane swap
// (it trades lo's upper lanes for hi's lower ones), no LDS round trip.  With
// lo == hi every lane gets the sum over the bit.
template <int O> TM_DEV float fold_swap(float lo, float hi) {
  static_assert(O == 16 || O == 32, "lane bit 4 or 5");
  const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(lo),
                                                            __float_as_uint(hi), false, false)
                         : __builtin_amdgcn_permlane32_swap(__float_as_uint(lo),
                                                            __float_as_uint(hi), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same swap for a maximum over lane bit 4 or 5 (every lane receives it).
template <int O> TM_DEV float max_swap(float v) {
  static_assert(O == 16 || O == 32, "lane bit 4 or 5");
  const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                            __float_as_uint(v), false, false)
                         : __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                            __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over lane bits 2 and 3, every lane receiving it (lanes i, i + 4, i + 8, i + 12 of a 16-lane row:
// two row rotations).
TM_DEV float sum_bits23(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
  return v;
}
// Wave-wide sum (64 lanes, every lane receives it): DPP within rows of 16,
// then the two permlane swaps.
TM_DEV float wave_sum(float v) {
  v = row16_sum(v);
  v = fold_swap<16>(v, v);
  return fold_swap<32>(v, v);
}
