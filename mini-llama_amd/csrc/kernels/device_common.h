// Device helpers shared by the gfx950 kernels.
//
// Weight decode without integer->float converts: a 4-bit (or biased 8-bit)
// code c placed in the mantissa of an fp16 whose exponent gives a unit ulp
// is the exact value bias + c:
//   0x6400 | c        = 1024 + c   (c in bits 0..9, ulp 1 at 1024)
//   0x5400 | (c << 4) = 64 + c     (c in bits 4..7, ulp 1/16 at 64)
// so one AND-OR turns two codes of a 32-bit word into an fp16 pair. The bias
// is removed either exactly in fp16 (pre-scaled MFMA operands) or once per
// block from a precomputed sum over the activations (GEMV dot2 path).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace mlq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) {
  return __builtin_bit_cast(h2_t, v);
}
__device__ __forceinline__ uint32_t as_u32(h2_t v) {
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 += a.x*b.x + a.y*b.y (v_dot2c_f32_f16: fp16 products are exact in
// fp32).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}

// (v & mask) | bits in one VALU op: gfx950's three-input v_bitop3_b32 with
// truth table (a & b) | c. Left to itself the compiler emits a separate AND
// and OR (VOP3 takes no literals and one scalar operand); through the
// builtin the mask sits in an SGPR and the OR constant in a hoisted VGPR, and
// the instruction stays visible to the compiler's hazard tracking (an
// inline-asm version is not: it can overwrite MFMA source registers that are
// still being read).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask,
                                           uint32_t bits) {
  constexpr unsigned kAndOr = (0xF0 & 0xCC) | 0xAA;  // f(a, b, c) = (a & b) | c
  return __builtin_amdgcn_bitop3_b32(v, mask, bits, kAndOr);
}

// q4 word -> four fp16 pairs (elements 0-1, 2-3, 4-5, 6-7 of the word's 8),
// biased by 1024 (pairs 0, 2) and 64 (pairs 1, 3).
struct Q4Pairs {
  uint32_t p0, p1, p2, p3;
};
__device__ __forceinline__ Q4Pairs q4_pairs(uint32_t v) {
  const uint32_t s = v >> 8;
  Q4Pairs p;
  p.p0 = and_or(v, 0x000F000Fu, 0x64006400u);
  p.p1 = and_or(v, 0x00F000F0u, 0x54005400u);
  p.p2 = and_or(s, 0x000F000Fu, 0x64006400u);
  p.p3 = and_or(s, 0x00F000F0u, 0x54005400u);
  return p;
}

// q8 word (codes q+128) -> two fp16 pairs (elements 0-1, 2-3), biased by
// 1024 + 128 relative to q. One v_perm_b32 per pair: the pair's two code
// bytes (bytes 0 and 2, or 1 and 3) become the low bytes of two halves
// whose high bytes are 0x64 (selector 4 picks a byte of the 0x64646464
// operand). The AND-OR form needs a shift for the second pair: 3 VALU per
// word instead of 2 (measured 2 % fewer cycles per stage in the prefill
// GEMM, same bits).
__device__ __forceinline__ void q8_pairs(uint32_t v, uint32_t& p0, uint32_t& p1) {
  p0 = __builtin_amdgcn_perm(0x64646464u, v, 0x04020400u);
  p1 = __builtin_amdgcn_perm(0x64646464u, v, 0x04030401u);
}

// Buffer resources: a scalar base address plus a byte range. A load whose
// offset lies past the range returns zeros without touching memory, which
// lets kernels read ragged tails (and skip whole groups) with no branches.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw (untyped, stride 0) buffer: word 3 selects 32-bit dword data.
constexpr int kRawBufferFlags = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)bytes, kRawBufferFlags);
}
__device__ __forceinline__ uint4 buf_load16(rsrc_t r, uint32_t voff,
                                            uint32_t soff) {
  return __builtin_bit_cast(
      uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
// Cache-policy bits of a buffer load: NT marks data read once (weight lines
// streamed by the decode kernels), so the caches do not keep it at the
// expense of reused data (activations). Measured 3-9% faster GEMVs on MI355X.
constexpr int kLoadNonTemporal = 2;
__device__ __forceinline__ uint4 buf_load16_stream(rsrc_t r, uint32_t voff,
                                                   uint32_t soff) {
  return __builtin_bit_cast(
      uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff,
                                                   kLoadNonTemporal));
}
__device__ __forceinline__ uint2 buf_load8(rsrc_t r, uint32_t voff,
                                           uint32_t soff) {
  return __builtin_bit_cast(
      uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t voff,
                                              uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

// 32-bit store through a buffer resource: offsets past the range are
// dropped (no write, no fault).
__device__ __forceinline__ void buf_store4(float v, rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)voff, (int)soff,
                                        0);
}

// Two fp32 -> packed fp16 pair (round to nearest even).
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  h2_t h;
  h.x = (_Float16)a;
  h.y = (_Float16)b;
  return as_u32(h);
}

// Power-of-two exponent that scales a set of values whose largest magnitude
// is amax into [2^14, 2^15): amax * 2^e lies there (amax zero or not finite:
// e = 0, values pass through and inf / NaN propagate). fp16 copies (and fp16
// hi/lo pairs) of x * 2^e then hold any finite fp32 activations without
// overflow, with the fp16 subnormal floor 2^-39 below the largest element;
// the fp32 results are scaled back by 2^-e (exact: ldexp).
__device__ __forceinline__ int pow2_scale_exp(float amax) {
  if (!(amax > 0.0f) || !(amax <= 3.402823466e38f)) return 0;
  return 15 - __builtin_amdgcn_frexp_expf(amax);
}
__device__ __forceinline__ float ldexp_f(float v, int e) { return __builtin_amdgcn_ldexpf(v, e); }
__device__ __forceinline__ float abs_max4(float m, float4 v) {
  return fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Largest of a non-negative value over the 64 lanes of a wave, wave-uniform
// (a scalar register): DPP within each 16-lane row, then the four row
// results on the scalar unit, compared as integers (non-negative floats
// order like their bit patterns). No LDS round trips, unlike shuffles.
__device__ __forceinline__ float wave_max_nonneg(float v) {
  int b = __builtin_bit_cast(int, v);
  b = max(b, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  b = max(b, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  b = max(b, __builtin_amdgcn_mov_dpp(b, 0x124, 0xF, 0xF, false));  // row_ror:4
  b = max(b, __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false));  // row_ror:8
  const int r = max(max(__builtin_amdgcn_readlane(b, 0), __builtin_amdgcn_readlane(b, 16)),
                    max(__builtin_amdgcn_readlane(b, 32), __builtin_amdgcn_readlane(b, 48)));
  return __builtin_bit_cast(float, r);
}

// Bitwise OR over the 64 lanes of a wave, wave-uniform: DPP within each
// 16-lane row, then the four row results on the scalar unit.
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
  int b = (int)v;
  b |= __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  b |= __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  b |= __builtin_amdgcn_mov_dpp(b, 0x124, 0xF, 0xF, false);  // row_ror:4
  b |= __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false);  // row_ror:8
  return (uint32_t)(__builtin_amdgcn_readlane(b, 0) | __builtin_amdgcn_readlane(b, 16) |
                    __builtin_amdgcn_readlane(b, 32) | __builtin_amdgcn_readlane(b, 48));
}

// Sum / max over the 64 lanes of a wave (every lane gets the result).
// ---- cross-lane reductions without LDS round trips -------------------------
// Within a 16-lane row: DPP (xor 1 and xor 2 as quad permutes, then
// row_half_mirror, lane i <-> 7 - i, pairing the two quads of 8 lanes, and
// row_mirror, i <-> 15 - i, pairing the two halves). Across rows: gfx950's
// v_permlane16_swap (rows 0 <-> 1, 2 <-> 3) and v_permlane32_swap (lanes
// 0..31 <-> 32..63) on two copies of the value, whose two results are the
// pair's low and high member in every lane. Every step combines the same
// two values in every lane of a group, so all lanes end with bit-identical
// results (a rotation would pair them in another order per lane).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppRor8 = 0x128;       // row_ror:8 = xor 8 within a row
struct LanePair {
  float lo, hi;
};
__device__ __forceinline__ LanePair xor16_pair(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ LanePair xor32_pair(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ float xor16_sum(float v) {
  const LanePair p = xor16_pair(v);
  return p.lo + p.hi;
}
__device__ __forceinline__ float xor32_sum(float v) {
  const LanePair p = xor32_pair(v);
  return p.lo + p.hi;
}
__device__ __forceinline__ float xor16_max(float v) {
  const LanePair p = xor16_pair(v);
  return fmaxf(p.lo, p.hi);
}
__device__ __forceinline__ float xor32_max(float v) {
  const LanePair p = xor32_pair(v);
  return fmaxf(p.lo, p.hi);
}
// Over the N-lane groups (N = 2 .. 64) of the wave; every lane of a group
// ends with the group's result.
template <int N>
__device__ __forceinline__ float row_sum(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "row_sum width");
  v += dpp<kDppXor1>(v);
  if constexpr (N >= 4) v += dpp<kDppXor2>(v);
  if constexpr (N >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp<kDppMirror>(v);
  if constexpr (N >= 32) v = xor16_sum(v);
  if constexpr (N >= 64) v = xor32_sum(v);
  return v;
}
template <int N>
__device__ __forceinline__ float row_max(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "row_max width");
  v = fmaxf(v, dpp<kDppXor1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<kDppXor2>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<kDppHalfMirror>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<kDppMirror>(v));
  if constexpr (N >= 32) v = xor16_max(v);
  if constexpr (N >= 64) v = xor32_max(v);
  return v;
}
__device__ __forceinline__ float wave_sum(float v) { return row_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return row_max<64>(v); }

// ---- output epilogue (Epilogue, kEpi* in launch.h) ---------------------------
// silu in fp32 with the hardware exp (v_exp_f32 on g * log2(e)): within a
// few ulp of g / (1 + expf(-g))
__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }
// output column of gate row `row` (row % 16 < 8) under kEpiSwiGLU
__device__ __forceinline__ int glu_col(int row) { return (row >> 4) * 8 + (row & 7); }
__device__ __forceinline__ float add_bias(const Epilogue& e, float v, int row) {
  return e.bias != nullptr ? v + e.bias[row] : v;
}

}  // namespace mlq
