// q8_0 quantization of fp32 activations with the reference's quantizeToQ80
// rules (src/quant.cc:130-190), shared by the GGUF-block quantizer
// (repack.hip) and the int8 GEMM's fragment-order quantizer (gemm_i8.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlq {

// fp32 -> fp16 bits as the reference's floatToFp16 (src/quant.cc:32-70)
// rounds: the 23-bit mantissa is cut to 10 bits after adding one unit at
// the first dropped bit (bit 12) when that bit is set (ties and above go up,
// lower bits ignored), a carry out of the mantissa bumps the exponent;
// exponents below the fp16 subnormal range give signed zero, above it (inf
// and NaN included) signed infinity.
__device__ __forceinline__ uint32_t fp16_bits_ref(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (b >> 16) & 0x8000u;
  int e = (int)((b >> 23) & 0xffu) - 112;  // exponent rebiased 127 -> 15
  uint32_t man = b & 0x7fffffu;
  if (e <= 0) {
    if (e < -10) return sign;
    uint32_t s = (man | 0x800000u) >> (1 - e);  // implicit bit made explicit
    s += (s & 0x1000u) << 1;
    return sign | (s >> 13);
  }
  if (e >= 31) return sign | 0x7c00u;
  man += (man & 0x1000u) << 1;
  if (man & 0x800000u) {
    man = 0;
    if (++e >= 31) return sign | 0x7c00u;
  }
  return sign | ((uint32_t)e << 10) | (man >> 13);
}

// Sixteen lanes per 32-element block, two elements each.
constexpr int kActLanes = 16;

// One block quantized by an aligned group of kActLanes lanes: each lane
// passes its two elements (0 for padding past the row) and gets the block's
// fp16 scale bits and its two codes. Every lane of the group must call it
// (the block maximum is a shuffle reduction).
struct Q8Codes {
  uint32_t dbits;
  int q0, q1;
};
__device__ __forceinline__ Q8Codes q8_block_codes(float v0, float v1) {
  // a NaN never becomes the maximum (the reference's strict-greater scan)
  float amax = fmaxf(fmaxf(0.0f, fabsf(v0)), fabsf(v1));
#pragma unroll
  for (int o = 1; o < kActLanes; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kActLanes));
  Q8Codes c = {0u, 0, 0};
  if (amax > 0.0f) {
    c.dbits = fp16_bits_ref(amax / 127.0f);
    const float ds = (float)__builtin_bit_cast(_Float16, (uint16_t)c.dbits);
    const float inv = ds == 0.0f ? 0.0f : 1.0f / ds;
    // round half away from zero, clamp to +-127; a value no int holds
    // (NaN, or inf * 0 under an infinite scale) takes the x86 conversion's
    // INT_MIN the reference compiles to, i.e. -127 after the clamp
    auto code = [&](float v) {
      const float q = v * inv;
      const int qi = fabsf(q) < 2147483648.0f ? (int)roundf(q) : -127;
      return qi > 127 ? 127 : (qi < -127 ? -127 : qi);
    };
    c.q0 = code(v0);
    c.q1 = code(v1);
  }
  return c;
}

}  // namespace mlq
