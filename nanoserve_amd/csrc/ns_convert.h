// Bit-exact dtype conversions for the cache writers, in integer arithmetic so
// the result does not depend on the wave's denormal mode: f16/bf16 -> f32 is
// exact, f32 -> f16/bf16 rounds to nearest even like torch's Tensor.to (NaN
// becomes a canonical quiet NaN).
#pragma once

#include "ns_common.h"

namespace ns {

__device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  if (e == 0) {
    if (m == 0) return sign;
    // Subnormal: m * 2^-24 is exactly representable as a normal f32.
    return sign | __float_as_uint(static_cast<float>(m) * 5.9604644775390625e-08f);
  }
  if (e == 31) return sign | 0x7F800000u | (m << 13);
  return sign | ((e + 112u) << 23) | (m << 13);
}

// IEEE binary32 -> binary16, round to nearest even, subnormals kept, NaN -> quiet NaN.
__device__ __forceinline__ uint32_t f32_bits_to_f16_bits(uint32_t u) {
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;            // NaN
  if (a >= 0x477FF000u) return sign | 0x7C00u;           // >= 65520 rounds to inf
  if (a >= 0x38800000u) {                                // normal f16 range (>= 2^-14)
    const uint32_t mant = a - 0x38000000u;               // rebias exponent 127 -> 15
    return sign | ((mant + 0xFFFu + ((mant >> 13) & 1u)) >> 13);
  }
  if (a <= 0x33000000u) return sign;                     // <= 2^-25 rounds to zero
  // f16 subnormal: value = q * 2^-24 with q = round(full_mantissa >> shift).
  const uint32_t e = a >> 23;                            // 102..112
  const uint32_t fm = (a & 0x7FFFFFu) | 0x800000u;
  const uint32_t rs = 126u - e;                          // 14..24
  uint32_t q = fm >> rs;
  const uint32_t rem = fm & ((1u << rs) - 1u);
  const uint32_t half = 1u << (rs - 1u);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return sign | q;
}

// IEEE binary32 -> bfloat16, round to nearest even, NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_bits_to_bf16_bits(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t load_as_f32_bits(const char* p, int dtype) {
  if (dtype == NS_DTYPE_F32) return *reinterpret_cast<const uint32_t*>(p);
  const uint32_t h = *reinterpret_cast<const uint16_t*>(p);
  return dtype == NS_DTYPE_F16 ? f16_bits_to_f32_bits(h) : (h << 16);
}

__device__ __forceinline__ uint32_t f32_bits_to(uint32_t f, int dtype) {
  if (dtype == NS_DTYPE_F32) return f;
  return dtype == NS_DTYPE_F16 ? f32_bits_to_f16_bits(f) : f32_bits_to_bf16_bits(f);
}

int dtype_size(int dtype);

}  // namespace ns
