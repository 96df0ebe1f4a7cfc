// Host-side IEEE binary16 conversions (round to nearest, ties to even).
//
// Behaviour matches the reference's FloatToHalfBitsRNE / HalfBitsToFloat
// (src/vapoursynth/hip_engine.cc:1190-1276): NaN stays a quiet NaN, overflow
// saturates to inf, subnormals are rounded correctly.
#pragma once

#include <cstdint>
#include <cstring>

namespace arthip {

inline uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
  // Below half of the smallest subnormal (2^-25): signed zero.
  if (a <= 0x33000000u) return static_cast<uint16_t>(sign);
  const int e = static_cast<int>(a >> 23) - 127;  // unbiased exponent
  uint32_t mant = (a & 0x7fffffu) | 0x800000u;     // 24-bit significand
  uint32_t bits;
  if (e < -14) {
    // Subnormal half: value = mant * 2^(e-23); half ulp is 2^-24.
    const int shift = -e - 14 + 13;  // 14..24
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    bits = q;  // may carry into the exponent field: that is the correct rounding
  } else {
    uint32_t q = mant >> 13;
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    // q in [0x400, 0x800]; exponent field e+15, carry handled by the addition
    bits = (static_cast<uint32_t>(e + 15) << 10) + (q - 0x400u);
    if (bits >= 0x7c00u) bits = 0x7c00u;  // overflow to inf
  }
  return static_cast<uint16_t>(sign | bits);
}

// fp32 -> fp16 as the reference's load-time model converter rounds
// initializers (src/vapoursynth/convert_float_to_float16.cpp:165-186): round to
// nearest even for results in the normal range, but every |x| < 2^-14 (the
// smallest normal half) becomes a signed zero instead of a subnormal, and NaN
// becomes a signed inf.
inline uint16_t f32_to_f16_no_subnormals(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u);
  if (a < 0x38800000u) return static_cast<uint16_t>(sign);  // |x| < 2^-14
  return f32_to_f16(f);
}

inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t x;
  if (e == 0x1fu) {
    x = sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u);
  } else if (e != 0) {
    x = sign | ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    x = sign;
  } else {
    int s = 0;
    while ((m & 0x400u) == 0) {
      m <<= 1;
      ++s;
    }
    x = sign | (static_cast<uint32_t>(113 - s) << 23) | ((m & 0x3ffu) << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

}  // namespace arthip
