// half_bits.h -- host-side 16-bit rounding by integer arithmetic.
//
// The storage formats' rounding rules (src/shaders.rs:27-179, src/half16.rs):
// f16 is IEEE binary16 round-to-nearest-even, bf16 is
// (u + 0x7FFF + ((u >> 16) & 1)) >> 16.  Host code computes them on the f32
// bits rather than with a `(_Float16)` cast: compiled as HIP at -O3, clang
// folds `(_Float16)(float)x` for a double x into one double -> half
// conversion, which rounds an f32 value that lies exactly halfway between two
// f16 values away from the even one whenever x itself is slightly above the
// halfway point (seen in the RoPE tables: cos(11.50136...) -> f32 0.48449707
// = 1984.5 * 2^-12 rounded to 1985 * 2^-12).  Integer code has no such
// latitude.  Device code keeps v_cvt_f16_f32, which rounds its f32 operand.
#pragma once

#include <stdint.h>
#include <string.h>

namespace qa_half {

inline uint32_t f32_bits(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return u;
}

// f32 -> f16 bits, IEEE round to nearest even (subnormals, overflow to
// infinity, NaN kept quiet).
inline uint16_t f16_from_f32(float v) {
  const uint32_t x = f32_bits(v);
  const uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));  // quiet NaN
  if (a >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);  // >= 2^16: infinity
  if (a < 0x33000000u) return (uint16_t)sign;                // <= 2^-25 (ties to 0)
  const int e = (int)(a >> 23) - 127;                        // -25 .. 15
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;         // 24 significant bits
  const int shift = e < -14 ? 13 + (-14 - e) : 13;           // subnormal: fewer bits kept
  uint32_t r = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (r & 1u))) ++r;
  if (e < -14) return (uint16_t)(sign | r);  // r == 0x400 encodes the smallest normal
  // r in [0x400, 0x800]; a carry to 0x800 steps the exponent (to infinity at 15)
  return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) + (r - 0x400u));
}

// f16 bits -> f32 (exact).
inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0x1f) {
    u = sign | 0x7f800000u | (m << 13);
  } else if (e != 0) {
    u = sign | ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    u = sign;
  } else {  // subnormal: normalise
    int k = 0;
    uint32_t mm = m;
    while (!(mm & 0x400u)) {
      mm <<= 1;
      ++k;
    }
    u = sign | ((uint32_t)(113 - k) << 23) | ((mm & 0x3ffu) << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// f32 -> bf16 bits, the reference's rule (src/shaders.rs:169-179).
inline uint16_t bf16_from_f32(float v) {
  const uint32_t u = f32_bits(v);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

inline float bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace qa_half
