// IEEE binary16 <-> binary32 conversions for host code (bit-exact, round to
// nearest even). f16 -> f32 follows the decode in
// apps/seeker-cli/src/commands/run.rs:4115-4129 (subnormal = mant * 2^-24).
#pragma once
#include <cstdint>
#include <cstring>

static inline float sh_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F;
  uint32_t mant = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      // subnormal: renormalise
      int e = -1;
      do { mant <<= 1; ++e; } while (!(mant & 0x400));
      mant &= 0x3FF;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
    }
  } else if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

static inline uint16_t sh_f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000;
  uint32_t absx = x & 0x7FFFFFFF;
  if (absx >= 0x7F800000) {  // inf / nan
    return (uint16_t)(sign | 0x7C00 | (absx > 0x7F800000 ? 0x200 : 0));
  }
  if (absx >= 0x477FF000) return (uint16_t)(sign | 0x7C00);  // rounds to inf
  if (absx < 0x38800000) {  // result is subnormal or zero
    if (absx < 0x33000000) return (uint16_t)sign;  // < 2^-25 -> 0 (ties at 2^-25 handled below)
    uint32_t e = absx >> 23;
    uint32_t m = (absx & 0x7FFFFF) | 0x800000;
    uint32_t shift = 126 - e;  // 14 + (113 - e)
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = (absx - 0x38000000) >> 13;  // rebias exponent, truncate mantissa
  uint32_t rem = absx & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) ++q;
  return (uint16_t)(sign | q);
}
