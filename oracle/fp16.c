/* fp16 conversions, restated from internal/vecops/vecops.go:297-352 (F16Bits, F16Value).
 * Test infrastructure only (see oracle.h). */
#include <string.h>

#include "oracle.h"

static uint32_t bits_of(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  return x;
}

static float float_of(uint32_t x) {
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* vecops.go:297-331: round to nearest even, overflow to infinity, NaN -> sign|0x7e00 */
uint16_t or_f16_bits(float f) {
  uint32_t x = bits_of(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  int exp = (int)((x >> 23) & 0xff) - 127 + 15;
  uint32_t mant = x & 0x7fffff;
  if (((x >> 23) & 0xff) == 0xff) {
    if (mant != 0) return sign | 0x7e00;
    return sign | 0x7c00;
  }
  if (exp >= 0x1f) return sign | 0x7c00;
  if (exp <= 0) {
    if (exp < -10) return sign;
    mant |= 0x800000;
    unsigned shift = (unsigned)(14 - exp);
    uint16_t h = (uint16_t)(mant >> shift);
    uint32_t rem = mant & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1) == 1)) h++;
    return sign | h;
  }
  uint16_t h = (uint16_t)(sign | (uint16_t)(exp << 10) | (uint16_t)(mant >> 13));
  uint32_t rem = mant & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1) == 1)) h++; /* may carry into the exponent */
  return h;
}

/* vecops.go:334-352: exact; subnormals normalized; NaN keeps its payload */
float or_f16_value(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (uint32_t)(h >> 10) & 0x1f;
  uint32_t mant = (uint32_t)(h & 0x3ff);
  if (exp == 0) {
    if (mant == 0) return float_of(sign);
    uint32_t e = 127 - 15 + 1;
    while ((mant & 0x400) == 0) {
      mant <<= 1;
      e--;
    }
    return float_of(sign | e << 23 | (mant & 0x3ff) << 13);
  }
  if (exp == 0x1f) return float_of(sign | 0xffu << 23 | mant << 13);
  return float_of(sign | (exp + 127 - 15) << 23 | mant << 13);
}

void or_f32_to_f16(uint16_t *dst, const float *src, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = or_f16_bits(src[i]);
}

void or_f16_to_f32(float *dst, const uint16_t *src, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = or_f16_value(src[i]);
}
