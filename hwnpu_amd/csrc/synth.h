// Counter-based synthetic draws: element i of a stream keyed by `key` reads splitmix64's output
// at state key + (i+1)*gamma, so any element can be drawn on its own, in any order, on any thread.
#pragma once

#include "hwk_common.h"

namespace hwk {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t splitmix_at(uint64_t key, uint64_t i) {
  uint64_t z = key + (i + 1) * kGamma;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Element i of a normal stream: pair i/2 takes draws i&~1 and i|1, u = (draw >> 11) * 2^-53 in
// [0, 1); r = sqrt(-2 ln(1 - u1)), t = 2 pi u2; even elements r cos t, odd r sin t (float64).
__device__ __forceinline__ double normal_at(uint64_t key, uint64_t i) {
  uint64_t p = i & ~1ull;
  double u1 = (double)(splitmix_at(key, p) >> 11) * 0x1.0p-53;
  double u2 = (double)(splitmix_at(key, p + 1) >> 11) * 0x1.0p-53;
  double r = sqrt(-2.0 * log(1.0 - u1));
  double t = 6.283185307179586 * u2;
  return (i & 1) ? r * sin(t) : r * cos(t);
}

}  // namespace hwk
