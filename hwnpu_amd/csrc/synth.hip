// Synthetic inputs drawn on the device from counter-based splitmix64 streams, so that the
// model's 1.4G weights and 311M embedding values are made in place without host copies, and any
// element can be re-drawn on the host to check them.
#include "synth.h"

namespace {

__global__ void k_bytes(uint8_t *__restrict__ out, uint64_t n, uint64_t key) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (uint8_t)hwk::splitmix_at(key, i);
}

__global__ void k_uniform(void *__restrict__ out, uint64_t n, uint64_t key, int32_t lo, uint32_t span, int elem) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t top = hwk::splitmix_at(key, i) >> 32;
  const int32_t v = lo + (int32_t)((top * span) >> 32);
  if (elem == 1) ((int8_t *)out)[i] = (int8_t)v;
  else ((int32_t *)out)[i] = v;
}

__global__ void k_normal(void *__restrict__ out, uint64_t n, uint64_t key, float stdv, int f16out) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = (float)(hwk::normal_at(key, i) * (double)stdv);
  if (f16out) ((f16 *)out)[i] = (f16)v;
  else ((float *)out)[i] = v;
}

uint32_t grid_of(uint64_t n) { return (uint32_t)((n + 255) / 256); }

// The reference's synthetic tensors (internal/llm/synth.go:17-35): seed = FNV-64a(name), then per
// element seed = seed * A + C (Knuth's MMIX LCG) and v = float32(int64(seed >> 40) - 2^23) / 2^23 *
// float32(0.2), uniform in [-0.2, 0.2) (the comment there says +-0.1; the code is followed). A thread
// takes kRefRun consecutive elements: it jumps the
// generator to its first element by composing the affine step with itself (binary powers), then
// steps sequentially.
constexpr uint64_t kLcgA = 6364136223846793005ull, kLcgC = 1442695040888963407ull;
constexpr uint32_t kRefRun = 64;

__global__ void k_synth_ref(void *__restrict__ out, uint64_t n, uint64_t seed, int f16out) {
#pragma clang fp contract(off)
  const uint64_t i0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * kRefRun;
  if (i0 >= n) return;
  // (a, c) = the step applied i0 times: x -> a x + c
  uint64_t a = 1, c = 0, pa = kLcgA, pc = kLcgC;
  for (uint64_t k = i0; k; k >>= 1) {
    if (k & 1) {
      c = pa * c + pc;
      a = pa * a;
    }
    pc = pa * pc + pc;
    pa = pa * pa;
  }
  uint64_t s = a * seed + c;
  const uint64_t end = i0 + kRefRun < n ? i0 + kRefRun : n;
  for (uint64_t i = i0; i < end; i++) {
    s = s * kLcgA + kLcgC;
    const float v = (float)((int64_t)(s >> 40) - (1 << 23)) / 8388608.0f * 0.2f;
    if (f16out) ((f16 *)out)[i] = (f16)f32_value(v);
    else ((float *)out)[i] = v;
  }
}

}  // namespace

extern "C" {

HWK_API char *hwk_synth_bytes(void *stream, void *out, uint64_t n, uint64_t key) {
  HWK_CHECK(out, "hwk_synth_bytes: null pointer");
  HWK_CHECK(n < (1ull << 38), "hwk_synth_bytes: n=%llu too large", (unsigned long long)n);
  if (n == 0) return nullptr;
  hipLaunchKernelGGL(k_bytes, dim3(grid_of(n)), dim3(256), 0, (hipStream_t)stream, (uint8_t *)out, n, key);
  return hwk::launched("hwk_synth_bytes");
}

HWK_API char *hwk_synth_uniform(void *stream, void *out, uint64_t n, uint64_t key, int32_t lo, uint32_t span,
                                int elem_size) {
  HWK_CHECK(out, "hwk_synth_uniform: null pointer");
  HWK_CHECK(elem_size == 1 || elem_size == 4, "hwk_synth_uniform: elem_size %d is not 1 or 4", elem_size);
  HWK_CHECK(span > 0, "hwk_synth_uniform: empty span");
  HWK_CHECK(elem_size == 4 || (lo >= -128 && (int64_t)lo + span - 1 <= 127), "hwk_synth_uniform: range past int8");
  HWK_CHECK(n < (1ull << 38), "hwk_synth_uniform: n too large");
  HWK_CHECK(elem_size == 1 || hwk::aligned(out, 4), "hwk_synth_uniform: out misaligned");
  if (n == 0) return nullptr;
  hipLaunchKernelGGL(k_uniform, dim3(grid_of(n)), dim3(256), 0, (hipStream_t)stream, out, n, key, lo, span,
                     elem_size);
  return hwk::launched("hwk_synth_uniform");
}

HWK_API char *hwk_synth_normal(void *stream, void *out, uint64_t n, uint64_t key, uint32_t std_bits, int out_f16) {
  HWK_CHECK(out, "hwk_synth_normal: null pointer");
  HWK_CHECK(hwk::aligned(out, out_f16 ? 2 : 4), "hwk_synth_normal: out misaligned");
  HWK_CHECK(n < (1ull << 38), "hwk_synth_normal: n too large");
  if (n == 0) return nullptr;
  hipLaunchKernelGGL(k_normal, dim3(grid_of(n)), dim3(256), 0, (hipStream_t)stream, out, n, key,
                     hwk::f32_of_bits(std_bits), out_f16);
  return hwk::launched("hwk_synth_normal");
}

HWK_API char *hwk_synth_reference(void *stream, void *out, uint64_t n, const char *name, int out_f16) {
  HWK_CHECK(out && name, "hwk_synth_reference: null pointer");
  HWK_CHECK(hwk::aligned(out, out_f16 ? 2 : 4), "hwk_synth_reference: out misaligned");
  HWK_CHECK(n < (1ull << 38), "hwk_synth_reference: n too large");
  if (n == 0) return nullptr;
  uint64_t h = 0xCBF29CE484222325ull;  // FNV-64a (Go hash/fnv New64a)
  for (const unsigned char *q = (const unsigned char *)name; *q; q++) {
    h ^= *q;
    h *= 0x100000001B3ull;
  }
  const uint64_t threads = (n + kRefRun - 1) / kRefRun;
  hipLaunchKernelGGL(k_synth_ref, dim3(grid_of(threads)), dim3(256), 0, (hipStream_t)stream, out, n, h, out_f16);
  return hwk::launched("hwk_synth_reference");
}

}  // extern "C"
