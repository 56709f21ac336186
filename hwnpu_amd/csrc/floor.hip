// The read floor (a measurement kernel, no counterpart in the reference): one launch that reads a
// buffer once in 16-byte loads and does nothing else, to show the shortest time in which a single
// launch can stream a given number of bytes from HBM on this device. The batch-1 GEMV (K1) reads its
// matrix the same way once; its time against this floor's separates the cost of the launch, ramp
// and drain of a few-MB read (which no GEMV avoids) from that of its own work.
#include "hwk_common.h"

namespace {

// Thread t of T reads 16-byte chunks t, t + T, ...: loads_per_lane (LPL) of them issued before any is
// used. The chunks are folded together and a value that the data never gives in practice is the
// only one written, so the loads stay and the kernel writes nothing.
template <int LPL>
__global__ __launch_bounds__(256) void k_read_floor(const u32x4 *__restrict__ src, uint64_t chunks,
                                                    uint32_t *__restrict__ out) {
  const uint64_t T = (uint64_t)gridDim.x * 256;
  uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; c + (LPL - 1) * T < chunks; c += LPL * T) {
    u32x4 v[LPL];
#pragma unroll
    for (int j = 0; j < LPL; j++) v[j] = __builtin_nontemporal_load(&src[c + j * T]);
#pragma unroll
    for (int j = 0; j < LPL; j++) acc ^= v[j];
  }
  for (; c < chunks; c += T) acc ^= src[c];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[0] = 1u;
}

}  // namespace

extern "C" {

HWK_API char *hwk_read_floor(void *stream, const void *src, size_t bytes, uint32_t *out, uint32_t waves_per_cu,
                             uint32_t loads_per_lane) {
  HWK_CHECK(src && out, "hwk_read_floor: null pointer");
  HWK_CHECK(bytes % 16 == 0 && hwk::aligned(src, 16), "hwk_read_floor: %zu bytes: a 16-byte aligned multiple of 16",
            bytes);
  HWK_CHECK(waves_per_cu >= 1 && waves_per_cu <= 32, "hwk_read_floor: %u waves a CU (1..32)", waves_per_cu);
  int dev = 0, cus = 0;
  HWK_TRY("hipGetDevice", hipGetDevice(&dev));
  HWK_TRY("hipDeviceGetAttribute", hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const uint64_t chunks = bytes / 16;
  const uint32_t blocks = (uint32_t)((waves_per_cu * (uint64_t)cus + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  const u32x4 *s = (const u32x4 *)src;
  switch (loads_per_lane) {
    case 1: hipLaunchKernelGGL(k_read_floor<1>, dim3(blocks), dim3(256), 0, st, s, chunks, out); break;
    case 2: hipLaunchKernelGGL(k_read_floor<2>, dim3(blocks), dim3(256), 0, st, s, chunks, out); break;
    case 4: hipLaunchKernelGGL(k_read_floor<4>, dim3(blocks), dim3(256), 0, st, s, chunks, out); break;
    case 8: hipLaunchKernelGGL(k_read_floor<8>, dim3(blocks), dim3(256), 0, st, s, chunks, out); break;
    default: return hwk::errf("hwk_read_floor: %u loads a lane (1, 2, 4 or 8)", loads_per_lane);
  }
  return hwk::launched("hwk_read_floor");
}

}  // extern "C"
