// The gfx950 code object libhwk's runtime calls load (hwk_module_load): kernels with C names and a
// launch manifest, built with `hipcc --genco` into lib/hwk_gfx950.hsaco. It holds
//   hwk_co_mxfp4_gemv  K1, the batch-1 MXFP4 GEMV (the same kernel as hwk_mxfp4_gemv's for rows of
//                      up to 64 blocks): y fp16 (n) = W (n, nb*32) x; rows past 64 blocks are
//                      outside this build, and such a call writes NaN to y instead of a wrong sum
//   hwk_co_stream_read a read of n16 16-byte chunks, one a lane, nothing written unless the data's
//                      XOR hits a fixed value: the time one launch takes to stream a buffer
#include "../co_manifest.h"
#include "../mxfp4_gemv.h"

extern "C" {

__attribute__((used)) __constant__ hwk_co_geometry hwk_co_manifest[2] = {
    // 8 waves of 2 rows: grid.x = ceil(n / 16), n is argument 4
    {"hwk_co_mxfp4_gemv", 512, 4, 16, 0, 0, {0, 0, 0}},
    // a lane a chunk: grid.x = ceil(n16 / 256), n16 is argument 1
    {"hwk_co_stream_read", 256, 1, 256, 0, 0, {0, 0, 0}},
};
__attribute__((used)) __constant__ uint32_t hwk_co_manifest_count = 2;

__global__ __launch_bounds__(512) void hwk_co_mxfp4_gemv(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                         const uint4 *__restrict__ x, f16 *__restrict__ y, uint32_t n,
                                                         uint32_t nb) {
  if (n == 0) return;        // nothing to read (the runtime launches no grid for n = 0)
  if (nb == 0 || nb > 64) {  // uniform: the whole grid takes this branch
    const uint32_t r = blockIdx.x * 16 + threadIdx.x;
    if (threadIdx.x < 16 && r < n) y[r] = (f16)__builtin_nanf("");
    return;
  }
  mxfp4_gemv_lds<8, 2, 1, HWK_OUT_F16>(w, e, x, y, n, nb);
}

__global__ __launch_bounds__(256) void hwk_co_stream_read(const uint4 *__restrict__ p, uint32_t n16,
                                                          uint32_t *__restrict__ sink) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (n16 == 0) return;
  const uint4 v = load_stream(&p[min(i, n16 - 1)]);
  const uint32_t a = v.x ^ v.y ^ v.z ^ v.w;
  if (a == 0x9e3779b9u && i < n16) sink[blockIdx.x] = a;
}

}  // extern "C"
