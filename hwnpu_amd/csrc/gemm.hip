// Prefill / verify GEMM (K3) on gfx950: the kernels of hwk_i8_gemm and hwk_mxfp4_gemm and the choice
// of tile shape (the device code is in gemm_kernels.h).
#include "gemm_kernels.h"
#include "hwk_common.h"

namespace {

using namespace hwk_gemm;

template <int BM, int BN, bool MX, int WM, int WN, int KG>
__global__ __launch_bounds__(64 * WM * WN * KG) __attribute__((amdgpu_waves_per_eu(MX && WM * WN * KG == 4 ? 2 : 1))) void k_gemm(
    const u32x4 *__restrict__ X, const uint8_t *__restrict__ W, const uint8_t *__restrict__ E,
    const uint16_t *__restrict__ S, void *__restrict__ Y, uint32_t M, uint32_t N, uint32_t K, int mode, bool equads) {
  gemm_wg<BM, BN, MX, WM, WN, KG>(blockIdx.x, X, W, E, S, Y, M, N, K, mode, equads);
}

template <int BM, int BN, bool MX, int WM, int WN, int KG, int RS>
__global__ __launch_bounds__(64 * WM * WN * KG) void k_gemm_ring(const u32x4 *__restrict__ X, const uint8_t *__restrict__ W,
                                                              const uint8_t *__restrict__ E,
                                                              const uint16_t *__restrict__ S, void *__restrict__ Y,
                                                              uint32_t M, uint32_t N, uint32_t K, int mode,
                                                              bool equads) {
  gemm_ring_wg<BM, BN, MX, WM, WN, KG, RS>(blockIdx.x, X, W, E, S, Y, M, N, K, mode, equads);
}

// The tile shape for (m, n): the fewest rounds of workgroups over the CUs, a round weighted by the
// tile's work and its per-tile overheads (larger tiles reuse their loads more). When every tile
// gets a CU of its own, 8 waves (2 x 4, two a SIMD: one computes while the other waits) beat 4 by
// 5-12 % on the prompt's shapes; with several tiles a CU, 4-wave workgroups fill the SIMDs as well.
// An int8 tile of 2 x 2 waves can be doubled into two k groups (8 waves) instead: its SIMDs then
// split the tile's k, which lets a smaller tile use 8 waves (128 x 96 fills the 256 CUs at 512 x 6144).
struct Shape {
  int bm, bn, wm, wn, kg, rs;  // tile, waves over its rows and columns, k groups, ring depth (ring form)
};
constexpr Shape kShapes[] = {{128, 128, 2, 2, 1, 0}, {128, 96, 2, 2, 1, 0}, {128, 64, 2, 2, 1, 0}, {64, 128, 2, 2, 1, 0},
                             {128, 128, 2, 4, 1, 0}, {128, 64, 2, 4, 1, 0}, {128, 96, 2, 2, 2, 0}};
Shape pick_shape(uint32_t m, uint32_t n, int cus, bool mx) {
  Shape best = kShapes[0];
  double best_cost = 1e300;
  for (const Shape &s : kShapes) {
    if (mx && s.kg != 1) continue;
    const uint64_t tiles = (uint64_t)((m + s.bm - 1) / s.bm) * ((n + s.bn - 1) / s.bn);
    const uint64_t rounds = (tiles + cus - 1) / cus;
    const bool eight = s.wm * s.wn * s.kg == 8;
    if (eight && tiles > (uint64_t)cus) continue;
    const double cost = (double)rounds * s.bm * s.bn * (1.0 + 32.0 / s.bm + 32.0 / s.bn) * (eight ? 0.75 : 1.0);
    if (cost < best_cost) {
      best_cost = cost;
      best = s;
    }
  }
  return best;
}

// The ring form (K a multiple of 128; see gemm_kernels.h) for the tiles 128 columns wide, as 8 waves
// (2 x 4; its LDS holds one workgroup a CU), and for the int8 128 x 96 tile of two k groups. Measured
// against the register-staged form, bit for bit the same results: 1024 x 4096 x 2048 MXFP4 31.3 ->
// 28.3 us, 1024 x 12288 x 2048 82.4 -> 79.9, int8 512 x 6144 x 2048 29.9 -> 24.1; its LDS reads
// software-pipelined (over 32 weight copies, past the memory-side cache): 25.6 -> 25.1, 86.7 -> 84.9
// (SwiGLU output), 21.8 -> 21.3. The MXFP4 tiles 64 columns
// wide stay register-staged: in the ring form (2 x 4 waves, or two k groups of one wave row) the
// prompt's down and o_proj projections measured no faster alone and the prompt 1.2 % slower
// (6.42 against 6.35 ms), and so did 64-row tiles with deeper rings.
bool ring_shape(Shape &sh, bool mx) {
  if (sh.bm == 128 && sh.bn == 128) {
    sh = {128, 128, 2, 4, 1, 3};
    return true;
  }
  if (!mx && sh.bm == 128 && sh.bn == 96 && sh.kg == 2) {
    sh.rs = 3;
    return true;
  }
  return false;
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

template <bool MX>
char *launch(hipStream_t st, const void *x, const void *w, const void *e, const void *s, void *y, uint32_t m,
             uint32_t n, uint32_t k, int mode, const char *what) {
  static const int cus = device_cus();
  // the ring form needs whole 128-column steps and 4-byte aligned scale rows
  Shape sh = pick_shape(m, n, cus, MX);
  // the ring form addresses its operands by 32-bit byte offsets (under 4 GiB an operand)
  const bool small = (uint64_t)m * k * 2 < (1ull << 32) && (uint64_t)n * (MX ? k / 2 : k) < (1ull << 32);
  const bool ring = k % 128 == 0 && (!MX || hwk::aligned(e, 4)) && small && ring_shape(sh, MX);
  const uint32_t tiles = ((m + sh.bm - 1) / sh.bm) * ((n + sh.bn - 1) / sh.bn);
  const bool equads = MX && (k / 32) % 16 == 0 && hwk::aligned(e, 16);
  const dim3 grid(tiles);
  const u32x4 *X = (const u32x4 *)x;
  const uint8_t *W = (const uint8_t *)w, *E = (const uint8_t *)e;
  const uint16_t *S = (const uint16_t *)s;
#define HWK_RING_IF(BMv, BNv, WMv, WNv, KGv, RSv)                                                              \
  if (sh.bm == BMv && sh.bn == BNv && sh.wm == WMv && sh.wn == WNv && sh.kg == KGv && sh.rs == RSv)               \
    hipLaunchKernelGGL((k_gemm_ring<BMv, BNv, MX, WMv, WNv, KGv, RSv>), grid, dim3(64 * WMv * WNv * KGv), 0, st, X, W, \
                       E, S, y, m, n, k, mode, equads);                                                           \
  else
  if (ring) {
    HWK_RING_IF(128, 128, 2, 4, 1, 3)
    if constexpr (!MX) {
      HWK_RING_IF(128, 96, 2, 2, 2, 3)
      HWK_CHECK(false, "%s: no ring kernel for the %dx%d tile", what, sh.bm, sh.bn);
    } else {
      HWK_CHECK(false, "%s: no ring kernel for the %dx%d tile", what, sh.bm, sh.bn);
    }
    return hwk::launched(what);
  }
#undef HWK_RING_IF
#define HWK_GEMM_IF(BMv, BNv, WMv, WNv, KGv)                                                                   \
  if (sh.bm == BMv && sh.bn == BNv && sh.wm == WMv && sh.wn == WNv && sh.kg == KGv)                               \
    hipLaunchKernelGGL((k_gemm<BMv, BNv, MX, WMv, WNv, KGv>), grid, dim3(64 * WMv * WNv * KGv), 0, st, X, W, E, S, \
                       y, m, n, k, mode, equads);                                                                 \
  else
  HWK_GEMM_IF(128, 128, 2, 2, 1)
  HWK_GEMM_IF(128, 96, 2, 2, 1)
  HWK_GEMM_IF(128, 64, 2, 2, 1)
  HWK_GEMM_IF(64, 128, 2, 2, 1)
  HWK_GEMM_IF(128, 128, 2, 4, 1)
  HWK_GEMM_IF(128, 64, 2, 4, 1)
  if constexpr (!MX) {
    HWK_GEMM_IF(128, 96, 2, 2, 2)
    HWK_CHECK(false, "%s: no kernel for the %dx%d tile", what, sh.bm, sh.bn);
  } else {
    HWK_CHECK(false, "%s: no kernel for the %dx%d tile", what, sh.bm, sh.bn);
  }
#undef HWK_GEMM_IF
  return hwk::launched(what);
}

}  // namespace

extern "C" {

HWK_API char *hwk_i8_gemm(void *stream, const void *x, const void *q, const void *scale16, void *y, uint32_t m,
                          uint32_t n, uint32_t k, int out_mode) {
  HWK_CHECK(x && q && scale16 && y, "hwk_i8_gemm: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_i8_gemm: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_SWIGLU_F16, "hwk_i8_gemm: out_mode %d", out_mode);
  HWK_CHECK(out_mode != HWK_OUT_SWIGLU_F16 || n % 16 == 0, "hwk_i8_gemm: SwiGLU output needs n %% 16 == 0 (n=%u)", n);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(q, 16), "hwk_i8_gemm: x and q must be 16-byte aligned");
  if (m == 0 || n == 0) return nullptr;
  return launch<false>((hipStream_t)stream, x, q, nullptr, scale16, y, m, n, k, out_mode, "hwk_i8_gemm");
}

HWK_API char *hwk_mxfp4_gemm(void *stream, const void *x, const void *w, const void *e, void *y, uint32_t m,
                             uint32_t n, uint32_t k, int out_mode) {
  HWK_CHECK(x && w && e && y, "hwk_mxfp4_gemm: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_mxfp4_gemm: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_SWIGLU_F16, "hwk_mxfp4_gemm: out_mode %d", out_mode);
  HWK_CHECK(out_mode != HWK_OUT_SWIGLU_F16 || n % 16 == 0, "hwk_mxfp4_gemm: SwiGLU output needs n %% 16 == 0 (n=%u)", n);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(w, 16), "hwk_mxfp4_gemm: x and w must be 16-byte aligned");
  if (m == 0 || n == 0) return nullptr;
  return launch<true>((hipStream_t)stream, x, w, e, nullptr, y, m, n, k, out_mode, "hwk_mxfp4_gemm");
}

}  // extern "C"
