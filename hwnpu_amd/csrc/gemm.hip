// Prefill / verify GEMM (K3) on gfx950: Y (M, N) = X (M, K) W^T, X fp16, W int8 per output channel
// or MXFP4, fp32 accumulation on the fp16 MFMA.
//
// A workgroup computes a 128 x 128 tile of Y with eight waves (2 x 4, 64 x 32 each, 8 MFMA
// 16x16x32 tiles a wave; two waves a SIMD). K goes 64 at a time, double-buffered in LDS: while the
// waves multiply
// one buffer, the next step's X rows and weight rows are already loading into registers; the
// weights are dequantized to fp16 on their way into LDS (int8 exactly, with the channel scale
// applied in the epilogue; MXFP4 with the hardware fp4 -> fp16 conversion, its 32-value block
// scale folded in, exact for e8m0 exponents within [-23, 13] where every code times the scale is
// an fp16 value). Tile order is XCD-aware: the workgroups that share a weight panel run on the
// same XCD, so its L2 holds the panel once.
#include "hwk_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDSK = BK + 8;  // row stride padded against bank conflicts

// 4 int8 codes (one dword) as 4 exact fp16 values (two dwords).
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const h2 bias = {(f16)1152.0f, (f16)1152.0f};
  const h2 lo = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
  const h2 hi = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

template <int SEL>
__device__ __forceinline__ uint32_t fp4x2_scaled(uint32_t w, float s) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, SEL));
}

constexpr int NT = 512;  // threads a workgroup: 8 waves, 2 a SIMD

// The step's global loads (BK = 64 values of K), held in registers until they go to LDS.
template <bool MX>
struct Stage {
  uint4 a[2];  // X: chunks t and t+512 of the 128 x 64 tile (row c/8, 8 halves at (c%8)*8)
  uint4 b;     // W int8: row t/4, 16 codes at (t%4)*16; MXFP4 (t < 256): row t/2, block t%2
  uint32_t e;  // MXFP4 scale byte of that block
};

template <bool MX>
__device__ __forceinline__ void load_stage(Stage<MX> &s, const uint4 *__restrict__ X, const uint8_t *__restrict__ W,
                                           const uint8_t *__restrict__ E, uint32_t M, uint32_t N, uint32_t K,
                                           uint32_t m0, uint32_t n0, uint32_t k0, int t) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = t + NT * i, row = c >> 3, q = c & 7;
    s.a[i] = (m0 + row < M && k0 + q * 8 < K) ? X[((size_t)(m0 + row) * K + k0) / 8 + q] : make_uint4(0, 0, 0, 0);
  }
  if constexpr (MX) {
    const uint32_t row = n0 + (t >> 1);
    const bool kin = k0 + (t & 1) * 32 < K;  // a K that is an odd multiple of 32 ends on a half step
    if (t < 256 && row < N && kin) {
      const uint32_t blk = k0 / 32 + (t & 1);
      s.b = load_stream((const uint4 *)(W + ((size_t)row * (K / 32) + blk) * 16));
      s.e = E[(size_t)row * (K / 32) + blk];
    } else {
      s.b = make_uint4(0, 0, 0, 0);
      s.e = 0;
    }
  } else {
    const uint32_t row = n0 + (t >> 2), col = k0 + (t & 3) * 16;
    s.b = (row < N && col < K) ? load_stream((const uint4 *)(W + (size_t)row * K + col)) : make_uint4(0, 0, 0, 0);
  }
}

template <bool MX>
__device__ __forceinline__ void store_stage(const Stage<MX> &s, f16 (*As)[LDSK], f16 (*Bs)[LDSK], int t) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = t + NT * i, row = c >> 3, q = c & 7;
    *(uint4 *)&As[row][q * 8] = s.a[i];
  }
  if constexpr (MX) {
    if (t < 256) {
      const int row = t >> 1, col = (t & 1) * 32;
      const float sc = e8m0_scale(s.e);
      const uint32_t cw[4] = {s.b.x, s.b.y, s.b.z, s.b.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint4 v = make_uint4(fp4x2_scaled<0>(cw[q], sc), fp4x2_scaled<1>(cw[q], sc), fp4x2_scaled<2>(cw[q], sc),
                             fp4x2_scaled<3>(cw[q], sc));
        *(uint4 *)&Bs[row][col + q * 8] = v;
      }
    }
  } else {
    const int row = t >> 2, col = (t & 3) * 16;
    const uint2 v0 = i8x4_to_f16x4(s.b.x), v1 = i8x4_to_f16x4(s.b.y);
    const uint2 v2 = i8x4_to_f16x4(s.b.z), v3 = i8x4_to_f16x4(s.b.w);
    *(uint4 *)&Bs[row][col] = make_uint4(v0.x, v0.y, v1.x, v1.y);
    *(uint4 *)&Bs[row][col + 8] = make_uint4(v2.x, v2.y, v3.x, v3.y);
  }
}

// Workgroup id -> tile: consecutive ids go round the XCDs, so ids x, x+8, x+16, ... share an XCD;
// those take the M tiles of one N panel in turn.
__device__ __forceinline__ void tile_of(uint32_t id, uint32_t mt, uint32_t nt, uint32_t &tm, uint32_t &tn) {
  const uint32_t total = mt * nt;
  const uint32_t xcd = id % 8, j = id / 8;
  uint32_t lin = id;
  if (total % 8 == 0) {
    const uint32_t per = total / 8;  // tiles an XCD runs
    lin = xcd * per + j;
  }
  tn = lin / mt;
  tm = lin % mt;
}

template <bool MX>
__global__ __launch_bounds__(NT) void k_gemm(const uint4 *__restrict__ X, const uint8_t *__restrict__ W,
                                             const uint8_t *__restrict__ E, const uint16_t *__restrict__ S,
                                             void *__restrict__ Y, uint32_t M, uint32_t N, uint32_t K, int mode) {
  __shared__ __attribute__((aligned(16))) f16 As[2][BM][LDSK];
  __shared__ __attribute__((aligned(16))) f16 Bs[2][BN][LDSK];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves of 64 x 32
  uint32_t tm, tn;
  tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;

  floatx4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};

  // K steps: LDS holds step it (being multiplied) and step it+1 (written at the end of step it from
  // registers whose global loads were issued a step earlier).
  const uint32_t steps = (K + BK - 1) / BK;
  Stage<MX> st;
  load_stage<MX>(st, X, W, E, M, N, K, m0, n0, 0, t);
  store_stage<MX>(st, As[0], Bs[0], t);
  if (steps > 1) load_stage<MX>(st, X, W, E, M, N, K, m0, n0, BK, t);
  __syncthreads();
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  for (uint32_t it = 0; it < steps; it++) {
    const int buf = it & 1;
    // both 32-wide substeps' fragments first, then the 16 MFMAs
    half8 a[2][4], b[2][2];
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
#pragma unroll
      for (int i = 0; i < 4; i++) a[kk][i] = *(const half8 *)&As[buf][wm * 64 + i * 16 + r16][kk * 32 + kq];
#pragma unroll
      for (int j = 0; j < 2; j++) b[kk][j] = *(const half8 *)&Bs[buf][wn * 32 + j * 16 + r16][kk * 32 + kq];
    }
#pragma unroll
    for (int kk = 0; kk < 2; kk++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[kk][i], b[kk][j], acc[i][j], 0, 0, 0);
    if (it + 1 < steps) {
      store_stage<MX>(st, As[buf ^ 1], Bs[buf ^ 1], t);
      if (it + 2 < steps) load_stage<MX>(st, X, W, E, M, N, K, m0, n0, (it + 2) * BK, t);
    }
    __syncthreads();
  }
  // D of tile (i, j): lane holds rows (lane/16)*4 + r, column lane%16
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const uint32_t n = n0 + wn * 32 + j * 16 + r16;
    if (n >= N) continue;
    const float sc = MX ? 1.0f : (float)__builtin_bit_cast(f16, S[n]);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (m < M) store_out(Y, (size_t)m * N + n, acc[i][j][r] * sc, mode);
      }
  }
}

}  // namespace

extern "C" {

HWK_API char *hwk_i8_gemm(void *stream, const void *x, const void *q, const void *scale16, void *y, uint32_t m,
                          uint32_t n, uint32_t k, int out_mode) {
  HWK_CHECK(x && q && scale16 && y, "hwk_i8_gemm: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_i8_gemm: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_i8_gemm: out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(q, 16), "hwk_i8_gemm: x and q must be 16-byte aligned");
  if (m == 0 || n == 0) return nullptr;
  const uint32_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  hipLaunchKernelGGL((k_gemm<false>), dim3(tiles), dim3(NT), 0, (hipStream_t)stream, (const uint4 *)x,
                     (const uint8_t *)q, nullptr, (const uint16_t *)scale16, y, m, n, k, out_mode);
  return hwk::launched("hwk_i8_gemm");
}

HWK_API char *hwk_mxfp4_gemm(void *stream, const void *x, const void *w, const void *e, void *y, uint32_t m,
                             uint32_t n, uint32_t k, int out_mode) {
  HWK_CHECK(x && w && e && y, "hwk_mxfp4_gemm: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_mxfp4_gemm: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_mxfp4_gemm: out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(w, 16), "hwk_mxfp4_gemm: x and w must be 16-byte aligned");
  if (m == 0 || n == 0) return nullptr;
  const uint32_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  hipLaunchKernelGGL((k_gemm<true>), dim3(tiles), dim3(NT), 0, (hipStream_t)stream, (const uint4 *)x,
                     (const uint8_t *)w, (const uint8_t *)e, nullptr, y, m, n, k, out_mode);
  return hwk::launched("hwk_mxfp4_gemm");
}

}  // extern "C"
