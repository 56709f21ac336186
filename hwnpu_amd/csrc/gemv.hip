// Batch-1 GEMV over int8 per-channel weights (K2) and fp16 weights (K7, the tied head).
//
// Both stream a row once in 16-byte chunks per lane, hold x in registers across a wave's rows,
// multiply in fp16 pairs with fp32 accumulation (v_dot2) and reduce a row across its lanes. int8
// codes become fp16 exactly with the exponent trick: byte b+128 placed under exponent bits 0x64
// is the half 1024+b+128, less 1152 is b (exact for every int8).
#include "hwk_common.h"

namespace {

__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, h2 &lo, h2 &hi) {
  const uint32_t u = w ^ 0x80808080u;
  const h2 bias = {(f16)1152.0f, (f16)1152.0f};
  lo = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
  hi = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
}

// WIDE: bytes of x a chunk covers per byte of weight (2 for int8: 16 codes <-> 16 halves; 1 for
// fp16: 8 halves <-> 8 halves). LPR lanes a row, CPL chunks a lane a pass, RPW row sets a wave.
template <bool INT8, int LPR, int CPL, int RPW>
__global__ __launch_bounds__(256) void k_gemv(const uint4 *__restrict__ w, const uint16_t *__restrict__ scale16,
                                              const uint4 *__restrict__ x, void *__restrict__ y, uint32_t n,
                                              uint32_t nc, int mode) {
  constexpr int RS = 64 / LPR;
  constexpr int XQ = INT8 ? 2 : 1;  // uint4s of x a chunk multiplies
  const int lane = threadIdx.x & 63;
  const int l = lane % LPR, sub = lane / LPR;
  const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t row0 = wave * (RPW * RS) + sub;
  float acc[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) acc[i] = 0.0f;
  for (uint32_t base = 0; base < nc; base += LPR * CPL) {
    // x first, then the weights, every load issued unconditionally from a clamped row / chunk (a
    // load under a branch is waited for where the branches join); a chunk past nc is zeroed where it
    // is used, rows past n are not stored
    uint4 xr[CPL][XQ];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
      const uint32_t ch = min(base + j * LPR + l, nc - 1);
#pragma unroll
      for (int q = 0; q < XQ; q++) xr[j][q] = x[(size_t)ch * XQ + q];
    }
    issue_order();
    uint4 c[RPW][CPL];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const uint32_t r = min(row0 + i * RS, n - 1), ch = min(base + j * LPR + l, nc - 1);
        c[i][j] = load_stream(&w[(size_t)r * nc + ch]);
      }
    }
#pragma unroll
    for (int j = 0; j < CPL; j++)
      if (base + j * LPR + l >= nc) {
#pragma unroll
        for (int q = 0; q < XQ; q++) xr[j][q] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const uint32_t cw[4] = {c[i][j].x, c[i][j].y, c[i][j].z, c[i][j].w};
        if constexpr (INT8) {
          const uint32_t xw[8] = {xr[j][0].x, xr[j][0].y, xr[j][0].z, xr[j][0].w,
                                  xr[j][1].x, xr[j][1].y, xr[j][1].z, xr[j][1].w};
#pragma unroll
          for (int q = 0; q < 4; q++) {
            h2 lo, hi;
            i8x4_to_h2x2(cw[q], lo, hi);
            d0 = __builtin_amdgcn_fdot2(lo, h2_of_bits(xw[2 * q]), d0, false);
            d1 = __builtin_amdgcn_fdot2(hi, h2_of_bits(xw[2 * q + 1]), d1, false);
          }
        } else {
          const uint32_t xw[4] = {xr[j][0].x, xr[j][0].y, xr[j][0].z, xr[j][0].w};
#pragma unroll
          for (int q = 0; q < 4; q += 2) {
            d0 = __builtin_amdgcn_fdot2(h2_of_bits(cw[q]), h2_of_bits(xw[q]), d0, false);
            d1 = __builtin_amdgcn_fdot2(h2_of_bits(cw[q + 1]), h2_of_bits(xw[q + 1]), d1, false);
          }
        }
      }
      acc[i] += d0 + d1;
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    float v = group_sum<LPR>(acc[i]);
    const uint32_t r = row0 + i * RS;
    if (l == 0 && r < n) {
      if constexpr (INT8) v *= (float)__builtin_bit_cast(f16, scale16[r]);
      store_out(y, r, v, mode);
    }
  }
}

template <bool INT8, int LPR, int CPL, int RPW>
void launch(hipStream_t st, const void *w, const void *s, const void *x, void *y, uint32_t n, uint32_t nc,
            int mode) {
  constexpr uint32_t rows_per_wave = RPW * (64 / LPR);
  const uint32_t waves = (n + rows_per_wave - 1) / rows_per_wave;
  hipLaunchKernelGGL((k_gemv<INT8, LPR, CPL, RPW>), dim3((waves + 3) / 4), dim3(256), 0, st, (const uint4 *)w,
                     (const uint16_t *)s, (const uint4 *)x, y, n, nc, mode);
}

// nc chunks a row: 64 lanes over up to 4 chunks a pass; narrower rows share a wave. The fp16 head
// (151,936 rows of 256 chunks) takes 32 lanes a row, 8 chunks a lane, two rows a wave: the decode step
// 1,521-1,523 tokens/s with 64 lanes over two rows a wave, 1,528-1,530 over one, 1,532.7-1,532.9 so
// (16 lanes a row: 1,522; four or eight rows a wave of 64-lane rows: 1,497-1,517). The int8 GEMV of
// 2,048-code rows (K2, 8192 x 2048) takes two row sets a wave: 5.17 -> 4.94 µs a launch against four
// (one: 5.00-5.02; 32 lanes a row and one or two sets: 4.99-5.07; 16 lanes: 5.39).
template <bool INT8>
void dispatch(hipStream_t st, const void *w, const void *s, const void *x, void *y, uint32_t n, uint32_t nc,
              int mode) {
  if (nc >= 256 && !INT8) launch<INT8, 32, 8, 1>(st, w, s, x, y, n, nc, mode);
  else if (nc >= 256) launch<INT8, 64, 4, 2>(st, w, s, x, y, n, nc, mode);
  else if (nc > 128) launch<INT8, 64, 3, 2>(st, w, s, x, y, n, nc, mode);
  else if (nc > 64) launch<INT8, 64, 2, INT8 ? 2 : 4>(st, w, s, x, y, n, nc, mode);
  else if (nc > 32) launch<INT8, 64, 1, 4>(st, w, s, x, y, n, nc, mode);
  else if (nc > 16) launch<INT8, 32, 1, 4>(st, w, s, x, y, n, nc, mode);
  else if (nc > 8) launch<INT8, 16, 1, 4>(st, w, s, x, y, n, nc, mode);
  else launch<INT8, 8, 1, 4>(st, w, s, x, y, n, nc, mode);
}

// K7r: Y (T, n) = X W^T for fp16 W (n, k) and T <= 8 fp16 vectors X (T, k): the tied head over the
// rows of a speculative verify, each weight row read once for all T vectors. The workgroup copies X
// into LDS; a wave walks rows (grid-stride), 64 lanes over a row's 16-byte chunks, 4 chunks a lane
// a pass, and with a single pass (k <= 2048) the next row's chunks are loaded before this row's
// products.
template <int TT, bool ONEPASS>
__global__ __launch_bounds__(256) void k_f16_gemv_rows(const uint4 *__restrict__ w, const uint4 *__restrict__ x,
                                                       void *__restrict__ y, uint32_t n, uint32_t nc, int mode) {
  extern __shared__ uint4 xsr[];  // (TT, nc)
  const int lane = threadIdx.x & 63;
  const uint32_t waves = gridDim.x * 4;
  uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  // every load issued unconditionally (a chunk past nc reads the last one; dot4 skips it): a load
  // under a branch is waited for where the branches join
  auto load4 = [&](uint32_t row, uint32_t base, uint4 (&c)[4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t ch = min(base + j * 64 + lane, nc - 1);
      c[j] = load_stream(&w[(size_t)row * nc + ch]);
    }
  };
  // x's chunks (up to 8 a thread) loaded first, then the first row's weights (single pass), then x
  // written to LDS waiting on x only (past x's end the last chunk again, into its own slot)
  constexpr int XF = TT < 8 ? TT : 8;
  const uint32_t xn = TT * nc;
  uint4 xv[XF];
#pragma unroll
  for (int j = 0; j < XF; j++) xv[j] = x[min((uint32_t)(threadIdx.x + j * 256), xn - 1)];
  issue_order();
  uint4 cur[4];
  if constexpr (ONEPASS) load4(min(r, n - 1), 0, cur);
  issue_order();
#pragma unroll
  for (int j = 0; j < XF; j++) xsr[min((uint32_t)(threadIdx.x + j * 256), xn - 1)] = xv[j];
  for (uint32_t i = threadIdx.x + XF * 256; i < xn; i += 256) xsr[i] = x[i];
  __syncthreads();
  auto dot4 = [&](const uint4 (&c)[4], uint32_t base, float (&acc)[TT]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t ch = base + j * 64 + lane;
      if (ch >= nc) continue;
      const uint32_t cw[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
#pragma unroll
      for (int v = 0; v < TT; v++) {
        const uint4 xv = xsr[(size_t)v * nc + ch];
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
        float d0 = 0.0f, d1 = 0.0f;
        d0 = __builtin_amdgcn_fdot2(h2_of_bits(cw[0]), h2_of_bits(xw[0]), d0, false);
        d1 = __builtin_amdgcn_fdot2(h2_of_bits(cw[1]), h2_of_bits(xw[1]), d1, false);
        d0 = __builtin_amdgcn_fdot2(h2_of_bits(cw[2]), h2_of_bits(xw[2]), d0, false);
        d1 = __builtin_amdgcn_fdot2(h2_of_bits(cw[3]), h2_of_bits(xw[3]), d1, false);
        acc[v] += d0 + d1;
      }
    }
  };
  if (r >= n) return;
  for (; r < n; r += waves) {
    float acc[TT];
#pragma unroll
    for (int v = 0; v < TT; v++) acc[v] = 0.0f;
    if constexpr (ONEPASS) {
      uint4 nxt[4];
      const uint32_t rn = r + waves < n ? r + waves : r;
      load4(rn, 0, nxt);
      dot4(cur, 0, acc);
#pragma unroll
      for (int j = 0; j < 4; j++) cur[j] = nxt[j];
    } else {
      for (uint32_t base = 0; base < nc; base += 256) {
        uint4 c[4];
        load4(r, base, c);
        dot4(c, base, acc);
      }
    }
#pragma unroll
    for (int v = 0; v < TT; v++) {
      const float s = group_sum<64>(acc[v]);
      if (lane == 0) store_out(y, (size_t)v * n + r, s, mode);
    }
  }
}

template <int TT>
void launch_f16_rows(hipStream_t st, const void *w, const void *x, void *y, uint32_t n, uint32_t nc, int mode) {
  const uint32_t blocks = (n + 3) / 4 < 1024u ? (n + 3) / 4 : 1024u;
  const size_t lds = (size_t)TT * nc * 16;
  if (nc <= 256)
    hipLaunchKernelGGL((k_f16_gemv_rows<TT, true>), dim3(blocks), dim3(256), lds, st, (const uint4 *)w,
                       (const uint4 *)x, y, n, nc, mode);
  else
    hipLaunchKernelGGL((k_f16_gemv_rows<TT, false>), dim3(blocks), dim3(256), lds, st, (const uint4 *)w,
                       (const uint4 *)x, y, n, nc, mode);
}

}  // namespace

extern "C" {

HWK_API char *hwk_f16_gemv_rows(void *stream, const void *w, const void *x, void *y, uint32_t n, uint32_t k,
                                uint32_t tokens, int out_mode) {
  HWK_CHECK(w && x && y, "hwk_f16_gemv_rows: null pointer");
  HWK_CHECK(k % 8 == 0 && k > 0, "hwk_f16_gemv_rows: k=%u is not a positive multiple of 8", k);
  HWK_CHECK(tokens >= 1 && tokens <= 8, "hwk_f16_gemv_rows: %u vectors (1..8)", tokens);
  HWK_CHECK((size_t)tokens * k * 2 <= 64 * 1024, "hwk_f16_gemv_rows: %u x %u fp16 vectors exceed 64 KB", tokens, k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_f16_gemv_rows: out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(w, 16) && hwk::aligned(x, 16), "hwk_f16_gemv_rows: w and x must be 16-byte aligned");
  HWK_CHECK(hwk::aligned(y, out_mode == HWK_OUT_F16 ? 2 : 4), "hwk_f16_gemv_rows: y misaligned");
  if (n == 0) return nullptr;
  hipStream_t st = (hipStream_t)stream;
  const uint32_t nc = k / 8;
  switch (tokens) {
    case 1: launch_f16_rows<1>(st, w, x, y, n, nc, out_mode); break;
    case 2: launch_f16_rows<2>(st, w, x, y, n, nc, out_mode); break;
    case 3: launch_f16_rows<3>(st, w, x, y, n, nc, out_mode); break;
    case 4: launch_f16_rows<4>(st, w, x, y, n, nc, out_mode); break;
    case 5: launch_f16_rows<5>(st, w, x, y, n, nc, out_mode); break;
    case 6: launch_f16_rows<6>(st, w, x, y, n, nc, out_mode); break;
    case 7: launch_f16_rows<7>(st, w, x, y, n, nc, out_mode); break;
    default: launch_f16_rows<8>(st, w, x, y, n, nc, out_mode); break;
  }
  return hwk::launched("hwk_f16_gemv_rows");
}

HWK_API char *hwk_i8_gemv(void *stream, const void *q, const void *scale16, const void *x, void *y, uint32_t n,
                          uint32_t k, int out_mode) {
  HWK_CHECK(q && scale16 && x && y, "hwk_i8_gemv: null pointer");
  HWK_CHECK(k % 16 == 0 && k > 0, "hwk_i8_gemv: k=%u is not a positive multiple of 16", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_i8_gemv: unknown out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(q, 16) && hwk::aligned(x, 16), "hwk_i8_gemv: q and x must be 16-byte aligned");
  HWK_CHECK(hwk::aligned(scale16, 2) && hwk::aligned(y, out_mode == HWK_OUT_F16 ? 2 : 4), "hwk_i8_gemv: misaligned");
  if (n == 0) return nullptr;
  dispatch<true>((hipStream_t)stream, q, scale16, x, y, n, k / 16, out_mode);
  return hwk::launched("hwk_i8_gemv");
}

HWK_API char *hwk_f16_gemv(void *stream, const void *w, const void *x, void *y, uint32_t n, uint32_t k,
                           int out_mode) {
  HWK_CHECK(w && x && y, "hwk_f16_gemv: null pointer");
  HWK_CHECK(k % 8 == 0 && k > 0, "hwk_f16_gemv: k=%u is not a positive multiple of 8", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_f16_gemv: unknown out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(w, 16) && hwk::aligned(x, 16), "hwk_f16_gemv: w and x must be 16-byte aligned");
  HWK_CHECK(hwk::aligned(y, out_mode == HWK_OUT_F16 ? 2 : 4), "hwk_f16_gemv: y misaligned");
  if (n == 0) return nullptr;
  dispatch<false>((hipStream_t)stream, w, nullptr, x, y, n, k / 8, out_mode);
  return hwk::launched("hwk_f16_gemv");
}

}  // extern "C"
