// K1, the batch-1 MXFP4 GEMV kernel, shared by libhwk (mxfp4.hip) and the gfx950 code object that
// the runtime calls load (co/hwk_co.hip).
//
// Every lane of a wave reads one 32-value block of a row (16 code bytes as one 128-bit load, and its
// scale byte) per block slot, so a launch issues its whole matrix at once: one row set a wave, the
// grid as large as the matrix. Measured on MI355X, one launch over a C1 matrix (8.9 MB) reaches its
// shortest time this way, not by fewer waves with more loads each in flight. x (k fp16 values) is
// loaded before the weights, so that it arrives first, and put in LDS once for the workgroup's
// waves; a wave then reads the 32 x values of its lanes' blocks from LDS while its weight loads are
// still in flight. Codes become fp16 pairs in registers (the hardware fp4 conversion, exact at
// scale 1), multiply x in fp16 pairs with fp32 sums (v_dot2), and each block's fp32 sum takes its
// power-of-two scale (exact). The lanes' terms are summed by DPP row shifts into lane 63, which
// writes the row.
#pragma once

#include <type_traits>

#include "hwk_common.h"

// The fp32 sum of a 32-value block's codes times its x: 16 code bytes against x's 32 fp16 values.
__device__ __forceinline__ float mxfp4_block_dot(uint4 c, const uint4 (&xr)[4]) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<0>(cw[q]), h2_of_bits(xr[q].x), d0, false);
    d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<1>(cw[q]), h2_of_bits(xr[q].y), d1, false);
    d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<2>(cw[q]), h2_of_bits(xr[q].z), d0, false);
    d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<3>(cw[q]), h2_of_bits(xr[q].w), d1, false);
  }
  return d0 + d1;
}

// y (n) = W (n, nb*32) x: W rows of nb blocks (codes w (n, nb) x 16 bytes, scales e (n, nb)),
// nb <= 64*BPL, x fp16 (nb*32). W waves a workgroup, RPW consecutive rows a wave (row r0 + i), BPL
// blocks a lane (block j*64 + lane). y per MODE: fp32, fp16 (RNE of the fp32 sum) or added to fp32 y.
// Loads are issued unconditionally from clamped rows and blocks (a predicated load would make the
// compiler wait for it before issuing the next); the terms of blocks past nb are dropped and rows
// past n are not written.
template <int W, int RPW, int BPL, int MODE>
__device__ __forceinline__ void mxfp4_gemv_lds(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                               const uint4 *__restrict__ x, void *__restrict__ y, uint32_t n,
                                               uint32_t nb) {
  constexpr int NT = 64 * W;
  // x is staged in units of 16 bytes when the threads divide its 64*BPL*4 chunks, else of 4 bytes
  constexpr int XU = (64 * BPL * 4) % NT == 0 ? 16 : 4;           // bytes a unit
  constexpr int XN = (64 * BPL * 64 / XU + NT - 1) / NT;          // units a thread stages
  using XT = std::conditional_t<XU == 16, uint4, uint32_t>;
  __shared__ uint4 xs[NT * XN * XU / 16];
  const int lane = threadIdx.x & 63, t = threadIdx.x;
  const uint32_t r0 = (blockIdx.x * W + (t >> 6)) * RPW;
  constexpr bool add = MODE == HWK_OUT_ADD_F32;
  // every thread loads and writes units t, t + NT, ... of x (past x's end the last unit again, into
  // slots no lane reads): no thread loads a unit that others load too, and no write sits under a
  // branch (the compiler would sink x's load into it, behind the weight loads, and wait for those)
  const XT *xu = (const XT *)x;
  XT xv[XN];
#pragma unroll
  for (int j = 0; j < XN; j++) xv[j] = xu[min((uint32_t)(t + j * NT), nb * 64 / XU - 1)];
  // the old y of an ADD-mode call, loaded before the weights so that the sum at the end waits on
  // no load
  float yo[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) yo[i] = add ? ((const float *)y)[min(r0 + i, n - 1)] : 0.0f;
  issue_order();
  uint4 c[RPW][BPL];
  uint32_t s[RPW][BPL];
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const size_t row = min(r0 + i, n - 1);
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const size_t blk = row * nb + min((uint32_t)(j * 64 + lane), nb - 1);
      c[i][j] = load_stream(&w[blk]);
      s[i][j] = e[blk];
    }
  }
  issue_order();  // every weight load issued before the wait for x
#pragma unroll
  for (int j = 0; j < XN; j++) ((XT *)xs)[t + j * NT] = xv[j];
  __syncthreads();
  uint4 xr[BPL][4];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const uint32_t b = min((uint32_t)(j * 64 + lane), nb - 1);
#pragma unroll
    for (int q = 0; q < 4; q++) xr[j][q] = xs[b * 4 + q];
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const float term = mxfp4_block_dot(c[i][j], xr[j]) * e8m0_scale(s[i][j]);
      acc += (uint32_t)(j * 64 + lane) < nb ? term : 0.0f;
    }
    const float v = wave_sum_to_63(acc);
    const uint32_t r = r0 + i;
    if (lane == 63 && r < n) {
      if constexpr (MODE == HWK_OUT_F16)
        ((f16 *)y)[r] = (f16)f32_value(v);
      else if constexpr (add)
        ((float *)y)[r] = yo[i] + v;
      else
        ((float *)y)[r] = v;
    }
  }
}

template <int W, int RPW, int BPL, int MODE>
__global__ __launch_bounds__(64 * W) void k_mxfp4_gemv_lds(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                           const uint4 *__restrict__ x, void *__restrict__ y,
                                                           uint32_t n, uint32_t nb) {
  mxfp4_gemv_lds<W, RPW, BPL, MODE>(w, e, x, y, n, nb);
}
