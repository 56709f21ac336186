// The decoder's elementwise and row ops (K6), shared by their C-ABI entry points (glue.hip) and the
// Qwen3 model (qwen3.hip), so that the entry points' parity tests run the code the model runs.
//
// Numerics:
//   RMSNorm   r = float(1 / sqrt(sum(x^2) / n + eps)), the sum of squares in float64; y = (x * r) * w
//             (reference internal/llm/blocks/blocks.go:351-395)
//   RoPE      rotate_half over cat(freqs, freqs) tables: y[j] = x[j] c[j] - x[j+h] s[j] for j < h,
//             y[j+h] = x[j+h] c[j] + x[j] s[j] (blocks.go:412-445), no fused multiply-add; the per-head
//             RMSNorm before it as head_norm_rope (internal.h) computes it
//   SiLU*up   g / (1 + float(exp(-g))) * u with exp in float64 (blocks.go:395-401; the reference's
//             expert act, internal/llm/experts/host.go:45-57)
#pragma once

#include "hwk_common.h"
#include "internal.h"

namespace hwk_glue {
namespace {  // each translation unit that launches them holds its own copy

// One workgroup a row. V > 0: the row (at most 256*V values) is loaded once into registers, all of a
// thread's loads (x and w) issued before the sum; V = 0: two passes over the row. Either way thread t
// sums x[t], x[t+256], ... in that order, then the wave (DPP row shifts into lane 63) and the
// workgroup sums are added alike.
template <bool F16OUT, int V = 0>
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, double eps,
                                                 void *__restrict__ out, uint32_t n) {
#pragma clang fp contract(off)
  __shared__ double red[4];
  const int t = threadIdx.x, lane = t & 63;
  const float *xr = x + (size_t)blockIdx.x * n;
  double ss = 0.0;
  float xv[V > 0 ? V : 1], wv[V > 0 ? V : 1];
  if constexpr (V > 0) {
#pragma unroll
    for (int j = 0; j < V; j++) {
      const uint32_t i = min((uint32_t)(t + 256 * j), n - 1);  // past n: the last value again, not summed
      xv[j] = xr[i];
      wv[j] = w[i];
    }
#pragma unroll
    for (int j = 0; j < V; j++)
      if ((uint32_t)(t + 256 * j) < n) {
        const double v = (double)xv[j];
        ss += v * v;
      }
  } else {
    for (uint32_t i = t; i < n; i += 256) {
      const double v = (double)xr[i];
      ss += v * v;
    }
  }
  ss = wave_sum_f64_to_63(ss);
  if (lane == 63) red[t >> 6] = ss;
  __syncthreads();
  ss = ((red[0] + red[1]) + red[2]) + red[3];
  const float r = (float)(1.0 / sqrt(ss / (double)n + eps));
  auto put = [&](uint32_t i, float y) {
    if (F16OUT)
      ((f16 *)out)[(size_t)blockIdx.x * n + i] = (f16)y;
    else
      ((float *)out)[(size_t)blockIdx.x * n + i] = y;
  };
  if constexpr (V > 0) {
#pragma unroll
    for (int j = 0; j < V; j++) {
      const uint32_t i = t + 256 * j;
      if (i < n) put(i, f32_value((xv[j] * r) * wv[j]));
    }
  } else {
    for (uint32_t i = t; i < n; i += 256) put(i, f32_value((xr[i] * r) * w[i]));
  }
}

// One wave a row of n = 256*C values (4 rows a workgroup): lane l holds the 16-byte pieces
// j*64 + l of x and w, loaded at once; the float64 sum of squares over the wave by DPP, no LDS and no
// barrier. The numerics are k_rmsnorm's; only the order of the float64 sum differs.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
template <bool F16OUT, int C>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *__restrict__ x, const float *__restrict__ w,
                                                      double eps, void *__restrict__ out, uint32_t rows) {
#pragma clang fp contract(off)
  constexpr uint32_t n = 256 * C;
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves leave together
  const int lane = threadIdx.x & 63;
  const f32x4 *xr = (const f32x4 *)(x + (size_t)row * n), *wr = (const f32x4 *)w;
  f32x4 xv[C], wv[C];
#pragma unroll
  for (int j = 0; j < C; j++) xv[j] = xr[j * 64 + lane];
#pragma unroll
  for (int j = 0; j < C; j++) wv[j] = wr[j * 64 + lane];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < C; j++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const double v = (double)xv[j][c];
      ss += v * v;
    }
  ss = wave_sum_f64_all(ss);
  const float r = (float)(1.0 / sqrt(ss / (double)n + eps));
#pragma unroll
  for (int j = 0; j < C; j++) {
    f32x4 y;
#pragma unroll
    for (int c = 0; c < 4; c++) y[c] = f32_value((xv[j][c] * r) * wv[j][c]);
    const size_t i = (size_t)row * n / 4 + j * 64 + lane;  // 4-value piece
    if constexpr (F16OUT)
      ((f16x4 *)out)[i] = (f16x4){(f16)y[0], (f16)y[1], (f16)y[2], (f16)y[3]};
    else
      ((f32x4 *)out)[i] = y;
  }
}

// Launches the RMSNorm of rows of n values: a wave a row for n = 256, 512, 1024, 2048 or 4096 with
// 16-byte aligned rows (the 1,024-token prompt of 2,048-value rows: 6.55 -> 6.52 ms; a decode step
// unchanged), else k_rmsnorm, its one-pass form up to 4096 values a row.
template <bool F16OUT>
inline void launch_rmsnorm(hipStream_t st, const float *x, const float *w, double eps, void *out, uint32_t rows,
                           uint32_t n) {
  const bool vec = hwk::aligned(x, 16) && hwk::aligned(w, 16) && hwk::aligned(out, F16OUT ? 8 : 16);
  const dim3 g4((rows + 3) / 4);
#define HWK_RMS_ROWS(Cv)                                                                                    \
  if (vec && n == 256 * Cv) {                                                                               \
    hipLaunchKernelGGL((k_rmsnorm_rows<F16OUT, Cv>), g4, dim3(256), 0, st, x, w, eps, out, rows);          \
    return;                                                                                                 \
  }
  HWK_RMS_ROWS(1)
  HWK_RMS_ROWS(2)
  HWK_RMS_ROWS(4)
  HWK_RMS_ROWS(8)
  HWK_RMS_ROWS(16)
#undef HWK_RMS_ROWS
  const uint32_t per = (n + 255) / 256;
  if (per <= 4)
    hipLaunchKernelGGL((k_rmsnorm<F16OUT, 4>), dim3(rows), dim3(256), 0, st, x, w, eps, out, n);
  else if (per <= 8)
    hipLaunchKernelGGL((k_rmsnorm<F16OUT, 8>), dim3(rows), dim3(256), 0, st, x, w, eps, out, n);
  else if (per <= 16)
    hipLaunchKernelGGL((k_rmsnorm<F16OUT, 16>), dim3(rows), dim3(256), 0, st, x, w, eps, out, n);
  else
    hipLaunchKernelGGL((k_rmsnorm<F16OUT, 0>), dim3(rows), dim3(256), 0, st, x, w, eps, out, n);
}

// One wave a (token, head) of 128 dims: lane l holds dims l and l + 64, the pair rotate_half mixes.
// The head's RMSNorm (when nw is given) then RoPE at position pos0 + token.
template <bool F16OUT>
__global__ __launch_bounds__(256) void k_norm_rope(const float *__restrict__ x, const float *__restrict__ nw,
                                                   const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                   double eps, void *__restrict__ out, uint32_t heads, uint32_t rows,
                                                   uint32_t pos0) {
#pragma clang fp contract(off)
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves leave together
  const uint32_t l = threadIdx.x & 63, t = row / heads;
  const float *xr = x + (size_t)row * 128;
  const float y0 = xr[l], y1 = xr[l + 64];
  const size_t p = (size_t)pos0 + t;
  const float c = cos_t[p * 64 + l], s = sin_t[p * 64 + l];
  float o0, o1;
  if (nw) {
    head_norm_rope(y0, y1, nw[l], nw[l + 64], c, s, eps, o0, o1);
  } else {
    o0 = f32_value(y0 * c + (-y1) * s);
    o1 = f32_value(y1 * c + y0 * s);
  }
  if (F16OUT) {
    ((f16 *)out)[(size_t)row * 128 + l] = (f16)o0;
    ((f16 *)out)[(size_t)row * 128 + l + 64] = (f16)o1;
  } else {
    ((float *)out)[(size_t)row * 128 + l] = o0;
    ((float *)out)[(size_t)row * 128 + l + 64] = o1;
  }
}

// kc/vc (kvh, cap, dim) rows pos0 + t of k/v (T, kvh, dim), fp16, 16 bytes a thread.
__global__ __launch_bounds__(256) void k_kv_append(const uint4 *__restrict__ k, const uint4 *__restrict__ v,
                                                   uint4 *__restrict__ kc, uint4 *__restrict__ vc, uint32_t kvh,
                                                   uint32_t cap, uint32_t vecs, uint32_t pos0, uint64_t total) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const uint64_t row = i / vecs, c = i % vecs;  // row = t * kvh + head
  const uint64_t t = row / kvh, hd = row % kvh;
  const uint64_t dst = (hd * cap + pos0 + t) * vecs + c;
  kc[dst] = k[i];
  vc[dst] = v[i];
}

template <bool F16OUT>
__global__ __launch_bounds__(256) void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u,
                                                  void *__restrict__ out, uint64_t n, uint32_t stride) {
#pragma clang fp contract(off)
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float y = swiglu_value(g[i * stride], u[i * stride]);
  if (F16OUT)
    ((f16 *)out)[i] = (f16)y;
  else
    ((float *)out)[i] = y;
}

__global__ __launch_bounds__(256) void k_add(float *__restrict__ y, const float *__restrict__ x, uint64_t n) {
#pragma clang fp contract(off)
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = y[i] + x[i];
}

// out (T, hidden) fp32 = rows ids[t] of the fp16 table, ids read at (*pos when pos is given) + base + t
// (the model's token history at its device position); a row whose id is outside [0, vocab) is NaN.
__global__ __launch_bounds__(256) void k_embed_ids(const int32_t *__restrict__ ids, const int32_t *__restrict__ pos,
                                                   uint32_t base, const f16 *__restrict__ table,
                                                   float *__restrict__ out, uint32_t hidden, uint32_t vocab) {
  const uint32_t t = blockIdx.y;
  const int32_t id = ids[(pos ? (uint32_t)*pos : 0u) + base + t];
  const bool ok = id >= 0 && (uint32_t)id < vocab;
  const f16 *row = table + (size_t)(ok ? id : 0) * hidden;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < hidden; i += gridDim.x * 256)
    out[(size_t)t * hidden + i] = ok ? (float)row[i] : __builtin_nanf("");
}

// Workgroups across hidden for k_embed_ids (at most 8).
uint32_t embed_blocks(uint32_t hidden) { return (hidden + 255) / 256 < 8 ? (hidden + 255) / 256 : 8; }

}  // namespace
}  // namespace hwk_glue
