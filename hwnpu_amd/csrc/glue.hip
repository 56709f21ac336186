// The decoder's small ops as C-ABI entry points (K6): RMSNorm, the per-head norm + RoPE, KV append,
// SiLU(gate)*up, the residual add, the embedding gather and the greedy argmax. Their kernels (but the
// argmax's) are the model's own (glue_kernels.h): the decode step's prompt path, final norm and
// embedding launch them, and its attention prologue computes the per-head norm + RoPE with the same
// function. The argmax: strict > from index 0 (internal/chat/sample.go:80-87), the lowest index of
// the largest value; NaNs never win except at index 0, where the reference keeps it.
#include <math.h>

#include "glue_kernels.h"
#include "hwk_common.h"

namespace {

using namespace hwk_glue;

constexpr uint32_t kArgParts = 64;  // workgroups a row

__device__ __forceinline__ void arg_better(float &bv, uint32_t &bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// Pass 1: workgroup (part, row) takes a contiguous share of the row; its best (value, index) goes
// to the workspace.
__global__ __launch_bounds__(256) void k_argmax_part(const float *__restrict__ x, uint64_t n,
                                                     float *__restrict__ part_v, uint32_t *__restrict__ part_i) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  const uint32_t t = threadIdx.x, lane = t & 63;
  const uint64_t per = (n + kArgParts - 1) / kArgParts;
  const uint64_t lo = blockIdx.x * per, hi = lo + per < n ? lo + per : n;
  const float *xr = x + (size_t)blockIdx.y * n;
  float bv = -__builtin_inff();
  uint32_t bi = 0xffffffffu;
  for (uint64_t i = lo + t; i < hi; i += 256) arg_better(bv, bi, xr[i], (uint32_t)i);
  wave_best(bv, bi);
  if (lane == 0) {
    sv[t >> 6] = bv;
    si[t >> 6] = bi;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < 4; w++) arg_better(bv, bi, sv[w], si[w]);
    part_v[(size_t)blockIdx.y * kArgParts + blockIdx.x] = bv;
    part_i[(size_t)blockIdx.y * kArgParts + blockIdx.x] = bi;
  }
}

// Pass 2: one wave a row over its kArgParts partials.
__global__ __launch_bounds__(64) void k_argmax_final(const float *__restrict__ x, uint64_t n,
                                                     const float *__restrict__ part_v,
                                                     const uint32_t *__restrict__ part_i, int32_t *__restrict__ out) {
  const uint32_t lane = threadIdx.x, row = blockIdx.x;
  float bv = part_v[(size_t)row * kArgParts + lane];
  uint32_t bi = part_i[(size_t)row * kArgParts + lane];
  wave_best(bv, bi);
  if (lane == 0) {
    const float x0 = x[(size_t)row * n];
    out[row] = (x0 != x0 || bi == 0xffffffffu) ? 0 : (int32_t)bi;
  }
}

uint32_t blocks_of(uint64_t n) { return (uint32_t)((n + 255) / 256); }

}  // namespace

extern "C" {

HWK_API char *hwk_rope_tables(uint64_t theta_bits, uint32_t start, uint32_t n, uint32_t head_dim, float *cos_out,
                              float *sin_out) {
  HWK_CHECK(cos_out && sin_out, "hwk_rope_tables: null output");
  HWK_CHECK(head_dim >= 2 && head_dim % 2 == 0, "hwk_rope_tables: head_dim %u is not even", head_dim);
  double theta;
  memcpy(&theta, &theta_bits, 8);
  HWK_CHECK(theta > 1.0 && isfinite(theta), "hwk_rope_tables: theta %g", theta);
  const uint32_t half = head_dim / 2;
  for (uint32_t i = 0; i < n; i++)
    for (uint32_t j = 0; j < half; j++) {
      const double inv = 1.0 / pow(theta, (double)(2 * j) / (double)head_dim);
      const double a = (double)(start + i) * inv;
      cos_out[(size_t)i * half + j] = (float)cos(a);
      sin_out[(size_t)i * half + j] = (float)sin(a);
    }
  return nullptr;
}

HWK_API char *hwk_rmsnorm(void *stream, const void *x, const void *w, void *out, uint32_t rows, uint32_t n,
                          uint64_t eps_bits, int out_mode) {
  HWK_CHECK((x && out) || rows == 0, "hwk_rmsnorm: null pointer");
  HWK_CHECK(w, "hwk_rmsnorm: null weights");
  HWK_CHECK(out_mode == HWK_OUT_F32 || out_mode == HWK_OUT_F16, "hwk_rmsnorm: out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(x, 4) && hwk::aligned(w, 4) && hwk::aligned(out, out_mode == HWK_OUT_F16 ? 2 : 4),
            "hwk_rmsnorm: misaligned pointer");
  double eps;
  memcpy(&eps, &eps_bits, 8);
  HWK_CHECK(eps >= 0.0 && isfinite(eps), "hwk_rmsnorm: eps %g", eps);
  HWK_CHECK(n > 0 || rows == 0, "hwk_rmsnorm: rows of 0 values");
  if (rows == 0) return nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (out_mode == HWK_OUT_F16)
    launch_rmsnorm<true>(st, (const float *)x, (const float *)w, eps, out, rows, n);
  else
    launch_rmsnorm<false>(st, (const float *)x, (const float *)w, eps, out, rows, n);
  return hwk::launched("hwk_rmsnorm");
}

HWK_API char *hwk_rope(void *stream, const void *x, const void *norm_w, const void *cos_t, const void *sin_t,
                       void *out, uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t pos0,
                       uint32_t table_rows, uint64_t eps_bits, int out_mode) {
  HWK_CHECK(((x && out) || (uint64_t)tokens * heads == 0) && cos_t && sin_t, "hwk_rope: null pointer");
  HWK_CHECK(head_dim == 128, "hwk_rope: head_dim %u (128 only)", head_dim);
  HWK_CHECK(out_mode == HWK_OUT_F32 || out_mode == HWK_OUT_F16, "hwk_rope: out_mode %d", out_mode);
  HWK_CHECK((uint64_t)pos0 + tokens <= table_rows, "hwk_rope: positions %u..%u past the %u table rows", pos0,
            pos0 + tokens, table_rows);
  double eps;
  memcpy(&eps, &eps_bits, 8);
  HWK_CHECK(!norm_w || (eps >= 0.0 && isfinite(eps)), "hwk_rope: eps %g", eps);
  const uint64_t rows = (uint64_t)tokens * heads;
  HWK_CHECK(rows < (1ull << 31), "hwk_rope: %llu rows", (unsigned long long)rows);
  if (rows == 0) return nullptr;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((uint32_t)((rows + 3) / 4));
  if (out_mode == HWK_OUT_F16)
    hipLaunchKernelGGL(k_norm_rope<true>, grid, dim3(256), 0, st, (const float *)x, (const float *)norm_w,
                       (const float *)cos_t, (const float *)sin_t, eps, out, heads, (uint32_t)rows, pos0);
  else
    hipLaunchKernelGGL(k_norm_rope<false>, grid, dim3(256), 0, st, (const float *)x, (const float *)norm_w,
                       (const float *)cos_t, (const float *)sin_t, eps, out, heads, (uint32_t)rows, pos0);
  return hwk::launched("hwk_rope");
}

HWK_API char *hwk_kv_append(void *stream, const void *k, const void *v, void *k_cache, void *v_cache, uint32_t tokens,
                            uint32_t kv_heads, uint32_t head_dim, uint32_t capacity, uint32_t pos0) {
  HWK_CHECK((k && v) || tokens == 0, "hwk_kv_append: null pointer");
  HWK_CHECK(k_cache && v_cache, "hwk_kv_append: null cache");
  HWK_CHECK(head_dim % 8 == 0 && head_dim > 0, "hwk_kv_append: head_dim %u is not a multiple of 8", head_dim);
  HWK_CHECK((uint64_t)pos0 + tokens <= capacity, "hwk_kv_append: rows %u..%u past capacity %u", pos0, pos0 + tokens,
            capacity);
  const uint64_t total = (uint64_t)tokens * kv_heads * (head_dim / 8);
  if (total == 0) return nullptr;  // nothing to write: k and v may be NULL
  HWK_CHECK(hwk::aligned(k, 16) && hwk::aligned(v, 16) && hwk::aligned(k_cache, 16) && hwk::aligned(v_cache, 16),
            "hwk_kv_append: pointers must be 16-byte aligned");
  hipLaunchKernelGGL(k_kv_append, dim3(blocks_of(total)), dim3(256), 0, (hipStream_t)stream, (const uint4 *)k,
                     (const uint4 *)v, (uint4 *)k_cache, (uint4 *)v_cache, kv_heads, capacity, head_dim / 8, pos0,
                     total);
  return hwk::launched("hwk_kv_append");
}

HWK_API char *hwk_silu_mul(void *stream, const void *gate, const void *up, void *out, uint64_t n, uint32_t stride,
                           int out_mode) {
  HWK_CHECK((gate && up && out) || n == 0, "hwk_silu_mul: null pointer");
  HWK_CHECK(stride >= 1, "hwk_silu_mul: stride 0");
  HWK_CHECK(out_mode == HWK_OUT_F32 || out_mode == HWK_OUT_F16, "hwk_silu_mul: out_mode %d", out_mode);
  if (n == 0) return nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (out_mode == HWK_OUT_F16)
    hipLaunchKernelGGL(k_silu_mul<true>, dim3(blocks_of(n)), dim3(256), 0, st, (const float *)gate, (const float *)up,
                       out, n, stride);
  else
    hipLaunchKernelGGL(k_silu_mul<false>, dim3(blocks_of(n)), dim3(256), 0, st, (const float *)gate,
                       (const float *)up, out, n, stride);
  return hwk::launched("hwk_silu_mul");
}

HWK_API char *hwk_add(void *stream, void *y, const void *x, uint64_t n) {
  HWK_CHECK((y && x) || n == 0, "hwk_add: null pointer");
  if (n == 0) return nullptr;
  hipLaunchKernelGGL(k_add, dim3(blocks_of(n)), dim3(256), 0, (hipStream_t)stream, (float *)y, (const float *)x, n);
  return hwk::launched("hwk_add");
}

HWK_API char *hwk_embed(void *stream, const void *table, const void *ids, void *out, uint32_t tokens, uint32_t hidden,
                        uint32_t vocab) {
  HWK_CHECK(table && ((ids && out) || tokens == 0), "hwk_embed: null pointer");
  HWK_CHECK(vocab > 0 && hidden > 0, "hwk_embed: empty table");
  HWK_CHECK(tokens <= 65535, "hwk_embed: %u tokens (at most 65535)", tokens);
  if (tokens == 0) return nullptr;
  hipLaunchKernelGGL(k_embed_ids, dim3(embed_blocks(hidden), tokens), dim3(256), 0, (hipStream_t)stream,
                     (const int32_t *)ids, nullptr, 0u, (const f16 *)table, (float *)out, hidden, vocab);
  return hwk::launched("hwk_embed");
}

HWK_API size_t hwk_argmax_workspace_bytes(uint32_t rows) { return (size_t)rows * kArgParts * 8; }

HWK_API char *hwk_argmax(void *stream, const void *x, void *out, uint32_t rows, uint64_t n, void *workspace,
                         size_t workspace_bytes) {
  HWK_CHECK(x && out && workspace, "hwk_argmax: null pointer");
  HWK_CHECK(n > 0 && n < 0xffffffffull, "hwk_argmax: %llu values a row (1 .. 2^32 - 2)", (unsigned long long)n);
  HWK_CHECK(rows <= 65535, "hwk_argmax: %u rows (at most 65535)", rows);
  HWK_CHECK(workspace_bytes >= hwk_argmax_workspace_bytes(rows), "hwk_argmax: workspace %zu bytes, %zu needed",
            workspace_bytes, hwk_argmax_workspace_bytes(rows));
  HWK_CHECK(hwk::aligned(workspace, 4) && hwk::aligned(x, 4) && hwk::aligned(out, 4), "hwk_argmax: misaligned pointer");
  if (rows == 0) return nullptr;
  float *pv = (float *)workspace;
  uint32_t *pi = (uint32_t *)(pv + (size_t)rows * kArgParts);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_argmax_part, dim3(kArgParts, rows), dim3(256), 0, st, (const float *)x, n, pv, pi);
  if (char *e = hwk::launched("hwk_argmax")) return e;
  hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, st, (const float *)x, n, pv, pi, (int32_t *)out);
  return hwk::launched("hwk_argmax (final)");
}

}  // extern "C"

char *hwk::rmsnorm_f16(hipStream_t st, const float *h, const float *nw, double eps, void *out, uint32_t rows,
                       uint32_t k) {
  HWK_CHECK(h && nw && out, "rmsnorm_f16: null pointer");
  if (rows == 0 || k == 0) return nullptr;
  launch_rmsnorm<true>(st, h, nw, eps, out, rows, k);
  return hwk::launched("rmsnorm_f16");
}
