/* The decoder's elementwise ops on the CPU, restated from internal/llm/blocks/blocks.go,
 * internal/llm/qwen3/{config.go,qwen3_test.go} and internal/chat/sample.go.
 * Test infrastructure only (see oracle.h). */
#include <math.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

/* Qwen3RMSNorm (qwen3_test.go:83-97, blocks.go:355-380): w * x * rsqrt(mean(x^2) + eps), here in
 * fp32 with the mean of squares accumulated in float64 and the inverse root taken in float64 (as
 * milcpu's rsqrt, internal/milcpu/ops.go:181-189) then rounded to float32; the products are
 * (x * r) * w in float32. */
void or_rmsnorm(float *out, const float *x, const float *w, int rows, int n, float eps) {
  for (int r = 0; r < rows; r++) {
    const float *xr = x + (size_t)r * n;
    double ms = 0;
    for (int j = 0; j < n; j++) ms += (double)xr[j] * (double)xr[j];
    float inv = (float)(1 / sqrt(ms / n + (double)eps));
    for (int j = 0; j < n; j++) out[(size_t)r * n + j] = (xr[j] * inv) * w[j];
  }
}

/* config.go:152-159 (RopeInvFreq) and blocks.go:412-425 (RopeValues): cat(freqs, freqs) */
void or_rope_tables(float *cos_t, float *sin_t, double theta, int start, int n, int head_dim) {
  int half = head_dim / 2;
  for (int i = 0; i < n; i++) {
    int pos = start + i;
    for (int j = 0; j < half; j++) {
      double inv = 1 / pow(theta, (double)(2 * j) / (double)head_dim);
      double a = (double)pos * inv;
      float c = (float)cos(a), s = (float)sin(a);
      cos_t[(size_t)i * head_dim + j] = c;
      cos_t[(size_t)i * head_dim + j + half] = c;
      sin_t[(size_t)i * head_dim + j] = s;
      sin_t[(size_t)i * head_dim + j + half] = s;
    }
  }
}

/* blocks.go:427-445 (ApplyRope): x*cos + rotate_half(x)*sin, rotate_half = cat(-x2, x1) */
void or_apply_rope(float *x, int heads, int head_dim, const float *cos_row, const float *sin_row) {
  int half = head_dim / 2;
  float tmp[1024];
  for (int h = 0; h < heads; h++) {
    float *v = x + (size_t)h * head_dim;
    for (int j = 0; j < head_dim; j++) {
      float rot = j < half ? -v[j + half] : v[j - half];
      tmp[j] = v[j] * cos_row[j] + rot * sin_row[j];
    }
    for (int j = 0; j < head_dim; j++) v[j] = tmp[j];
  }
}

/* blocks.go:395-401 (SiLU as x / (1 + exp(-x))) times up (qwen3 build.go mlp) */
void or_silu_mul(float *out, const float *g, const float *u, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = g[i] / (1 + (float)exp((double)(-g[i]))) * u[i];
}

/* internal/chat/sample.go:80-87: strict >, ties to the lowest index */
int32_t or_argmax(const float *x, size_t n) {
  size_t best = 0;
  for (size_t i = 0; i < n; i++)
    if (x[i] > x[best]) best = i;
  return (int32_t)best;
}

int or_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
