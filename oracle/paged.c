/* Chunk attention and the Flash-Decoding merge on the CPU, restated from
 * internal/llm/paged/paged.go:70-310, internal/llm/decode/decode.go:1435-1483 and the milcpu
 * evaluation of the chunk program (internal/milcpu/ops.go: matmul through sgemm, exp through
 * f32.Exp). Test infrastructure only (see oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* internal/f32/f32.go:46-66: Cephes expf (a published method: S. L. Moshier, Cephes Math
 * Library), the exp milcpu evaluates */
static float cephes_exp(float x) {
  if (x != x) return x;
  x = x < -86.6f ? -86.6f : x;
  x = x > 88.72283f ? 88.72283f : x;
  const float log2e = 1.44269504088896341f, c1 = 0.693359375f, c2 = -2.12194440e-4f;
  float n = (float)floor((double)(x * log2e + 0.5f));
  float r = x - n * c1 - n * c2;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  float y = p * r * r + r + 1;
  uint32_t bits = (uint32_t)((int32_t)n + 126) << 23;
  float f;
  memcpy(&f, &bits, 4);
  return (y + y) * f;
}

struct or_merge {
  int rows, dim;
  float *acc, *top, *sum;
};

/* paged.go:236-240 (NewMerge) */
or_merge *or_merge_new(int rows, int dim) {
  or_merge *c = calloc(1, sizeof(*c));
  c->rows = rows;
  c->dim = dim;
  c->acc = calloc((size_t)rows * dim, sizeof(float));
  c->top = calloc((size_t)rows, sizeof(float));
  c->sum = calloc((size_t)rows, sizeof(float));
  or_merge_reset(c);
  return c;
}

void or_merge_free(or_merge *c) {
  if (!c) return;
  free(c->acc);
  free(c->top);
  free(c->sum);
  free(c);
}

/* paged.go:243-249 */
void or_merge_reset(or_merge *c) {
  memset(c->acc, 0, sizeof(float) * (size_t)c->rows * c->dim);
  memset(c->sum, 0, sizeof(float) * (size_t)c->rows);
  for (int i = 0; i < c->rows; i++) c->top[i] = -INFINITY;
}

/* paged.go:255-279 (Add): a row with l <= 0 is skipped; a larger m rescales what came before */
void or_merge_add(or_merge *c, const float *o, const float *m, const float *l) {
  for (int r = 0; r < c->rows; r++) {
    if (l[r] <= 0) continue;
    float mj = m[r];
    float *row = c->acc + (size_t)r * c->dim;
    if (mj > c->top[r]) {
      if (c->sum[r] > 0) {
        float f = (float)exp((double)(c->top[r] - mj));
        c->sum[r] *= f;
        for (int i = 0; i < c->dim; i++) row[i] *= f;
      }
      c->top[r] = mj;
    }
    float w = l[r] * (float)exp((double)(mj - c->top[r]));
    c->sum[r] += w;
    const float *oj = o + (size_t)r * c->dim;
    for (int i = 0; i < c->dim; i++) row[i] += w * oj[i];
  }
}

/* paged.go:284-299 (AddSink) */
void or_merge_add_sink(or_merge *c, const float *sinks, int tokens) {
  for (int r = 0; r < c->rows; r++) {
    float mj = sinks[r / tokens];
    if (mj > c->top[r]) {
      if (c->sum[r] > 0) {
        float f = (float)exp((double)(c->top[r] - mj));
        c->sum[r] *= f;
        float *row = c->acc + (size_t)r * c->dim;
        for (int i = 0; i < c->dim; i++) row[i] *= f;
      }
      c->top[r] = mj;
    }
    c->sum[r] += (float)exp((double)(mj - c->top[r]));
  }
}

/* paged.go:302-310 (Result) */
void or_merge_result(or_merge *c, float *out) {
  for (int r = 0; r < c->rows; r++) {
    float inv = 0;
    if (c->sum[r] > 0) inv = 1 / c->sum[r];
    for (int i = 0; i < c->dim; i++) out[(size_t)r * c->dim + i] = c->acc[(size_t)r * c->dim + i] * inv;
  }
}

/* paged.go:70-203, the grouped form as milcpu evaluates it, in fp32: s = (q.k^T)*scale + mask;
 * m = rowmax; e = exp(s - m); l = sum e; o = ((e * (1024/l)) . v) * (1/1024). The scale is a
 * parameter here (the program stores 1/sqrt(d) as an fp16 constant; the GPU path takes the
 * fp32 value the caller passes, and so does this restatement). */
void or_paged_chunk(const float *q, const float *k, const float *v, size_t kv_stride,
                    const float *mask, float *o, float *m, float *l, int heads, int kv_heads,
                    int tokens, int chunk, int d, float scale) {
  const float out_scale = 1024.0f, inv_scale = 1.0f / 1024.0f; /* paged.go:48 (OutScale) */
  int rep = heads / kv_heads;
  float *s = malloc(sizeof(float) * (size_t)chunk);
  for (int h = 0; h < heads; h++) {
    const float *kh = k + (size_t)(h / rep) * kv_stride * d;
    const float *vh = v + (size_t)(h / rep) * kv_stride * d;
    for (int t = 0; t < tokens; t++) {
      const float *qr = q + ((size_t)h * tokens + t) * d;
      float top = -INFINITY;
      for (int c = 0; c < chunk; c++) {
        float dot = 0;
        for (int i = 0; i < d; i++) dot += qr[i] * kh[(size_t)c * d + i];
        float sc = dot * scale;
        if (mask) sc += mask[(size_t)t * chunk + c];
        s[c] = sc;
        top = sc > top ? sc : top;
      }
      float sum = 0;
      for (int c = 0; c < chunk; c++) {
        s[c] = cephes_exp(s[c] - top);
        sum += s[c];
      }
      float f = out_scale / sum;
      float *orow = o + ((size_t)h * tokens + t) * d;
      for (int i = 0; i < d; i++) orow[i] = 0;
      for (int c = 0; c < chunk; c++) {
        float w = s[c] * f;
        for (int i = 0; i < d; i++) orow[i] += w * vh[(size_t)c * d + i];
      }
      for (int i = 0; i < d; i++) orow[i] *= inv_scale;
      m[h * tokens + t] = top;
      l[h * tokens + t] = sum;
    }
  }
  free(s);
}

/* decode.go:1435-1483 (attend): the program per used chunk, merged in fp32. One query row per
 * head at the last position: every cached key is visible, so no chunk needs a mask. The heads
 * of one kv head are independent of the others', so the kv heads run on threads. */
void or_attn_decode(const float *q, const float *k, const float *v, float *out, int heads,
                    int kv_heads, int L, int d, float scale, int chunk, int threads) {
  if (threads <= 0) threads = or_max_threads();
  if (chunk <= 0) chunk = 8192; /* paged.go:62 (DefaultChunk) */
  int rep = heads / kv_heads;
#pragma omp parallel for schedule(static, 1) num_threads(threads)
  for (int g = 0; g < kv_heads; g++) {
    or_merge *mg = or_merge_new(rep, d);
    float *o = malloc(sizeof(float) * (size_t)rep * d);
    float m[64], l[64];
    for (int c0 = 0; c0 < L; c0 += chunk) {
      int n = L - c0 < chunk ? L - c0 : chunk;
      or_paged_chunk(q + (size_t)g * rep * d, k + ((size_t)g * L + c0) * d,
                     v + ((size_t)g * L + c0) * d, (size_t)L, NULL, o, m, l, rep, 1, 1, n, d, scale);
      or_merge_add(mg, o, m, l);
    }
    or_merge_result(mg, out + (size_t)g * rep * d);
    free(o);
    or_merge_free(mg);
  }
}
