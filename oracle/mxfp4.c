/* MXFP4 on the CPU, restated from internal/mxfp4/mxfp4.go, encode.go and matvec.go.
 * Test infrastructure only (see oracle.h). */
#include <float.h>
#include <math.h>
#include <string.h>

#include "oracle.h"

enum { BLOCK = 32, CHUNK = 32 };

/* mxfp4.go:17: e2m1's values by their 4 bits (code 8 is -0) */
static const float values[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                 -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
/* mxfp4.go:20: the values doubled, integers */
static const int8_t doubled[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

float or_mxfp4_value(int code) { return values[code & 15]; }

/* mxfp4.go:77: Float32frombits(e << 23): e=0 gives +0, e=255 gives +Inf */
float or_mxfp4_scale(uint8_t e) {
  uint32_t x = (uint32_t)e << 23;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* mxfp4.go:120-128: the even value in the low nibble */
void or_mxfp4_dequantize(float *dst, const uint8_t *w, const uint8_t *e, size_t nb) {
  for (size_t b = 0; b < nb; b++) {
    float s = or_mxfp4_scale(e[b]);
    const uint8_t *blk = w + 16 * b;
    for (int j = 0; j < 16; j++) {
      dst[b * BLOCK + 2 * j] = values[blk[j] & 15] * s;
      dst[b * BLOCK + 2 * j + 1] = values[blk[j] >> 4] * s;
    }
  }
}

void or_mxfp4_dequantize_rows(float *dst, const uint8_t *w, const uint8_t *e, size_t rows,
                              size_t nb, int threads) {
  if (threads <= 0) threads = or_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
  for (size_t r = 0; r < rows; r++)
    or_mxfp4_dequantize(dst + r * nb * BLOCK, w + r * nb * 16, e + r * nb, nb);
}

/* encode.go:62-78: nearest e2m1 code, clipped to +-6, halfway to the even code, 0 as +0 */
uint8_t or_mxfp4_nearest(double x) {
  uint8_t sign = 0;
  if (x < 0) {
    sign = 8;
    x = -x;
  }
  uint8_t c = 7;
  for (uint8_t k = 0; k < 7; k++) {
    double mid = (double)(values[k] + values[k + 1]) / 2;
    if (x < mid || (x == mid && k % 2 == 0)) {
      c = k;
      break;
    }
    if (x == mid) {
      c = k + 1;
      break;
    }
  }
  if (c == 0) return 0;
  return sign | c;
}

/* encode.go:11-59: per block the least-squared-error scale among OCP's rule and its neighbours */
void or_mxfp4_encode(uint8_t *w, uint8_t *e, const float *row, size_t n) {
  uint8_t codes[BLOCK];
  for (size_t b = 0; b < n / BLOCK; b++) {
    const float *blk = row + b * BLOCK;
    float m = 0;
    for (int j = 0; j < BLOCK; j++) {
      float a = (float)fabs((double)blk[j]);
      m = a > m ? a : m; /* Go's max(m, a) with m >= 0 and no NaN input */
    }
    uint8_t best = 0;
    double best_err = INFINITY;
    if (m > 0) {
      int exp;
      frexp((double)m, &exp); /* m = f 2^exp, f in [0.5, 1) */
      int rule = exp - 1 - 2;
      for (int x = rule - 1; x <= rule + 1; x++) {
        int eb = x + 127;
        if (eb < 1 || eb > 254) continue;
        double s = (double)or_mxfp4_scale((uint8_t)eb);
        double se = 0;
        for (int j = 0; j < BLOCK; j++) {
          double v = (double)blk[j];
          double d = v - (double)values[or_mxfp4_nearest(v / s)] * s;
          se += d * d;
        }
        if (se < best_err) {
          best = (uint8_t)eb;
          best_err = se;
        }
      }
    }
    if (best == 0) {
      memset(w + 16 * b, 0, 16);
      e[b] = 0;
      continue;
    }
    double s = (double)or_mxfp4_scale(best);
    for (int j = 0; j < BLOCK; j++) codes[j] = or_mxfp4_nearest((double)blk[j] / s);
    for (int j = 0; j < BLOCK / 2; j++) w[16 * b + j] = (uint8_t)(codes[2 * j] | codes[2 * j + 1] << 4);
    e[b] = best;
  }
}

void or_mxfp4_encode_rows(uint8_t *w, uint8_t *e, const float *m, size_t rows, size_t n,
                          int threads) {
  if (threads <= 0) threads = or_max_threads();
  size_t nb = n / BLOCK;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (size_t r = 0; r < rows; r++) or_mxfp4_encode(w + r * nb * 16, e + r * nb, m + r * n, n);
}

/* mxfp4.go:33-53: int8 by blocks; a block's 16 even values then its 16 odd ones */
void or_vec_quantize(int8_t *q, float *s, const float *x, size_t n) {
  for (size_t b = 0; b < n / BLOCK; b++) {
    const float *blk = x + b * BLOCK;
    float m = 0;
    for (int j = 0; j < BLOCK; j++) {
      float a = (float)fabs((double)blk[j]);
      m = a > m ? a : m;
    }
    int8_t *qb = q + b * BLOCK;
    if (m == 0) {
      memset(qb, 0, BLOCK);
      s[b] = 0;
      continue;
    }
    float inv = 127 / m;
    for (int j = 0; j < BLOCK / 2; j++) {
      /* float32 product, then RoundToEven in float64 (math.RoundToEven) */
      float p0 = blk[2 * j] * inv, p1 = blk[2 * j + 1] * inv;
      qb[j] = (int8_t)nearbyint((double)p0);
      qb[BLOCK / 2 + j] = (int8_t)nearbyint((double)p1);
    }
    s[b] = m / 127;
  }
}

/* mxfp4.go:80-91 (dotGo, the x86 path: mxfp4_other.go:5-14) */
float or_mxfp4_dot(const uint8_t *w, const uint8_t *e, size_t nb, const int8_t *q, const float *s) {
  float sum = 0;
  for (size_t b = 0; b < nb; b++) {
    int32_t acc = 0;
    const uint8_t *blk = w + 16 * b;
    const int8_t *qb = q + b * BLOCK;
    for (int j = 0; j < 16; j++) {
      uint8_t by = blk[j];
      acc += (int32_t)doubled[by & 15] * (int32_t)qb[j] + (int32_t)doubled[by >> 4] * (int32_t)qb[16 + j];
    }
    float t = (float)acc * or_mxfp4_scale(e[b]);
    t = t * s[b];
    sum += t;
  }
  return sum / 2;
}

/* matvec.go:33-160 (Run) without the arm64 kernels: spans of CHUNK rows taken by the workers as
 * they finish one (the atomic counter there is OpenMP's dynamic schedule here); a row is read
 * once for all the vectors. */
void or_mxfp4_run(float *out, const uint8_t *w, const uint8_t *e, size_t rows, size_t nb,
                  const int8_t *q, const float *s, size_t nvec, int threads) {
  if (threads <= 0) threads = or_max_threads();
  size_t spans = (rows + CHUNK - 1) / CHUNK;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (size_t sp = 0; sp < spans; sp++) {
    size_t lo = sp * CHUNK, hi = lo + CHUNK < rows ? lo + CHUNK : rows;
    for (size_t r = lo; r < hi; r++)
      for (size_t v = 0; v < nvec; v++)
        out[v * rows + r] = or_mxfp4_dot(w + r * nb * 16, e + r * nb, nb, q + v * nb * BLOCK,
                                         s + v * nb);
  }
}
