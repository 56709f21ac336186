/* int8 per-channel weights and the int8 KV rule on the CPU.
 * Test infrastructure only (see oracle.h). */
#include <math.h>

#include "oracle.h"

/* internal/milcpu/ops.go:1589-1610 (shiftScale without offset, one scale per row): float32(q) *
 * scale, exact in float32 for int8 q and an fp16 scale */
void or_i8_dequant(float *dst, const int8_t *q, const uint16_t *scale16, size_t rows, size_t cols,
                   int threads) {
  if (threads <= 0) threads = or_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
  for (size_t r = 0; r < rows; r++) {
    float s = or_f16_value(scale16[r]);
    for (size_t c = 0; c < cols; c++) dst[r * cols + c] = (float)q[r * cols + c] * s;
  }
}

/* The int8 KV rule, per row (one KV head's key or value at one position): the scale is the row's
 * largest magnitude over 127 rounded to fp16 first, 1 for a row of zeros
 * (internal/llm/experts/weights.go:229-252), and the codes are v/scale rounded to even and
 * clamped to +-127 (internal/vecops/vecops.go:179-185). */
void or_i8_quantize_rows(int8_t *q, uint16_t *scale16, const float *x, size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; r++) {
    const float *row = x + r * cols;
    float m = 0;
    for (size_t c = 0; c < cols; c++) {
      float a = (float)fabs((double)row[c]);
      m = a > m ? a : m;
    }
    float s = m / 127;
    if (s == 0) s = 1;
    uint16_t h = or_f16_bits(s);
    s = or_f16_value(h);
    scale16[r] = h;
    for (size_t c = 0; c < cols; c++) {
      float v = (float)nearbyint((double)(row[c] / s));
      v = v < -127 ? -127 : v > 127 ? 127 : v;
      q[r * cols + c] = (int8_t)v;
    }
  }
}
