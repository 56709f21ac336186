/* MoE routing and experts on the CPU, restated from internal/llm/experts/weights.go:33-81
 * (Routing.Choose) and internal/llm/experts/host.go:478-579,723-882 (Host.runRow, Host.Run).
 * Test infrastructure only (see oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* weights.go:33-81. Scores in float32 (exp in float64 rounded to float32, a sequential float32
 * sum, a float32 divide), a stable sort descending (ties keep the lower index first), the chosen
 * scores over their float32 sum plus 1e-6 when norm. */
void or_choose(const float *logits, const float *bias, int n, int k, int score, int norm,
               double scale, int32_t *idx, float *w) {
  float *sc = malloc(sizeof(float) * n), *key = sc;
  int *order = malloc(sizeof(int) * n);
  if (score == 0) {
    float m = -INFINITY;
    for (int e = 0; e < n; e++) m = logits[e] > m ? logits[e] : m;
    float sum = 0;
    for (int e = 0; e < n; e++) {
      sc[e] = (float)exp((double)(logits[e] - m));
      sum += sc[e];
    }
    for (int e = 0; e < n; e++) sc[e] /= sum;
  } else {
    for (int e = 0; e < n; e++) sc[e] = 1 / (1 + (float)exp((double)(-logits[e])));
  }
  if (bias) {
    key = malloc(sizeof(float) * n);
    for (int e = 0; e < n; e++) key[e] = sc[e] + bias[e];
  }
  /* sort.SliceStable with a[i] before a[j] when key[a[i]] > key[a[j]]: insertion sort is stable */
  for (int e = 0; e < n; e++) order[e] = e;
  for (int i = 1; i < n; i++) {
    int v = order[i], j = i;
    while (j > 0 && key[v] > key[order[j - 1]]) {
      order[j] = order[j - 1];
      j--;
    }
    order[j] = v;
  }
  float sum = 0;
  for (int j = 0; j < k; j++) {
    idx[j] = order[j];
    w[j] = sc[order[j]];
    sum += w[j];
  }
  for (int j = 0; j < k; j++) {
    if (norm) w[j] /= sum + 1e-6f;
    if (scale != 0) w[j] *= (float)scale;
  }
  if (key != sc) free(key);
  free(sc);
  free(order);
}

/* The gated unit (host.go:516-527): SiLU g/(1+e^-g)*u, or gpt-oss's: g = min(g, limit),
 * u = clamp(u, -limit, limit), g/(1+e^(-alpha*g))*(u+1); exp in float64 rounded to float32, every
 * other step a float32 operation (Go evaluates left to right, no fused multiply-add on amd64). */
static float act_unit(float g, float u, int act, float alpha, float limit) {
  if (act == 1) {
    g = g < limit ? g : limit;
    u = u > -limit ? u : -limit;
    u = u < limit ? u : limit;
    float ag = alpha * g;
    return g / (1 + (float)exp((double)(-ag))) * (u + 1);
  }
  return g / (1 + (float)exp((double)(-g))) * u;
}

/* The experts each row chose, run once for all the rows that chose them (host.go:769-773), added
 * to the rows' outputs in ascending expert id (host.go:566-578, :866-881 walks experts by id). */
static void experts_common(int quantized, const float *x, int T, const int32_t *idx,
                           const float *w, int k, const uint8_t *gu_w, const uint8_t *gu_e,
                           const float *gu_b, const uint8_t *dn_w, const uint8_t *dn_e,
                           const float *dn_b, int E, int H, int I, int act_kind, float alpha,
                           float limit, float *out, int threads) {
  if (threads <= 0) threads = or_max_threads();
  size_t gb = (size_t)2 * I * H / 2, ge = (size_t)2 * I * H / 32; /* an expert's gate_up bytes */
  size_t db = (size_t)H * I / 2, de = (size_t)H * I / 32;
  int nbG = H / 32, nbD = I / 32;
  float *gu = malloc(sizeof(float) * 2 * I);
  float *act = malloc(sizeof(float) * I);
  const int actk = act_kind;
  float *y = malloc(sizeof(float) * H);
  float *rowbuf = malloc(sizeof(float) * (size_t)(H > I ? H : I));
  int8_t *qx = malloc((size_t)H), *qa = malloc((size_t)I);
  float *sx = malloc(sizeof(float) * nbG), *sa = malloc(sizeof(float) * nbD);
  for (int e = 0; e < E; e++) {
    for (int t = 0; t < T; t++) {
      int kk = -1;
      for (int j = 0; j < k; j++)
        if (idx[t * k + j] == e) kk = j;
      if (kk < 0) continue;
      const uint8_t *gw = gu_w + e * gb, *gs = gu_e + e * ge;
      const uint8_t *dw = dn_w + e * db, *ds = dn_e + e * de;
      const float *xr = x + (size_t)t * H;
      if (quantized) {
        or_vec_quantize(qx, sx, xr, H);
        or_mxfp4_run(gu, gw, gs, 2 * I, nbG, qx, sx, 1, threads);
      } else {
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int r = 0; r < 2 * I; r++) {
          float wr[8192];
          or_mxfp4_dequantize(wr, gw + (size_t)r * nbG * 16, gs + (size_t)r * nbG, nbG);
          float acc = 0;
          for (int c = 0; c < H; c++) acc += wr[c] * xr[c];
          gu[r] = acc;
        }
      }
      if (gu_b) /* host.go:505-512: the bias after the product */
        for (int r = 0; r < 2 * I; r++) gu[r] += gu_b[(size_t)e * 2 * I + r];
      for (int j = 0; j < I; j++) /* gate the even rows */
        act[j] = act_unit(gu[2 * j], gu[2 * j + 1], actk, alpha, limit);
      if (quantized) {
        or_vec_quantize(qa, sa, act, I);
        or_mxfp4_run(y, dw, ds, H, nbD, qa, sa, 1, threads);
      } else {
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int r = 0; r < H; r++) {
          float wr[8192];
          or_mxfp4_dequantize(wr, dw + (size_t)r * nbD * 16, ds + (size_t)r * nbD, nbD);
          float acc = 0;
          for (int c = 0; c < I; c++) acc += wr[c] * act[c];
          y[r] = acc;
        }
      }
      float wt = w[t * k + kk];
      float *o = out + (size_t)t * H;
      const float *b = dn_b ? dn_b + (size_t)e * H : NULL;
      for (int c = 0; c < H; c++) o[c] += wt * (y[c] + (b ? b[c] : 0.0f)); /* host.go:570-577 */
    }
  }
  free(gu);
  free(act);
  free(y);
  free(rowbuf);
  free(qx);
  free(qa);
  free(sx);
  free(sa);
}

void or_experts_f32(const float *x, int T, const int32_t *idx, const float *w, int k,
                    const uint8_t *gu_w, const uint8_t *gu_e, const float *gu_b,
                    const uint8_t *dn_w, const uint8_t *dn_e, const float *dn_b, int E, int H,
                    int I, int act, float alpha, float limit, float *out, int threads) {
  experts_common(0, x, T, idx, w, k, gu_w, gu_e, gu_b, dn_w, dn_e, dn_b, E, H, I, act, alpha,
                 limit, out, threads);
}

void or_experts_host(const float *x, int T, const int32_t *idx, const float *w, int k,
                     const uint8_t *gu_w, const uint8_t *gu_e, const float *gu_b,
                     const uint8_t *dn_w, const uint8_t *dn_e, const float *dn_b, int E, int H,
                     int I, int act, float alpha, float limit, float *out, int threads) {
  experts_common(1, x, T, idx, w, k, gu_w, gu_e, gu_b, dn_w, dn_e, dn_b, E, H, I, act, alpha,
                 limit, out, threads);
}
