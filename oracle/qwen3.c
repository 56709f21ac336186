/* The Qwen3 decoder on the CPU, restated from the reference's float64 forward of Qwen3ForCausalLM
 * (internal/llm/qwen3/qwen3_test.go:77-207), its ops (internal/llm/blocks/blocks.go:351-445,
 * internal/llm/qwen3/config.go:152-162) and the decode session's chunked attention
 * (internal/llm/decode/decode.go:1391-1483 over internal/llm/paged/paged.go:70-310), in float32
 * with the linears through the sgemm restatement (milcpu's linear, internal/milcpu/ops.go:940),
 * rounding to fp16 where the device path stores fp16:
 *   x = f16((h * r) * w), r = float(1 / sqrt(mean(h^2) + eps)) with the mean in float64
 *   q, k = f16(rope(rmsnorm(q))), v = f16(v): the KV cache holds fp16 values
 *   attn = f16(chunk attention + merge), act = f16(silu(gate) * up)
 * and the greedy pick of internal/chat/sample.go:80-87.
 *
 * The synthetic checkpoint: each linear's values float32(N(0,1) * std) from the counter stream
 * of its Hugging Face name (splitmix64 at key + (i+1)*gamma, Box-Muller in float64; key = seed ^
 * fnv64a(name)), encoded to MXFP4 (or_mxfp4_encode) and dequantized; the embedding
 * f16(float32(N(0,1) * std)); norm weights 1. With std 0 nothing is drawn: linears and embedding
 * start at zero. or_qwen3_set then replaces any tensor by its Hugging Face name with a
 * checkpoint's values, the norm weights included (Qwen3RMSNorm's weight, applied as
 * (x * r) * w in float32: input_layernorm, post_attention_layernorm, q_norm/k_norm per head before
 * RoPE, model.norm before the head; qwen3_test.go:155-163,196,205, build.go:108,150,188,283).
 *
 * Test infrastructure only (see oracle.h). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define GAMMA 0x9E3779B97F4A7C15ull

static uint64_t splitmix_at(uint64_t key, uint64_t i) {
  uint64_t z = key + (i + 1) * GAMMA;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

double or_normal_at(uint64_t key, uint64_t i) {
  uint64_t p = i & ~1ull;
  double u1 = (double)(splitmix_at(key, p) >> 11) * 0x1.0p-53;
  double u2 = (double)(splitmix_at(key, p + 1) >> 11) * 0x1.0p-53;
  double r = sqrt(-2.0 * log(1.0 - u1));
  double t = 6.283185307179586 * u2;
  return (i & 1) ? r * sin(t) : r * cos(t);
}

uint64_t or_fnv64a(const char *s) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (; *s; s++) {
    h ^= (unsigned char)*s;
    h *= 0x100000001B3ull;
  }
  return h;
}

struct or_qwen3 {
  or_qwen3_cfg c;
  int threads;
  float **wqkv, **wo, **wg, **wu, **wd; /* dequantized linears (out, in) */
  float *emb;                           /* f16 values widened (vocab, hidden) */
  float *kc, *vc;                       /* (layers, kv_heads, max_ctx, head_dim), fp16 values */
  float *cos_t, *sin_t;                 /* (max_ctx, head_dim) */
  float *in_nw, *post_nw;               /* (layers, hidden) */
  float *q_nw, *k_nw;                   /* (layers, head_dim) */
  float *final_nw;                      /* (hidden) */
  uint64_t sum_blocks, sum_scales, sum_embed;
};

/* rows x cols synthetic MXFP4 values of one name, dequantized into dst rows; the codes and
 * scales are added into the checksums */
static void synth_linear(or_qwen3 *m, float *dst, int rows, int cols, uint64_t key, float sd) {
  int nb = cols / 32;
  uint64_t sb = 0, ss = 0;
#pragma omp parallel for schedule(static) num_threads(m->threads) reduction(+ : sb, ss)
  for (int r = 0; r < rows; r++) {
    float *row = malloc(sizeof(float) * (size_t)cols);
    uint8_t *w = malloc((size_t)nb * 16), *e = malloc((size_t)nb);
    for (int j = 0; j < cols; j++) row[j] = (float)(or_normal_at(key, (uint64_t)r * cols + j) * (double)sd);
    or_mxfp4_encode(w, e, row, (size_t)cols);
    for (int b = 0; b < nb * 16; b++) sb += w[b];
    for (int b = 0; b < nb; b++) ss += e[b];
    or_mxfp4_dequantize(dst + (size_t)r * cols, w, e, (size_t)nb);
    free(row);
    free(w);
    free(e);
  }
  m->sum_blocks += sb;
  m->sum_scales += ss;
}

or_qwen3 *or_qwen3_new(const or_qwen3_cfg *cfg, uint64_t seed, float sd, int threads) {
  or_qwen3 *m = calloc(1, sizeof(*m));
  m->c = *cfg;
  m->threads = threads > 0 ? threads : or_max_threads();
  const or_qwen3_cfg *c = &m->c;
  int hd = c->head_dim, qn = c->heads * hd, kn = c->kv_heads * hd;
  m->wqkv = calloc(c->layers, sizeof(float *));
  m->wo = calloc(c->layers, sizeof(float *));
  m->wg = calloc(c->layers, sizeof(float *));
  m->wu = calloc(c->layers, sizeof(float *));
  m->wd = calloc(c->layers, sizeof(float *));
  char name[128];
  for (int i = 0; i < c->layers; i++) {
    m->wqkv[i] = malloc(sizeof(float) * (size_t)(qn + 2 * kn) * c->hidden);
    m->wo[i] = malloc(sizeof(float) * (size_t)c->hidden * qn);
    m->wg[i] = malloc(sizeof(float) * (size_t)c->inter * c->hidden);
    m->wu[i] = malloc(sizeof(float) * (size_t)c->inter * c->hidden);
    m->wd[i] = malloc(sizeof(float) * (size_t)c->hidden * c->inter);
    if (!(sd > 0)) {
      memset(m->wqkv[i], 0, sizeof(float) * (size_t)(qn + 2 * kn) * c->hidden);
      memset(m->wo[i], 0, sizeof(float) * (size_t)c->hidden * qn);
      memset(m->wg[i], 0, sizeof(float) * (size_t)c->inter * c->hidden);
      memset(m->wu[i], 0, sizeof(float) * (size_t)c->inter * c->hidden);
      memset(m->wd[i], 0, sizeof(float) * (size_t)c->hidden * c->inter);
      continue;
    }
#define KEY(n)                                                      \
  (snprintf(name, sizeof name, "model.layers.%d.%s", i, n), seed ^ or_fnv64a(name))
    synth_linear(m, m->wqkv[i], qn, c->hidden, KEY("self_attn.q_proj.weight"), sd);
    synth_linear(m, m->wqkv[i] + (size_t)qn * c->hidden, kn, c->hidden, KEY("self_attn.k_proj.weight"), sd);
    synth_linear(m, m->wqkv[i] + (size_t)(qn + kn) * c->hidden, kn, c->hidden, KEY("self_attn.v_proj.weight"), sd);
    synth_linear(m, m->wo[i], c->hidden, qn, KEY("self_attn.o_proj.weight"), sd);
    synth_linear(m, m->wg[i], c->inter, c->hidden, KEY("mlp.gate_proj.weight"), sd);
    synth_linear(m, m->wu[i], c->inter, c->hidden, KEY("mlp.up_proj.weight"), sd);
    synth_linear(m, m->wd[i], c->hidden, c->inter, KEY("mlp.down_proj.weight"), sd);
#undef KEY
  }
  size_t ne = (size_t)c->vocab * c->hidden;
  m->emb = malloc(sizeof(float) * ne);
  uint64_t ekey = seed ^ or_fnv64a("model.embed_tokens.weight"), se = 0;
#pragma omp parallel for schedule(static) num_threads(m->threads) reduction(+ : se)
  for (size_t i = 0; i < ne; i++) {
    uint16_t b = sd > 0 ? or_f16_bits((float)(or_normal_at(ekey, i) * (double)sd)) : 0;
    se += b;
    m->emb[i] = or_f16_value(b);
  }
  m->sum_embed = se;
  m->in_nw = malloc(sizeof(float) * (size_t)c->layers * c->hidden);
  m->post_nw = malloc(sizeof(float) * (size_t)c->layers * c->hidden);
  m->q_nw = malloc(sizeof(float) * (size_t)c->layers * hd);
  m->k_nw = malloc(sizeof(float) * (size_t)c->layers * hd);
  m->final_nw = malloc(sizeof(float) * (size_t)c->hidden);
  for (size_t i = 0; i < (size_t)c->layers * c->hidden; i++) m->in_nw[i] = m->post_nw[i] = 1.0f;
  for (size_t i = 0; i < (size_t)c->layers * hd; i++) m->q_nw[i] = m->k_nw[i] = 1.0f;
  for (int i = 0; i < c->hidden; i++) m->final_nw[i] = 1.0f;
  size_t kv = (size_t)c->layers * c->kv_heads * c->max_ctx * hd;
  m->kc = calloc(kv, sizeof(float));
  m->vc = calloc(kv, sizeof(float));
  m->cos_t = malloc(sizeof(float) * (size_t)c->max_ctx * hd);
  m->sin_t = malloc(sizeof(float) * (size_t)c->max_ctx * hd);
  or_rope_tables(m->cos_t, m->sin_t, c->theta, 0, c->max_ctx, hd);
  return m;
}

void or_qwen3_free(or_qwen3 *m) {
  if (!m) return;
  for (int i = 0; i < m->c.layers; i++) {
    free(m->wqkv[i]);
    free(m->wo[i]);
    free(m->wg[i]);
    free(m->wu[i]);
    free(m->wd[i]);
  }
  free(m->wqkv);
  free(m->wo);
  free(m->wg);
  free(m->wu);
  free(m->wd);
  free(m->emb);
  free(m->kc);
  free(m->vc);
  free(m->cos_t);
  free(m->sin_t);
  free(m->in_nw);
  free(m->post_nw);
  free(m->q_nw);
  free(m->k_nw);
  free(m->final_nw);
  free(m);
}

/* The destination of a Hugging Face tensor name: its float32 storage, the row stride and row
 * count it occupies there (a stacked q/k/v matrix takes its rows at an offset). */
static float *tensor_of(or_qwen3 *m, const char *name, size_t *count) {
  const or_qwen3_cfg *c = &m->c;
  size_t H = (size_t)c->hidden, hd = (size_t)c->head_dim, qn = (size_t)c->heads * hd, kn = (size_t)c->kv_heads * hd,
         I = (size_t)c->inter;
  if (!strcmp(name, "model.norm.weight")) return *count = H, m->final_nw;
  if (!strcmp(name, "model.embed_tokens.weight")) return *count = (size_t)c->vocab * H, m->emb;
  int li, used = 0;
  char rest[96];
  if (sscanf(name, "model.layers.%d.%95s%n", &li, rest, &used) != 2 || name[used] != 0 || li < 0 || li >= c->layers)
    return NULL;
  if (!strcmp(rest, "input_layernorm.weight")) return *count = H, m->in_nw + (size_t)li * H;
  if (!strcmp(rest, "post_attention_layernorm.weight")) return *count = H, m->post_nw + (size_t)li * H;
  if (!strcmp(rest, "self_attn.q_norm.weight")) return *count = hd, m->q_nw + (size_t)li * hd;
  if (!strcmp(rest, "self_attn.k_norm.weight")) return *count = hd, m->k_nw + (size_t)li * hd;
  if (!strcmp(rest, "self_attn.q_proj.weight")) return *count = qn * H, m->wqkv[li];
  if (!strcmp(rest, "self_attn.k_proj.weight")) return *count = kn * H, m->wqkv[li] + qn * H;
  if (!strcmp(rest, "self_attn.v_proj.weight")) return *count = kn * H, m->wqkv[li] + (qn + kn) * H;
  if (!strcmp(rest, "self_attn.o_proj.weight")) return *count = H * qn, m->wo[li];
  if (!strcmp(rest, "mlp.gate_proj.weight")) return *count = I * H, m->wg[li];
  if (!strcmp(rest, "mlp.up_proj.weight")) return *count = I * H, m->wu[li];
  if (!strcmp(rest, "mlp.down_proj.weight")) return *count = H * I, m->wd[li];
  return NULL;
}

int or_qwen3_set(or_qwen3 *m, const char *name, const float *v, size_t n) {
  size_t want = 0;
  float *dst = tensor_of(m, name, &want);
  if (!dst) return -1;
  if (n != want) return -2;
  if (dst == m->emb) {
    for (size_t i = 0; i < n; i++) dst[i] = or_f16_value(or_f16_bits(v[i]));
  } else {
    memcpy(dst, v, sizeof(float) * n);
  }
  return 0;
}

void or_qwen3_checksums(const or_qwen3 *m, uint64_t out[3]) {
  out[0] = m->sum_blocks;
  out[1] = m->sum_scales;
  out[2] = m->sum_embed;
}

static float f16r(float x) { return or_f16_value(or_f16_bits(x)); }

/* Qwen3RMSNorm rounded to fp16: (x * r) * w, r = float32(1 / sqrt(mean(x^2) + eps)), with w the
 * norm's weight (qwen3_test.go:155-163) */
static void rms_f16(float *out, const float *x, const float *w, int rows, int n, double eps) {
  for (int r = 0; r < rows; r++) {
    const float *xr = x + (size_t)r * n;
    double ss = 0;
    for (int j = 0; j < n; j++) ss += (double)xr[j] * (double)xr[j];
    float inv = (float)(1.0 / sqrt(ss / (double)n + eps));
    for (int j = 0; j < n; j++) out[(size_t)r * n + j] = f16r((xr[j] * inv) * w[j]);
  }
}

/* y (T, out) = x (T, in) W^T */
static void linear(or_qwen3 *m, float *y, const float *x, const float *w, int T, int in, int out) {
  memset(y, 0, sizeof(float) * (size_t)T * out);
  or_sgemm(T, out, in, x, in, 0, w, in, 1, y, out, m->threads);
}

/* Rows [0, T) at positions start .. start+T-1: the final hidden state of the last row into hlast,
 * the KV cache written at the rows' positions. */
static void forward(or_qwen3 *m, const int32_t *tokens, int T, int start, float *hlast) {
  const or_qwen3_cfg *c = &m->c;
  int H = c->hidden, hd = c->head_dim, nh = c->heads, nkv = c->kv_heads, I = c->inter;
  int qn = nh * hd, kn = nkv * hd, qkv_n = qn + 2 * kn, L = start + T;
  float scale = (float)(1.0 / sqrt((double)hd));
  float *h = malloc(sizeof(float) * (size_t)T * H);
  float *x = malloc(sizeof(float) * (size_t)T * (H > I ? H : I));
  float *qkv = malloc(sizeof(float) * (size_t)T * qkv_n);
  float *q = malloc(sizeof(float) * (size_t)nh * T * hd);
  float *att = malloc(sizeof(float) * (size_t)T * qn);
  float *g = malloc(sizeof(float) * (size_t)T * I), *u = malloc(sizeof(float) * (size_t)T * I);
  float *y = malloc(sizeof(float) * (size_t)T * H);
  for (int t = 0; t < T; t++) memcpy(h + (size_t)t * H, m->emb + (size_t)tokens[t] * H, sizeof(float) * H);
  for (int li = 0; li < c->layers; li++) {
    float *kc = m->kc + (size_t)li * nkv * c->max_ctx * hd, *vc = m->vc + (size_t)li * nkv * c->max_ctx * hd;
    rms_f16(x, h, m->in_nw + (size_t)li * H, T, H, c->eps);
    linear(m, qkv, x, m->wqkv[li], T, H, qkv_n);
    for (int t = 0; t < T; t++) {
      int p = start + t;
      float *row = qkv + (size_t)t * qkv_n, tmp[128];
      for (int j = 0; j < nh + nkv; j++) {
        float *v = row + (size_t)j * hd;
        /* per-head RMSNorm (q_norm for query heads, k_norm for key heads; qwen3_test.go:196) in
         * float32, rounded to fp16 only after RoPE */
        const float *nw = (j < nh ? m->q_nw : m->k_nw) + (size_t)li * hd;
        double ss = 0;
        for (int d = 0; d < hd; d++) ss += (double)v[d] * (double)v[d];
        float r = (float)(1.0 / sqrt(ss / (double)hd + c->eps));
        for (int d = 0; d < hd; d++) tmp[d] = (v[d] * r) * nw[d];
        or_apply_rope(tmp, 1, hd, m->cos_t + (size_t)p * hd, m->sin_t + (size_t)p * hd);
        if (j < nh) {
          for (int d = 0; d < hd; d++) q[((size_t)j * T + t) * hd + d] = f16r(tmp[d]);
        } else {
          float *dst = kc + ((size_t)(j - nh) * c->max_ctx + p) * hd;
          for (int d = 0; d < hd; d++) dst[d] = f16r(tmp[d]);
        }
      }
      for (int j = 0; j < nkv; j++) {
        float *v = row + (size_t)(nh + nkv + j) * hd, *dst = vc + ((size_t)j * c->max_ctx + p) * hd;
        for (int d = 0; d < hd; d++) dst[d] = f16r(v[d]);
      }
    }
    /* the session's chunked attention: chunks of 8192 keys (paged.DefaultChunk) with the causal
     * mask (0 / -1e4), merged in fp32 */
    const int chunk = 8192;
    or_merge *mg = or_merge_new(nh * T, hd);
    float *o = malloc(sizeof(float) * (size_t)nh * T * hd), *mm = malloc(sizeof(float) * (size_t)nh * T),
          *ll = malloc(sizeof(float) * (size_t)nh * T);
    for (int c0 = 0; c0 < L; c0 += chunk) {
      int n = L - c0 < chunk ? L - c0 : chunk;
      float *mask = malloc(sizeof(float) * (size_t)T * n);
      for (int t = 0; t < T; t++)
        for (int k = 0; k < n; k++) mask[(size_t)t * n + k] = (c0 + k <= start + t) ? 0.0f : -1e4f;
#pragma omp parallel for schedule(static, 1) num_threads(m->threads)
      for (int g2 = 0; g2 < nkv; g2++) {
        int rep = nh / nkv;
        or_paged_chunk(q + (size_t)g2 * rep * T * hd, kc + ((size_t)g2 * c->max_ctx + c0) * hd,
                       vc + ((size_t)g2 * c->max_ctx + c0) * hd, (size_t)c->max_ctx, mask,
                       o + (size_t)g2 * rep * T * hd, mm + (size_t)g2 * rep * T, ll + (size_t)g2 * rep * T, rep, 1, T,
                       n, hd, scale);
      }
      or_merge_add(mg, o, mm, ll);
      free(mask);
    }
    or_merge_result(mg, o);
    or_merge_free(mg);
    for (int hh = 0; hh < nh; hh++)
      for (int t = 0; t < T; t++)
        for (int d = 0; d < hd; d++) att[(size_t)t * qn + (size_t)hh * hd + d] = f16r(o[((size_t)hh * T + t) * hd + d]);
    free(o);
    free(mm);
    free(ll);
    linear(m, y, att, m->wo[li], T, qn, H);
    for (size_t i = 0; i < (size_t)T * H; i++) h[i] += y[i];
    rms_f16(x, h, m->post_nw + (size_t)li * H, T, H, c->eps);
    linear(m, g, x, m->wg[li], T, H, I);
    linear(m, u, x, m->wu[li], T, H, I);
    or_silu_mul(g, g, u, (size_t)T * I);
    for (size_t i = 0; i < (size_t)T * I; i++) g[i] = f16r(g[i]);
    linear(m, y, g, m->wd[li], T, I, H);
    for (size_t i = 0; i < (size_t)T * H; i++) h[i] += y[i];
  }
  memcpy(hlast, h + (size_t)(T - 1) * H, sizeof(float) * H);
  free(h);
  free(x);
  free(qkv);
  free(q);
  free(att);
  free(g);
  free(u);
  free(y);
}

int32_t or_qwen3_run(or_qwen3 *m, const int32_t *tokens, int T, int start, float *logits) {
  const or_qwen3_cfg *c = &m->c;
  float *hl = malloc(sizeof(float) * c->hidden), *x = malloc(sizeof(float) * c->hidden);
  forward(m, tokens, T, start, hl);
  rms_f16(x, hl, m->final_nw, 1, c->hidden, c->eps);
  linear(m, logits, x, m->emb, 1, c->hidden, c->vocab);
  free(hl);
  free(x);
  return or_argmax(logits, (size_t)c->vocab);
}
