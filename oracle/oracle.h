/*
 * oracle.h - CPU restatement of hwnpu's quantized-decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker and the timed CPU baseline. Only the
 * test suite (tests/), the package smoke check (__graft_entry__.smoke) and the cpu_baseline leg
 * of bench.py may load it. The product path (libhwk and the hwnpu_amd package) never links,
 * loads or calls anything here, and has no CPU fallback.
 *
 * Every function restates a function of the reference (shibukawa/hwnpu, Go) from its source read
 * as text; each definition cites the file:line it follows. The reference is Go plus Go assembly
 * and there is no Go toolchain in this image, so nothing of it is compiled here (no oracle/_ref).
 *
 * How each part is pinned (besides the cross-checks between the parts):
 *   or_f16_bits / or_f16_value   all 65,536 halves round trip; halfCases of
 *                                internal/vecops/vecops_test.go:404-489; IEEE RNE vs numpy.
 *   or_mxfp4_scale/dequantize    closed form 16 codes x 256 exponents; -0 for code 8; e=0 -> +0;
 *                                e=255 -> +Inf.
 *   or_mxfp4_nearest/encode      the nearest() KAT of internal/mxfp4/mxfp4_test.go:168-175 and
 *                                TestEncode's invariants (:131-176); brute-force argmin of the
 *                                block error over every e8m0 exponent.
 *   or_vec_quantize/or_mxfp4_dot TestDot's invariants (mxfp4_test.go:21-55): Dot equals the f64
 *                                sum of dequantized x int8 x scale.
 *   or_sgemm                     brute-force f64 GEMM, tolerance 1e-4*sqrt(k)+1e-5
 *                                (internal/sgemm/sgemm_test.go:31-62).
 *   or_i8_dequant                closed form q*s; the int4 shift-scale KAT of
 *                                internal/milcpu/milcpu_test.go:297-308 restated for int8.
 *   or_paged_* / or_merge_*      TestMergeOrder and TestMergeSink KATs (paged_test.go:133-186);
 *                                one f64 softmax over the whole cache vs chunks+merge (:17-131).
 *   or_choose                    TestChooseSigmoidBias KAT (experts/weights_test.go:11-26);
 *                                top-k equals a full stable sort's first k.
 *   or_experts_*                 f64 dequantized-experts brute force; the int8-activation path
 *                                against the fp32 path (cosine >= 0.999, experts/host_test.go:211-285);
 *                                with biases and the gpt-oss gated unit, TestHostRunSmall's float64
 *                                form (host_test.go:208-284), which fails when the clamp, the +1 on
 *                                up, alpha or a bias is dropped.
 *   or_rmsnorm/rope/silu/argmax  closed forms (rotation preserves norms, RMS of output = |w|).
 *   or_fnv64a / or_synth_reference  FNV-1a 64 published test vectors; the MMIX LCG sequence against
 *                                its recurrence and the [-0.2, 0.2) range and mean of the values.
 *   or_qwen3_*                   a float64 forward written from the model's semantics on the same
 *                                weights (relative RMS < 5e-3 at every position); cached stepping
 *                                equals the full prompt; fails when RoPE is dropped or gate/up swap.
 */
#ifndef HWNPU_ORACLE_H
#define HWNPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (internal/vecops/vecops.go:297-352) ---- */
uint16_t or_f16_bits(float f);
float or_f16_value(uint16_t h);
void or_f32_to_f16(uint16_t *dst, const float *src, size_t n);
void or_f16_to_f32(float *dst, const uint16_t *src, size_t n);

/* ---- MXFP4 (internal/mxfp4/mxfp4.go, encode.go, matvec.go) ---- */
float or_mxfp4_value(int code);
float or_mxfp4_scale(uint8_t e);
/* one row: nb blocks; w = nb*16 bytes, e = nb bytes, dst = nb*32 floats */
void or_mxfp4_dequantize(float *dst, const uint8_t *w, const uint8_t *e, size_t nb);
/* rows x nb blocks, threads over rows */
void or_mxfp4_dequantize_rows(float *dst, const uint8_t *w, const uint8_t *e, size_t rows,
                              size_t nb, int threads);
uint8_t or_mxfp4_nearest(double x);
void or_mxfp4_encode(uint8_t *w, uint8_t *e, const float *row, size_t n);
void or_mxfp4_encode_rows(uint8_t *w, uint8_t *e, const float *m, size_t rows, size_t n,
                          int threads);
void or_vec_quantize(int8_t *q, float *s, const float *x, size_t n);
float or_mxfp4_dot(const uint8_t *w, const uint8_t *e, size_t nb, const int8_t *q, const float *s);
/* mxfp4.Run over one job with V vectors: out[v*rows + r]; threads workers, chunks of 32 rows */
void or_mxfp4_run(float *out, const uint8_t *w, const uint8_t *e, size_t rows, size_t nb,
                  const int8_t *q, const float *s, size_t nvec, int threads);

/* ---- fp32 GEMM (internal/sgemm/sgemm.go) ----
 * C (m x n, ldc) += A (m x k, lda; transposed if transa) * B (k x n, ldb; given as its
 * transpose n x k if transb). */
void or_sgemm(int m, int n, int k, const float *a, int lda, int transa, const float *b, int ldb,
              int transb, float *c, int ldc, int threads);

/* ---- int8 per-channel weights (internal/milcpu/ops.go:1589-1610,
 *      internal/llm/experts/weights.go:229-252, internal/vecops/vecops.go:179-202) ---- */
void or_i8_dequant(float *dst, const int8_t *q, const uint16_t *scale16, size_t rows, size_t cols,
                   int threads);
/* the KV rule: scale = f16(absmax/127) (1 for a zero row), q = RoundToEven(v/scale) clamped +-127 */
void or_i8_quantize_rows(int8_t *q, uint16_t *scale16, const float *x, size_t rows, size_t cols);

/* ---- chunk attention and merge (internal/llm/paged/paged.go:70-310) ---- */
typedef struct or_merge or_merge;
or_merge *or_merge_new(int rows, int dim);
void or_merge_free(or_merge *c);
void or_merge_reset(or_merge *c);
void or_merge_add(or_merge *c, const float *o, const float *m, const float *l);
void or_merge_add_sink(or_merge *c, const float *sinks, int tokens);
void or_merge_result(or_merge *c, float *out);
/* one chunk, grouped form: q (heads, tokens, d), k/v (kv_heads, chunk, d) with stride
 * kv_stride between heads (in rows), mask (tokens, chunk) or NULL; o (heads, tokens, d),
 * m/l (heads, tokens). */
void or_paged_chunk(const float *q, const float *k, const float *v, size_t kv_stride,
                    const float *mask, float *o, float *m, float *l, int heads, int kv_heads,
                    int tokens, int chunk, int d, float scale);
/* decode attention: one query row per head over L cached keys in chunks of chunk, merged
 * (internal/llm/decode/decode.go:1435-1483). q (heads, d); k/v (kv_heads, L, d); out (heads, d).
 * The cache is given as floats (fp16 values widened, or int8 x scale dequantized by the
 * caller). */
void or_attn_decode(const float *q, const float *k, const float *v, float *out, int heads,
                    int kv_heads, int L, int d, float scale, int chunk, int threads);

/* ---- MoE (internal/llm/experts/weights.go:33-81, host.go:478-579,723-882) ---- */
/* score: 0 softmax, 1 sigmoid; bias may be NULL; scale 0 for none */
void or_choose(const float *logits, const float *bias, int n, int k, int score, int norm,
               double scale, int32_t *idx, float *w);
/* The experts of T rows, the parity form: gate_up/down dequantized, fp32 GEMV, gate/up biases
 * gu_b (E, 2I) after the product (NULL: none), the gated unit in fp32 (act 0 SiLU, 1 gpt-oss with
 * alpha and limit), out += w * (y + dn_b) with dn_b (E, H) (NULL: none) in ascending expert id.
 * gu_w (E, 2I, H/32, 16), gu_e (E, 2I, H/32); dn_w (E, H, I/32, 16), dn_e (E, H, I/32).
 * x (T, H) floats; idx/w (T, k); out (T, H) added to. */
void or_experts_f32(const float *x, int T, const int32_t *idx, const float *w, int k,
                    const uint8_t *gu_w, const uint8_t *gu_e, const float *gu_b,
                    const uint8_t *dn_w, const uint8_t *dn_e, const float *dn_b, int E, int H,
                    int I, int act, float alpha, float limit, float *out, int threads);
/* The same with the reference's production numerics (Host.Run): x and the activations quantized
 * to int8 by blocks (Vec.Quantize), MXFP4 dot in int32 (dotGo). The timed CPU baseline. */
void or_experts_host(const float *x, int T, const int32_t *idx, const float *w, int k,
                     const uint8_t *gu_w, const uint8_t *gu_e, const float *gu_b,
                     const uint8_t *dn_w, const uint8_t *dn_e, const float *dn_b, int E, int H,
                     int I, int act, float alpha, float limit, float *out, int threads);

/* ---- model ops (internal/llm/blocks/blocks.go, internal/llm/qwen3, internal/chat/sample.go) ---- */
/* rows of n: out = x * (1/sqrt(mean(x^2) + eps)) * w, in fp32 */
void or_rmsnorm(float *out, const float *x, const float *w, int rows, int n, float eps);
/* cos/sin tables (n positions from start, head_dim each, cat(freqs, freqs)) */
void or_rope_tables(float *cos_t, float *sin_t, double theta, int start, int n, int head_dim);
/* x (heads, head_dim) rotated in place at one position's tables */
void or_apply_rope(float *x, int heads, int head_dim, const float *cos_row, const float *sin_row);
/* silu(g)*u, elementwise: g / (1 + float32(exp(-g))) * u */
void or_silu_mul(float *out, const float *g, const float *u, size_t n);
/* greedy pick: the first index of the largest value (strict >) */
int32_t or_argmax(const float *x, size_t n);

/* ---- the Qwen3 decoder (internal/llm/qwen3/qwen3_test.go:77-207 with the decode session's
 *      chunked attention and fp16 storage points; see qwen3.c) ---- */
typedef struct or_qwen3_cfg {
  int layers, hidden, heads, kv_heads, head_dim, inter, vocab, max_ctx;
  double theta, eps;
} or_qwen3_cfg;
typedef struct or_qwen3 or_qwen3;
/* element i of the normal stream keyed by key (splitmix64 + Box-Muller in float64) */
double or_normal_at(uint64_t key, uint64_t i);
uint64_t or_fnv64a(const char *s);
/* the synthetic checkpoint of seed with weight std sd (norm weights 1); sd 0 draws nothing (zero
 * linears and embedding, for or_qwen3_set to fill) */
or_qwen3 *or_qwen3_new(const or_qwen3_cfg *cfg, uint64_t seed, float sd, int threads);
/* replaces the tensor of a Hugging Face Qwen3 name (model.layers.N.{input_layernorm,
 * post_attention_layernorm,self_attn.{q,k}_norm,self_attn.{q,k,v,o}_proj,mlp.{gate,up,down}_proj}
 * .weight, model.norm.weight, model.embed_tokens.weight) by n float32 values (row-major (out, in)
 * for a linear: the values it computes with, e.g. a dequantized MXFP4 matrix; the embedding is
 * rounded to fp16); 0 on success, -1 for an unknown name, -2 for a wrong count */
int or_qwen3_set(or_qwen3 *m, const char *name, const float *v, size_t n);
void or_qwen3_free(or_qwen3 *m);
/* sums of every linear's code bytes, of their scale bytes, and of the embedding's fp16 bits */
void or_qwen3_checksums(const or_qwen3 *m, uint64_t out[3]);
/* T tokens at positions start .. start+T-1 (KV cache written there; earlier positions must be
 * cached): logits (vocab) of the last row, returns the greedy token */
int32_t or_qwen3_run(or_qwen3 *m, const int32_t *tokens, int T, int start, float *logits);

/* ---- the reference's synthetic checkpoint (internal/llm/synth.go:17-35) ---- */
/* n values of tensor name: FNV-64a seed, MMIX LCG, uniform in [-0.2, 0.2) (synth.go's comment
 * says +-0.1; its code gives +-0.2) */
void or_synth_reference(const char *name, size_t n, float *out);

/* ---- threads ---- */
int or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
