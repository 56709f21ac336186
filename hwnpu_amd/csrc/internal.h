// Launchers that libhwk's sources share with the Qwen3 runtime (qwen3.hip) but do not export:
// the decode-step forms of the GEMVs (RMSNorm fused on the input side, SwiGLU fused on the
// output side) and the attention with its length read from the device, which a captured step
// graph needs. Every launcher checks its shapes and returns an error string like the C ABI.
#pragma once

#include "hwk_common.h"

namespace hwk {

// y = W x for MXFP4 W (n, k) with x = fp16((h * r) * nw), r = float(1 / sqrt(mean(h^2) + eps))
// in float64, computed by every workgroup from fp32 h (k values) and fp32 norm weights nw; or,
// with h null, x fp16 given. swiglu: rows come in (gate, up) pairs and the output is the fp16
// vector silu(gate) * up (n/2 values), silu(g) = g / (1 + float(exp(-g))) with exp in float64;
// otherwise y per out_mode.
char *mxfp4_gemv_x(hipStream_t st, const void *w, const void *e, const void *x16, const float *h, const float *nw,
                   double eps, void *y, uint32_t n, uint32_t k, int out_mode, bool swiglu);

// Synthetic MXFP4 rows (hwk_synth_mxfp4's draws) with source row r written at row row0 + r*stride.
char *synth_mxfp4_rows(hipStream_t st, void *w, void *e, uint32_t rows, uint32_t k, uint64_t key, float stdv,
                       uint32_t stride, uint32_t row0);

// fp32 h (rows, k) -> fp16 (h * r) * nw per row, r as above (one workgroup a row).
char *rmsnorm_f16(hipStream_t st, const float *h, const float *nw, double eps, void *out, uint32_t rows, uint32_t k);

// hwk_attn_decode with the number of keys read on the device: len = *pos + len_add when pos is
// not null (the grid is sized by p->len, which must then be the cache's capacity).
char *attn_decode_dev(hipStream_t st, const void *q, const void *k, const void *v, const void *k_scale,
                      const void *v_scale, void *out, void *workspace, size_t workspace_bytes,
                      const hwk_attn_params *p, const int32_t *pos, uint32_t len_add);

// The model's decode attention for the token at position *pos, split over the context, with the
// per-head q/k RMSNorm, RoPE and the KV append folded in: q, k, v come from the stacked projection
// qkv (fp32, heads + 2 * kv_heads rows of 128); the workgroup whose chunk holds *pos writes the new
// k (normed, rotated) and v into the caches before it reads them. The chunks' partials go to the
// workspace (o (slots, 128) | m (slots) | l (slots), slot = (kv head * nchunk + chunk) * G + g) for
// a consumer to merge (attn_merge_ws). p: the decode
// grid (its capacity sizes the chunks), fp16 caches. *nchunk_out: the chunks a kv head.
uint32_t attn_step_chunks(const hwk_attn_params *p);
size_t attn_step_workspace_bytes(const hwk_attn_params *p);
char *attn_decode_step(hipStream_t st, const float *qkv, const float *qn, const float *kn, const float *cos_t,
                       const float *sin_t, double eps, void *kc, void *vc, void *workspace, size_t workspace_bytes,
                       const hwk_attn_params *p, const int32_t *pos, uint32_t *nchunk_out);
// The model's decode attention for the token at *pos (k_attn_head): the per-head q/k RMSNorm, RoPE
// and the KV append folded into its prologue (q, k, v from the stacked fp32 projection qkv), a few
// workgroups a kv head over the keys [0, *pos], the last of them to arrive merging the partials
// into out (heads, 128) fp16. counters (kv_heads) start at zero and are left at zero; workspace:
// attn_head_workspace_bytes.
uint32_t attn_head_split(const hwk_attn_params *p);
size_t attn_head_workspace_bytes(const hwk_attn_params *p);
char *attn_head(hipStream_t st, const float *qkv, const float *qn, const float *kn, const float *cos_t,
                const float *sin_t, double eps, void *kc, void *vc, void *out, void *workspace, size_t workspace_bytes,
                uint32_t *counters, const hwk_attn_params *p, const int32_t *pos);

// The merge of attn_decode_step's partials into out (heads, 128) fp16.
char *attn_merge_ws(hipStream_t st, const void *workspace, void *out, const hwk_attn_params *p, uint32_t nchunk);

}  // namespace hwk

// Per-head RMSNorm then RoPE of one 128-wide head held as dims (l, l+64) by lane l: (x * r) * w
// with r = float(1 / sqrt(mean(x^2) + eps)) (mean in float64), then x*cos + rotate_half(x)*sin
// with the position's float32 tables (rotate_half = cat(-x2, x1); reference internal/llm/blocks/
// blocks.go:427-445), each product and sum rounded on its own.
__device__ __forceinline__ void head_norm_rope(float x0, float x1, float nw0, float nw1, float c, float s,
                                               double eps, float &o0, float &o1) {
#pragma clang fp contract(off)
  double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float r = (float)(1.0 / sqrt(ss / 128.0 + eps));
  const float y0 = (x0 * r) * nw0, y1 = (x1 * r) * nw1;
  o0 = f32_value(y0 * c + (-y1) * s);  // j < half: x*cos + (-x[j+half])*sin
  o1 = f32_value(y1 * c + y0 * s);     // j >= half: x*cos + x[j-half]*sin
}
