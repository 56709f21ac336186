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

// y = W x for MXFP4 W (n, heads*128) with x the fp16 attention output merged from attn_step's partials
// in the workgroup's prologue (the reference's Merge rule, internal/llm/paged/paged.go:252-310): for
// query head hq, x = fp16(sum_c w_c o_c / sum_c w_c l_c) over the chunks c < nchunk with l_c > 0 (a
// chunk past the position has l = 0), w_c = exp(m_c - top), top their largest m. nchunk <= 16. y per
// out_mode.
char *mxfp4_gemv_merge(hipStream_t st, const void *w, const void *e, const void *workspace, uint32_t heads, uint32_t G,
                       uint32_t nchunk, void *y, uint32_t n, int out_mode);

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

// The model's decode attention for the token at *pos (k_attn_step): the per-head q/k RMSNorm, RoPE
// (rope: the position's cos | sin rows, 64 values each) and the KV append in its prologue (q, k, v
// from the stacked fp32 projection qkv), workgroups of a kv head over chunks of the keys [0, *pos],
// each leaving its partial (o unnormalized, m in natural-log units, l) per query head at slot
// (kv head * nchunk + chunk) * G + g of the workspace: o (slots, 128) | m (slots) | l (slots). Every
// chunk of the capacity is written; a chunk past *pos has l = 0 and weighs nothing in the merge.
// attn_step_layout gives the chunking (fixed by the capacity), which the merging consumer needs.
// keep: the cache rows are read with cache-allocating loads (for a caller whose rows of every layer
// fit the memory-side cache together), else with nontemporal loads. The kernel finds kn at qn + 128,
// vc right after kc (kv_heads * capacity rows) and pos right after the RoPE row (rope + 128).
void attn_step_layout(const hwk_attn_params *p, uint32_t *chunk, uint32_t *nchunk);
size_t attn_step_workspace_bytes(const hwk_attn_params *p);
char *attn_step(hipStream_t st, const float *qkv, const float *qn, const float *kn, const float *rope, double eps,
                void *kc, void *vc, void *workspace, size_t workspace_bytes, const hwk_attn_params *p,
                const int32_t *pos, bool keep);

}  // namespace hwk

// A double's DPP move (both halves moved alike; lanes the row mask leaves out get 0.0).
template <int CTRL, int ROW_MASK, bool BOUND>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xf, BOUND);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xf, BOUND);
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Sum of a double over the 64 lanes by DPP row shifts and row broadcasts, as wave_sum_to_63 (no LDS
// round trip): lane 63 ends with the total.
__device__ __forceinline__ double wave_sum_f64_to_63(double v) {
  v += dpp_f64<0x111, 0xf, true>(v);   // row_shr:1
  v += dpp_f64<0x112, 0xf, true>(v);   // row_shr:2
  v += dpp_f64<0x114, 0xf, true>(v);   // row_shr:4
  v += dpp_f64<0x118, 0xf, true>(v);   // row_shr:8
  v += dpp_f64<0x142, 0xa, false>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f64<0x143, 0xc, false>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// The sum of a double over the 64 lanes, in every lane (lane 63's total read back as a scalar).
__device__ __forceinline__ double wave_sum_f64_all(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, wave_sum_f64_to_63(v));
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Per-head RMSNorm then RoPE of one 128-wide head held as dims (l, l+64) by lane l: (x * r) * w
// with r = float(1 / sqrt(mean(x^2) + eps)) (mean in float64), then x*cos + rotate_half(x)*sin
// with the position's float32 tables (rotate_half = cat(-x2, x1); reference internal/llm/blocks/
// blocks.go:427-445), each product and sum rounded on its own.
__device__ __forceinline__ void head_norm_rope(float x0, float x1, float nw0, float nw1, float c, float s,
                                               double eps, float &o0, float &o1) {
#pragma clang fp contract(off)
  const double ss = wave_sum_f64_all((double)x0 * (double)x0 + (double)x1 * (double)x1);
  const float r = (float)(1.0 / sqrt(ss / 128.0 + eps));
  const float y0 = (x0 * r) * nw0, y1 = (x1 * r) * nw1;
  o0 = f32_value(y0 * c + (-y1) * s);  // j < half: x*cos + (-x[j+half])*sin
  o1 = f32_value(y1 * c + y0 * s);     // j >= half: x*cos + x[j-half]*sin
}

