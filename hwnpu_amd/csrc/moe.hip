// MoE on gfx950: the kernels of hwk_moe_route, hwk_moe_experts and hwk_moe_layer and their launch
// choices (the device code is in moe_kernels.h).
#include "hwk_common.h"
#include "moe_kernels.h"

#define HWK_Q(call)                  \
  do {                               \
    if (char *e_ = (call)) return e_; \
  } while (0)

namespace {

using namespace hwk_moe;

// hwk_moe_route: one wave a row.
__global__ __launch_bounds__(256) void k_moe_route(const float *__restrict__ logits, const float *__restrict__ bias,
                                                   int32_t *__restrict__ idx, float *__restrict__ w, uint32_t rows,
                                                   uint32_t E, uint32_t k, int score, int norm, float scale) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  choose_wave(logits + (size_t)row * E, bias, E, k, score, norm, scale, idx + (size_t)row * k, w + (size_t)row * k);
}

template <int BPL, int PPW, bool ROUTE>
__global__ __launch_bounds__(256) void k_moe_gate_up(const uint4 *__restrict__ x, const float *__restrict__ logits,
                                                     const float *__restrict__ rbias, int32_t *__restrict__ idx,
                                                     float *__restrict__ wout, const uint4 *__restrict__ gw,
                                                     const uint8_t *__restrict__ ge, const float *__restrict__ gb,
                                                     float *__restrict__ act, MoeArgs a) {
  moe_gate_up_wg<BPL, PPW, ROUTE>(blockIdx.x, blockIdx.y, x, logits, rbias, idx, wout, gw, ge, gb, act, a);
}

template <int LPR, int BPL, int EPW, bool AL, int NW>
__global__ __launch_bounds__(64 * NW) void k_moe_down(const float *__restrict__ act, const int32_t *__restrict__ idx,
                                                  const float *__restrict__ w, const uint4 *__restrict__ dw,
                                                  const uint8_t *__restrict__ de, const float *__restrict__ db,
                                                  float *__restrict__ out, MoeArgs a) {
  moe_down_wg<LPR, BPL, EPW, AL, NW>(blockIdx.x, act, idx, w, dw, de, db, out, a);
}

// LDS the staging copies may take (gfx950: 160 KB a workgroup, 64 KB without the attribute).
constexpr size_t kMoeStageLds = 128 * 1024;

template <int LPR, int BPL, int EPW, int NW>
void launch_down_cfg(hipStream_t st, const float *act, const int32_t *idx, const float *w, const void *dw,
                     const void *de, const float *db, float *out, const MoeArgs &a) {
  constexpr int RS = 64 / LPR;
  const size_t lds = (size_t)a.T * a.k * a.I * 4;
  const dim3 grid((a.H + RS - 1) / RS);
  if (lds <= kMoeStageLds) {
    static bool attr = false;  // once per instance: the dynamic LDS past 64 KB
    if (!attr) {
      (void)hipFuncSetAttribute((const void *)k_moe_down<LPR, BPL, EPW, true, NW>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMoeStageLds);
      attr = true;
    }
    hipLaunchKernelGGL((k_moe_down<LPR, BPL, EPW, true, NW>), grid, dim3(64 * NW), lds, st, act, idx, w,
                       (const uint4 *)dw, (const uint8_t *)de, db, out, a);
  } else {
    hipLaunchKernelGGL((k_moe_down<LPR, BPL, EPW, false, NW>), grid, dim3(64 * NW), 0, st, act, idx, w,
                       (const uint4 *)dw, (const uint8_t *)de, db, out, a);
  }
}

// The waves of a down workgroup and the experts a wave loads at once, by the chosen (token, expert)
// slots n = T*k (at most n distinct experts): every slot a wave of its own up to 4 (no load is a
// padding copy), one a wave for 16 waves up to 32 (16 at once, a second round past 16 distinct
// experts; at T = 5 30.5-30.8 µs a layer against 31.4 for two a wave in 8 waves, and 31.6 for one in
// 8), else as many as the registers take.
template <int LPR, int BPL>
void launch_down(hipStream_t st, const float *act, const int32_t *idx, const float *w, const void *dw, const void *de,
                 const float *db, float *out, const MoeArgs &a) {
  const uint32_t n = a.T * a.k;
  if (n <= 4)
    launch_down_cfg<LPR, BPL, 1, 4>(st, act, idx, w, dw, de, db, out, a);
  else if (n <= 32)
    launch_down_cfg<LPR, BPL, 1, 16>(st, act, idx, w, dw, de, db, out, a);
  else
    launch_down_cfg<LPR, BPL, BPL <= 1 ? 8 : 12 / BPL, 8>(st, act, idx, w, dw, de, db, out, a);
}

char *check_params(const char *what, const hwk_moe_params *p) {
  HWK_CHECK(p, "%s: null params", what);
  HWK_CHECK(p->tokens >= 1 && p->tokens <= 8, "%s: %u tokens (1..8)", what, p->tokens);
  HWK_CHECK(p->experts >= 1 && p->experts <= 64, "%s: %u experts (1..64)", what, p->experts);
  HWK_CHECK(p->k >= 1 && p->k <= p->experts && p->tokens * p->k <= 64, "%s: k=%u", what, p->k);
  HWK_CHECK(p->hidden % 32 == 0 && p->hidden > 0 && p->hidden <= 8192, "%s: hidden %u", what, p->hidden);
  HWK_CHECK(p->inter % 32 == 0 && p->inter > 0 && p->inter <= 8192, "%s: inter %u", what, p->inter);
  HWK_CHECK(p->out_mode == HWK_OUT_F32 || p->out_mode == HWK_OUT_ADD_F32, "%s: out_mode %u", what, p->out_mode);
  HWK_CHECK(p->act == HWK_ACT_SILU || p->act == HWK_ACT_GPTOSS, "%s: act %u", what, p->act);
  return nullptr;
}

MoeArgs args_of(const hwk_moe_params *p) {
  MoeArgs a;
  a.T = p->tokens;
  a.H = p->hidden;
  a.I = p->inter;
  a.E = p->experts;
  a.k = p->k;
  a.act = (int)p->act;
  a.alpha = hwk::f32_of_bits(p->alpha_bits);
  a.limit = hwk::f32_of_bits(p->limit_bits);
  a.score = (int)p->score;
  a.norm = (int)p->norm;
  a.scale = hwk::f32_of_bits(p->scale_bits);
  a.mode = (int)p->out_mode;
  return a;
}

template <int PPW, bool ROUTE>
void launch_gate_up(hipStream_t st, const void *x, const float *logits, const float *rbias, int32_t *idx, float *w,
                    const void *gu_w, const void *gu_e, const float *gu_b, float *act, const MoeArgs &a) {
  const uint32_t unique_max = a.T * a.k < a.E ? a.T * a.k : a.E;
  // with the route folded in, one more column of workgroups: the route's own (moe_gate_up_wg)
  const dim3 g1((a.I + 4 * PPW - 1) / (4 * PPW) + (ROUTE ? 1 : 0), unique_max);
  const int bpl1 = (int)((a.H / 32 + 63) / 64);
#define HWK_GU(B)                                                                                         \
  hipLaunchKernelGGL((k_moe_gate_up<B, PPW, ROUTE>), g1, dim3(256), 0, st, (const uint4 *)x, logits, rbias, idx, w, \
                     (const uint4 *)gu_w, (const uint8_t *)gu_e, gu_b, act, a)
  switch (bpl1) {
    case 1: HWK_GU(1); break;
    case 2: HWK_GU(2); break;
    case 3: HWK_GU(3); break;
    default: HWK_GU(4); break;
  }
#undef HWK_GU
}

// K5b: gate_up (with the route folded in when ROUTE), then down with the ordered combine. Past 2
// tokens a workgroup takes 4 row pairs a wave instead of 2: fewer waves repeat the per-token work.
template <bool ROUTE>
char *run_experts(hipStream_t st, const void *x, const float *logits, const float *rbias, int32_t *idx, float *w,
                  const void *gu_w, const void *gu_e, const float *gu_b, const void *dn_w, const void *dn_e,
                  const float *dn_b, float *out, float *act, const MoeArgs &a, const char *what) {
  if (a.T <= 2)
    launch_gate_up<2, ROUTE>(st, x, logits, rbias, idx, w, gu_w, gu_e, gu_b, act, a);
  else
    launch_gate_up<4, ROUTE>(st, x, logits, rbias, idx, w, gu_w, gu_e, gu_b, act, a);
  if (char *err = hwk::launched(what)) return err;
  // down: lanes a row by I/32 blocks, the fewest idle slots (8 lanes x 3 blocks for I = 768)
  const uint32_t nbi = a.I / 32;
  if (nbi <= 8) launch_down<8, 1>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else if (nbi <= 16) launch_down<16, 1>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else if (nbi <= 24) launch_down<8, 3>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else if (nbi <= 32) launch_down<32, 1>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else if (nbi <= 64) launch_down<64, 1>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else if (nbi <= 128) launch_down<64, 2>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else if (nbi <= 192) launch_down<64, 3>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  else launch_down<64, 4>(st, act, idx, w, dn_w, dn_e, dn_b, out, a);
  return hwk::launched(what);
}

// Tokens up to which hwk_moe_layer folds the route into the gate_up launch: every workgroup routes
// every token, which past a few tokens costs more vector issue than the route launch it saves.
constexpr uint32_t kFoldRouteMaxTokens = 2;

}  // namespace

extern "C" {

HWK_API char *hwk_moe_route(void *stream, const void *logits, const void *bias, void *idx, void *w, uint32_t rows,
                            uint32_t experts, uint32_t k, int score, int norm, uint32_t scale_bits) {
  HWK_CHECK(logits && idx && w, "hwk_moe_route: null pointer");
  HWK_CHECK(experts >= 1 && experts <= 64, "hwk_moe_route: %u experts (1..64)", experts);
  HWK_CHECK(k >= 1 && k <= experts, "hwk_moe_route: k=%u of %u experts", k, experts);
  HWK_CHECK(score == HWK_SCORE_SOFTMAX || score == HWK_SCORE_SIGMOID, "hwk_moe_route: score %d", score);
  if (rows == 0) return nullptr;
  hipLaunchKernelGGL(k_moe_route, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, (const float *)logits,
                     (const float *)bias, (int32_t *)idx, (float *)w, rows, experts, k, score, norm,
                     hwk::f32_of_bits(scale_bits));
  return hwk::launched("hwk_moe_route");
}

// Layout: act (tokens, k, I) fp32.
HWK_API size_t hwk_moe_workspace_bytes(const hwk_moe_params *p) {
  if (!p) return 0;
  return (size_t)p->tokens * p->k * p->inter * sizeof(float);
}

HWK_API char *hwk_moe_experts(void *stream, const void *x, const void *idx, const void *w, const void *gu_w,
                              const void *gu_e, const void *gu_b, const void *dn_w, const void *dn_e,
                              const void *dn_b, void *out, void *workspace, size_t workspace_bytes,
                              const hwk_moe_params *p) {
  HWK_Q(check_params("hwk_moe_experts", p));
  HWK_CHECK(x && idx && w && gu_w && gu_e && dn_w && dn_e && out && workspace, "hwk_moe_experts: null pointer");
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(gu_w, 16) && hwk::aligned(dn_w, 16) && hwk::aligned(workspace, 16),
            "hwk_moe_experts: x, weights and workspace must be 16-byte aligned");
  HWK_CHECK(workspace_bytes >= hwk_moe_workspace_bytes(p), "hwk_moe_experts: workspace %zu bytes, %zu needed",
            workspace_bytes, hwk_moe_workspace_bytes(p));
  return run_experts<false>((hipStream_t)stream, x, nullptr, nullptr, (int32_t *)idx, (float *)w, gu_w, gu_e,
                            (const float *)gu_b, dn_w, dn_e, (const float *)dn_b, (float *)out, (float *)workspace,
                            args_of(p), "hwk_moe_experts");
}

HWK_API char *hwk_moe_layer(void *stream, const void *x, const void *logits, const void *router_bias, void *idx,
                            void *w, const void *gu_w, const void *gu_e, const void *gu_b, const void *dn_w,
                            const void *dn_e, const void *dn_b, void *out, void *workspace, size_t workspace_bytes,
                            const hwk_moe_params *p) {
  HWK_Q(check_params("hwk_moe_layer", p));
  HWK_CHECK(x && logits && idx && w && gu_w && gu_e && dn_w && dn_e && out && workspace,
            "hwk_moe_layer: null pointer");
  HWK_CHECK(p->score == HWK_SCORE_SOFTMAX || p->score == HWK_SCORE_SIGMOID, "hwk_moe_layer: score %u", p->score);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(gu_w, 16) && hwk::aligned(dn_w, 16) && hwk::aligned(workspace, 16),
            "hwk_moe_layer: x, weights and workspace must be 16-byte aligned");
  HWK_CHECK(workspace_bytes >= hwk_moe_workspace_bytes(p), "hwk_moe_layer: workspace %zu bytes, %zu needed",
            workspace_bytes, hwk_moe_workspace_bytes(p));
  const MoeArgs a = args_of(p);
  hipStream_t st = (hipStream_t)stream;
  if (p->tokens <= kFoldRouteMaxTokens)
    return run_experts<true>(st, x, (const float *)logits, (const float *)router_bias, (int32_t *)idx, (float *)w,
                             gu_w, gu_e, (const float *)gu_b, dn_w, dn_e, (const float *)dn_b, (float *)out,
                             (float *)workspace, a, "hwk_moe_layer");
  hipLaunchKernelGGL(k_moe_route, dim3((p->tokens + 3) / 4), dim3(256), 0, st, (const float *)logits,
                     (const float *)router_bias, (int32_t *)idx, (float *)w, p->tokens, p->experts, p->k,
                     (int)p->score, (int)p->norm, a.scale);
  HWK_Q(hwk::launched("hwk_moe_layer (route)"));
  return run_experts<false>(st, x, nullptr, nullptr, (int32_t *)idx, (float *)w, gu_w, gu_e, (const float *)gu_b,
                            dn_w, dn_e, (const float *)dn_b, (float *)out, (float *)workspace, a, "hwk_moe_layer");
}

}  // extern "C"
