// MoE on gfx950: the router's top-k choice (K5a) and the chosen experts' SwiGLU FFNs (K5b).
//
// K5a is one wave per token and restates the reference's Routing.Choose operation for operation
// (float64 exp rounded to float32, a sequential float32 sum, a stable descending order), so that
// the chosen expert ids are the reference's bit for bit.
//
// K5b is three launches and needs nothing from the host between them: every workgroup derives the
// sorted set of chosen experts from idx itself (a 64-bit ballot of the expert ids). The gate_up
// kernel gives each (chosen expert, row-pair tile) to a workgroup, reads the expert's rows once
// for all tokens that chose it, and writes silu(gate)*up in fp32 (it overflows fp16 at the
// benchmark's scales). The down kernel does the same for (chosen expert, row tile), so that every
// expert's rows stream in parallel, and leaves each token's per-expert outputs in fp32; the combine
// adds w * y for each token in ascending expert id, the reference's summation order
// (host.go:566-578,866-881), with no atomics.
#include "hwk_common.h"

namespace {

// ---- K5a ----

__global__ __launch_bounds__(64) void k_moe_route(const float *__restrict__ logits, const float *__restrict__ bias,
                                                  int32_t *__restrict__ idx, float *__restrict__ w, uint32_t E,
                                                  uint32_t k, int score, int norm, float scale) {
#pragma clang fp contract(off)
  __shared__ float sc[64], key[64], chosen_w[64];
  __shared__ int chosen_e[64];
  __shared__ float total;
  const uint32_t row = blockIdx.x, lane = threadIdx.x;
  const bool live = lane < E;
  const float v = live ? logits[(size_t)row * E + lane] : -__builtin_inff();
  float s;
  if (score == HWK_SCORE_SOFTMAX) {
    float m = v;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    const float d = v - m;
    const float ex = live ? (float)exp((double)d) : 0.0f;
    sc[lane] = ex;
    __syncthreads();
    if (lane == 0) {
      float sum = 0.0f;
      for (uint32_t j = 0; j < E; j++) sum += sc[j];
      total = sum;
    }
    __syncthreads();
    s = ex / total;
  } else {
    s = 1.0f / (1.0f + (float)exp((double)(-v)));
  }
  const float kv = bias && live ? s + bias[lane] : s;
  key[lane] = kv;
  __syncthreads();
  // position in a stable descending sort: larger keys first, equal keys by index
  uint32_t rank = 0;
  for (uint32_t j = 0; j < E; j++) {
    const float kj = key[j];
    rank += (kj > kv) || (kj == kv && j < lane);
  }
  if (live && rank < k) {
    chosen_e[rank] = (int)lane;
    chosen_w[rank] = s;
  }
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (uint32_t j = 0; j < k; j++) sum += chosen_w[j];
    total = sum;
  }
  __syncthreads();
  if (lane < k) {
    float wj = chosen_w[lane];
    if (norm) wj /= total + 1e-6f;
    if (scale != 0.0f) wj *= scale;
    idx[(size_t)row * k + lane] = chosen_e[lane];
    w[(size_t)row * k + lane] = wj;
  }
}

// ---- K5b helpers ----

// The set of experts idx names (n entries, experts < 64) as a bit mask, the same in every lane.
__device__ __forceinline__ uint64_t chosen_mask(const int32_t *__restrict__ idx, uint32_t n) {
  const int lane = threadIdx.x & 63;
  bool hit = false;
  for (uint32_t j = 0; j < n; j++) hit |= idx[j] == lane;
  return __ballot(hit);
}

// The slot of expert e among token t's k choices, -1 if none (uniform).
__device__ __forceinline__ int slot_of(const int32_t *__restrict__ idx, uint32_t t, uint32_t k, int e) {
  for (uint32_t j = 0; j < k; j++)
    if (idx[t * k + j] == e) return (int)j;
  return -1;
}

// sum over a 32-value block: codes (16 bytes) as fp16 pairs against x in fp16 pairs (v_dot2)
__device__ __forceinline__ float dot_block_f16(uint4 c, const uint4 (&x)[4]) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<0>(cw[q]), h2_of_bits(x[q].x), d0, false);
    d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<1>(cw[q]), h2_of_bits(x[q].y), d1, false);
    d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<2>(cw[q]), h2_of_bits(x[q].z), d0, false);
    d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<3>(cw[q]), h2_of_bits(x[q].w), d1, false);
  }
  return d0 + d1;
}

// the same against fp32 activations a[32] (mixed-precision multiply-adds)
__device__ __forceinline__ float dot_block_f32(uint4 c, const float4 (&a)[8]) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const h2 p0 = fp4x2_to_h2<0>(cw[q]), p1 = fp4x2_to_h2<1>(cw[q]);
    const h2 p2 = fp4x2_to_h2<2>(cw[q]), p3 = fp4x2_to_h2<3>(cw[q]);
    const float4 a0 = a[2 * q], a1 = a[2 * q + 1];
    d0 = fmaf((float)p0.x, a0.x, d0);
    d1 = fmaf((float)p0.y, a0.y, d1);
    d0 = fmaf((float)p1.x, a0.z, d0);
    d1 = fmaf((float)p1.y, a0.w, d1);
    d0 = fmaf((float)p2.x, a1.x, d0);
    d1 = fmaf((float)p2.y, a1.y, d1);
    d0 = fmaf((float)p3.x, a1.z, d0);
    d1 = fmaf((float)p3.y, a1.w, d1);
  }
  return d0 + d1;
}

// ---- K5b stage 1: gate_up + SwiGLU ----
// Workgroup (row-pair tile blockIdx.x, chosen expert number blockIdx.y in ascending id). 64 lanes
// a row, BPL blocks a lane (nb = H/32 <= 64*BPL); a wave takes PPW row pairs (gate 2j, up 2j+1).
template <int BPL, int PPW>
__global__ __launch_bounds__(256) void k_moe_gate_up(const uint4 *__restrict__ x, const int32_t *__restrict__ idx,
                                                     const uint4 *__restrict__ gw, const uint8_t *__restrict__ ge,
                                                     float *__restrict__ act, uint32_t T, uint32_t H, uint32_t I,
                                                     uint32_t k) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t mask = chosen_mask(idx, T * k);
  const uint32_t u = blockIdx.y;
  if (u >= (uint32_t)__builtin_popcountll(mask)) return;
  for (uint32_t i = 0; i < u; i++) mask &= mask - 1;
  const int e = __builtin_ctzll(mask);
  const uint32_t nb = H / 32;
  const uint32_t pair0 = (blockIdx.x * 4 + wave) * PPW;
  const size_t erow = (size_t)e * 2 * I;  // the expert's first row
  uint4 c[PPW][2][BPL];
  uint32_t s[PPW][2][BPL];
#pragma unroll
  for (int p = 0; p < PPW; p++)
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int j = 0; j < BPL; j++) {
        const uint32_t pair = pair0 + p, b = j * 64 + lane;
        if (pair < I && b < nb) {
          const size_t blk = (erow + 2 * pair + r) * nb + b;
          c[p][r][j] = load_stream(&gw[blk]);
          s[p][r][j] = ge[blk];
        } else {
          c[p][r][j] = make_uint4(0, 0, 0, 0);
          s[p][r][j] = 0;
        }
      }
  for (uint32_t t = 0; t < T; t++) {
    const int slot = slot_of(idx, t, k, e);
    if (slot < 0) continue;
    uint4 xr[BPL][4];
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const uint32_t b = j * 64 + lane;
#pragma unroll
      for (int q = 0; q < 4; q++) xr[j][q] = b < nb ? x[((size_t)t * H + b * 32) / 8 + q] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < PPW; p++) {
      float gu[2];
#pragma unroll
      for (int r = 0; r < 2; r++) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < BPL; j++) a += dot_block_f16(c[p][r][j], xr[j]) * e8m0_scale(s[p][r][j]);
        gu[r] = group_sum<64>(a);
      }
      const uint32_t pair = pair0 + p;
      if (lane == 0 && pair < I) {
        const float g = gu[0];
        act[((size_t)t * k + slot) * I + pair] = g / (1.0f + expf(-g)) * gu[1];
      }
    }
  }
}

// ---- K5b stage 2: down, one chosen expert a workgroup column ----
// Workgroup (row tile blockIdx.x, chosen expert number blockIdx.y in ascending id), one wave: LPR
// lanes a row (RS = 64/LPR rows), BPL blocks a lane (nb = I/32 <= LPR*BPL). The expert's rows are
// read once for all the tokens that chose it; y = down(act) goes unweighted to ydown (tokens, k, H)
// at the token's slot of that expert.
template <int LPR, int BPL>
__global__ __launch_bounds__(64) void k_moe_down(const float *__restrict__ act, const int32_t *__restrict__ idx,
                                                 const uint4 *__restrict__ dw, const uint8_t *__restrict__ de,
                                                 float *__restrict__ ydown, uint32_t T, uint32_t H, uint32_t I,
                                                 uint32_t k) {
  constexpr int RS = 64 / LPR;
  const int lane = threadIdx.x & 63, l = lane % LPR;
  const uint32_t row = blockIdx.x * RS + lane / LPR;
  uint64_t mask = chosen_mask(idx, T * k);
  const uint32_t u = blockIdx.y;
  if (u >= (uint32_t)__builtin_popcountll(mask)) return;
  for (uint32_t i = 0; i < u; i++) mask &= mask - 1;
  const int e = __builtin_ctzll(mask);
  const uint32_t nb = I / 32;
  uint4 c[BPL];
  uint32_t sc[BPL];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const uint32_t b = j * LPR + l;
    if (row < H && b < nb) {
      const size_t blk = ((size_t)e * H + row) * nb + b;
      c[j] = load_stream(&dw[blk]);
      sc[j] = de[blk];
    } else {
      c[j] = make_uint4(0, 0, 0, 0);
      sc[j] = 0;
    }
  }
  for (uint32_t t = 0; t < T; t++) {
    const int slot = slot_of(idx, t, k, e);
    if (slot < 0) continue;
    const float *ar = act + ((size_t)t * k + slot) * I;
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const uint32_t b = j * LPR + l;
      float4 av[8];
#pragma unroll
      for (int q = 0; q < 8; q++) av[q] = b < nb ? ((const float4 *)(ar + b * 32))[q] : make_float4(0, 0, 0, 0);
      a += dot_block_f32(c[j], av) * e8m0_scale(sc[j]);
    }
    const float y = group_sum<LPR>(a);
    if (l == 0 && row < H) ydown[((size_t)t * k + slot) * H + row] = y;
  }
}

// ---- K5b stage 3: the ordered combine ----
// out[t][r] (+)= sum over token t's experts in ascending expert id of w * y (the reference's order,
// host.go:566-578,866-881), one thread an output.
__global__ __launch_bounds__(256) void k_moe_combine(const float *__restrict__ ydown, const int32_t *__restrict__ idx,
                                                     const float *__restrict__ w, float *__restrict__ out, uint32_t T,
                                                     uint32_t H, uint32_t k, int mode) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= T * H) return;
  const uint32_t t = i / H, r = i % H;
  float acc = mode == HWK_OUT_ADD_F32 ? out[i] : 0.0f;
  int prev = -1;
  for (uint32_t n = 0; n < k; n++) {
    int best = 1 << 30;
    uint32_t bs = 0;
    for (uint32_t j = 0; j < k; j++) {
      const int e = idx[t * k + j];
      if (e > prev && e < best) {
        best = e;
        bs = j;
      }
    }
    acc += w[t * k + bs] * ydown[((size_t)t * k + bs) * H + r];
    prev = best;
  }
  out[i] = acc;
}

template <int LPR, int BPL>
void launch_down(hipStream_t st, const float *act, const int32_t *idx, const void *dw, const void *de, float *ydown,
                 const hwk_moe_params *p, uint32_t unique_max) {
  constexpr uint32_t rows = 64 / LPR;
  hipLaunchKernelGGL((k_moe_down<LPR, BPL>), dim3((p->hidden + rows - 1) / rows, unique_max), dim3(64), 0, st, act,
                     idx, (const uint4 *)dw, (const uint8_t *)de, ydown, p->tokens, p->hidden, p->inter, p->k);
}

}  // namespace

extern "C" {

HWK_API char *hwk_moe_route(void *stream, const void *logits, const void *bias, void *idx, void *w, uint32_t rows,
                            uint32_t experts, uint32_t k, int score, int norm, uint32_t scale_bits) {
  HWK_CHECK(logits && idx && w, "hwk_moe_route: null pointer");
  HWK_CHECK(experts >= 1 && experts <= 64, "hwk_moe_route: %u experts (1..64)", experts);
  HWK_CHECK(k >= 1 && k <= experts, "hwk_moe_route: k=%u of %u experts", k, experts);
  HWK_CHECK(score == HWK_SCORE_SOFTMAX || score == HWK_SCORE_SIGMOID, "hwk_moe_route: score %d", score);
  if (rows == 0) return nullptr;
  hipLaunchKernelGGL(k_moe_route, dim3(rows), dim3(64), 0, (hipStream_t)stream, (const float *)logits,
                     (const float *)bias, (int32_t *)idx, (float *)w, experts, k, score, norm,
                     hwk::f32_of_bits(scale_bits));
  return hwk::launched("hwk_moe_route");
}

// Layout: act (tokens, k, I) fp32 | ydown (tokens, k, H) fp32.
HWK_API size_t hwk_moe_workspace_bytes(const hwk_moe_params *p) {
  if (!p) return 0;
  return (size_t)p->tokens * p->k * (p->inter + p->hidden) * sizeof(float);
}

HWK_API char *hwk_moe_experts(void *stream, const void *x, const void *idx, const void *w, const void *gu_w,
                              const void *gu_e, const void *dn_w, const void *dn_e, void *out, void *workspace,
                              size_t workspace_bytes, const hwk_moe_params *p) {
  HWK_CHECK(p, "hwk_moe_experts: null params");
  HWK_CHECK(x && idx && w && gu_w && gu_e && dn_w && dn_e && out && workspace, "hwk_moe_experts: null pointer");
  HWK_CHECK(p->tokens >= 1 && p->tokens <= 8, "hwk_moe_experts: %u tokens (1..8)", p->tokens);
  HWK_CHECK(p->experts >= 1 && p->experts <= 64, "hwk_moe_experts: %u experts (1..64)", p->experts);
  HWK_CHECK(p->k >= 1 && p->k <= p->experts && p->tokens * p->k <= 64, "hwk_moe_experts: k=%u", p->k);
  HWK_CHECK(p->hidden % 32 == 0 && p->hidden > 0 && p->hidden <= 8192, "hwk_moe_experts: hidden %u", p->hidden);
  HWK_CHECK(p->inter % 32 == 0 && p->inter > 0 && p->inter <= 8192, "hwk_moe_experts: inter %u", p->inter);
  HWK_CHECK(p->out_mode == HWK_OUT_F32 || p->out_mode == HWK_OUT_ADD_F32, "hwk_moe_experts: out_mode %u", p->out_mode);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(gu_w, 16) && hwk::aligned(dn_w, 16) && hwk::aligned(workspace, 16),
            "hwk_moe_experts: x, weights and workspace must be 16-byte aligned");
  HWK_CHECK(workspace_bytes >= hwk_moe_workspace_bytes(p), "hwk_moe_experts: workspace %zu bytes, %zu needed",
            workspace_bytes, hwk_moe_workspace_bytes(p));
  hipStream_t st = (hipStream_t)stream;
  float *act = (float *)workspace;
  const int32_t *id = (const int32_t *)idx;
  const uint32_t unique_max = p->tokens * p->k < p->experts ? p->tokens * p->k : p->experts;
  constexpr int PPW = 2;
  const dim3 g1((p->inter + 4 * PPW - 1) / (4 * PPW), unique_max);
  const uint32_t nbh = p->hidden / 32;
  const int bpl1 = (int)((nbh + 63) / 64);
#define HWK_GU(B) \
  hipLaunchKernelGGL((k_moe_gate_up<B, PPW>), g1, dim3(256), 0, st, (const uint4 *)x, id, (const uint4 *)gu_w, \
                     (const uint8_t *)gu_e, act, p->tokens, p->hidden, p->inter, p->k)
  switch (bpl1) {
    case 1: HWK_GU(1); break;
    case 2: HWK_GU(2); break;
    case 3: HWK_GU(3); break;
    default: HWK_GU(4); break;
  }
#undef HWK_GU
  if (char *err = hwk::launched("hwk_moe_experts (gate_up)")) return err;
  // down: lanes a row by I/32 blocks, the fewest idle slots (8 lanes x 3 blocks for I = 768)
  const uint32_t nbi = p->inter / 32;
  float *yd = act + (size_t)p->tokens * p->k * p->inter;
  if (nbi <= 8) launch_down<8, 1>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else if (nbi <= 16) launch_down<16, 1>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else if (nbi <= 24) launch_down<8, 3>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else if (nbi <= 32) launch_down<32, 1>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else if (nbi <= 64) launch_down<64, 1>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else if (nbi <= 128) launch_down<64, 2>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else if (nbi <= 192) launch_down<64, 3>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  else launch_down<64, 4>(st, act, id, dn_w, dn_e, yd, p, unique_max);
  if (char *err = hwk::launched("hwk_moe_experts (down)")) return err;
  const uint32_t n = p->tokens * p->hidden;
  hipLaunchKernelGGL(k_moe_combine, dim3((n + 255) / 256), dim3(256), 0, st, yd, id, (const float *)w, (float *)out,
                     p->tokens, p->hidden, p->k, (int)p->out_mode);
  return hwk::launched("hwk_moe_experts (combine)");
}

}  // extern "C"
