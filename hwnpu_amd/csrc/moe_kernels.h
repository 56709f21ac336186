// The device code of the MoE path (K5a routing, K5b experts), shared by libhwk's kernels (moe.hip) and
// the kernels of the library's code object (co/hwk_co.hip), so that both run the same instructions.
//
// MoE on gfx950: the router's top-k choice (K5a) and the chosen experts' gated FFNs (K5b).
//
// K5a restates the reference's Routing.Choose operation for operation (float64 exp rounded to
// float32, a sequential float32 sum, a stable descending order) in one wave per token with lane j
// holding expert j, so that the chosen expert ids are the reference's bit for bit.
//
// K5b is two launches and needs nothing from the host between them. The gate_up kernel gives each
// (chosen expert, row-pair tile) to a workgroup: with the route folded in (hwk_moe_layer) every
// workgroup derives the token's choice from the router logits itself (read off the logits' order
// where that provably equals Choose's, so that its weight loads issue before Choose has run, in a
// workgroup of its own that writes idx and w; else by Choose first); otherwise it reads the given
// idx. It reads the expert's rows once for all tokens that chose it, adds the gate/up biases,
// and writes the gated unit (SiLU, or gpt-oss's clamped one) in fp32 (it overflows fp16 at the
// benchmark's scales). The down kernel gives each workgroup a tile of output rows for every chosen
// expert (its waves take the experts in turn, all their rows' loads issued at once) and then adds,
// for each token, w * (y + down bias) in ascending expert id, the reference's summation order
// (host.go:566-578,866-881), with no atomics.
#pragma once

#include "hwk_common.h"

namespace hwk_moe {


// ---- K5a ----

// A lane's float as a wave-uniform value (v_readlane: no LDS round trip).
__device__ __forceinline__ float lane_f(float v, uint32_t j) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)j));
}

// Routing.Choose (internal/llm/experts/weights.go:33-81) of one row of E <= 64 logits by one wave,
// lane j holding expert j, reading other lanes' values with v_readlane only (no LDS, no barrier):
// softmax scores in float32 (exp in float64 rounded to float32, the sum taken in expert order), or
// sigmoid; the rank of each expert in a stable descending sort of score + bias (ties to the lower
// index); the first k (idx, w) with w the chosen scores over their float32 sum + 1e-6 (norm), times
// scale unless 0. Lanes < k write idx_out/w_out.
__device__ void choose_wave(const float *__restrict__ logits, const float *__restrict__ bias, uint32_t E, uint32_t k,
                            int score, int norm, float scale, int32_t *idx_out, float *w_out) {
#pragma clang fp contract(off)
  const uint32_t lane = threadIdx.x & 63;
  const bool live = lane < E;
  const float v = live ? logits[lane] : -__builtin_inff();
  const float bl = bias && live ? bias[lane] : 0.0f;
  float s;
  if (score == HWK_SCORE_SOFTMAX) {
    const float m = group_max_dpp<64>(v);
    const float ex = live ? (float)exp((double)(v - m)) : 0.0f;
    float total = 0.0f;
    for (uint32_t j = 0; j < E; j++) total += lane_f(ex, j);
    s = ex / total;
  } else {
    s = 1.0f / (1.0f + (float)exp((double)(-v)));
  }
  const float kv = bias && live ? s + bl : s;
  uint32_t rank = 0;
  for (uint32_t j = 0; j < E; j++) {
    const float kj = lane_f(kv, j);
    rank += (kj > kv) || (kj == kv && j < lane);
  }
  // the k chosen in rank order: lane r learns the expert of rank r and its score
  int my_e = -1;
  float my_w = 0.0f, sum = 0.0f;
  for (uint32_t r = 0; r < k; r++) {
    const uint64_t who = __ballot(live && rank == r);
    const uint32_t src = who ? (uint32_t)__builtin_ctzll(who) : 0u;  // no such rank only with NaN scores
    const float wr = lane_f(s, src);
    sum += wr;
    if (lane == r) {
      my_e = (int)src;
      my_w = wr;
    }
  }
  if (lane < k) {
    float wj = my_w;
    if (norm) wj /= sum + 1e-6f;
    if (scale != 0.0f) wj *= scale;
    idx_out[lane] = my_e;
    w_out[lane] = wj;
  }
}

// Routing.Choose's choice read off the logits alone, where that provably gives Choose's experts in
// Choose's order (softmax scores, no bias): rank by d = logit - max (the float32 difference Choose
// exponentiates; softmax is monotone in it), ties to the lower index. The choice is Choose's when the
// d of consecutive ranks 0 .. min(k, E-1) differ by at least 2^-20 (their float64 exps then differ by
// a factor above 1 + 9.5e-7, so their float32 roundings, and the roundings of those over the same
// sum, differ: a float32 rounding moves a value by at most 2^-24 of it) and the last chosen has
// d >= -80 (every chosen score a normal float32). Returns that, the same in every wave; every wave
// gets the chosen set of the T tokens as mask, and wave 0 writes token t's choice in rank order to
// ch[t*k ..].
__device__ __forceinline__ bool spec_choice(const float *__restrict__ logits, uint32_t T, uint32_t E, uint32_t k,
                                            int32_t *ch, uint64_t &mask) {
  const uint32_t lane = threadIdx.x & 63;
  const bool live = lane < E, w0 = threadIdx.x < 64;
  const uint32_t kk = k < E ? k : E;  // the chosen a token
  bool ok = true;
  mask = 0;
  for (uint32_t t = 0; t < T; t++) {
    const float v = live ? logits[(size_t)t * E + lane] : -__builtin_inff();
    const float m = group_max_dpp<64>(v);
    const float d = v - m;
    uint32_t rank = 0;
    for (uint32_t j = 0; j < E; j++) {
      const float dj = lane_f(d, j);
      rank += (dj > d) || (dj == d && j < lane);
    }
    ok = ok && !__ballot(live && !(d == d));  // no NaN
    float prev = 0.0f;
    for (uint32_t r = 0; r <= kk && r < E; r++) {
      const uint64_t who = __ballot(live && rank == r);
      if (!who) {
        ok = false;
        break;
      }
      const float dr = lane_f(d, (uint32_t)__builtin_ctzll(who));
      if (r > 0 && !(prev - dr >= 0x1p-20f)) ok = false;
      if (r + 1 == kk && !(dr >= -80.0f)) ok = false;
      prev = dr;
    }
    if (w0 && live && rank < k) ch[t * k + rank] = (int32_t)lane;
    mask |= __ballot(live && rank < k);
  }
  return ok;
}

// ---- K5b helpers ----

// dst[0, n) = src[0, n) (16-byte items) by the 256 threads of a workgroup, every thread's loads of
// a pass (up to SPT) issued before its stores, so that a pass waits on one memory latency, not SPT.
// Native vectors: an array of HIP's uint4 (a union) would be left in scratch memory.
template <int SPT, int NT = 256>
__device__ __forceinline__ void stage_copy(void *dstv, const void *__restrict__ srcv, uint32_t n) {
  typedef uint32_t V __attribute__((ext_vector_type(4)));
  V *dst = (V *)dstv;
  const V *src = (const V *)srcv;
  for (uint32_t base = 0; base < n; base += NT * SPT) {
    V r[SPT];
#pragma unroll
    for (int j = 0; j < SPT; j++) r[j] = src[min(base + j * NT + threadIdx.x, n - 1)];
#pragma unroll
    for (int j = 0; j < SPT; j++) {
      const uint32_t i = base + j * NT + threadIdx.x;
      if (i < n) dst[i] = r[j];
    }
  }
}

// The set of experts idx names (n entries) as a bit mask, the same in every lane: ids outside
// [0, E) name none (E <= 64).
__device__ __forceinline__ uint64_t chosen_mask(const int32_t *idx, uint32_t n, uint32_t E) {
  const int lane = threadIdx.x & 63;
  bool hit = false;
  for (uint32_t j = 0; j < n; j++) hit |= idx[j] == lane;
  return __ballot(hit && (uint32_t)lane < E);
}

// The slot of expert e among token t's k choices, -1 if none (uniform).
__device__ __forceinline__ int slot_of(const int32_t *idx, uint32_t t, uint32_t k, int e) {
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

// ---- K5b stage 1: route (optional), gate_up + bias, the gated unit ----

struct MoeArgs {
  uint32_t T, H, I, E, k;
  int act;  // HWK_ACT_SILU or HWK_ACT_GPTOSS
  int score, norm;
  float alpha, limit, scale;
  int mode;  // out_mode of the down stage
};

// The gated unit of one (gate, up) pair (host.go:516-527): SiLU g/(1+e^-g)*u, or gpt-oss's
// min(g, L)/(1+e^(-a*min(g, L))) * (clamp(u, -L, L) + 1), exp in float64 rounded to float32, every
// other step a float32 operation of its own.
__device__ __forceinline__ float gated(float g, float u, const MoeArgs &a) {
#pragma clang fp contract(off)
  if (a.act == HWK_ACT_GPTOSS) {
    g = fminf(g, a.limit);
    u = fminf(fmaxf(u, -a.limit), a.limit);
    return g / (1.0f + (float)exp((double)(-(a.alpha * g)))) * (u + 1.0f);
  }
  return g / (1.0f + (float)exp((double)(-g))) * u;
}

// Workgroup (row-pair tile bx, chosen expert number by in ascending id). 64 lanes
// a row, BPL blocks a lane (nb = H/32 <= 64*BPL); a wave takes PPW row pairs (gate 2j, up 2j+1).
// ROUTE: the workgroup routes every token from the logits first (waves over tokens), and workgroup
// (0, 0) writes idx and w; else idx is given. x is read from global memory per token after the
// weight loads are issued (an LDS copy of x first only delays the weight loads).
template <int BPL, int PPW, bool ROUTE>
__device__ __forceinline__ void moe_gate_up_wg(uint32_t bx, uint32_t by, const uint4 *__restrict__ x,
                                               const float *__restrict__ logits, const float *__restrict__ rbias,
                                               int32_t *__restrict__ idx, float *__restrict__ wout,
                                               const uint4 *__restrict__ gw, const uint8_t *__restrict__ ge,
                                               const float *__restrict__ gb, float *__restrict__ act, MoeArgs a) {
  __shared__ int32_t sidx[64];
  __shared__ float sw[64];
  __shared__ float gsum[PPW == 2 ? 1 : 2 * 64 * 4 * PPW];  // (token, wave, pair) -> (gate, up) sums
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t n = a.T * a.k;
  uint64_t mask = 0;
  bool spec = false;  // the choice read off the logits (spec_choice), the weight loads issued before Choose
  if constexpr (ROUTE) {
    if (!rbias && a.score == HWK_SCORE_SOFTMAX) spec = spec_choice(logits, a.T, a.E, a.k, sidx, mask);
    if (bx == (a.I + 4 * PPW - 1) / (4 * PPW)) {
      // the route's own workgroup (one column past the experts' tiles): Choose's idx and w, beside
      // the experts' loads; without the logits' choice the experts' workgroups route themselves
      if (spec && by == 0)
        for (uint32_t t = wave; t < a.T; t += 4)
          choose_wave(logits + (size_t)t * a.E, rbias, a.E, a.k, a.score, a.norm, a.scale, idx + t * a.k,
                      wout + t * a.k);
      return;
    }
    if (!spec) {
      for (uint32_t t = wave; t < a.T; t += 4)
        choose_wave(logits + (size_t)t * a.E, rbias, a.E, a.k, a.score, a.norm, a.scale, sidx + t * a.k,
                    sw + t * a.k);
      __syncthreads();
      if (bx == 0 && by == 0 && threadIdx.x < n) {
        idx[threadIdx.x] = sidx[threadIdx.x];
        wout[threadIdx.x] = sw[threadIdx.x];
      }
      mask = chosen_mask(sidx, n, a.E);
    }
  } else {
    if (threadIdx.x < n) sidx[threadIdx.x] = idx[threadIdx.x];
    __syncthreads();
    mask = chosen_mask(sidx, n, a.E);
  }
  const uint32_t u = by;
  if (u >= (uint32_t)__builtin_popcountll(mask)) return;
  for (uint32_t i = 0; i < u; i++) mask &= mask - 1;
  const int e = __builtin_ctzll(mask);
  const uint32_t nb = a.H / 32, I = a.I;
  const uint32_t pair0 = (bx * 4 + wave) * PPW;
  const size_t erow = (size_t)e * 2 * I;  // the expert's first row
  // every load issued unconditionally from a clamped row / block (a load under a branch is waited
  // for where the branches join): terms of blocks past nb are dropped, rows past I not written
  uint4 c[PPW][2][BPL];
  uint32_t s[PPW][2][BPL];
#pragma unroll
  for (int p = 0; p < PPW; p++)
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int j = 0; j < BPL; j++) {
        const uint32_t pair = min(pair0 + p, I - 1), b = min((uint32_t)(j * 64 + lane), nb - 1);
        const size_t blk = (erow + 2 * pair + r) * nb + b;
        c[p][r][j] = load_stream(&gw[blk]);
        s[p][r][j] = ge[blk];
      }
  float bias[PPW][2];
#pragma unroll
  for (int p = 0; p < PPW; p++)
#pragma unroll
    for (int r = 0; r < 2; r++) bias[p][r] = gb ? gb[erow + 2 * min(pair0 + p, I - 1) + r] : 0.0f;
  if (spec) {
    // wave 0's choice in sidx: its LDS writes done, then a bare barrier (__syncthreads would wait
    // for the weight loads above too)
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
  }
  for (uint32_t t = 0; t < a.T; t++) {
    const int slot = slot_of(sidx, t, a.k, e);
    if (slot < 0) continue;
    uint4 xr[BPL][4];
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const uint32_t b = min((uint32_t)(j * 64 + lane), nb - 1);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const size_t xi = ((size_t)t * a.H + b * 32) / 8 + q;
        xr[j][q] = x[xi];
      }
    }
    float gl = 0.0f, ul = 0.0f;  // PPW == 2: lane p's pair
#pragma unroll
    for (int p = 0; p < PPW; p++) {
      float gu[2];
#pragma unroll
      for (int r = 0; r < 2; r++) {
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < BPL; j++) {
          const float term = dot_block_f16(c[p][r][j], xr[j]) * e8m0_scale(s[p][r][j]);
          v += (uint32_t)(j * 64 + lane) < nb ? term : 0.0f;
        }
        gu[r] = group_sum<64>(v) + bias[p][r];
      }
      if constexpr (PPW == 2) {
        if (lane == p) {
          gl = gu[0];
          ul = gu[1];
        }
      } else if (lane == 0) {
        gsum[2 * ((t * 4 + wave) * PPW + p)] = gu[0];
        gsum[2 * ((t * 4 + wave) * PPW + p) + 1] = gu[1];
      }
    }
    // PPW == 2: both pairs' gated units (a float64 exp) in one instruction stream, a pair a lane
    if constexpr (PPW == 2) {
      const uint32_t pair = pair0 + lane;
      if (lane < PPW && pair < I) act[((size_t)t * a.k + slot) * I + pair] = gated(gl, ul, a);
    }
  }
  if constexpr (PPW == 2) return;
  // with 4 pairs a wave (past 2 tokens): the gated unit (a float64 exp) a (token, pair) a thread over
  // the workgroup, not by each wave with its lanes computing the same value (at 2 pairs a wave the
  // barrier costs more than it saves)
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < a.T * 4 * PPW; i += 256) {
    const uint32_t t = i / (4 * PPW), w = (i / PPW) % 4, p = i % PPW;
    const int slot = slot_of(sidx, t, a.k, e);
    const uint32_t pair = (bx * 4 + w) * PPW + p;
    if (slot >= 0 && pair < I) act[((size_t)t * a.k + slot) * I + pair] = gated(gsum[2 * i], gsum[2 * i + 1], a);
  }
}

// ---- K5b stage 2: down for every chosen expert, then the ordered combine ----
// Workgroup: RS = 64/LPR output rows (row0 + lane/LPR), 4 waves; wave wv takes the chosen experts
// u = wv, wv+4, ... (ascending id), EPW of them at a time with all their rows' loads issued at
// once; LPR lanes a row, BPL blocks a lane (nb = I/32 <= LPR*BPL). Each expert's rows are read once
// for every token that chose it, its unweighted y kept in LDS by (token slot, row). Then one thread
// a (token, row) adds w * (y + down bias) over the token's experts in ascending expert id. AL: the
// activations (T*k, I) fp32 are copied into LDS (dynamic) after the first experts' weight loads are
// issued, so that the products wait on no global load.
template <int LPR, int BPL, int EPW, bool AL, int NW>
__device__ __forceinline__ void moe_down_wg(uint32_t bx, const float *__restrict__ act, const int32_t *__restrict__ idx,
                                            const float *__restrict__ w, const uint4 *__restrict__ dw,
                                            const uint8_t *__restrict__ de, const float *__restrict__ db,
                                            float *__restrict__ out, MoeArgs a) {
  constexpr int RS = 64 / LPR;
  __shared__ int32_t sidx[64];
  __shared__ float sw[64];
  __shared__ float ys[64 * RS];  // (token slot, row)
  extern __shared__ float4 ash[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l = lane % LPR;
  const uint32_t n = a.T * a.k, H = a.H, nb = a.I / 32;
  if (threadIdx.x < n) {
    sidx[threadIdx.x] = idx[threadIdx.x];
    sw[threadIdx.x] = w[threadIdx.x];
  }
  __syncthreads();
  const uint64_t mask = chosen_mask(sidx, n, a.E);
  const uint32_t U = (uint32_t)__builtin_popcountll(mask);
  const uint32_t e0 = mask ? (uint32_t)__builtin_ctzll(mask) : 0u;  // the rows padding slots read
  const uint32_t row0 = bx * RS, row = row0 + lane / LPR;
  const uint32_t rowc = row < H ? row : H - 1;
  const float4 *act4 = (const float4 *)act;
  bool staged = !AL;
  for (uint32_t base = wave; base < U + NW * EPW * (staged ? 0 : 1); base += NW * EPW) {
    uint4 c[EPW][BPL];
    uint32_t sc[EPW][BPL];
    int ex[EPW];
    // every load issued unconditionally (a load under a branch is waited for where the branches
    // join): slots past the chosen experts read the first chosen expert's rows, blocks past nb the
    // last block; their terms are dropped
#pragma unroll
    for (int i = 0; i < EPW; i++) {
      const uint32_t u = base + NW * i;
      uint64_t m = mask;
      for (uint32_t q = 0; q < u && m; q++) m &= m - 1;
      ex[i] = u < U ? __builtin_ctzll(m) : -1;
      const uint32_t el = u < U ? (uint32_t)__builtin_ctzll(m) : e0;
#pragma unroll
      for (int j = 0; j < BPL; j++) {
        const uint32_t b = min((uint32_t)(j * LPR + l), nb - 1);
        const size_t blk = ((size_t)el * H + rowc) * nb + b;
        c[i][j] = load_stream(&dw[blk]);
        sc[i][j] = de[blk];
      }
    }
    if (!staged) {  // once, behind the first weight loads: every wave of the workgroup takes part
      stage_copy<16, 64 * NW>(ash, act4, n * a.I / 4);
      __syncthreads();
      staged = true;
    }
#pragma unroll
    for (int i = 0; i < EPW; i++) {
      if (ex[i] < 0) continue;
      for (uint32_t t = 0; t < a.T; t++) {
        const int slot = slot_of(sidx, t, a.k, ex[i]);
        if (slot < 0) continue;
        const size_t a0 = ((size_t)t * a.k + slot) * a.I / 4;
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < BPL; j++) {
          const uint32_t b = min((uint32_t)(j * LPR + l), nb - 1);
          float4 av[8];
#pragma unroll
          for (int q = 0; q < 8; q++) av[q] = AL ? ash[a0 + b * 8 + q] : act4[a0 + b * 8 + q];
          const float term = dot_block_f32(c[i][j], av) * e8m0_scale(sc[i][j]);
          v += (uint32_t)(j * LPR + l) < nb ? term : 0.0f;
        }
        const float y = group_sum<LPR>(v);
        if (l == 0) ys[(t * a.k + slot) * RS + lane / LPR] = y;
      }
    }
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < a.T * RS; i += 64 * NW) {
#pragma clang fp contract(off)
    const uint32_t t = i / RS, r = i % RS, orow = row0 + r;
    if (orow >= H) continue;
    float acc = a.mode == HWK_OUT_ADD_F32 ? out[(size_t)t * H + orow] : 0.0f;
    int prev = -1;
    for (uint32_t q = 0; q < a.k; q++) {
      int best = 1 << 30;
      uint32_t bs = 0;
      for (uint32_t j = 0; j < a.k; j++) {
        const int e = sidx[t * a.k + j];
        if (e > prev && e < best) {
          best = e;
          bs = j;
        }
      }
      if (best >= (int)a.E) break;  // an id outside [0, E) (a caller's error): no term
      const float bias = db ? db[(size_t)best * H + orow] : 0.0f;
      acc += sw[t * a.k + bs] * (ys[(t * a.k + bs) * RS + r] + bias);
      prev = best;
    }
    out[(size_t)t * H + orow] = acc;
  }
}

}  // namespace hwk_moe
