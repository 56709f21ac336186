// GQA decode attention (K4) on gfx950: one query token per head over an fp16 or int8 KV cache.
//
// The context is split over workgroups (split-K). A workgroup owns one KV head and a chunk of
// keys; its four waves take the chunk's 16-key tiles in turn, each with the next tile's loads in
// flight while it computes the current one:
//   - scores: the G query heads of the KV head (padded to the MFMA's 16 rows) times the tile's
//     keys on the fp16 MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation); a lane loads 16 bytes
//     of one key row straight from HBM as its B operand, so no cross-lane reduction is needed;
//   - an online softmax in fp32 (base 2) per head, the running max kept wave-uniform;
//   - P.V on the vector ALUs in fp32 (P stays fp32; a lane holds 8 dims of one key), so the
//     weights are never rounded to fp16.
// The waves merge in LDS; with one chunk a head the workgroup writes the output, else one
// unnormalized output, max and sum per query head to a workspace that a merge kernel combines
// with the rule of the reference's Merge (internal/llm/paged/paged.go:252-310).
#include <mutex>
#include <vector>

#include "hwk_common.h"
#include "internal.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint32_t kMaxChunks = 4096;  // chunks a merge row takes (its weights live in LDS)

__device__ __forceinline__ half8 half8_of(uint4 u) { return __builtin_bit_cast(half8, u); }

// 8 int8 values (two dwords) as 8 exact fp16 values.
__device__ __forceinline__ half8 i8x8_to_half8(uint2 w) {
  const h2 bias = {(f16)1152.0f, (f16)1152.0f};
  const uint32_t a = w.x ^ 0x80808080u, b = w.y ^ 0x80808080u;
  h2 r0 = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u)) - bias;
  h2 r1 = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, a, 0x04030402u)) - bias;
  h2 r2 = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, b, 0x04010400u)) - bias;
  h2 r3 = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)) - bias;
  half8 out;
  out[0] = r0.x; out[1] = r0.y; out[2] = r1.x; out[3] = r1.y;
  out[4] = r2.x; out[5] = r2.y; out[6] = r3.x; out[7] = r3.y;
  return out;
}

// ---- K4, the split-K decode attention of hwk_attn_decode ----
//
// A lane's view of a 16-key tile:
//   scores   D = K_tile . Q^T on v_mfma_f32_16x16x32_f16, K as the A operand (lane l: key l%16, a
//            k-step's 8 dims), Q as B with the G query heads repeated over the 16 columns, so that
//            lane l ends with the scores of keys 4*(l/16) .. +3 for query head l%G: no lane idles;
//   softmax  a key's scores of one head sit in the 4 row groups of the wave (lanes l, l^16, l^32,
//            l^48): max and sum over them with two permlane swaps (VALU, no LDS);
//   P.V      on the VALUs in fp32 (P never rounded): lane l holds V rows 4*(l/16) + r (r = 0..3), dims
//            (l%16)*8 .. +8, and takes head g's weight of key 4*(l/16)+r from lane (l & ~3) + g of its
//            quad by a DPP broadcast.
// Every load is issued unconditionally from a clamped row (a predicated load makes the compiler wait
// for it before issuing the next), and the terms of keys past the attended range are dropped.

// The value of lane (l & ~3) + Q of the lane's quad (DPP quad_perm broadcast).
template <int Q>
__device__ __forceinline__ float quad_lane(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), Q * 0x55, 0xf, 0xf, false));
}
template <int G>
__device__ __forceinline__ void quad_heads(float v, float (&out)[G]) {
  if constexpr (G == 1) out[0] = v;
  if constexpr (G == 2) {
    out[0] = quad_lane<0>(v);
    out[1] = quad_lane<1>(v);
  }
  if constexpr (G == 4) {
    out[0] = quad_lane<0>(v);
    out[1] = quad_lane<1>(v);
    out[2] = quad_lane<2>(v);
    out[3] = quad_lane<3>(v);
  }
}

// 16 int8 values (four dwords) as 16 exact fp16 values.
__device__ __forceinline__ void i8x16_to_half8x2(uint4 w, half8 &lo, half8 &hi) {
  lo = i8x8_to_half8(make_uint2(w.x, w.y));
  hi = i8x8_to_half8(make_uint2(w.z, w.w));
}

template <bool I8>
struct KTile {
  half8 k[4];      // A operand of the 4 k-steps
  uint4 kraw[2];   // int8: the two 16-byte loads the k operands come from
  half8 v[4];      // fp16 V rows 4*(l/16) + r, dims (l%16)*8 .. +8
  uint2 vraw[4];   // int8 V: the same rows and dims as 8 codes
  uint16_t ksc[4], vsc[4];  // int8: the fp16 scales of keys 4*(l/16) .. +3
};

// The dims of k-step s a lane takes: fp16 K: 32s + 8*(l/16) .. +8 (one 16-byte load each); int8 K:
// 64*(s/2) + 16*(l/16) + 8*(s%2) .. +8 (two 16-byte loads of 16 codes). Q's B operand follows the
// same map, so the contraction sees every dim once.
template <bool I8>
__device__ __forceinline__ uint32_t kstep_dim(int s, int lane) {
  return I8 ? 64 * (s >> 1) + 16 * (lane >> 4) + 8 * (s & 1) : 32 * s + 8 * (lane >> 4);
}

template <bool I8>
__device__ __forceinline__ void load_ktile(KTile<I8> &t, const void *__restrict__ k, const void *__restrict__ v,
                                           const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs,
                                           size_t head_base, uint32_t key0, uint32_t rows, int lane) {
  const size_t rk = head_base + min(key0 + (lane & 15), rows - 1);
  if constexpr (I8) {
#pragma unroll
    for (int j = 0; j < 2; j++)
      t.kraw[j] = load_stream((const uint4 *)((const int8_t *)k + rk * 128 + 64 * j + 16 * (lane >> 4)));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const size_t rv = head_base + min(key0 + 4 * (lane >> 4) + r, rows - 1);
      t.vraw[r] = *(const uint2 *)((const int8_t *)v + rv * 128 + (lane & 15) * 8);
      t.ksc[r] = ks[rv];
      t.vsc[r] = vs[rv];
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; s++) t.k[s] = half8_of(load_stream((const uint4 *)((const f16 *)k + rk * 128 + kstep_dim<false>(s, lane))));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const size_t rv = head_base + min(key0 + 4 * (lane >> 4) + r, rows - 1);
      t.v[r] = half8_of(load_stream((const uint4 *)((const f16 *)v + rv * 128 + (lane & 15) * 8)));
    }
  }
}

// One tile into the wave's running state: m, ls of head l%G (base 2, the same in the lane's 4 row
// groups), acc[g][8] of dims (l%16)*8 .. +8 over the lane's row group's keys.
template <int G, bool I8>
__device__ __forceinline__ void attend_ktile(KTile<I8> &t, const half8 (&qb)[4], uint32_t key0, uint32_t end,
                                             float scale_log2, int lane, float &m, float &ls, float (&acc)[G][8]) {
  if constexpr (I8) {
    i8x16_to_half8x2(t.kraw[0], t.k[0], t.k[1]);
    i8x16_to_half8x2(t.kraw[1], t.k[2], t.k[3]);
  }
  floatx4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; s++) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(t.k[s], qb[s], sc, 0, 0, 0);
  const uint32_t kr = key0 + 4 * (lane >> 4);  // the lane's first key
  float ksc[4] = {1.0f, 1.0f, 1.0f, 1.0f}, vsc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if constexpr (I8) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      ksc[r] = (float)__builtin_bit_cast(f16, t.ksc[r]);
      vsc[r] = (float)__builtin_bit_cast(f16, t.vsc[r]);
    }
  }
  float s2[4];
  float tmax = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float x = sc[i] * scale_log2;
    if constexpr (I8) x *= ksc[i];
    s2[i] = kr + i < end ? x : -__builtin_inff();
    tmax = fmaxf(tmax, s2[i]);
  }
  tmax = row_groups_max(tmax);
  const float mnew = fmaxf(m, tmax);
  const bool none = mnew == -__builtin_inff();  // no key seen yet
  const float alpha = none ? 1.0f : exp2f(m - mnew);
  float p[4], psum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    p[i] = none ? 0.0f : exp2f(s2[i] - mnew);
    psum += p[i];
  }
  ls = ls * alpha + row_groups_sum(psum);
  m = mnew;
  float ag[G];
  quad_heads<G>(alpha, ag);
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[g][d] *= ag[g];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    // a row past end was loaded from another row: zero it (p = 0 times NaN would be NaN)
    const bool ok = kr + r < end;
    half8 vr;
    if constexpr (I8) vr = ok ? i8x8_to_half8(t.vraw[r]) : half8_of(make_uint4(0, 0, 0, 0));
    else vr = ok ? t.v[r] : half8_of(make_uint4(0, 0, 0, 0));
    float pg[G];
    quad_heads<G>(I8 ? p[r] * vsc[r] : p[r], pg);
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int d = 0; d < 8; d++) acc[g][d] = fmaf(pg[g], (float)vr[d], acc[g][d]);
  }
}

// Workgroup (kv head h, chunk c) of W waves over keys [c*chunk, min((c+1)*chunk, len)) (len plus *pos
// when pos is given); wave w takes keys [c*chunk + w*kpw, +kpw) a tile at a time with the next tile's
// loads in flight. With one chunk a head the workgroup writes out; otherwise its partial (o
// unnormalized, m in natural-log units, l) per query head g to workspace slot (h*nchunk + c)*G + g,
// with plain stores, for k_attn_merge.
template <int G, bool I8, int W>
__global__ __launch_bounds__(64 * W) void k_attn_decode(const f16 *__restrict__ q, const void *__restrict__ k,
                                                        const void *__restrict__ v, const uint16_t *__restrict__ ks,
                                                        const uint16_t *__restrict__ vs, float *__restrict__ ws_o,
                                                        float *__restrict__ ws_m, float *__restrict__ ws_l,
                                                        void *__restrict__ out, int mode, const int32_t *__restrict__ pos,
                                                        uint32_t len, uint32_t cap, uint32_t chunk, uint32_t nchunk,
                                                        uint32_t kpw, float scale_log2) {
  __shared__ float sm[W][G], sl[W][G];
  __shared__ float sacc[W][G][128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t h = blockIdx.x / nchunk, c = blockIdx.x % nchunk;
  if (pos) len += (uint32_t)*pos;  // the keys in use, read on the device (a replayed step graph)
  const uint32_t begin = c * chunk, end = min(begin + chunk, len);
  const size_t head_base = (size_t)h * cap;
  const uint32_t kb = begin + wave * kpw, ke = min(kb + kpw, end);
  const uint32_t nt = kb < ke ? (ke - kb + 15) / 16 : 0;
  // q first, then the two tiles (loads complete in issue order for the wait counter: the first
  // tile's scores wait on q and that tile only)
  half8 qb[4];
#pragma unroll
  for (int s = 0; s < 4; s++) qb[s] = half8_of(*(const uint4 *)(q + ((size_t)h * G + (lane % G)) * 128 + kstep_dim<I8>(s, lane)));
  issue_order();
  KTile<I8> ta, tb;
  load_ktile<I8>(ta, k, v, ks, vs, head_base, kb, cap, lane);
  issue_order();
  load_ktile<I8>(tb, k, v, ks, vs, head_base, kb + 16, cap, lane);
  float m = -__builtin_inff(), ls = 0.0f, acc[G][8];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[g][d] = 0.0f;
  uint32_t i = 0, key = kb;
  for (; i + 3 < nt; i += 2, key += 32) {
    attend_ktile<G, I8>(ta, qb, key, ke, scale_log2, lane, m, ls, acc);
    load_ktile<I8>(ta, k, v, ks, vs, head_base, key + 32, cap, lane);
    attend_ktile<G, I8>(tb, qb, key + 16, ke, scale_log2, lane, m, ls, acc);
    load_ktile<I8>(tb, k, v, ks, vs, head_base, key + 48, cap, lane);
  }
  const uint32_t rem = nt - i;  // 0 .. 3
  if (rem >= 1) attend_ktile<G, I8>(ta, qb, key, ke, scale_log2, lane, m, ls, acc);
  if (rem == 3) load_ktile<I8>(ta, k, v, ks, vs, head_base, key + 32, cap, lane);
  if (rem >= 2) attend_ktile<G, I8>(tb, qb, key + 16, ke, scale_log2, lane, m, ls, acc);
  if (rem == 3) attend_ktile<G, I8>(ta, qb, key + 32, ke, scale_log2, lane, m, ls, acc);
  // the 4 row groups hold the same dims for different keys (under one m): sum them
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[g][d] = row_groups_sum(acc[g][d]);
  if (lane < 16) {
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int d = 0; d < 8; d++) sacc[wave][g][lane * 8 + d] = acc[g][d];
  }
  if (lane < G) {
    sm[wave][lane] = m;
    sl[wave][lane] = ls;
  }
  __syncthreads();
  // the waves' states merged: weights 2^(m_w - top)
  const size_t base = ((size_t)h * nchunk + c) * G;
  for (uint32_t t = threadIdx.x; t < (uint32_t)G * 128; t += 64 * W) {
    const uint32_t g = t / 128, d = t % 128;
    float top = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < W; w++) top = fmaxf(top, sm[w][g]);
    float o = 0.0f, lsum = 0.0f;
    if (top != -__builtin_inff()) {
#pragma unroll
      for (int w = 0; w < W; w++) {
        const float wt = exp2f(sm[w][g] - top);
        o += wt * sacc[w][g][d];
        lsum += wt * sl[w][g];
      }
    }
    if (nchunk == 1) {
      store_out(out, (size_t)(h * G + g) * 128 + d, lsum > 0.0f ? o / lsum : 0.0f, mode);
    } else {
      ws_o[(base + g) * 128 + d] = o;
      if (d == 0) {
        ws_m[base + g] = top * kLn2;
        ws_l[base + g] = lsum;
      }
    }
  }
}
// ---- the model's decode attention (K4m): k_attn_decode's tiles with the step's own q, k, v ----
//
// Workgroup (kv head h, chunk c) of W waves over the keys [c*chunk, min((c+1)*chunk, p+1)) for the token
// at position p = *pos; the grid covers the cache's capacity and a workgroup whose chunk starts past p
// attends no key and leaves a partial of weight 0 (l = 0). Prologue: q for the kv head's G query heads
// comes from the fp32 projection qkv (heads + 2*kvh rows of 128) through the per-head RMSNorm and RoPE
// (the step's cos/sin row, cos | sin of 64 values each, made by the step's first kernel); the workgroup
// whose chunk holds p (the owner) also makes the new k (normed, rotated) and v, writes them to the
// caches at p for later steps and keeps them in LDS: the tile holding p takes them from there in place
// of its load of row p, so the owner waits on no store. Every load of the prologue and both tiles is
// issued before the first wait (the tiles' rows do not depend on p). Each workgroup leaves its partial
// (o unnormalized, m in natural-log units, l) per query head with plain stores at slot
// (h*nchunk + c)*G + g; the o_proj GEMV merges them (mxfp4_gemv_x's X_MERGE).
template <int G, int W, bool ONE>
__global__ __launch_bounds__(64 * W) void k_attn_step(const float *__restrict__ qkv, const float *__restrict__ qn,
                                                      const float *__restrict__ kn, const float *__restrict__ rope,
                                                      double eps, f16 *__restrict__ kc, f16 *__restrict__ vc,
                                                      float *__restrict__ ws_o, float *__restrict__ ws_m,
                                                      float *__restrict__ ws_l, const int32_t *__restrict__ pos,
                                                      uint32_t heads, uint32_t kvh, uint32_t cap, uint32_t chunk,
                                                      uint32_t nchunk, uint32_t kpw, float scale_log2) {
  __shared__ float sm[W][G], sl[W][G];
  __shared__ float sacc[W][G][128];
  __shared__ __attribute__((aligned(16))) f16 qs[G][128];
  __shared__ __attribute__((aligned(16))) f16 knew[128], vnew[128];
  kernarg_now(qkv, qn, kn, rope, eps, kc, vc, ws_o, ws_m, ws_l, pos, heads, kvh, cap, chunk, nchunk, kpw, scale_log2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t h = blockIdx.x / nchunk, c = blockIdx.x % nchunk;
  const uint32_t begin = c * chunk;
  const size_t head_base = (size_t)h * cap;
  // the position first (written by the previous step's argmax), then every load that does not depend
  // on it: wave j's prologue job j (query head j < G, then k, then v; a wave past the jobs repeats the
  // last one, every workgroup loads the k and v jobs and only the owner keeps them), the RoPE row,
  // and the wave's two tiles (rows clamped to the capacity). Loads complete in issue order for the
  // wait counter: the position's wait holds nothing else, the RoPE's none of the tiles.
  const int32_t pv = load_first(pos);
  const uint32_t j0 = (uint32_t)wave < (uint32_t)G + 2 ? (uint32_t)wave : (uint32_t)G + 1;
  auto job_row = [&](uint32_t j) { return j < G ? h * G + j : j == G ? heads + h : heads + kvh + h; };
  const float *nwp = j0 < G ? qn : kn;
  const float x0 = qkv[(size_t)job_row(j0) * 128 + lane], x1 = qkv[(size_t)job_row(j0) * 128 + lane + 64];
  const float nw0 = nwp[lane], nw1 = nwp[lane + 64];
  const float cp = rope[lane], sp = rope[64 + lane];
  issue_order();
  const uint32_t kb = begin + wave * kpw;
  KTile<false> ta, tb;
  load_ktile<false>(ta, kc, vc, nullptr, nullptr, head_base, kb, cap, lane);
  issue_order();
  if constexpr (!ONE) load_ktile<false>(tb, kc, vc, nullptr, nullptr, head_base, kb + 16, cap, lane);
  issue_order();
  const uint32_t p = (uint32_t)__builtin_amdgcn_readfirstlane(pv), len = p + 1;
  // a workgroup whose chunk starts past p attends no key (no early exit: the compiler would move the
  // loads above behind the branch, and so behind the read of the position) and leaves a partial of
  // weight 0 (l = 0), which the merge skips
  const bool owner = p - begin < chunk;  // the chunk holds p (begin <= p)
  const uint32_t end = begin >= len ? begin : owner ? len : begin + chunk;
  const uint32_t jobs = owner ? G + 2 : G;
  const uint32_t ke = min(kb + kpw, end);
  const uint32_t nt = kb < ke ? (ke - kb + 15) / 16 : 0;
  auto make_job = [&](uint32_t j, float a0, float a1, float w0, float w1, bool keep) {
    float o0, o1;
    head_norm_rope(a0, a1, w0, w1, cp, sp, eps, o0, o1);
    if (!keep) return;
    if (j == G + 1) {
      vnew[lane] = (f16)a0;
      vnew[lane + 64] = (f16)a1;
      vc[(head_base + p) * 128 + lane] = (f16)a0;
      vc[(head_base + p) * 128 + lane + 64] = (f16)a1;
    } else if (j < G) {
      qs[j][lane] = (f16)o0;
      qs[j][lane + 64] = (f16)o1;
    } else {
      knew[lane] = (f16)o0;
      knew[lane + 64] = (f16)o1;
      kc[(head_base + p) * 128 + lane] = (f16)o0;
      kc[(head_base + p) * 128 + lane + 64] = (f16)o1;
    }
  };
  make_job(j0, x0, x1, nw0, nw1, (uint32_t)wave < jobs);
  for (uint32_t j = wave + W; j < jobs; j += W) {  // more jobs than waves (W < G + 2)
    const float *nj = j < G ? qn : kn;
    make_job(j, qkv[(size_t)job_row(j) * 128 + lane], qkv[(size_t)job_row(j) * 128 + lane + 64], nj[lane],
             nj[lane + 64], true);
  }
  __syncthreads();  // q, and the owner's new k/v, in LDS
  half8 qb[4];
#pragma unroll
  for (int s = 0; s < 4; s++) qb[s] = *(const half8 *)&qs[lane % G][kstep_dim<false>(s, lane)];
  // the owner's tile holding p takes row p from LDS
  auto patch = [&](KTile<false> &t, uint32_t key0) {
    if (!owner || p - key0 >= 16) return;
    const uint32_t j = p - key0;
    if ((uint32_t)(lane & 15) == j) {
#pragma unroll
      for (int s = 0; s < 4; s++) t.k[s] = *(const half8 *)&knew[kstep_dim<false>(s, lane)];
    }
#pragma unroll
    for (int r = 0; r < 4; r++)
      if ((uint32_t)(4 * (lane >> 4) + r) == j) t.v[r] = *(const half8 *)&vnew[(lane & 15) * 8];
  };
  float m = -__builtin_inff(), ls = 0.0f, acc[G][8];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[g][d] = 0.0f;
  if constexpr (ONE) {  // one tile a wave (kpw 16)
    if (nt) {
      patch(ta, kb);
      attend_ktile<G, false>(ta, qb, kb, ke, scale_log2, lane, m, ls, acc);
    }
  } else {
    uint32_t i = 0, key = kb;
    for (; i + 3 < nt; i += 2, key += 32) {
      patch(ta, key);
      attend_ktile<G, false>(ta, qb, key, ke, scale_log2, lane, m, ls, acc);
      load_ktile<false>(ta, kc, vc, nullptr, nullptr, head_base, key + 32, cap, lane);
      patch(tb, key + 16);
      attend_ktile<G, false>(tb, qb, key + 16, ke, scale_log2, lane, m, ls, acc);
      load_ktile<false>(tb, kc, vc, nullptr, nullptr, head_base, key + 48, cap, lane);
    }
    const uint32_t rem = nt - i;  // 0 .. 3
    if (rem >= 1) {
      patch(ta, key);
      attend_ktile<G, false>(ta, qb, key, ke, scale_log2, lane, m, ls, acc);
    }
    if (rem == 3) load_ktile<false>(ta, kc, vc, nullptr, nullptr, head_base, key + 32, cap, lane);
    if (rem >= 2) {
      patch(tb, key + 16);
      attend_ktile<G, false>(tb, qb, key + 16, ke, scale_log2, lane, m, ls, acc);
    }
    if (rem == 3) {
      patch(ta, key + 32);
      attend_ktile<G, false>(ta, qb, key + 32, ke, scale_log2, lane, m, ls, acc);
    }
  }
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[g][d] = row_groups_sum(acc[g][d]);
  if (lane < 16) {
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int d = 0; d < 8; d++) sacc[wave][g][lane * 8 + d] = acc[g][d];
  }
  if (lane < G) {
    sm[wave][lane] = m;
    sl[wave][lane] = ls;
  }
  __syncthreads();
  const size_t base = ((size_t)h * nchunk + c) * G;
  for (uint32_t t = threadIdx.x; t < (uint32_t)G * 128; t += 64 * W) {
    const uint32_t g = t / 128, d = t % 128;
    float top = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < W; w++) top = fmaxf(top, sm[w][g]);
    float o = 0.0f, lsum = 0.0f;
    if (top != -__builtin_inff()) {
#pragma unroll
      for (int w = 0; w < W; w++) {
        const float wt = exp2f(sm[w][g] - top);
        o += wt * sacc[w][g][d];
        lsum += wt * sl[w][g];
      }
    }
    ws_o[(base + g) * 128 + d] = o;
    if (d == 0) {
      ws_m[base + g] = top * kLn2;
      ws_l[base + g] = lsum;
    }
  }
}

// Merge of chunks (the reference's Merge rule, paged.go:252-310): top = the largest m among
// chunks with l > 0; a chunk weighs exp(m - top), times l when its o is normalized; out = the
// weighted sum of o over the weighted sum of l. Block (row, slice of 32 dims) of 256 threads: the
// chunks' weights go to LDS first (one pass of independent loads), then 8 chunk lanes x 32 dims
// sum o in batches of independent loads. o (chunks, rows, dim) normalized per chunk, m and l (chunks,
// rows): hwk_attn_merge's layout.
__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ o, const float *__restrict__ m,
                                                    const float *__restrict__ l, void *__restrict__ out,
                                                    uint32_t chunks, uint32_t rows, uint32_t dim, int mode) {
  __shared__ float wgt[kMaxChunks];
  __shared__ float red[256];
  const uint32_t row = blockIdx.x, t = threadIdx.x;
  const uint32_t d = blockIdx.y * 32 + (t & 31), cl = t >> 5;
  const size_t base = row, stride = rows;
  float top = -__builtin_inff();
  for (uint32_t c = t; c < chunks; c += 256) {
    const size_t i = base + c * stride;
    const float mc = m[i], lc = l[i];
    wgt[c] = lc;
    if (lc > 0.0f) top = fmaxf(top, mc);
  }
  red[t] = top;
  __syncthreads();
  for (uint32_t s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] = fmaxf(red[t], red[t + s]);
    __syncthreads();
  }
  top = red[0];
  __syncthreads();
  float den = 0.0f;
  for (uint32_t c = t; c < chunks; c += 256) {
    const float lc = wgt[c];
    float w = 0.0f;
    if (lc > 0.0f && top != -__builtin_inff()) {
      w = expf(m[base + c * stride] - top) * lc;
      den += w;
    }
    wgt[c] = w;
  }
  red[t] = den;
  __syncthreads();
  for (uint32_t s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] += red[t + s];
    __syncthreads();
  }
  den = red[0];
  __syncthreads();
  float num = 0.0f;
  if (d < dim) {
    constexpr uint32_t U = 8;
    uint32_t c = cl;
    for (; c + 8 * (U - 1) < chunks; c += 8 * U) {
      float ov[U];
#pragma unroll
      for (uint32_t u = 0; u < U; u++) ov[u] = o[(base + (size_t)(c + 8 * u) * stride) * dim + d];
      // a skipped chunk (weight 0) adds nothing, whatever its o holds (0 * NaN would be NaN)
#pragma unroll
      for (uint32_t u = 0; u < U; u++) {
        const float wu = wgt[c + 8 * u];
        num += wu > 0.0f ? wu * ov[u] : 0.0f;
      }
    }
    for (; c < chunks; c += 8) {
      const float wu = wgt[c];
      num += wu > 0.0f ? wu * o[(base + (size_t)c * stride) * dim + d] : 0.0f;
    }
  }
  red[t] = num;
  __syncthreads();
  if (cl == 0 && d < dim) {
    for (uint32_t j = 1; j < 8; j++) num += red[t + 32 * j];
    store_out(out, (size_t)row * dim + d, den > 0.0f ? num / den : 0.0f, mode);
  }
}

// The merge of k_attn_decode's partials (the reference's Merge rule, paged.go:252-310): workgroup =
// (query head, 64 dims), 4 waves = 4 chunk lanes x 64 dims. Every load is issued at once: each thread's
// share of the o values (chunks cl, cl+4, ...) is in flight while the chunks' m and l go to LDS. Then
// top = the largest m among chunks with l > 0, a chunk weighs w = exp(m - top) (0 for a chunk whose l
// is not positive, which adds nothing whatever its o holds), and out = sum(w * o) / sum(w * l).
template <int U>
__global__ __launch_bounds__(256) void k_attn_merge_fast(const float *__restrict__ o, const float *__restrict__ m,
                                                         const float *__restrict__ l, void *__restrict__ out,
                                                         uint32_t chunks, uint32_t G, int mode) {
  __shared__ float sm[kMaxChunks], sl[kMaxChunks];
  __shared__ float red[2][4];
  __shared__ float part[4][64];
  const uint32_t row = blockIdx.x, t = threadIdx.x, lane = t & 63, cl = t >> 6;
  const uint32_t d = blockIdx.y * 64 + lane;
  const size_t base = (size_t)(row / G) * chunks * G + row % G;  // slot of chunk c: base + c*G
  float ov[U];
#pragma unroll
  for (int u = 0; u < U; u++) ov[u] = o[(base + (size_t)min(cl + 4 * u, chunks - 1) * G) * 128 + d];
  for (uint32_t c = t; c < chunks; c += 256) {
    sm[c] = m[base + (size_t)c * G];
    sl[c] = l[base + (size_t)c * G];
  }
  __syncthreads();
  float top = -__builtin_inff();
  for (uint32_t c = t; c < chunks; c += 256)
    if (sl[c] > 0.0f) top = fmaxf(top, sm[c]);
  top = wave_max(top);
  if (lane == 0) red[0][cl] = top;
  __syncthreads();
  top = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float den = 0.0f;
  for (uint32_t c = t; c < chunks; c += 256) {
    const float w = (sl[c] > 0.0f && top != -__builtin_inff()) ? expf(sm[c] - top) : 0.0f;
    den += w * sl[c];
    sm[c] = w;  // the weight replaces m
  }
  den = group_sum<64>(den);
  if (lane == 0) red[1][cl] = den;
  __syncthreads();
  den = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  float num = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t c = cl + 4 * u;
    const float w = c < chunks ? sm[c] : 0.0f;
    num += w > 0.0f ? w * ov[u] : 0.0f;
  }
  for (uint32_t c = cl + 4 * U; c < chunks; c += 4) {  // chunks past the first 4*U: one load at a time
    const float w = sm[c];
    if (w > 0.0f) num += w * o[(base + (size_t)c * G) * 128 + d];
  }
  part[cl][lane] = num;
  __syncthreads();
  if (cl == 0) {
    num = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
    store_out(out, (size_t)row * 128 + d, den > 0.0f ? num / den : 0.0f, mode);
  }
}

// The merge of hwk_attn_decode's partials with one wave a (query head, 16 dims), for at most 4*U
// chunks: lane = (dim lane % 16, chunk group lane / 16), group g takes chunks g, g+4, ..., all its
// loads (o, m, l) issued at once; the reference's Merge rule (paged.go:252-310) as k_attn_merge_fast:
// top = the largest m among chunks with l > 0, w = exp(m - top), out = sum(w o) / sum(w l), a chunk
// with w = 0 (l <= 0) adding nothing (its o is never multiplied); the sums reduced over the four
// groups by permlane swaps. No LDS, no barrier.
template <int U>
__global__ __launch_bounds__(64) void k_attn_merge_wave(const float *__restrict__ o, const float *__restrict__ m,
                                                        const float *__restrict__ l, void *__restrict__ out,
                                                        uint32_t chunks, uint32_t G, int mode) {
  const uint32_t row = blockIdx.x, lane = threadIdx.x, g = lane >> 4;
  const uint32_t d = blockIdx.y * 16 + (lane & 15);
  const size_t base = (size_t)(row / G) * chunks * G + row % G;  // slot of chunk c: base + c*G
  float ov[U], mv[U], lv[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const size_t slot = base + (size_t)min(g + 4 * u, chunks - 1) * G;
    ov[u] = o[slot * 128 + d];
    mv[u] = m[slot];
    lv[u] = l[slot];
  }
  float top = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < U; u++)
    if (g + 4 * u < chunks && lv[u] > 0.0f) top = fmaxf(top, mv[u]);
  top = row_groups_max(top);
  float den = 0.0f, num = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const float w = (g + 4 * u < chunks && lv[u] > 0.0f && top != -__builtin_inff()) ? expf(mv[u] - top) : 0.0f;
    den += w * lv[u];
    num += w > 0.0f ? w * ov[u] : 0.0f;
  }
  den = row_groups_sum(den);
  num = row_groups_sum(num);
  if (g == 0) store_out(out, (size_t)row * 128 + d, den > 0.0f ? num / den : 0.0f, mode);
}

// One wave a row of head_dim (<= 512) fp16 values: absmax over the row, scale rounded to fp16,
// codes rounded to even against that scale.
__global__ void k_kv_quantize_i8(const f16 *__restrict__ x, int8_t *__restrict__ q, f16 *__restrict__ scale,
                                 uint32_t rows, uint32_t dim) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const f16 *xr = x + (size_t)row * dim;
  float mx = 0.0f;
  for (uint32_t c = lane; c < dim; c += 64) mx = fmaxf(mx, fabsf((float)xr[c]));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float s = mx / 127.0f;
  if (s == 0.0f) s = 1.0f;
  const f16 s16 = (f16)s;
  s = (float)s16;
  if (lane == 0) scale[row] = s16;
  for (uint32_t c = lane; c < dim; c += 64) {
    float v = rintf((float)xr[c] / s);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    q[(size_t)row * dim + c] = (int8_t)v;
  }
}

// The split of hwk_attn_decode: workgroups of W waves (8 from 8,192 keys, fp16 caches below 32,768;
// else 4: measured fastest for each), each wave kpw keys (a multiple of 16), chunk = W*kpw keys a
// workgroup. kpw is sized so that the launch runs about 2048 waves (8 a CU, each with two tiles of
// loads in flight), between 32 and 256 keys, more when a head would exceed kMaxChunks chunks. A
// caller's split (a multiple of 64) is the chunk.
uint32_t decode_waves(const hwk_attn_params *p) {
  return p->len >= 8192 && (p->kv_int8 || p->len < 32768) ? 8u : 4u;
}

uint32_t pick_kpw(const hwk_attn_params *p) {
  const uint32_t W = decode_waves(p);
  if (p->split) return p->split / W;
  const uint64_t keys = (uint64_t)p->len * p->kv_heads;
  uint64_t kpw = (keys + 2047) / 2048;
  kpw = (kpw + 15) / 16 * 16;
  if (kpw < 32) kpw = 32;
  if (kpw > 256) kpw = 256;
  const uint64_t min_kpw = ((uint64_t)p->len + (uint64_t)kMaxChunks * W - 1) / ((uint64_t)kMaxChunks * W);
  if (kpw < min_kpw) kpw = (min_kpw + 15) / 16 * 16;
  return (uint32_t)kpw;
}

uint32_t pick_chunk(const hwk_attn_params *p) { return pick_kpw(p) * decode_waves(p); }

uint32_t chunks_of(const hwk_attn_params *p, uint32_t chunk) { return p->len ? (p->len + chunk - 1) / chunk : 1; }

}  // namespace

extern "C" {

// Layout: o (slots, 128) | m (slots) | l (slots), slots = heads * chunks.
HWK_API size_t hwk_attn_workspace_bytes(const hwk_attn_params *p) {
  if (!p || p->kv_heads == 0 || p->heads % p->kv_heads) return 0;
  const uint32_t chunk = pick_chunk(p);
  const uint64_t slots = (uint64_t)p->heads * chunks_of(p, chunk);
  return (size_t)(slots * (p->head_dim + 2) * sizeof(float));
}

HWK_API char *hwk_attn_decode(void *stream, const void *q, const void *k, const void *v, const void *k_scale,
                              const void *v_scale, void *out, void *workspace, size_t workspace_bytes,
                              const hwk_attn_params *p) {
  return hwk::attn_decode_dev((hipStream_t)stream, q, k, v, k_scale, v_scale, out, workspace, workspace_bytes, p,
                              nullptr, 0);
}

}  // extern "C"

char *hwk::attn_decode_dev(hipStream_t st, const void *q, const void *k, const void *v, const void *k_scale,
                           const void *v_scale, void *out, void *workspace, size_t workspace_bytes,
                           const hwk_attn_params *p, const int32_t *pos, uint32_t len_add) {
  HWK_CHECK(p, "hwk_attn_decode: null params");
  HWK_CHECK(q && k && v && out && workspace, "hwk_attn_decode: null pointer");
  HWK_CHECK(p->head_dim == 128, "hwk_attn_decode: head_dim %u (128 only)", p->head_dim);
  HWK_CHECK(p->kv_heads > 0 && p->heads % p->kv_heads == 0, "hwk_attn_decode: %u heads over %u kv heads", p->heads,
            p->kv_heads);
  const uint32_t G = p->heads / p->kv_heads;
  HWK_CHECK(G == 1 || G == 2 || G == 4, "hwk_attn_decode: %u query heads a kv head (1, 2 or 4)", G);
  HWK_CHECK(p->len <= p->capacity, "hwk_attn_decode: len %u past capacity %u", p->len, p->capacity);
  HWK_CHECK(!p->kv_int8 || (k_scale && v_scale), "hwk_attn_decode: int8 cache without scales");
  HWK_CHECK(p->out_mode == HWK_OUT_F32 || p->out_mode == HWK_OUT_F16, "hwk_attn_decode: out_mode %u", p->out_mode);
  HWK_CHECK(p->split % 64 == 0, "hwk_attn_decode: split %u is not a multiple of 64", p->split);
  HWK_CHECK(hwk::aligned(q, 16) && hwk::aligned(workspace, 16), "hwk_attn_decode: q and workspace 16-byte aligned");
  HWK_CHECK(p->kv_int8 ? (hwk::aligned(k, 16) && hwk::aligned(v, 8)) : (hwk::aligned(k, 16) && hwk::aligned(v, 16)),
            "hwk_attn_decode: k, v misaligned (k 16-byte aligned; v 16-byte for fp16, 8-byte for int8)");
  const size_t need = hwk_attn_workspace_bytes(p);
  HWK_CHECK(workspace_bytes >= need, "hwk_attn_decode: workspace %zu bytes, %zu needed", workspace_bytes, need);
  const uint32_t chunk = pick_chunk(p);
  const uint32_t nchunk = chunks_of(p, chunk);
  HWK_CHECK(nchunk <= kMaxChunks, "hwk_attn_decode: %u chunks of %u keys (at most %u)", nchunk, chunk, kMaxChunks);
  const uint64_t slots = (uint64_t)p->heads * nchunk;
  float *ws_o = (float *)workspace;
  float *ws_m = ws_o + slots * 128;
  float *ws_l = ws_m + slots;
  const float scale_log2 = hwk::f32_of_bits(p->scale_bits) * kLog2e;
  HWK_CHECK(!pos || p->len == p->capacity, "attn_decode_dev: a device length needs the grid of the capacity");
  const uint32_t len = pos ? len_add : p->len;
  const uint32_t W = decode_waves(p);
  const uint32_t kpw = chunk / W;
  const dim3 grid(p->kv_heads * nchunk), block(64 * W);
  const uint16_t *ks = (const uint16_t *)k_scale, *vs = (const uint16_t *)v_scale;
  const int mode = (int)p->out_mode;
#define HWK_ATTN_LAUNCH(GG)                                                                                          \
  if (p->kv_int8 && W == 8)                                                                                          \
    hipLaunchKernelGGL((k_attn_decode<GG, true, 8>), grid, block, 0, st, (const f16 *)q, k, v, ks, vs, ws_o, ws_m,   \
                       ws_l, out, mode, pos, len, p->capacity, chunk, nchunk, kpw, scale_log2);                      \
  else if (p->kv_int8)                                                                                               \
    hipLaunchKernelGGL((k_attn_decode<GG, true, 4>), grid, block, 0, st, (const f16 *)q, k, v, ks, vs, ws_o, ws_m,   \
                       ws_l, out, mode, pos, len, p->capacity, chunk, nchunk, kpw, scale_log2);                      \
  else if (W == 8)                                                                                                   \
    hipLaunchKernelGGL((k_attn_decode<GG, false, 8>), grid, block, 0, st, (const f16 *)q, k, v, ks, vs, ws_o, ws_m,  \
                       ws_l, out, mode, pos, len, p->capacity, chunk, nchunk, kpw, scale_log2);                      \
  else                                                                                                               \
    hipLaunchKernelGGL((k_attn_decode<GG, false, 4>), grid, block, 0, st, (const f16 *)q, k, v, ks, vs, ws_o, ws_m,  \
                       ws_l, out, mode, pos, len, p->capacity, chunk, nchunk, kpw, scale_log2);
  if (G == 1) {
    HWK_ATTN_LAUNCH(1)
  } else if (G == 2) {
    HWK_ATTN_LAUNCH(2)
  } else {
    HWK_ATTN_LAUNCH(4)
  }
#undef HWK_ATTN_LAUNCH
  if (char *err = hwk::launched("hwk_attn_decode")) return err;
  if (nchunk == 1) return nullptr;
  const dim3 mgrid(p->heads, 8);
  if (nchunk <= 4 * 4)
    hipLaunchKernelGGL((k_attn_merge_wave<4>), mgrid, dim3(64), 0, st, ws_o, ws_m, ws_l, out, nchunk, G, mode);
  else if (nchunk <= 4 * 8)
    hipLaunchKernelGGL((k_attn_merge_wave<8>), mgrid, dim3(64), 0, st, ws_o, ws_m, ws_l, out, nchunk, G, mode);
  else if (nchunk <= 4 * 16)
    hipLaunchKernelGGL((k_attn_merge_wave<16>), mgrid, dim3(64), 0, st, ws_o, ws_m, ws_l, out, nchunk, G, mode);
  else
    hipLaunchKernelGGL((k_attn_merge_fast<32>), dim3(p->heads, 2), dim3(256), 0, st, ws_o, ws_m, ws_l, out, nchunk, G, mode);
  return hwk::launched("hwk_attn_decode (merge)");
}


// The model step's split: 4 waves a workgroup, kpw keys a wave (32: two tiles, both in flight), chunk =
// 4*kpw keys; kpw grows past 32 so that a kv head has at most kStepMaxChunks chunks (the o_proj GEMV
// merges every chunk's partial in its prologue). (Eight waves of one tile each were measured no faster.)
constexpr int kStepWaves = 4;
constexpr uint32_t kStepMaxChunks = 16;

void hwk::attn_step_layout(const hwk_attn_params *p, uint32_t *chunk, uint32_t *nchunk) {
  uint32_t kpw = 32;
  const uint32_t need = (p->capacity + kStepWaves * kStepMaxChunks - 1) / (kStepWaves * kStepMaxChunks);
  if (kpw < need) kpw = (need + 15) / 16 * 16;
  *chunk = kpw * kStepWaves;
  *nchunk = (p->capacity + *chunk - 1) / *chunk;
}

size_t hwk::attn_step_workspace_bytes(const hwk_attn_params *p) {
  uint32_t chunk, nchunk;
  attn_step_layout(p, &chunk, &nchunk);
  return (size_t)p->heads * nchunk * (128 + 2) * sizeof(float);
}

char *hwk::attn_step(hipStream_t st, const float *qkv, const float *qn, const float *kn, const float *rope, double eps,
                     void *kc, void *vc, void *workspace, size_t workspace_bytes, const hwk_attn_params *p,
                     const int32_t *pos) {
  HWK_CHECK(p && qkv && qn && kn && rope && kc && vc && workspace && pos, "attn_step: null argument");
  HWK_CHECK(p->head_dim == 128 && !p->kv_int8, "attn_step: fp16 caches of head_dim 128 only");
  HWK_CHECK(p->kv_heads > 0 && p->heads % p->kv_heads == 0, "attn_step: %u heads over %u", p->heads, p->kv_heads);
  const uint32_t G = p->heads / p->kv_heads;
  HWK_CHECK(G == 1 || G == 2 || G == 4, "attn_step: %u query heads a kv head", G);
  HWK_CHECK(workspace_bytes >= attn_step_workspace_bytes(p), "attn_step: workspace too small");
  uint32_t chunk, nchunk;
  attn_step_layout(p, &chunk, &nchunk);
  const uint64_t slots = (uint64_t)p->heads * nchunk;
  float *ws_o = (float *)workspace, *ws_m = ws_o + slots * 128, *ws_l = ws_m + slots;
  const float scale_log2 = hwk::f32_of_bits(p->scale_bits) * kLog2e;
  constexpr int W = kStepWaves;
  const uint32_t kpw = chunk / W;
#define HWK_STEP2(GG, ONE)                                                                                        \
  hipLaunchKernelGGL((k_attn_step<GG, W, ONE>), dim3(p->kv_heads * nchunk), dim3(64 * W), 0, st, qkv, qn, kn, rope,   \
                     eps, (f16 *)kc, (f16 *)vc, ws_o, ws_m, ws_l, pos, p->heads, p->kv_heads, p->capacity, chunk,      \
                     nchunk, kpw, scale_log2)
  if (G == 1) HWK_STEP2(1, false);
  else if (G == 2) HWK_STEP2(2, false);
  else HWK_STEP2(4, false);
#undef HWK_STEP2
  return hwk::launched("attn_step");
}

extern "C" {

HWK_API char *hwk_kv_quantize_i8(void *stream, const void *x, void *q, void *scale, uint32_t rows,
                                 uint32_t head_dim) {
  HWK_CHECK(x && q && scale, "hwk_kv_quantize_i8: null pointer");
  HWK_CHECK(head_dim > 0 && head_dim <= 512, "hwk_kv_quantize_i8: head_dim %u (1..512)", head_dim);
  if (rows == 0) return nullptr;
  hipLaunchKernelGGL(k_kv_quantize_i8, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, (const f16 *)x,
                     (int8_t *)q, (f16 *)scale, rows, head_dim);
  return hwk::launched("hwk_kv_quantize_i8");
}

HWK_API char *hwk_attn_merge(void *stream, const void *o, const void *m, const void *l, void *out, uint32_t chunks,
                             uint32_t rows, uint32_t dim, int out_mode) {
  HWK_CHECK(o && m && l && out, "hwk_attn_merge: null pointer");
  HWK_CHECK(dim > 0 && dim <= 1024, "hwk_attn_merge: dim %u (1..1024)", dim);
  HWK_CHECK(chunks <= kMaxChunks, "hwk_attn_merge: %u chunks (at most %u)", chunks, kMaxChunks);
  HWK_CHECK(out_mode == HWK_OUT_F32 || out_mode == HWK_OUT_F16, "hwk_attn_merge: out_mode %d", out_mode);
  if (rows == 0) return nullptr;
  hipLaunchKernelGGL(k_attn_merge, dim3(rows, (dim + 31) / 32), dim3(256), 0, (hipStream_t)stream, (const float *)o,
                     (const float *)m, (const float *)l, out, chunks, rows, dim, out_mode);
  return hwk::launched("hwk_attn_merge");
}

}  // extern "C"

// ---- the allocation-free decode attention: hwk_attn_decode with its split-K partials in a
// file-scope device array instead of a caller's workspace ----

namespace {

constexpr size_t kScratchBytes = 4u << 20;  // HWK_ATTN_SCRATCH_BYTES in include/hwk.h

// Every device the library runs on holds one copy until the process ends; calls on one device
// share it (and race when they overlap).
__device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];

std::mutex scratch_mu;
std::vector<void *> scratch_ptrs;  // the array's device address, per device

// The address of the current device's copy of `scratch`, looked up once per device (the host-side
// name of the array is a stand-in that must never reach a kernel).
char *scratch_of_current_device(void **out) {
  int dev = 0;
  HWK_TRY("hipGetDevice", hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(scratch_mu);
  if ((size_t)dev >= scratch_ptrs.size()) scratch_ptrs.resize((size_t)dev + 1, nullptr);
  if (!scratch_ptrs[dev]) {
    void *p = nullptr;
    HWK_TRY("hipGetSymbolAddress (attention scratch)", hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    HWK_CHECK(p != nullptr, "hipGetSymbolAddress (attention scratch): null address");
    scratch_ptrs[dev] = p;
  }
  *out = scratch_ptrs[dev];
  return nullptr;
}

}  // namespace

extern "C" {

HWK_API char *hwk_attn_decode_noalloc(void *stream, const void *q, const void *k, const void *v,
                                      const void *k_scale, const void *v_scale, void *out,
                                      const hwk_attn_params *p) {
  HWK_CHECK(p, "hwk_attn_decode_noalloc: null params");
  const size_t need = hwk_attn_workspace_bytes(p);
  HWK_CHECK(need <= kScratchBytes,
            "hwk_attn_decode_noalloc: %zu bytes of partials needed, past the library's %zu-byte scratch "
            "(use hwk_attn_decode with a workspace)",
            need, kScratchBytes);
  void *ws = nullptr;
  if (char *err = scratch_of_current_device(&ws)) return err;
  return hwk::attn_decode_dev((hipStream_t)stream, q, k, v, k_scale, v_scale, out, ws, kScratchBytes, p, nullptr, 0);
}

}  // extern "C"
