// The device code of K4, the split-K GQA decode attention (one query token per head over an fp16 or
// int8 KV cache), and of its merge, shared by libhwk's kernels (attn.hip) and the kernels of the
// library's code object (co/hwk_co.hip), so that both run the same instructions.
//
// The context is split over workgroups (split-K). A workgroup owns one KV head and a chunk of
// keys; its waves take the chunk's 16-key tiles in turn, each with the next tile's loads in flight
// while it computes the current one:
//   - scores: the G query heads of the KV head (padded to the MFMA's 16 rows) times the tile's
//     keys on the fp16 MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation); a lane loads 16 bytes
//     of one key row straight from HBM as its B operand, so no cross-lane reduction is needed;
//   - an online softmax in fp32 (base 2) per head, the running max kept wave-uniform;
//   - P.V on the vector ALUs in fp32 (P stays fp32; a lane holds 8 dims of one key), so the
//     weights are never rounded to fp16.
// The waves merge in LDS; with one chunk a head the workgroup writes the output, else one
// unnormalized output, max and sum per query head to a workspace that the merge combines with the
// rule of the reference's Merge (internal/llm/paged/paged.go:252-310).
#pragma once

#include "hwk_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace hwk_attn {

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

// KEEP: the cache rows are read with ordinary (cache-allocating) loads, for rows that later calls read
// again and that fit the memory-side cache together (the model's decode step keeps a prefix of every
// layer's cache there; its weights stream with nontemporal loads and do not evict it); otherwise
// with nontemporal loads, which leave the memory-side cache to other data.
template <bool I8, bool KEEP = false>
__device__ __forceinline__ void load_ktile(KTile<I8> &t, const void *__restrict__ k, const void *__restrict__ v,
                                           const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs,
                                           size_t head_base, uint32_t key0, uint32_t rows, int lane) {
  auto ld = [](const void *a) { return KEEP ? *(const uint4 *)a : load_stream((const uint4 *)a); };
  const size_t rk = head_base + min(key0 + (lane & 15), rows - 1);
  if constexpr (I8) {
#pragma unroll
    for (int j = 0; j < 2; j++)
      t.kraw[j] = ld((const int8_t *)k + rk * 128 + 64 * j + 16 * (lane >> 4));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const size_t rv = head_base + min(key0 + 4 * (lane >> 4) + r, rows - 1);
      t.vraw[r] = *(const uint2 *)((const int8_t *)v + rv * 128 + (lane & 15) * 8);
      t.ksc[r] = ks[rv];
      t.vsc[r] = vs[rv];
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; s++) t.k[s] = half8_of(ld((const f16 *)k + rk * 128 + kstep_dim<false>(s, lane)));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const size_t rv = head_base + min(key0 + 4 * (lane >> 4) + r, rows - 1);
      t.v[r] = half8_of(ld((const f16 *)v + rv * 128 + (lane & 15) * 8));
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

// Two tiles (keys key0 .. key0+31) into the wave's running state at once: both tiles' scores (two
// independent MFMA chains), one max, one rescale and one sum over the 32 keys, then both tiles' V
// rows. The same arithmetic as attend_ktile over the pair's keys, with the running max taken over
// both tiles before any exp (one online-softmax update instead of two: the serial chain of a tile's
// softmax, issued by one wave a SIMD, is most of a tile's time).
template <int G, bool I8>
__device__ __forceinline__ void attend_pair(KTile<I8> &ta, KTile<I8> &tb, const half8 (&qb)[4], uint32_t key0,
                                            uint32_t end, float scale_log2, int lane, float &m, float &ls,
                                            float (&acc)[G][8]) {
  KTile<I8> *tt[2] = {&ta, &tb};
  if constexpr (I8) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
      i8x16_to_half8x2(tt[u]->kraw[0], tt[u]->k[0], tt[u]->k[1]);
      i8x16_to_half8x2(tt[u]->kraw[1], tt[u]->k[2], tt[u]->k[3]);
    }
  }
  floatx4 sc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (int s = 0; s < 4; s++)
#pragma unroll
    for (int u = 0; u < 2; u++) sc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tt[u]->k[s], qb[s], sc[u], 0, 0, 0);
  float s2[2][4];
  float tmax = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const uint32_t kr = key0 + 16 * u + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float x = sc[u][i] * scale_log2;
      if constexpr (I8) x *= (float)__builtin_bit_cast(f16, tt[u]->ksc[i]);
      s2[u][i] = kr + i < end ? x : -__builtin_inff();
      tmax = fmaxf(tmax, s2[u][i]);
    }
  }
  tmax = row_groups_max(tmax);
  const float mnew = fmaxf(m, tmax);
  const bool none = mnew == -__builtin_inff();  // no key seen yet
  const float alpha = none ? 1.0f : exp2f(m - mnew);
  float p[2][4], psum = 0.0f;
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p[u][i] = none ? 0.0f : exp2f(s2[u][i] - mnew);
      psum += p[u][i];
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
  for (int u = 0; u < 2; u++) {
    const uint32_t kr = key0 + 16 * u + 4 * (lane >> 4);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      // a row past end was loaded from another row: zero it (p = 0 times NaN would be NaN)
      const bool ok = kr + r < end;
      half8 vr;
      if constexpr (I8) vr = ok ? i8x8_to_half8(tt[u]->vraw[r]) : half8_of(make_uint4(0, 0, 0, 0));
      else vr = ok ? tt[u]->v[r] : half8_of(make_uint4(0, 0, 0, 0));
      float pg[G];
      quad_heads<G>(I8 ? p[u][r] * (float)__builtin_bit_cast(f16, tt[u]->vsc[r]) : p[u][r], pg);
#pragma unroll
      for (int g = 0; g < G; g++)
#pragma unroll
        for (int d = 0; d < 8; d++) acc[g][d] = fmaf(pg[g], (float)vr[d], acc[g][d]);
    }
  }
}

// Workgroup bx = (kv head h, chunk c) of W waves over keys [c*chunk, min((c+1)*chunk, len)) (len plus
// *pos when pos is given); wave w takes keys [c*chunk + w*kpw, +kpw) a tile at a time with the next tile's
// loads in flight. With one chunk a head the workgroup writes out; otherwise its partial (o
// unnormalized, m in natural-log units, l) per query head g to workspace slot (h*nchunk + c)*G + g,
// with plain stores, for k_attn_merge.
template <int G, bool I8, int W>
__device__ __forceinline__ void attn_decode_wg(uint32_t bx, const f16 *__restrict__ q, const void *__restrict__ k,
                                               const void *__restrict__ v, const uint16_t *__restrict__ ks,
                                               const uint16_t *__restrict__ vs, float *__restrict__ ws_o,
                                               float *__restrict__ ws_m, float *__restrict__ ws_l,
                                               void *__restrict__ out, int mode, const int32_t *__restrict__ pos,
                                               uint32_t len, uint32_t cap, uint32_t chunk, uint32_t nchunk,
                                               uint32_t kpw, float scale_log2) {
  __shared__ float sm[W][G], sl[W][G];
  __shared__ float sacc[W][G][128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t h = bx / nchunk, c = bx % nchunk;
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
  const uint32_t rem = nt - i;  // 0 .. 3 (attend_pair measured slower here: 8,192 fp16 keys 11.6 -> 12.1 us)
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
// The merge of hwk_attn_decode's partials with one wave a (query head row, 16 dims slice), for at
// most 4*U chunks: lane = (dim lane % 16, chunk group lane / 16), group g takes chunks g, g+4, ..., all its
// loads (o, m, l) issued at once; the reference's Merge rule (paged.go:252-310) as k_attn_merge_fast:
// top = the largest m among chunks with l > 0, w = exp(m - top), out = sum(w o) / sum(w l), a chunk
// with w = 0 (l <= 0) adding nothing (its o is never multiplied); the sums reduced over the four
// groups by permlane swaps. No LDS, no barrier.
template <int U>
__device__ __forceinline__ void attn_merge_wave_wg(uint32_t row, uint32_t slice, const float *__restrict__ o,
                                                   const float *__restrict__ m, const float *__restrict__ l,
                                                   void *__restrict__ out, uint32_t chunks, uint32_t G, int mode) {
  const uint32_t lane = threadIdx.x, g = lane >> 4;
  const uint32_t d = slice * 16 + (lane & 15);
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

}  // namespace hwk_attn
