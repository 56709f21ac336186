// GQA decode attention (K4) on gfx950: the kernels of hwk_attn_decode (split-K partials and their
// merge; the device code is in attn_kernels.h), the model's decode attention (K4m, with the step's
// q/k norm, RoPE and KV append in its prologue), the int8 KV quantizer, and the allocation-free
// entry point.
#include <mutex>
#include <vector>

#include "attn_kernels.h"
#include "hwk_common.h"
#include "internal.h"

namespace {

using namespace hwk_attn;

template <int G, bool I8, int W>
__global__ __launch_bounds__(64 * W) void k_attn_decode(const f16 *__restrict__ q, const void *__restrict__ k,
                                                        const void *__restrict__ v, const uint16_t *__restrict__ ks,
                                                        const uint16_t *__restrict__ vs, float *__restrict__ ws_o,
                                                        float *__restrict__ ws_m, float *__restrict__ ws_l,
                                                        void *__restrict__ out, int mode, const int32_t *__restrict__ pos,
                                                        uint32_t len, uint32_t cap, uint32_t chunk, uint32_t nchunk,
                                                        uint32_t kpw, float scale_log2) {
  attn_decode_wg<G, I8, W>(blockIdx.x, q, k, v, ks, vs, ws_o, ws_m, ws_l, out, mode, pos, len, cap, chunk, nchunk, kpw,
                           scale_log2);
}

// ---- the model's decode attention (K4m): k_attn_decode's tiles with the step's own q, k, v ----
//
// Workgroup (kv head h, chunk c, query-head group sub) of W waves over the keys [c*chunk, min((c+1)*chunk,
// p+1)) for the token at position p = *pos, for G of the kv head's gd query heads (heads h*gd + sub*G ..
// +G; blockIdx = sub * kvh * nchunk + h * nchunk + c). The gd/G workgroups of one (h, c) read the same
// cache rows: the grid spreads the attention's VALU work over that many more CUs (a kv head's two query
// heads in two workgroups of one head each: 1,393 -> 1,409 tokens/s on the C5 decode step), and with
// kvh * nchunk a multiple of 8 they run on one XCD and share its L2. The grid covers the cache's
// capacity and a workgroup whose chunk starts past p attends no key and leaves a partial of weight 0
// (l = 0). Prologue: q for the workgroup's G query heads comes from the fp32 projection qkv (heads +
// 2*kvh rows of 128) through the per-head RMSNorm and RoPE (the step's cos/sin row, cos | sin of 64
// values each, made by the step's first kernel); the workgroups whose chunk holds p (the owners) also
// make the new k (normed, rotated) and v and keep them in LDS, and the first of them (sub 0) writes
// them to the caches at p for later steps: the tile holding p takes them from LDS in place of its load
// of row p, so no owner waits on a store. Every load of the prologue and both tiles is issued before
// the first wait (the tiles' rows do not depend on p). Each workgroup leaves its partial (o
// unnormalized, m in natural-log units, l) per query head with plain stores at slot
// (h*nchunk + c)*gd + sub*G + g; the o_proj GEMV merges them (mxfp4_gemv_x's X_MERGE).
template <int G, int W, bool ONE, bool KEEP>
__device__ __forceinline__ void attn_step_wg(const float *__restrict__ qkv, const float *__restrict__ qn,
                                             const float *__restrict__ kn, const float *__restrict__ rope, double eps,
                                             f16 *__restrict__ kc, f16 *__restrict__ vc, float *__restrict__ ws_o,
                                             float *__restrict__ ws_m, float *__restrict__ ws_l,
                                             const int32_t *__restrict__ pos, uint32_t heads, uint32_t kvh,
                                             uint32_t cap, uint32_t chunk, uint32_t nchunk, uint32_t kpw,
                                             float scale_log2, uint32_t gd, uint32_t h, uint32_t c, uint32_t sub) {
  __shared__ float sm[W][G], sl[W][G];
  __shared__ float sacc[W][G][128];
  __shared__ __attribute__((aligned(16))) f16 qs[G][128];
  __shared__ __attribute__((aligned(16))) f16 knew[128], vnew[128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t q0 = h * gd + sub * G;
  const uint32_t begin = c * chunk;
  const size_t head_base = (size_t)h * cap;
  // the position first (written by the previous step's argmax), then every load that does not depend
  // on it: wave j's prologue job j (query head j < G, then k, then v; a wave past the jobs repeats the
  // last one, every workgroup loads the k and v jobs and only the owner keeps them), the RoPE row,
  // and the wave's two tiles (rows clamped to the capacity). Loads complete in issue order for the
  // wait counter: the position's wait holds nothing else, the RoPE's none of the tiles.
  const int32_t pv = load_first(pos);
  const uint32_t j0 = (uint32_t)wave < (uint32_t)G + 2 ? (uint32_t)wave : (uint32_t)G + 1;
  auto job_row = [&](uint32_t j) { return j < G ? q0 + j : j == G ? heads + h : heads + kvh + h; };
  const float *nwp = j0 < G ? qn : kn;
  const float x0 = qkv[(size_t)job_row(j0) * 128 + lane], x1 = qkv[(size_t)job_row(j0) * 128 + lane + 64];
  const float nw0 = nwp[lane], nw1 = nwp[lane + 64];
  const float cp = rope[lane], sp = rope[64 + lane];
  issue_order();
  const uint32_t kb = begin + wave * kpw;
  KTile<false> ta, tb;
  load_ktile<false, KEEP>(ta, kc, vc, nullptr, nullptr, head_base, kb, cap, lane);
  issue_order();
  if constexpr (!ONE) load_ktile<false, KEEP>(tb, kc, vc, nullptr, nullptr, head_base, kb + 16, cap, lane);
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
      if (sub == 0) {
        vc[(head_base + p) * 128 + lane] = (f16)a0;
        vc[(head_base + p) * 128 + lane + 64] = (f16)a1;
      }
    } else if (j < G) {
      qs[j][lane] = (f16)o0;
      qs[j][lane + 64] = (f16)o1;
    } else {
      knew[lane] = (f16)o0;
      knew[lane + 64] = (f16)o1;
      if (sub == 0) {
        kc[(head_base + p) * 128 + lane] = (f16)o0;
        kc[(head_base + p) * 128 + lane + 64] = (f16)o1;
      }
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
      load_ktile<false, KEEP>(ta, kc, vc, nullptr, nullptr, head_base, key + 32, cap, lane);
      patch(tb, key + 16);
      attend_ktile<G, false>(tb, qb, key + 16, ke, scale_log2, lane, m, ls, acc);
      load_ktile<false, KEEP>(tb, kc, vc, nullptr, nullptr, head_base, key + 48, cap, lane);
    }
    const uint32_t rem = nt - i;  // 0 .. 3: a pair at once (1,510 -> 1,521 tokens/s on the C5 decode step)
    if (rem == 2) {
      patch(ta, key);
      patch(tb, key + 16);
      attend_pair<G, false>(ta, tb, qb, key, ke, scale_log2, lane, m, ls, acc);
    } else {
      if (rem >= 1) {
        patch(ta, key);
        attend_ktile<G, false>(ta, qb, key, ke, scale_log2, lane, m, ls, acc);
      }
      if (rem == 3) load_ktile<false, KEEP>(ta, kc, vc, nullptr, nullptr, head_base, key + 32, cap, lane);
      if (rem == 3) {
        patch(tb, key + 16);
        attend_ktile<G, false>(tb, qb, key + 16, ke, scale_log2, lane, m, ls, acc);
      }
      if (rem == 3) {
        patch(ta, key + 32);
        attend_ktile<G, false>(ta, qb, key + 32, ke, scale_log2, lane, m, ls, acc);
      }
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
  const size_t base = ((size_t)h * nchunk + c) * gd + sub * G;
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

// The arguments fit the 56 bytes the hardware preloads into SGPRs at wave launch
// (-amdgpu-kernarg-preload-count), eps aside (loaded when first used): step = the step's RoPE row (cos
// | sin, 64 each) followed by the position (int32); kc = the K cache, the V cache right after it
// (kvh * cap rows of 128); ws = the partials o | m | l; qn = the q norm weights, the k norm weights
// right after them; nk = nchunk | kpw << 16; hk = kvh | gd << 8 | keep << 16 (keep: the chunks are
// read with cache-allocating loads, for a caller that keeps the rows in the memory-side cache, else
// with nontemporal ones).
template <int G, int W, bool ONE>
__global__ __launch_bounds__(64 * W) void k_attn_step(const float *__restrict__ step, const float *__restrict__ qkv,
                                                      f16 *__restrict__ kc, float *__restrict__ ws,
                                                      const float *__restrict__ qn, uint32_t cap, uint32_t nk,
                                                      uint32_t hk, float scale_log2, double eps) {
  kernarg_now(step, qkv, kc, ws, qn, cap, nk, hk, scale_log2);
  const uint32_t nchunk = nk & 0xffffu, kpw = nk >> 16, kvh = hk & 0xffu, gd = (hk >> 8) & 0xffu;
  const uint32_t heads = kvh * gd, chunk = kpw * W, slots = heads * nchunk;
  const int32_t *pos = (const int32_t *)(step + 128);
  f16 *vc = kc + (size_t)kvh * cap * 128;
  float *ws_m = ws + (size_t)slots * 128, *ws_l = ws_m + slots;
  const float *kn = qn + 128;
  const uint32_t nkc = kvh * nchunk, sub = blockIdx.x / nkc, rest = blockIdx.x % nkc;
  const uint32_t h = rest / nchunk, c = rest % nchunk;
  float *ws_o = ws;
  const float *rope = step;
  if ((hk >> 16) & 1u)
    attn_step_wg<G, W, ONE, true>(qkv, qn, kn, rope, eps, kc, vc, ws_o, ws_m, ws_l, pos, heads, kvh, cap, chunk,
                                  nchunk, kpw, scale_log2, gd, h, c, sub);
  else
    attn_step_wg<G, W, ONE, false>(qkv, qn, kn, rope, eps, kc, vc, ws_o, ws_m, ws_l, pos, heads, kvh, cap, chunk,
                                   nchunk, kpw, scale_log2, gd, h, c, sub);
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

template <int U>
__global__ __launch_bounds__(64) void k_attn_merge_wave(const float *__restrict__ o, const float *__restrict__ m,
                                                        const float *__restrict__ l, void *__restrict__ out,
                                                        uint32_t chunks, uint32_t G, int mode) {
  attn_merge_wave_wg<U>(blockIdx.x, blockIdx.y, o, m, l, out, chunks, G, mode);
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

// The split of hwk_attn_decode: workgroups of W waves, each wave kpw keys (a multiple of 16), chunk =
// W*kpw keys a workgroup. W = 8 for int8 caches from 8,192 keys, else 4. From 8,192 keys a kv head
// takes 32 chunks, so that the merge reads 32 partials a query head (measured at 8K, 16K and 32K keys
// over chunks of 128-2048 keys and 4 or 8 waves: the fastest, with the merge's cost growing with the
// chunks and the split's with the keys a workgroup; fp16 at 8,192 keys: 11.6 us a call in 4-wave
// workgroups against 12.0 in 8-wave ones). Below 8,192 keys kpw is sized so that the launch runs
// about 2048 waves (8 a CU, each with two tiles of loads in flight), between 32 and 256 keys, more
// when a head would exceed kMaxChunks chunks; and one 16-key tile a wave while a kv head then has at
// most 16 chunks (fp16) or 32 (int8): at 512 keys 7.2 / 7.1 us a call against 7.6 / 7.9 for two
// tiles, int8 at 2,048 keys 7.7 against 8.1 (fp16 at 2,048 keys, 32 chunks: 8.2 against 8.0).
// A caller's split (a multiple of 64) is the chunk.
uint32_t decode_waves(const hwk_attn_params *p) { return p->kv_int8 && p->len >= 8192 ? 8u : 4u; }

uint32_t pick_kpw(const hwk_attn_params *p) {
  const uint32_t W = decode_waves(p);
  if (p->split) return p->split / W;
  uint64_t kpw;
  if (p->len >= 8192) {
    kpw = ((uint64_t)p->len + 32ull * W - 1) / (32ull * W);
  } else {
    const uint64_t keys = (uint64_t)p->len * p->kv_heads;
    kpw = (keys + 2047) / 2048;
    if (kpw < 32) kpw = 32;
    if (kpw > 256) kpw = 256;
    if (kpw == 32 && ((uint64_t)p->len + 16ull * W - 1) / (16ull * W) <= (p->kv_int8 ? 32u : 16u)) kpw = 16;
  }
  kpw = (kpw + 15) / 16 * 16;
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
// merges every chunk's partial in its prologue); one query head a workgroup (two for 4 or more a kv
// head). (Eight waves of one tile each were measured no faster, with one or two heads a workgroup.)
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
                     const int32_t *pos, bool keep) {
  HWK_CHECK(p && qkv && qn && kn && rope && kc && vc && workspace && pos, "attn_step: null argument");
  HWK_CHECK(p->head_dim == 128 && !p->kv_int8, "attn_step: fp16 caches of head_dim 128 only");
  HWK_CHECK(p->kv_heads > 0 && p->heads % p->kv_heads == 0, "attn_step: %u heads over %u", p->heads, p->kv_heads);
  const uint32_t G = p->heads / p->kv_heads;
  HWK_CHECK(G == 1 || G == 2 || G == 4, "attn_step: %u query heads a kv head", G);
  HWK_CHECK(workspace_bytes >= attn_step_workspace_bytes(p), "attn_step: workspace too small");
  uint32_t chunk, nchunk;
  attn_step_layout(p, &chunk, &nchunk);
  float *ws_o = (float *)workspace;
  const float scale_log2 = hwk::f32_of_bits(p->scale_bits) * kLog2e;
  constexpr int W = kStepWaves;
  const uint32_t kpw = chunk / W;
  // the kernel's compact arguments: the k norm weights, the V cache and the position each lie at a
  // fixed offset from the q norm weights, the K cache and the RoPE row (the model's layout)
  HWK_CHECK(kn == qn + 128 && (const f16 *)vc == (const f16 *)kc + (size_t)p->kv_heads * p->capacity * 128 &&
                (const float *)pos == rope + 128,
            "attn_step: the k norm, V cache or position not where the kernel takes them");
  HWK_CHECK(p->kv_heads < 256 && G < 256 && nchunk < 65536 && kpw < 65536, "attn_step: %u kv heads, %u chunks",
            p->kv_heads, nchunk);
  const uint32_t nk = nchunk | kpw << 16, hk = p->kv_heads | G << 8 | (keep ? 1u : 0u) << 16;
#define HWK_STEP2(GG, ONE)                                                                                        \
  hipLaunchKernelGGL((k_attn_step<GG, W, ONE>), dim3(p->kv_heads * nchunk * (G / GG)), dim3(64 * W), 0, st, rope, qkv, \
                     (f16 *)kc, ws_o, qn, p->capacity, nk, hk, scale_log2, eps)
  if (G == 1 || G == 2) HWK_STEP2(1, false);
  else HWK_STEP2(2, false);
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
