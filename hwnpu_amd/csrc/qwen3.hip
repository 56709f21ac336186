// The Qwen3 decoder on gfx950 (the 28-layer synthetic model of the decode benchmark): a
// device-resident session in the shape of the reference's iron.Model (Step(token, pos) -> logits,
// internal/llm/iron/model.go:578) over the architecture of internal/llm/qwen3 (build.go:107-311;
// the float64 forward of qwen3_test.go:77-207 is the semantics restated here).
//
// Numerics: the residual stream h is fp32. Values cross kernels in fp16 exactly where noted:
//   x = fp16((h * r) * w)          RMSNorm into every linear (r = float(1/sqrt(mean h^2 + eps)))
//   q, k = fp16(rope(norm(q)))     per-head RMSNorm before RoPE (cos/sin tables in float32)
//   v = fp16(v); K/V cache fp16
//   attn = fp16(softmax(q k^T / sqrt(d)) v)   (fp32 softmax and P.V)
//   act = fp16(silu(gate) * up)
// Linears accumulate in fp32 (MXFP4 weights, the fp16 tied head); h += o_proj(attn) and
// h += down(act) in fp32. The greedy token is the first index of the largest logit.
//
// A decode step is five kernels a layer: the norm-fused qkv GEMV; the attention with the q/k norm,
// RoPE and KV append in its prologue (partials over chunks of the cache); o_proj, which merges the
// partials in its prologue; the norm- and SwiGLU-fused gate_up GEMV; down. Then four more: embed,
// final norm, head, argmax. Its token and position are read on the device (hist[pos], pos), and the
// argmax writes the next token and advances pos, so one captured graph replays for every step.
#include <math.h>
#include <algorithm>
#include <string>
#include <vector>

#include "glue_kernels.h"
#include "hwk_common.h"
#include "internal.h"
#include "synth.h"

namespace {

// ---- glue kernels (K6): the embedding gather, RMSNorm and SiLU*up are hwk_glue's (glue_kernels.h),
// the same kernels as the hwk_embed / hwk_rmsnorm / hwk_silu_mul entry points ----

using hwk_glue::embed_blocks;
using hwk_glue::k_embed_ids;
using hwk_glue::k_silu_mul;

// One wave a (token t, head slot): slots [0, heads) are query heads, [heads, heads+kvh) key heads,
// then value heads. A lane holds dims l and l+64, the pair rotate_half mixes. q and k: per-head
// RMSNorm with fp32 weights, then RoPE at position *pos + base + t with the float32 tables
// (reference internal/llm/blocks/blocks.go:412-445), rounded to fp16; q to q16 (t, heads, 128),
// k to the cache; v rounded to fp16 into the cache.
__global__ __launch_bounds__(256) void k_qk_rope(const float *__restrict__ qkv, const float *__restrict__ qn,
                                                 const float *__restrict__ kn, const float *__restrict__ cos_t,
                                                 const float *__restrict__ sin_t, const int32_t *__restrict__ pos,
                                                 uint32_t base, f16 *__restrict__ q16, f16 *__restrict__ kc,
                                                 f16 *__restrict__ vc, uint32_t heads, uint32_t kvh, uint32_t cap,
                                                 double eps) {
#pragma clang fp contract(off)
  const uint32_t slot = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t t = blockIdx.y, l = threadIdx.x & 63;
  const uint32_t slots = heads + 2 * kvh;
  if (slot >= slots) return;
  const uint32_t p = (uint32_t)*pos + base + t;
  const float *x = qkv + (size_t)t * slots * 128 + (size_t)slot * 128;
  float x0 = x[l], x1 = x[l + 64];
  if (slot >= heads + kvh) {
    const uint32_t j = slot - heads - kvh;
    f16 *dst = vc + ((size_t)j * cap + p) * 128;
    dst[l] = (f16)x0;
    dst[l + 64] = (f16)x1;
    return;
  }
  float o0, o1;
  const float *nw = slot < heads ? qn : kn;
  head_norm_rope(x0, x1, nw[l], nw[l + 64], cos_t[(size_t)p * 64 + l], sin_t[(size_t)p * 64 + l], eps, o0, o1);
  f16 *dst = slot < heads ? q16 + ((size_t)t * heads + slot) * 128
                          : kc + ((size_t)(slot - heads) * cap + p) * 128;
  dst[l] = (f16)o0;
  dst[l + 64] = (f16)o1;
}

__global__ void k_set_i32(int32_t *__restrict__ p, int32_t v) { *p = v; }

constexpr uint32_t kArgBlocks = 64;
constexpr int kArgPer = 10;  // values a thread takes a pass (151,936 logits: one pass)

__device__ __forceinline__ void better(float &bv, uint32_t &bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// Greedy pick (reference internal/chat/sample.go:80-87: strict >, so the lowest index of the
// largest value) over kArgBlocks workgroups; the last one to finish reduces their partials in
// a fixed order, writes the token at hist[*pos + 1], advances *pos and clears the counter for the
// next call.
__global__ __launch_bounds__(256) void k_argmax(const float *__restrict__ x, uint32_t n, float *__restrict__ part_v,
                                                uint32_t *__restrict__ part_i, uint32_t *__restrict__ counter,
                                                int32_t *__restrict__ hist, int32_t *__restrict__ pos) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  __shared__ bool last;
  kernarg_now(x, n, part_v, part_i, counter, hist, pos);
  const uint32_t t = threadIdx.x;
  const uint32_t per = (n + kArgBlocks - 1) / kArgBlocks;
  const uint32_t lo = blockIdx.x * per, hi = lo + per < n ? lo + per : n;
  float bv = -__builtin_inff();
  uint32_t bi = 0xffffffffu;
  // kArgPer values a thread, all loads issued at once (a slot past hi reads an in-range value and
  // is skipped)
  for (uint32_t base = lo; base < hi; base += kArgPer * 256) {
    float v[kArgPer];
#pragma unroll
    for (int j = 0; j < kArgPer; j++) v[j] = x[min(base + t + j * 256, hi - 1)];
#pragma unroll
    for (int j = 0; j < kArgPer; j++)
      if (base + t + j * 256 < hi) better(bv, bi, v[j], base + t + j * 256);
  }
  wave_best(bv, bi);
  if ((t & 63) == 0) {
    sv[t >> 6] = bv;
    si[t >> 6] = bi;
  }
  __syncthreads();
  // The handoff by the memory model: thread 0 stores the block's partial, then counts the block in
  // with an agent-scope acquire-release add, so every partial store happens before the adds that
  // follow it in the counter's modification order. The block that draws the last count acquires
  // all of them; its barrier carries that to the threads that read the partials.
  if (t == 0) {
    for (int w = 1; w < 4; w++) better(bv, bi, sv[w], si[w]);
    __hip_atomic_store(&part_v[blockIdx.x], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&part_i[blockIdx.x], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  if (t < 64) {
    const uint32_t c = t < gridDim.x ? t : gridDim.x - 1;
    float v = __hip_atomic_load(&part_v[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t i = __hip_atomic_load(&part_i[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int32_t p = *pos;
    const float x0 = x[0];  // a NaN at index 0 is kept: strict > never replaces it
    if (t >= gridDim.x) {
      v = -__builtin_inff();
      i = 0xffffffffu;
    }
    wave_best(v, i);
    if (t == 0) {
      hist[p + 1] = (int32_t)((i == 0xffffffffu || x0 != x0) ? 0 : i);
      *pos = p + 1;
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The decode step's first kernel: the embedding row of the token hist[*pos] into h (fp32), and the
// RoPE tables' row *pos into rope_now (cos | sin, 64 values each), so that the step's attention
// kernels read their cos/sin without first waiting for the position.
__global__ __launch_bounds__(256) void k_step_embed(const int32_t *__restrict__ hist, const int32_t *__restrict__ pos,
                                                    const f16 *__restrict__ table, float *__restrict__ h,
                                                    uint32_t hidden, uint32_t vocab, const float *__restrict__ cos_t,
                                                    const float *__restrict__ sin_t, float *__restrict__ rope_now) {
  kernarg_now(hist, pos, table, h, hidden, vocab, cos_t, sin_t, rope_now);
  const uint32_t p = (uint32_t)*pos;
  const int32_t id = hist[p];
  const bool ok = id >= 0 && (uint32_t)id < vocab;
  const f16 *row = table + (size_t)(ok ? id : 0) * hidden;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < hidden; i += gridDim.x * 256)
    h[i] = ok ? (float)row[i] : __builtin_nanf("");
  if (blockIdx.x == 0 && threadIdx.x < 128)
    rope_now[threadIdx.x] = threadIdx.x < 64 ? cos_t[(size_t)p * 64 + threadIdx.x] : sin_t[(size_t)p * 64 + threadIdx.x - 64];
}

uint64_t fnv64a(const std::string &s) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001B3ull;
  }
  return h;
}

double f64_of_bits(uint64_t b) {
  double d;
  memcpy(&d, &b, 8);
  return d;
}

__global__ void k_fill_f32(float *__restrict__ p, uint64_t n, float v) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// Rows of positions [from, from + gridDim.x) of every K/V cache, packed per position with the caches
// in the order of tab (their base pointers): cache c's row is kvh heads x 128 fp16 (16 uint4 a
// head). EXPORT copies the caches into packed, else packed into the caches.
template <bool EXPORT>
__global__ __launch_bounds__(256) void k_kv_rows(const uint64_t *__restrict__ tab, uint4 *__restrict__ packed,
                                                 uint32_t from, uint32_t ncache, uint32_t kvh, uint32_t cap) {
  const uint32_t p = blockIdx.x, c = blockIdx.y, per = kvh * 16;
  uint4 *cache = (uint4 *)tab[c];
  uint4 *pk = packed + ((size_t)p * ncache + c) * per;
  for (uint32_t i = threadIdx.x; i < per; i += 256) {
    uint4 *cell = cache + ((size_t)(i / 16) * cap + from + p) * 16 + i % 16;
    if constexpr (EXPORT)
      pk[i] = *cell;
    else
      *cell = pk[i];
  }
}

// The greedy token of each row of logits (rows, n), one workgroup a row: strict > (the lowest index
// of the largest value), a NaN at index 0 kept, as k_argmax.
__global__ __launch_bounds__(1024) void k_argmax_rows(const float *__restrict__ x, uint32_t n,
                                                      int32_t *__restrict__ out) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const float *row = x + (size_t)blockIdx.x * n;
  const uint32_t t = threadIdx.x;
  float bv = -__builtin_inff();
  uint32_t bi = 0xffffffffu;
  for (uint32_t i = t; i < n; i += 1024) better(bv, bi, row[i], i);
  wave_best(bv, bi);
  if ((t & 63) == 0) {
    sv[t >> 6] = bv;
    si[t >> 6] = bi;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < 16; w++) better(bv, bi, sv[w], si[w]);
    const float x0 = row[0];
    out[blockIdx.x] = (int32_t)((bi == 0xffffffffu || x0 != x0) ? 0 : bi);
  }
}

// Keep of a verify: the greedy token of row kept-1 becomes the next step's token, past the kept rows.
__global__ void k_keep(const int32_t *__restrict__ am, uint32_t kept, uint32_t start, int32_t *__restrict__ hist,
                       int32_t *__restrict__ pos) {
  hist[start + kept] = am[kept - 1];
  *pos = (int32_t)(start + kept);
}

// The sequence moved to position p, with the token there set when tok >= 0.
__global__ void k_rewind(int32_t *__restrict__ hist, int32_t *__restrict__ pos, uint32_t p, int32_t tok) {
  if (tok >= 0) hist[p] = tok;
  *pos = (int32_t)p;
}

}  // namespace

struct hwk_qwen3 {
  hwk_qwen3_config c;
  double theta, eps;
  uint32_t qkv_n, att_n;  // rows of the stacked q/k/v projection; width of the attention output
  size_t bytes = 0;
  uint8_t *base = nullptr;  // one allocation for weights, cache, state and scratch
  struct Lin {
    uint8_t *w, *e;
    uint32_t rows, cols;
  };
  struct Layer {
    Lin qkv, o, gu, down;
    float *in_norm, *post_norm, *q_norm, *k_norm;
    f16 *kc, *vc;
  };
  std::vector<Layer> L;
  float *norm;
  f16 *embed;
  float *cos_t, *sin_t;
  float *rope_now;  // the decode step's cos | sin rows at its position (head_dim/2 values each)
  int32_t *hist, *pos;
  uint32_t *counter, *part_i;
  uint32_t step_chunk = 0, step_nchunk = 0;  // the decode attention's chunking (attn_step_layout)
  // a decode step reading at most keep_rows cache rows of every layer reads them with cache-allocating
  // loads (they then stay in the memory-side cache from step to step), a later one with nontemporal
  // loads
  uint32_t keep_rows = 0;
  float *part_v, *logits;
  uint64_t *cache_tab;  // the K/V caches' base pointers in the export order (kv_k_N_new / kv_v_N_new sorted)
  float *vlogits;       // a verify's logits (kMaxVerify, vocab) and greedy tokens (kMaxVerify)
  int32_t *vargmax;
  uint32_t verify_start = 0, verify_n = 0;  // the last verify, until its keep (verify_n 0: none)
  float *h, *qkv, *gu;
  f16 *x16, *q16, *att16, *a16;
  void *ws;
  size_t ws_bytes;
  hwk_attn_params ap;  // decode attention: len = capacity (the grid), the length read on the device
  uint32_t host_pos = 0;  // mirror of *pos: where the next step writes
  bool started = false;
  hipStream_t cap = nullptr;
  // the decode step captured once as a graph of one step and one of kGraphSteps steps (a step
  // reads its token and position on the device and advances them, so consecutive replays chain),
  // each with the cache rows read nontemporally [0][.] or kept [1][.]
  hipGraphExec_t exec[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
  hipGraph_t graph[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
};

namespace {

constexpr uint32_t kMaxVerify = 8;  // rows a speculative verify takes
// The most KV cache bytes (all layers) a decode step reads with cache-allocating loads: up to that
// many, the rows stay in the device's 256 MB memory-side cache from one step to the next (the
// weights stream past it with nontemporal loads; their fp4 scale bytes, 1/17 of them, are the other
// data it keeps). Measured on the C5 decode (28 layers, 4 KB a position): keeping the rows gains
// 1.2-2.4 % up to position 1,695 (195 MB) and loses 1.5 % from 1,696 on; nontemporal loads past it.
constexpr uint64_t kKeepCacheBytes = 176ull << 20;

struct Carver {
  size_t off = 0;
  template <typename T>
  T *take(uint8_t *base, size_t bytes) {
    off = (off + 255) / 256 * 256;
    T *p = base ? (T *)(base + off) : nullptr;
    off += bytes;
    return p;
  }
};

// Lays the model out in one allocation (base null: only counts the bytes).
void layout(hwk_qwen3 *m, uint8_t *base) {
  const hwk_qwen3_config &c = m->c;
  Carver cv;
  auto lin = [&](uint32_t rows, uint32_t cols) {
    hwk_qwen3::Lin l;
    l.rows = rows;
    l.cols = cols;
    l.w = cv.take<uint8_t>(base, (size_t)rows * cols / 2);
    l.e = cv.take<uint8_t>(base, (size_t)rows * cols / 32);
    return l;
  };
  m->L.resize(c.layers);
  for (auto &ly : m->L) {
    ly.qkv = lin(m->qkv_n, c.hidden);
    ly.o = lin(c.hidden, m->att_n);
    ly.gu = lin(2 * c.inter, c.hidden);
    ly.down = lin(c.hidden, c.inter);
    ly.in_norm = cv.take<float>(base, 4ull * c.hidden);
    ly.post_norm = cv.take<float>(base, 4ull * c.hidden);
    ly.q_norm = cv.take<float>(base, 4ull * c.head_dim);
    ly.k_norm = cv.take<float>(base, 4ull * c.head_dim);
    ly.kc = cv.take<f16>(base, 2ull * c.kv_heads * c.max_ctx * c.head_dim);
    ly.vc = cv.take<f16>(base, 2ull * c.kv_heads * c.max_ctx * c.head_dim);
  }
  m->norm = cv.take<float>(base, 4ull * c.hidden);
  m->embed = cv.take<f16>(base, 2ull * c.vocab * c.hidden);
  m->cos_t = cv.take<float>(base, 4ull * c.max_ctx * (c.head_dim / 2));
  m->sin_t = cv.take<float>(base, 4ull * c.max_ctx * (c.head_dim / 2));
  // the step's RoPE row and, right after it, the position (the decode attention finds it there)
  m->rope_now = cv.take<float>(base, 4ull * c.head_dim + 4);
  m->pos = (int32_t *)(m->rope_now + c.head_dim);
  m->hist = cv.take<int32_t>(base, 4ull * (c.max_ctx + 1));
  m->counter = cv.take<uint32_t>(base, 4);
  m->part_i = cv.take<uint32_t>(base, 4 * kArgBlocks);
  m->part_v = cv.take<float>(base, 4 * kArgBlocks);
  m->logits = cv.take<float>(base, 4ull * c.vocab);
  m->cache_tab = cv.take<uint64_t>(base, 16ull * c.layers);
  m->vlogits = cv.take<float>(base, 4ull * kMaxVerify * c.vocab);
  m->vargmax = cv.take<int32_t>(base, 4ull * kMaxVerify);
  const size_t T = c.max_prompt;
  m->h = cv.take<float>(base, 4 * T * c.hidden);
  m->qkv = cv.take<float>(base, 4 * T * m->qkv_n);
  m->gu = cv.take<float>(base, 8 * T * c.inter);
  m->x16 = cv.take<f16>(base, 2 * T * (c.hidden > c.inter ? c.hidden : c.inter));
  m->q16 = cv.take<f16>(base, 2 * T * m->att_n);
  m->att16 = cv.take<f16>(base, 2 * T * m->att_n);
  m->a16 = cv.take<f16>(base, 2 * T * c.inter);
  m->ws = cv.take<uint8_t>(base, m->ws_bytes);
  m->bytes = cv.off;
}

#define HWK_Q(call)                  \
  do {                               \
    if (char *e_ = (call)) return e_; \
  } while (0)

// Steps a replay of the long graph runs: the gap between graph launches is paid once for them.
constexpr uint32_t kGraphSteps = 8;

// Captures graph slot [keep][i] (n decode steps) on the model's private stream the first time it is
// needed.
char *capture(hwk_qwen3 *m, int keep, int i, uint32_t n);

// Whether steps whose last one writes position last (and reads cache rows 0 .. last) keep the rows.
bool keeps(const hwk_qwen3 *m, uint32_t last) { return last < m->keep_rows; }

// The decode step on stream st: the token hist[*pos] at position *pos; keep: the attention reads the
// cache rows with cache-allocating loads.
char *step(hwk_qwen3 *m, hipStream_t st, bool keep) {
  const hwk_qwen3_config &c = m->c;
  hipLaunchKernelGGL(k_step_embed, dim3(embed_blocks(c.hidden)), dim3(256), 0, st, m->hist, m->pos, m->embed, m->h,
                     c.hidden, c.vocab, m->cos_t, m->sin_t, m->rope_now);
  HWK_Q(hwk::launched("qwen3 embed"));
  for (auto &ly : m->L) {
    HWK_Q(hwk::mxfp4_gemv_x(st, ly.qkv.w, ly.qkv.e, nullptr, m->h, ly.in_norm, m->eps, m->qkv, m->qkv_n, c.hidden,
                            HWK_OUT_F32, false));
    // attention partials over chunks of the cache, merged by the o_proj GEMV into its input
    HWK_Q(hwk::attn_step(st, m->qkv, ly.q_norm, ly.k_norm, m->rope_now, m->eps, ly.kc, ly.vc, m->ws, m->ws_bytes,
                         &m->ap, m->pos, keep));
    HWK_Q(hwk::mxfp4_gemv_merge(st, ly.o.w, ly.o.e, m->ws, c.heads, c.heads / c.kv_heads, m->step_nchunk, m->h,
                                c.hidden, HWK_OUT_ADD_F32));
    HWK_Q(hwk::mxfp4_gemv_x(st, ly.gu.w, ly.gu.e, nullptr, m->h, ly.post_norm, m->eps, m->a16, 2 * c.inter, c.hidden,
                            HWK_OUT_F16, true));
    HWK_Q(hwk_mxfp4_gemv(st, ly.down.w, ly.down.e, m->a16, m->h, c.hidden, c.inter, HWK_OUT_ADD_F32));
  }
  HWK_Q(hwk::rmsnorm_f16(st, m->h, m->norm, m->eps, m->x16, 1, c.hidden));
  HWK_Q(hwk_f16_gemv(st, m->embed, m->x16, m->logits, c.vocab, c.hidden, HWK_OUT_F32));
  hipLaunchKernelGGL(k_argmax, dim3(kArgBlocks), dim3(256), 0, st, m->logits, c.vocab, m->part_v, m->part_i,
                     m->counter, m->hist, m->pos);
  return hwk::launched("qwen3 argmax");
}

char *capture(hwk_qwen3 *m, int keep, int i, uint32_t n) {
  if (m->exec[keep][i]) return nullptr;
  HWK_TRY("hipStreamBeginCapture", hipStreamBeginCapture(m->cap, hipStreamCaptureModeRelaxed));
  char *err = nullptr;
  for (uint32_t s = 0; s < n && !err; s++) err = step(m, m->cap, keep != 0);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(m->cap, &g);
  if (err) {
    if (g) (void)hipGraphDestroy(g);
    return err;
  }
  if (e != hipSuccess) return hwk::hip_err("hipStreamEndCapture", e);
  m->graph[keep][i] = g;
  HWK_TRY("hipGraphInstantiate", hipGraphInstantiate(&m->exec[keep][i], g, nullptr, nullptr, 0));
  return nullptr;
}

// Rows [0, T) of a prompt piece at positions start .. start+T-1, whose tokens are in hist.
char *prefill_piece(hwk_qwen3 *m, hipStream_t st, uint32_t T, uint32_t start, bool last_piece) {
  const hwk_qwen3_config &c = m->c;
  hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(1), 0, st, m->pos, (int32_t)start);
  hipLaunchKernelGGL(k_embed_ids, dim3(embed_blocks(c.hidden), T), dim3(256), 0, st, m->hist, m->pos, 0u, m->embed,
                     m->h, c.hidden, c.vocab);
  HWK_Q(hwk::launched("qwen3 embed"));
  const uint32_t slots = c.heads + 2 * c.kv_heads;
  hwk_attn_params pp = m->ap;
  pp.len = start + T;
  pp.out_mode = HWK_OUT_F16;
  for (auto &ly : m->L) {
    HWK_Q(hwk::rmsnorm_f16(st, m->h, ly.in_norm, m->eps, m->x16, T, c.hidden));
    HWK_Q(hwk_mxfp4_gemm(st, m->x16, ly.qkv.w, ly.qkv.e, m->qkv, T, m->qkv_n, c.hidden, HWK_OUT_F32));
    hipLaunchKernelGGL(k_qk_rope, dim3((slots + 3) / 4, T), dim3(256), 0, st, m->qkv, ly.q_norm, ly.k_norm, m->cos_t,
                       m->sin_t, m->pos, 0u, m->q16, ly.kc, ly.vc, c.heads, c.kv_heads, c.max_ctx, m->eps);
    HWK_Q(hwk::launched("qwen3 qk_rope"));
    HWK_Q(hwk_attn_prefill(st, m->q16, ly.kc, ly.vc, m->att16, T, start, &pp));
    HWK_Q(hwk_mxfp4_gemm(st, m->att16, ly.o.w, ly.o.e, m->h, T, c.hidden, m->att_n, HWK_OUT_ADD_F32));
    HWK_Q(hwk::rmsnorm_f16(st, m->h, ly.post_norm, m->eps, m->x16, T, c.hidden));
    HWK_Q(hwk_mxfp4_gemm(st, m->x16, ly.gu.w, ly.gu.e, m->a16, T, 2 * c.inter, c.hidden, HWK_OUT_SWIGLU_F16));
    HWK_Q(hwk_mxfp4_gemm(st, m->a16, ly.down.w, ly.down.e, m->h, T, c.hidden, c.inter, HWK_OUT_ADD_F32));
  }
  if (!last_piece) return nullptr;
  // the head on the last row; the argmax writes hist[start+T] and sets pos = start+T
  hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(1), 0, st, m->pos, (int32_t)(start + T - 1));
  HWK_Q(hwk::rmsnorm_f16(st, m->h + (size_t)(T - 1) * c.hidden, m->norm, m->eps, m->x16, 1, c.hidden));
  HWK_Q(hwk_f16_gemv(st, m->embed, m->x16, m->logits, c.vocab, c.hidden, HWK_OUT_F32));
  hipLaunchKernelGGL(k_argmax, dim3(kArgBlocks), dim3(256), 0, st, m->logits, c.vocab, m->part_v, m->part_i,
                     m->counter, m->hist, m->pos);
  return hwk::launched("qwen3 argmax");
}

// y (T rows) = the linear of T fp16 vectors x, every weight row read once for each piece of
// vectors whose fp16 copy fits K1r's 64 KB of LDS. mode F32 or ADD (fp32 y).
char *rows_linear(hipStream_t st, const f16 *x, const hwk_qwen3::Lin &l, float *y, uint32_t T, int mode) {
  const uint32_t per = (64u * 1024u) / (2u * l.cols);
  for (uint32_t t0 = 0; t0 < T; t0 += per) {
    const uint32_t tn = T - t0 < per ? T - t0 : per;
    HWK_Q(hwk_mxfp4_gemv_rows(st, l.w, l.e, x + (size_t)t0 * l.cols, y + (size_t)t0 * l.rows, l.rows, l.cols, tn,
                              mode));
  }
  return nullptr;
}

// A speculative verify: the T tokens in hist[start .. start+T-1] at those positions, every row
// through the decoder (K1r linears, causal attention over the cache and the rows before it), the
// head on every row into vlogits and each row's greedy token into vargmax. The values cross
// kernels in fp16 where the decode step rounds them, so row t's logits are those of the decode
// step at position start+t up to fp32 summation order. *pos is start throughout.
char *verify_piece(hwk_qwen3 *m, hipStream_t st, uint32_t T, uint32_t start) {
  const hwk_qwen3_config &c = m->c;
  hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(1), 0, st, m->pos, (int32_t)start);
  hipLaunchKernelGGL(k_embed_ids, dim3(embed_blocks(c.hidden), T), dim3(256), 0, st, m->hist, m->pos, 0u, m->embed,
                     m->h, c.hidden, c.vocab);
  HWK_Q(hwk::launched("qwen3 verify embed"));
  const uint32_t slots = c.heads + 2 * c.kv_heads;
  hwk_attn_params pp = m->ap;
  pp.len = start + T;
  pp.out_mode = HWK_OUT_F16;
  for (auto &ly : m->L) {
    HWK_Q(hwk::rmsnorm_f16(st, m->h, ly.in_norm, m->eps, m->x16, T, c.hidden));
    HWK_Q(rows_linear(st, m->x16, ly.qkv, m->qkv, T, HWK_OUT_F32));
    hipLaunchKernelGGL(k_qk_rope, dim3((slots + 3) / 4, T), dim3(256), 0, st, m->qkv, ly.q_norm, ly.k_norm, m->cos_t,
                       m->sin_t, m->pos, 0u, m->q16, ly.kc, ly.vc, c.heads, c.kv_heads, c.max_ctx, m->eps);
    HWK_Q(hwk::launched("qwen3 verify qk_rope"));
    HWK_Q(hwk_attn_prefill(st, m->q16, ly.kc, ly.vc, m->att16, T, start, &pp));
    HWK_Q(rows_linear(st, m->att16, ly.o, m->h, T, HWK_OUT_ADD_F32));
    HWK_Q(hwk::rmsnorm_f16(st, m->h, ly.post_norm, m->eps, m->x16, T, c.hidden));
    HWK_Q(rows_linear(st, m->x16, ly.gu, m->gu, T, HWK_OUT_F32));
    const uint64_t n = (uint64_t)T * c.inter;
    hipLaunchKernelGGL(k_silu_mul<true>, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, m->gu, m->gu + 1, m->a16, n,
                       2u);
    HWK_Q(hwk::launched("qwen3 verify swiglu"));
    HWK_Q(rows_linear(st, m->a16, ly.down, m->h, T, HWK_OUT_ADD_F32));
  }
  HWK_Q(hwk::rmsnorm_f16(st, m->h, m->norm, m->eps, m->x16, T, c.hidden));
  HWK_Q(hwk_f16_gemv_rows(st, m->embed, m->x16, m->vlogits, c.vocab, c.hidden, T, HWK_OUT_F32));
  hipLaunchKernelGGL(k_argmax_rows, dim3(T), dim3(1024), 0, st, m->vlogits, c.vocab, m->vargmax);
  return hwk::launched("qwen3 verify argmax");
}

}  // namespace

extern "C" {

HWK_API char *hwk_qwen3_new(const hwk_qwen3_config *cfg, hwk_qwen3 **out) {
  HWK_CHECK(cfg && out, "hwk_qwen3_new: null argument");
  const hwk_qwen3_config &c = *cfg;
  HWK_CHECK(c.layers >= 1 && c.layers <= 256, "hwk_qwen3_new: %u layers", c.layers);
  HWK_CHECK(c.head_dim == 128, "hwk_qwen3_new: head_dim %u (128 only)", c.head_dim);
  HWK_CHECK(c.kv_heads > 0 && c.heads % c.kv_heads == 0 && (c.heads / c.kv_heads == 1 || c.heads / c.kv_heads == 2 ||
                                                           c.heads / c.kv_heads == 4),
            "hwk_qwen3_new: %u heads over %u kv heads", c.heads, c.kv_heads);
  HWK_CHECK(c.hidden % 32 == 0 && c.hidden > 0 && c.hidden <= 8192, "hwk_qwen3_new: hidden %u", c.hidden);
  HWK_CHECK(c.inter % 32 == 0 && c.inter > 0 && c.inter <= 8192, "hwk_qwen3_new: inter %u", c.inter);
  HWK_CHECK(c.heads * c.head_dim <= 8192, "hwk_qwen3_new: heads*head_dim %u past 8192", c.heads * c.head_dim);
  HWK_CHECK(c.vocab >= 1 && c.max_ctx >= 2 && c.max_prompt >= 1 && c.max_prompt <= c.max_ctx,
            "hwk_qwen3_new: vocab %u, max_ctx %u, max_prompt %u", c.vocab, c.max_ctx, c.max_prompt);
  hwk_qwen3 *m = new hwk_qwen3();
  m->c = c;
  m->theta = f64_of_bits(c.theta_bits);
  m->eps = f64_of_bits(c.eps_bits);
  m->qkv_n = (c.heads + 2 * c.kv_heads) * c.head_dim;
  m->att_n = c.heads * c.head_dim;
  hwk_attn_params &ap = m->ap;
  ap.heads = c.heads;
  ap.kv_heads = c.kv_heads;
  ap.head_dim = c.head_dim;
  ap.len = c.max_ctx;
  ap.capacity = c.max_ctx;
  ap.kv_int8 = 0;
  const float sc = (float)(1.0 / sqrt((double)c.head_dim));
  memcpy(&ap.scale_bits, &sc, 4);
  ap.out_mode = HWK_OUT_F16;
  ap.split = 0;
  hwk::attn_step_layout(&ap, &m->step_chunk, &m->step_nchunk);
  m->ws_bytes = hwk::attn_step_workspace_bytes(&ap);
  {
    const uint64_t row = (uint64_t)c.layers * c.kv_heads * c.head_dim * 2 * sizeof(uint16_t);
    m->keep_rows = (uint32_t)std::min<uint64_t>(kKeepCacheBytes / row, c.max_ctx);
  }
  layout(m, nullptr);
  hipError_t e = hipMalloc((void **)&m->base, m->bytes);
  if (e != hipSuccess) {
    char *err = hwk::errf("hwk_qwen3_new: hipMalloc of %zu bytes: %s", m->bytes, hipGetErrorString(e));
    delete m;
    return err;
  }
  layout(m, m->base);
  // the caches in the order of the reference's names sorted as strings (decode.go:484), for the
  // rows export_rows packs
  std::vector<std::pair<std::string, uint64_t>> caches;
  for (uint32_t i = 0; i < c.layers; i++) {
    caches.push_back({"kv_k_" + std::to_string(i) + "_new", (uint64_t)(uintptr_t)m->L[i].kc});
    caches.push_back({"kv_v_" + std::to_string(i) + "_new", (uint64_t)(uintptr_t)m->L[i].vc});
  }
  std::sort(caches.begin(), caches.end());
  std::vector<uint64_t> tab;
  for (auto &cp : caches) tab.push_back(cp.second);
  // RoPE tables in float32 of float64 cos/sin (reference blocks.go:412-425, config.go:152-159)
  const uint32_t half = c.head_dim / 2;
  std::vector<float> ct((size_t)c.max_ctx * half), stb((size_t)c.max_ctx * half);
  for (uint32_t p = 0; p < c.max_ctx; p++)
    for (uint32_t j = 0; j < half; j++) {
      const double inv = 1.0 / pow(m->theta, (double)(2 * j) / (double)c.head_dim);
      const double a = (double)p * inv;
      ct[(size_t)p * half + j] = (float)cos(a);
      stb[(size_t)p * half + j] = (float)sin(a);
    }
  char *err = nullptr;
  if ((e = hipMemcpy(m->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(m->cache_tab, tab.data(), tab.size() * 8, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(m->sin_t, stb.data(), stb.size() * 4, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemset(m->hist, 0, 4ull * (c.max_ctx + 1))) != hipSuccess || (e = hipMemset(m->pos, 0, 4)) != hipSuccess ||
      (e = hipMemset(m->counter, 0, 4)) != hipSuccess ||
      (e = hipStreamCreateWithFlags(&m->cap, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipDeviceSynchronize()) != hipSuccess)
    err = hwk::hip_err("hwk_qwen3_new", e);
  if (err) {
    hwk_qwen3_free(m);
    return err;
  }
  *out = m;
  return nullptr;
}

HWK_API void hwk_qwen3_free(hwk_qwen3 *m) {
  if (!m) return;
  for (int k = 0; k < 2; k++)
    for (int i = 0; i < 2; i++) {
      if (m->exec[k][i]) (void)hipGraphExecDestroy(m->exec[k][i]);
      if (m->graph[k][i]) (void)hipGraphDestroy(m->graph[k][i]);
    }
  if (m->cap) (void)hipStreamDestroy(m->cap);
  if (m->base) {
    (void)hipDeviceSynchronize();
    (void)hipFree(m->base);
  }
  delete m;
}

HWK_API char *hwk_qwen3_synth(hwk_qwen3 *m, void *stream, uint64_t seed, uint32_t std_bits) {
  HWK_CHECK(m, "hwk_qwen3_synth: null model");
  hipStream_t st = (hipStream_t)stream;
  const hwk_qwen3_config &c = m->c;
  const float sd = hwk::f32_of_bits(std_bits);
  const uint32_t hd = c.head_dim, qn = c.heads * hd, kn = c.kv_heads * hd;
  for (uint32_t i = 0; i < c.layers; i++) {
    hwk_qwen3::Layer &ly = m->L[i];
    const std::string p = "model.layers." + std::to_string(i) + ".";
    auto key = [&](const char *name) { return seed ^ fnv64a(p + name); };
    // q, k, v stacked; rows of one projection are one stream
    const uint32_t nb = c.hidden / 32;
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.qkv.w, ly.qkv.e, qn, c.hidden, key("self_attn.q_proj.weight"), sd, 1, 0));
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.qkv.w, ly.qkv.e, kn, c.hidden, key("self_attn.k_proj.weight"), sd, 1, qn));
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.qkv.w, ly.qkv.e, kn, c.hidden, key("self_attn.v_proj.weight"), sd, 1, qn + kn));
    (void)nb;
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.o.w, ly.o.e, c.hidden, qn, key("self_attn.o_proj.weight"), sd, 1, 0));
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.gu.w, ly.gu.e, c.inter, c.hidden, key("mlp.gate_proj.weight"), sd, 2, 0));
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.gu.w, ly.gu.e, c.inter, c.hidden, key("mlp.up_proj.weight"), sd, 2, 1));
    HWK_Q(hwk::synth_mxfp4_rows(st, ly.down.w, ly.down.e, c.hidden, c.inter, key("mlp.down_proj.weight"), sd, 1, 0));
    float *ones[4] = {ly.in_norm, ly.post_norm, ly.q_norm, ly.k_norm};
    const uint32_t lens[4] = {c.hidden, c.hidden, hd, hd};
    for (int j = 0; j < 4; j++)
      hipLaunchKernelGGL(k_fill_f32, dim3((lens[j] + 255) / 256), dim3(256), 0, st, ones[j], (uint64_t)lens[j], 1.0f);
  }
  hipLaunchKernelGGL(k_fill_f32, dim3((c.hidden + 255) / 256), dim3(256), 0, st, m->norm, (uint64_t)c.hidden, 1.0f);
  HWK_Q(hwk::launched("hwk_qwen3_synth (norms)"));
  return hwk_synth_normal(stream, m->embed, (uint64_t)c.vocab * c.hidden, seed ^ fnv64a("model.embed_tokens.weight"),
                          std_bits, 1);
}

HWK_API char *hwk_qwen3_tensor(hwk_qwen3 *m, const char *name, void **ptr, size_t *bytes) {
  HWK_CHECK(m && name && ptr && bytes, "hwk_qwen3_tensor: null argument");
  const hwk_qwen3_config &c = m->c;
  std::string n(name);
  auto put = [&](void *p, size_t b) {
    *ptr = p;
    *bytes = b;
    return (char *)nullptr;
  };
  if (n == "norm") return put(m->norm, 4ull * c.hidden);
  if (n == "embed") return put(m->embed, 2ull * c.vocab * c.hidden);
  unsigned li = 0;
  char rest[64] = {0};
  if (sscanf(name, "layers.%u.%63s", &li, rest) == 2 && li < c.layers) {
    hwk_qwen3::Layer &ly = m->L[li];
    std::string r(rest);
    hwk_qwen3::Lin *lin = nullptr;
    std::string part;
    const size_t dot = r.find('.');
    std::string head = dot == std::string::npos ? r : r.substr(0, dot);
    part = dot == std::string::npos ? "" : r.substr(dot + 1);
    if (head == "qkv") lin = &ly.qkv;
    else if (head == "o") lin = &ly.o;
    else if (head == "gate_up") lin = &ly.gu;
    else if (head == "down") lin = &ly.down;
    if (lin && part == "blocks") return put(lin->w, (size_t)lin->rows * lin->cols / 2);
    if (lin && part == "scales") return put(lin->e, (size_t)lin->rows * lin->cols / 32);
    if (r == "input_norm") return put(ly.in_norm, 4ull * c.hidden);
    if (r == "post_norm") return put(ly.post_norm, 4ull * c.hidden);
    if (r == "q_norm") return put(ly.q_norm, 4ull * c.head_dim);
    if (r == "k_norm") return put(ly.k_norm, 4ull * c.head_dim);
    if (r == "k_cache") return put(ly.kc, 2ull * c.kv_heads * c.max_ctx * c.head_dim);
    if (r == "v_cache") return put(ly.vc, 2ull * c.kv_heads * c.max_ctx * c.head_dim);
  }
  return hwk::errf("hwk_qwen3_tensor: no tensor %s", name);
}

HWK_API char *hwk_qwen3_state(hwk_qwen3 *m, void **logits, void **hist, void **pos) {
  HWK_CHECK(m, "hwk_qwen3_state: null model");
  if (logits) *logits = m->logits;
  if (hist) *hist = m->hist;
  if (pos) *pos = m->pos;
  return nullptr;
}

HWK_API char *hwk_qwen3_prefill(hwk_qwen3 *m, void *stream, const int32_t *tokens, uint32_t n, uint32_t start) {
  HWK_CHECK(m && tokens, "hwk_qwen3_prefill: null argument");
  HWK_CHECK(n >= 1, "hwk_qwen3_prefill: empty prompt");
  HWK_CHECK((uint64_t)start + n < m->c.max_ctx, "hwk_qwen3_prefill: positions %u+%u leave no room in %u", start, n,
            m->c.max_ctx);
  HWK_CHECK(start <= m->host_pos, "hwk_qwen3_prefill: start %u past the cached positions (%u)", start, m->host_pos);
  for (uint32_t i = 0; i < n; i++)
    HWK_CHECK(tokens[i] >= 0 && (uint32_t)tokens[i] < m->c.vocab, "hwk_qwen3_prefill: token %d at %u out of vocab %u",
              tokens[i], i, m->c.vocab);
  hipStream_t st = (hipStream_t)stream;
  HWK_TRY("hipStreamSynchronize", hipStreamSynchronize(st));
  HWK_TRY("hipMemcpy", hipMemcpy(m->hist + start, tokens, 4ull * n, hipMemcpyHostToDevice));
  for (uint32_t done = 0; done < n;) {
    const uint32_t T = n - done < m->c.max_prompt ? n - done : m->c.max_prompt;
    HWK_Q(prefill_piece(m, st, T, start + done, done + T == n));
    done += T;
  }
  m->host_pos = start + n;
  m->started = true;
  m->verify_n = 0;
  return nullptr;
}

HWK_API char *hwk_qwen3_step(hwk_qwen3 *m, void *stream) {
  HWK_CHECK(m, "hwk_qwen3_step: null model");
  HWK_CHECK(m->started, "hwk_qwen3_step: no prompt yet");
  HWK_CHECK((uint64_t)m->host_pos + 1 < m->c.max_ctx, "hwk_qwen3_step: position %u is the last of %u", m->host_pos,
            m->c.max_ctx);
  HWK_Q(step(m, (hipStream_t)stream, keeps(m, m->host_pos)));
  m->host_pos++;
  m->verify_n = 0;
  return nullptr;
}

HWK_API char *hwk_qwen3_decode(hwk_qwen3 *m, void *stream, uint32_t steps) {
  HWK_CHECK(m, "hwk_qwen3_decode: null model");
  HWK_CHECK(m->started, "hwk_qwen3_decode: no prompt yet");
  HWK_CHECK((uint64_t)m->host_pos + steps < m->c.max_ctx, "hwk_qwen3_decode: %u steps from %u pass %u", steps,
            m->host_pos, m->c.max_ctx);
  const uint32_t many = steps / kGraphSteps, one = steps % kGraphSteps;
  // each replay takes the graph of its last position's cache policy; every graph a replay needs is
  // captured before the first launch
  for (int pass = 0; pass < 2; pass++) {
    uint32_t p = m->host_pos;
    for (uint32_t i = 0; i < many + one; i++) {
      const int len = i < many ? 1 : 0;
      const uint32_t n = len ? kGraphSteps : 1;
      const int keep = keeps(m, p + n - 1) ? 1 : 0;
      if (pass == 0)
        HWK_Q(capture(m, keep, len, n));
      else
        HWK_TRY("hipGraphLaunch", hipGraphLaunch(m->exec[keep][len], (hipStream_t)stream));
      p += n;
    }
  }
  m->host_pos += steps;
  m->verify_n = 0;
  return nullptr;
}

HWK_API char *hwk_qwen3_capture(hwk_qwen3 *m) {
  HWK_CHECK(m, "hwk_qwen3_capture: null model");
  for (int keep = 0; keep < 2; keep++) {
    HWK_Q(capture(m, keep, 1, kGraphSteps));
    HWK_Q(capture(m, keep, 0, 1));
  }
  return nullptr;
}

HWK_API char *hwk_qwen3_row_bytes(hwk_qwen3 *m, size_t *bytes) {
  HWK_CHECK(m && bytes, "hwk_qwen3_row_bytes: null argument");
  *bytes = 2ull * m->c.layers * m->c.kv_heads * m->c.head_dim * 2;
  return nullptr;
}

HWK_API char *hwk_qwen3_export_rows(hwk_qwen3 *m, void *stream, uint32_t from, uint32_t to, void *dst) {
  HWK_CHECK(m, "hwk_qwen3_export_rows: null model");
  HWK_CHECK(from <= to && to <= m->c.max_ctx, "hwk_qwen3_export_rows: rows %u to %u of a cache of %u", from, to,
            m->c.max_ctx);
  if (to == from) return nullptr;
  HWK_CHECK(dst, "hwk_qwen3_export_rows: null dst");
  HWK_CHECK(hwk::aligned(dst, 16), "hwk_qwen3_export_rows: dst must be 16-byte aligned");
  hipLaunchKernelGGL(k_kv_rows<true>, dim3(to - from, 2 * m->c.layers), dim3(256), 0, (hipStream_t)stream,
                     m->cache_tab, (uint4 *)dst, from, 2 * m->c.layers, m->c.kv_heads, m->c.max_ctx);
  return hwk::launched("hwk_qwen3_export_rows");
}

HWK_API char *hwk_qwen3_import_rows(hwk_qwen3 *m, void *stream, uint32_t from, const void *src, size_t bytes) {
  HWK_CHECK(m, "hwk_qwen3_import_rows: null model");
  const size_t rb = 2ull * m->c.layers * m->c.kv_heads * m->c.head_dim * 2;
  HWK_CHECK(bytes % rb == 0, "hwk_qwen3_import_rows: %zu bytes of rows, not a multiple of %zu", bytes, rb);
  const uint64_t n = bytes / rb;
  HWK_CHECK((uint64_t)from + n <= m->c.max_ctx, "hwk_qwen3_import_rows: rows %u to %llu of a cache of %u", from,
            (unsigned long long)(from + n), m->c.max_ctx);
  if (n == 0) return nullptr;
  HWK_CHECK(src, "hwk_qwen3_import_rows: null src");
  HWK_CHECK(hwk::aligned(src, 16), "hwk_qwen3_import_rows: src must be 16-byte aligned");
  hipLaunchKernelGGL(k_kv_rows<false>, dim3((uint32_t)n, 2 * m->c.layers), dim3(256), 0, (hipStream_t)stream,
                     m->cache_tab, (uint4 *)src, from, 2 * m->c.layers, m->c.kv_heads, m->c.max_ctx);
  return hwk::launched("hwk_qwen3_import_rows");
}

HWK_API char *hwk_qwen3_position(hwk_qwen3 *m, uint32_t *pos) {
  HWK_CHECK(m && pos, "hwk_qwen3_position: null argument");
  *pos = m->host_pos;
  return nullptr;
}

HWK_API char *hwk_qwen3_rewind(hwk_qwen3 *m, void *stream, uint32_t pos, int32_t next_token) {
  HWK_CHECK(m, "hwk_qwen3_rewind: null model");
  HWK_CHECK((uint64_t)pos + 1 < m->c.max_ctx, "hwk_qwen3_rewind: position %u leaves no step in %u", pos,
            m->c.max_ctx);
  HWK_CHECK(next_token < 0 || (uint32_t)next_token < m->c.vocab, "hwk_qwen3_rewind: token %d out of vocab %u",
            next_token, m->c.vocab);
  hipLaunchKernelGGL(k_rewind, dim3(1), dim3(1), 0, (hipStream_t)stream, m->hist, m->pos, pos, next_token);
  HWK_Q(hwk::launched("hwk_qwen3_rewind"));
  m->host_pos = pos;
  m->started = true;
  m->verify_n = 0;
  return nullptr;
}

HWK_API char *hwk_qwen3_verify(hwk_qwen3 *m, void *stream, const int32_t *tokens, uint32_t n, void **logits,
                               void **argmax) {
  HWK_CHECK(m && tokens, "hwk_qwen3_verify: null argument");
  HWK_CHECK(m->started, "hwk_qwen3_verify: no prompt yet");
  HWK_CHECK(n >= 1 && n <= kMaxVerify && n <= m->c.max_prompt, "hwk_qwen3_verify: %u tokens (1..%u, at most %u)", n,
            kMaxVerify, m->c.max_prompt);
  HWK_CHECK((uint64_t)m->host_pos + n < m->c.max_ctx, "hwk_qwen3_verify: positions %u+%u leave no room in %u",
            m->host_pos, n, m->c.max_ctx);
  for (uint32_t i = 0; i < n; i++)
    HWK_CHECK(tokens[i] >= 0 && (uint32_t)tokens[i] < m->c.vocab, "hwk_qwen3_verify: token %d at %u out of vocab %u",
              tokens[i], i, m->c.vocab);
  hipStream_t st = (hipStream_t)stream;
  HWK_TRY("hipStreamSynchronize", hipStreamSynchronize(st));
  HWK_TRY("hipMemcpy", hipMemcpy(m->hist + m->host_pos, tokens, 4ull * n, hipMemcpyHostToDevice));
  m->verify_n = 0;
  HWK_Q(verify_piece(m, st, n, m->host_pos));
  m->verify_start = m->host_pos;
  m->verify_n = n;
  if (logits) *logits = m->vlogits;
  if (argmax) *argmax = m->vargmax;
  return nullptr;
}

HWK_API char *hwk_qwen3_keep(hwk_qwen3 *m, void *stream, uint32_t kept) {
  HWK_CHECK(m, "hwk_qwen3_keep: null model");
  HWK_CHECK(m->verify_n > 0, "hwk_qwen3_keep: no verify to keep rows of");
  HWK_CHECK(kept >= 1 && kept <= m->verify_n, "hwk_qwen3_keep: %u of %u rows kept", kept, m->verify_n);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_keep, dim3(1), dim3(1), 0, st, m->vargmax, kept, m->verify_start, m->hist, m->pos);
  HWK_Q(hwk::launched("hwk_qwen3_keep"));
  HWK_TRY("hipMemcpyAsync", hipMemcpyAsync(m->logits, m->vlogits + (size_t)(kept - 1) * m->c.vocab,
                                           4ull * m->c.vocab, hipMemcpyDeviceToDevice, st));
  m->host_pos = m->verify_start + kept;
  m->verify_n = 0;
  return nullptr;
}

}  // extern "C"
