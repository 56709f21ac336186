// GQA decode attention (K4) on gfx950: one query token per head over an fp16 or int8 KV cache.
//
// The context is split over waves (split-K). A wave owns one KV head and a run of keys, and walks
// it in tiles of 16 keys with the next tile's loads in flight:
//   - scores: the G query heads of the KV head (padded to the MFMA's 16 rows) times the tile's
//     keys on the fp16 MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation); a lane loads 16 bytes
//     of one key row straight from HBM as its B operand, so no cross-lane reduction is needed;
//   - an online softmax in fp32 (base 2) per head, the running max kept wave-uniform;
//   - P.V on the vector ALUs in fp32 (P stays fp32; a lane holds 8 dims of one key), so the
//     weights are never rounded to fp16.
// The wave writes its unnormalized output, max and sum to a workspace; a merge kernel combines
// the splits with the rule of the reference's Merge (internal/llm/paged/paged.go:252-310).
#include "hwk_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

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

template <bool I8>
struct Tile {
  half8 k[4];     // B operand of the 4 MFMA k-steps: key lane%16, dims t*32 + (lane/16)*8 .. +8
  half8 v[4];     // V rows: key 4r + lane/16, dims (lane%16)*8 .. +8
  float kscale;   // int8: the scale of key lane%16
  float vscale[4];
};

// Loads tile keys [key0, key0+16) of kv head h; keys at or past `end` read as zeros.
template <bool I8>
__device__ __forceinline__ void load_tile(Tile<I8> &t, const void *__restrict__ k, const void *__restrict__ v,
                                          const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs,
                                          size_t head_base, uint32_t key0, uint32_t end, int lane) {
  const uint32_t kk = key0 + (lane & 15);
  const int grp = lane >> 4;
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const size_t row = head_base + kk;
    if constexpr (I8) {
      const uint2 z = make_uint2(0, 0);
      uint2 w = kk < end ? *(const uint2 *)((const uint8_t *)k + row * 128 + s * 32 + grp * 8) : z;
      t.k[s] = i8x8_to_half8(w);
    } else {
      const uint4 z = make_uint4(0, 0, 0, 0);
      t.k[s] = half8_of(kk < end ? load_stream((const uint4 *)((const f16 *)k + row * 128 + s * 32 + grp * 8)) : z);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t key = key0 + 4 * r + grp;
    const size_t row = head_base + key;
    if constexpr (I8) {
      uint2 w = key < end ? *(const uint2 *)((const uint8_t *)v + row * 128 + (lane & 15) * 8) : make_uint2(0, 0);
      t.v[r] = i8x8_to_half8(w);
      t.vscale[r] = key < end ? (float)__builtin_bit_cast(f16, vs[row]) : 0.0f;
    } else {
      t.v[r] = half8_of(key < end ? load_stream((const uint4 *)((const f16 *)v + row * 128 + (lane & 15) * 8))
                                  : make_uint4(0, 0, 0, 0));
    }
  }
  if constexpr (I8) t.kscale = kk < end ? (float)__builtin_bit_cast(f16, ks[head_base + kk]) : 0.0f;
}

__device__ __forceinline__ float max16(float x) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}

__device__ __forceinline__ float sum16(float x) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// One wave per (kv head, split). G query heads per kv head (G <= 4: the heads are rows 0..G-1 of
// the MFMA, held by lanes 0..15). Workspace per (kv head, split, g): o[128] unnormalized, m (natural
// log units), l.
template <int G, bool I8>
__global__ __launch_bounds__(256) void k_attn_split(const uint4 *__restrict__ q, const void *__restrict__ k,
                                                    const void *__restrict__ v, const uint16_t *__restrict__ ks,
                                                    const uint16_t *__restrict__ vs, float *__restrict__ ws_o,
                                                    float *__restrict__ ws_m, float *__restrict__ ws_l,
                                                    uint32_t kv_heads, uint32_t len, uint32_t cap, uint32_t split,
                                                    uint32_t nsplit, float scale_log2) {
  const int lane = threadIdx.x & 63;
  const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= kv_heads * nsplit) return;
  const uint32_t h = wid / nsplit, sp = wid % nsplit;
  const uint32_t begin = sp * split;
  const uint32_t end = begin + split < len ? begin + split : len;
  const size_t head_base = (size_t)h * cap;

  // A operand: query head lane%16 (zero past G), dims t*32 + (lane/16)*8 .. +8
  half8 qa[4];
  {
    const int g = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int s = 0; s < 4; s++)
      qa[s] = half8_of(g < G ? q[((size_t)(h * G + g) * 128 + s * 32 + grp * 8) / 8] : make_uint4(0, 0, 0, 0));
  }
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[g][d] = 0.0f;
  float m[G], l[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -__builtin_inff();
    l[g] = 0.0f;
  }

  Tile<I8> cur, nxt;
  if (begin < end) load_tile<I8>(cur, k, v, ks, vs, head_base, begin, end, lane);
  for (uint32_t key0 = begin; key0 < end; key0 += 16) {
    if (key0 + 16 < end) load_tile<I8>(nxt, k, v, ks, vs, head_base, key0 + 16, end, lane);
    floatx4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; s++) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], cur.k[s], sc, 0, 0, 0);
    const bool valid = key0 + (lane & 15) < end;
    float p[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      float s2 = sc[g] * scale_log2;
      if constexpr (I8) s2 *= cur.kscale;
      s2 = valid ? s2 : -__builtin_inff();
      // the tile's largest score, wave-uniform (lanes 0..15 hold the real head rows)
      const float mt = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(max16(s2))));
      const float mnew = fmaxf(m[g], mt);
      float alpha = 1.0f;
      if (mnew == -__builtin_inff()) {
        p[g] = 0.0f;
      } else {
        alpha = exp2f(m[g] - mnew);
        p[g] = exp2f(s2 - mnew);
      }
      const float lt = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__float_as_uint(sum16(lane < 16 ? p[g] : 0.0f))));
      l[g] = l[g] * alpha + lt;
      m[g] = mnew;
      if (alpha != 1.0f) {
#pragma unroll
        for (int d = 0; d < 8; d++) acc[g][d] *= alpha;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int src = 4 * r + (lane >> 4);
#pragma unroll
      for (int g = 0; g < G; g++) {
        float pv = __shfl(p[g], src, 64);
        if constexpr (I8) pv *= cur.vscale[r];
#pragma unroll
        for (int d = 0; d < 8; d++) acc[g][d] = fmaf(pv, (float)cur.v[r][d], acc[g][d]);
      }
    }
    cur = nxt;
  }
  // sum the four key slots of the wave (lanes lane%16 + 16j hold the same dims)
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int d = 0; d < 8; d++) {
      float a = acc[g][d];
      a += __shfl_xor(a, 16, 64);
      a += __shfl_xor(a, 32, 64);
      acc[g][d] = a;
    }
  const size_t base = ((size_t)h * nsplit + sp) * G;
  if (lane < 16) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      float4 *dst = (float4 *)(ws_o + (base + g) * 128 + lane * 8);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      ws_m[base + g] = m[g] * kLn2;  // natural log units
      ws_l[base + g] = l[g];
    }
  }
}

// Merge of chunks per row (one block of `dim` threads a row): top = the largest m among chunks
// with l > 0; a chunk weighs exp(m - top), times l when its o is normalized (the reference's
// Merge); the sum of weights is over l. INTERNAL reads the split workspace of k_attn_split (row
// = query head, chunk c of kv head row/G at ((row/G)*nsplit + c)*G + row%G).
template <bool INTERNAL>
__global__ void k_attn_merge(const float *__restrict__ o, const float *__restrict__ m, const float *__restrict__ l,
                             void *__restrict__ out, uint32_t chunks, uint32_t rows, uint32_t dim, uint32_t G,
                             int mode) {
  const uint32_t row = blockIdx.x, t = threadIdx.x;
  size_t base, stride;
  if (INTERNAL) {
    base = (size_t)(row / G) * chunks * G + row % G;
    stride = G;
  } else {
    base = row;
    stride = rows;
  }
  float top = -__builtin_inff();
  for (uint32_t c = 0; c < chunks; c++) {
    const size_t i = base + c * stride;
    if (l[i] > 0.0f) top = fmaxf(top, m[i]);
  }
  float num = 0.0f, den = 0.0f;
  if (top != -__builtin_inff()) {
    for (uint32_t c = 0; c < chunks; c++) {
      const size_t i = base + c * stride;
      const float lc = l[i];
      if (!(lc > 0.0f)) continue;
      const float w = expf(m[i] - top);
      if (INTERNAL) {
        den += w * lc;
        if (t < dim) num += w * o[i * dim + t];
      } else {
        den += w * lc;
        if (t < dim) num += (w * lc) * o[i * dim + t];
      }
    }
  }
  if (t < dim) store_out(out, (size_t)row * dim + t, den > 0.0f ? num / den : 0.0f, mode);
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

uint32_t pick_split(const hwk_attn_params *p) {
  if (p->split) return p->split;
  // about 2048 waves over the device; at least one 16-key tile a wave
  uint64_t keys = (uint64_t)p->len * p->kv_heads;
  uint64_t s = (keys + 2047) / 2048;
  s = (s + 15) / 16 * 16;
  if (s < 16) s = 16;
  return (uint32_t)s;
}

}  // namespace

extern "C" {

HWK_API size_t hwk_attn_workspace_bytes(const hwk_attn_params *p) {
  if (!p || p->kv_heads == 0 || p->heads % p->kv_heads) return 0;
  const uint32_t split = pick_split(p);
  const uint64_t nsplit = p->len ? (p->len + split - 1) / split : 1;
  const uint64_t slots = (uint64_t)p->heads * nsplit;  // kv_heads * nsplit * G
  return (size_t)(slots * (p->head_dim + 2) * sizeof(float)) + 256;
}

HWK_API char *hwk_attn_decode(void *stream, const void *q, const void *k, const void *v, const void *k_scale,
                              const void *v_scale, void *out, void *workspace, size_t workspace_bytes,
                              const hwk_attn_params *p) {
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
  HWK_CHECK(p->split % 16 == 0, "hwk_attn_decode: split %u is not a multiple of 16", p->split);
  HWK_CHECK(hwk::aligned(q, 16) && hwk::aligned(workspace, 16), "hwk_attn_decode: q and workspace 16-byte aligned");
  HWK_CHECK(p->kv_int8 ? (hwk::aligned(k, 8) && hwk::aligned(v, 8)) : (hwk::aligned(k, 16) && hwk::aligned(v, 16)),
            "hwk_attn_decode: k, v misaligned");
  const size_t need = hwk_attn_workspace_bytes(p);
  HWK_CHECK(workspace_bytes >= need, "hwk_attn_decode: workspace %zu bytes, %zu needed", workspace_bytes, need);
  const uint32_t split = pick_split(p);
  const uint32_t nsplit = p->len ? (p->len + split - 1) / split : 1;
  const uint64_t slots = (uint64_t)p->heads * nsplit;
  float *ws_o = (float *)workspace;
  float *ws_m = ws_o + slots * 128;
  float *ws_l = ws_m + slots;
  const float scale_log2 = hwk::f32_of_bits(p->scale_bits) * kLog2e;
  const uint32_t waves = p->kv_heads * nsplit;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((waves + 3) / 4), block(256);
  const uint16_t *ks = (const uint16_t *)k_scale, *vs = (const uint16_t *)v_scale;
#define HWK_ATTN_LAUNCH(GG)                                                                                       \
  if (p->kv_int8)                                                                                                 \
    hipLaunchKernelGGL((k_attn_split<GG, true>), grid, block, 0, st, (const uint4 *)q, k, v, ks, vs, ws_o, ws_m, \
                       ws_l, p->kv_heads, p->len, p->capacity, split, nsplit, scale_log2);                       \
  else                                                                                                            \
    hipLaunchKernelGGL((k_attn_split<GG, false>), grid, block, 0, st, (const uint4 *)q, k, v, ks, vs, ws_o, ws_m, \
                       ws_l, p->kv_heads, p->len, p->capacity, split, nsplit, scale_log2);
  if (G == 1) {
    HWK_ATTN_LAUNCH(1)
  } else if (G == 2) {
    HWK_ATTN_LAUNCH(2)
  } else {
    HWK_ATTN_LAUNCH(4)
  }
#undef HWK_ATTN_LAUNCH
  if (char *err = hwk::launched("hwk_attn_decode (split)")) return err;
  hipLaunchKernelGGL((k_attn_merge<true>), dim3(p->heads), dim3(128), 0, st, ws_o, ws_m, ws_l, out, nsplit, p->heads,
                     128u, G, (int)p->out_mode);
  return hwk::launched("hwk_attn_decode (merge)");
}

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
  HWK_CHECK(out_mode == HWK_OUT_F32 || out_mode == HWK_OUT_F16, "hwk_attn_merge: out_mode %d", out_mode);
  if (rows == 0) return nullptr;
  const uint32_t threads = (dim + 63) / 64 * 64;
  hipLaunchKernelGGL((k_attn_merge<false>), dim3(rows), dim3(threads), 0, (hipStream_t)stream, (const float *)o,
                     (const float *)m, (const float *)l, out, chunks, rows, dim, 1u, out_mode);
  return hwk::launched("hwk_attn_merge");
}

}  // extern "C"
