// Causal attention of a prompt (prefill) on gfx950: T query rows at positions start .. start+T-1
// per head over an fp16 KV cache that already holds their keys, GQA (head j on kv head
// j/(heads/kv_heads)). This is the prompt form of the reference's per-chunk program with its
// causal mask (internal/llm/paged/paged.go:70-203 at tokens > 1, internal/llm/blocks/blocks.go:
// 516-540): every query sees the keys at or before its own position.
//
// A workgroup owns one kv head and a block of 64/G query positions; each of its four waves takes
// 16 positions of one query head. Key tiles of 32 go through LDS once for all four waves (K row
// major, V transposed). On the fp16 MFMA (v_mfma_f32_16x16x32_f16) a wave computes the scores
// transposed, S^T = K Q^T, so that a lane holds eight scores of one query: the online softmax
// (fp32, base 2) reduces them in-lane and across its four lane groups, and the probabilities
// already sit where the B operand of O^T = V^T P^T wants them (the MFMA's k index is permuted to
// the keys the lane holds, consistently in A and B). P is split into an fp16 high part and an
// fp16 residual, two MFMAs, so that P.V keeps the precision of fp32 probabilities.
#include "hwk_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int KT = 32;           // keys a tile
constexpr int KS = 128 + 8;      // K row stride in LDS (halves)
constexpr int VS = KT + 8;       // transposed V row stride in LDS (halves)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ half8 half8_of(uint4 u) { return __builtin_bit_cast(half8, u); }

template <int G>
__global__ __launch_bounds__(256) void k_attn_prefill(const f16 *__restrict__ q, const f16 *__restrict__ kc,
                                                      const f16 *__restrict__ vc, void *__restrict__ out, int mode,
                                                      uint32_t T, uint32_t start, uint32_t heads, uint32_t cap,
                                                      float scale_log2) {
  constexpr uint32_t QB = 64 / G;  // query positions a workgroup
  __shared__ __attribute__((aligned(16))) f16 Ks[KT][KS];
  __shared__ __attribute__((aligned(16))) f16 Vt[128][VS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n = lane & 15, grp = lane >> 4;
  const uint32_t nqb = (T + QB - 1) / QB;
  const uint32_t qb = nqb - 1 - blockIdx.x;  // the longest blocks first
  const uint32_t h = blockIdx.y;
  const uint32_t head = h * G + wave % G;
  const uint32_t tq = qb * QB + (wave / G) * 16 + n;  // this lane's query row
  const bool qlive = tq < T;
  const uint32_t qpos = start + tq;
  const uint32_t last = start + (qb * QB + QB < T ? qb * QB + QB : T);  // keys [0, last) seen by the block
  const size_t head_base = (size_t)h * cap;

  half8 qv[4];
#pragma unroll
  for (int s = 0; s < 4; s++)
    qv[s] = half8_of(qlive ? *(const uint4 *)(q + ((size_t)tq * heads + head) * 128 + s * 32 + grp * 8)
                           : make_uint4(0, 0, 0, 0));
  floatx4 acc[8];
#pragma unroll
  for (int d = 0; d < 8; d++) acc[d] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
  float m = -__builtin_inff(), l = 0.0f;

  // the tile's global loads: thread t takes chunks t and t+256 (key c/16, dims (c%16)*8 .. +8)
  uint4 kr[2], vr[2];
  auto load = [&](uint32_t key0) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t c = t + 256 * i, key = key0 + c / 16, d8 = (c % 16) * 8;
      const bool ok = key < last;
      kr[i] = ok ? *(const uint4 *)(kc + (head_base + key) * 128 + d8) : make_uint4(0, 0, 0, 0);
      vr[i] = ok ? *(const uint4 *)(vc + (head_base + key) * 128 + d8) : make_uint4(0, 0, 0, 0);
    }
  };
  const uint32_t tiles = (last + KT - 1) / KT;
  load(0);
  for (uint32_t ti = 0; ti < tiles; ti++) {
    const uint32_t key0 = ti * KT;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t c = t + 256 * i, key = c / 16, d8 = (c % 16) * 8;
      *(uint4 *)&Ks[key][d8] = kr[i];
      const half8 vv = half8_of(vr[i]);
#pragma unroll
      for (int j = 0; j < 8; j++) Vt[d8 + j][key] = vv[j];
    }
    __syncthreads();
    if (ti + 1 < tiles) load(key0 + KT);
    // S^T: keys kt*16 + grp*4 + r of this lane's query n
    floatx4 sc[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      sc[kt] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; s++)
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8 *)&Ks[kt * 16 + n][s * 32 + grp * 8], qv[s],
                                                        sc[kt], 0, 0, 0);
    }
    float s2[2][4], tmax = -__builtin_inff();
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t key = key0 + kt * 16 + grp * 4 + r;
        s2[kt][r] = (qlive && key <= qpos) ? sc[kt][r] * scale_log2 : -__builtin_inff();
        tmax = fmaxf(tmax, s2[kt][r]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(m, tmax);
    float p[2][4], psum = 0.0f, alpha = 1.0f;
    if (mnew == -__builtin_inff()) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) p[kt][r] = 0.0f;
    } else {
      alpha = exp2f(m - mnew);
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          p[kt][r] = exp2f(s2[kt][r] - mnew);
          psum += p[kt][r];
        }
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l = l * alpha + psum;
    m = mnew;
    half8 bhi, blo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float pv = p[i / 4][i % 4];
      const f16 hi = (f16)pv;
      bhi[i] = hi;
      blo[i] = (f16)(pv - (float)hi);
    }
#pragma unroll
    for (int d = 0; d < 8; d++) {
      acc[d] *= alpha;
      const uint2 a0 = *(const uint2 *)&Vt[d * 16 + n][grp * 4];
      const uint2 a1 = *(const uint2 *)&Vt[d * 16 + n][16 + grp * 4];
      const half8 av = half8_of(make_uint4(a0.x, a0.y, a1.x, a1.y));
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bhi, acc[d], 0, 0, 0);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, blo, acc[d], 0, 0, 0);
    }
    __syncthreads();
  }
  if (!qlive) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const size_t o0 = ((size_t)tq * heads + head) * 128;
#pragma unroll
  for (int d = 0; d < 8; d++) {
    const uint32_t dim = d * 16 + grp * 4;
    if (mode == HWK_OUT_F16) {
      half4 o;
#pragma unroll
      for (int r = 0; r < 4; r++) o[r] = (f16)f32_value(acc[d][r] * inv);
      *(half4 *)((f16 *)out + o0 + dim) = o;
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) ((float *)out)[o0 + dim + r] = acc[d][r] * inv;
    }
  }
}

}  // namespace

extern "C" {

HWK_API char *hwk_attn_prefill(void *stream, const void *q, const void *k, const void *v, void *out, uint32_t tokens,
                               uint32_t start, const hwk_attn_params *p) {
  HWK_CHECK(p, "hwk_attn_prefill: null params");
  HWK_CHECK(q && k && v && out, "hwk_attn_prefill: null pointer");
  HWK_CHECK(p->head_dim == 128, "hwk_attn_prefill: head_dim %u (128 only)", p->head_dim);
  HWK_CHECK(!p->kv_int8, "hwk_attn_prefill: fp16 caches only");
  HWK_CHECK(p->kv_heads > 0 && p->heads % p->kv_heads == 0, "hwk_attn_prefill: %u heads over %u kv heads", p->heads,
            p->kv_heads);
  const uint32_t G = p->heads / p->kv_heads;
  HWK_CHECK(G == 1 || G == 2 || G == 4, "hwk_attn_prefill: %u query heads a kv head (1, 2 or 4)", G);
  HWK_CHECK((uint64_t)start + tokens <= p->capacity, "hwk_attn_prefill: positions %u+%u past capacity %u", start,
            tokens, p->capacity);
  HWK_CHECK(p->len == start + tokens, "hwk_attn_prefill: len %u is not start + tokens = %u", p->len, start + tokens);
  HWK_CHECK(p->out_mode == HWK_OUT_F32 || p->out_mode == HWK_OUT_F16, "hwk_attn_prefill: out_mode %u", p->out_mode);
  HWK_CHECK(hwk::aligned(q, 16) && hwk::aligned(k, 16) && hwk::aligned(v, 16) && hwk::aligned(out, 8),
            "hwk_attn_prefill: q, k, v 16-byte and out 8-byte aligned");
  if (tokens == 0) return nullptr;
  const uint32_t QB = 64 / G;
  const dim3 grid((tokens + QB - 1) / QB, p->kv_heads);
  const float scale_log2 = hwk::f32_of_bits(p->scale_bits) * kLog2e;
  hipStream_t st = (hipStream_t)stream;
#define HWK_PF(GG)                                                                                                 \
  hipLaunchKernelGGL((k_attn_prefill<GG>), grid, dim3(256), 0, st, (const f16 *)q, (const f16 *)k, (const f16 *)v, \
                     out, (int)p->out_mode, tokens, start, p->heads, p->capacity, scale_log2)
  if (G == 1) HWK_PF(1);
  else if (G == 2) HWK_PF(2);
  else HWK_PF(4);
#undef HWK_PF
  return hwk::launched("hwk_attn_prefill");
}

}  // extern "C"
