// Causal attention of a prompt (prefill) on gfx950: T query rows at positions start .. start+T-1
// per head over an fp16 KV cache that already holds their keys, GQA (head j on kv head
// j/(heads/kv_heads)). This is the prompt form of the reference's per-chunk program with its
// causal mask (internal/llm/paged/paged.go:70-203 at tokens > 1, internal/llm/blocks/blocks.go:
// 516-540): every query sees the keys at or before its own position.
//
// A workgroup of four waves owns one kv head and a block of 64/G query positions (G query heads a kv
// head); each wave takes 16 positions of one query head over all of the block's keys in tiles of 32,
// in key order. The kv head is the workgroup index modulo kv_heads, so that with 8 kv heads every
// workgroup of a head runs on the same XCD and the head's K and V stay in that XCD's L2. The tiles go
// through LDS in three stages (rows padded so that every operand read is free of bank conflicts and
// addressed by one per-lane register plus constant offsets), loaded into registers a tile ahead.
// On the fp16 MFMA (v_mfma_f32_16x16x32_f16) a wave computes the scores transposed, S^T = K Q^T, so
// that a lane holds eight scores of one query: the online softmax (fp32, base 2) reduces them
// in-lane and across its four lane groups (permlane swaps), and the probabilities already sit where
// the B operand of O^T = V^T P^T wants them (the MFMA's k index is permuted to the keys the lane
// holds, consistently in A and B); V^T's operand comes from the row-major tile by LDS transpose reads
// (ds_read_b64_tr_b16). P is split into an fp16 high part and an fp16 residual, two MFMAs, so that
// P.V keeps the precision of fp32 probabilities. The scores of the next tile are issued before the
// softmax of the current one, so that their MFMAs run beside it.
#include "hwk_common.h"
#include "internal.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int KT = 32;  // keys a tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr int NST = 3;                        // LDS stages
constexpr uint32_t KROW = 272, VROW = 288;    // bytes of a K / V row in LDS (256 + padding)
constexpr uint32_t KBYTES = KT * KROW;        // a stage: K rows, then V rows
constexpr uint32_t STAGE = KBYTES + KT * VROW;
constexpr int PER = KT * 16 / 256;            // 16-byte chunks of K (and of V) a thread moves a tile

__device__ __forceinline__ half8 half8_of(u32x4 u) { return __builtin_bit_cast(half8, u); }

// LDS transpose read: in each 16-lane group, lane 4a + c receives element c of the 8-byte
// segments addressed by lanes a, a + 4, a + 8, a + 12 of the group.
typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ short4v tr_read(const lds_char *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v *)p);
}

// S key groups of four waves (S = 3: twelve waves, a CU's three waves a SIMD): group gi takes the
// tiles gi, gi + S, ... with stages of its own, so that the longest query blocks walk a third of
// their tiles in order; the other groups' (m, l, O^T) then meet the first's in LDS (the Merge rule in
// base 2). Measured on the C5 prefill (1,024 tokens): one group 36.3 µs a layer, two 28.6-29.0,
// three 27.1 (which fit the registers once a group's tiles were staged through one register set).
template <int G, int S>
__global__ __launch_bounds__(256 * S) void k_attn_prefill(const u32x4 *__restrict__ q, const u32x4 *__restrict__ kc,
                                                          const u32x4 *__restrict__ vc, void *__restrict__ out,
                                                          int mode, uint32_t T, uint32_t start, uint32_t heads,
                                                          uint32_t kvh, uint32_t cap, float scale_log2) {
  constexpr uint32_t QB = 64 / G;  // query positions a workgroup
  static_assert(S >= 1 && S <= 3, "one to three key groups");
  __shared__ __attribute__((aligned(16))) char lds_all[S * NST * STAGE];
  const int gi = threadIdx.x >> 8;  // key group
  char *lds = lds_all + gi * NST * STAGE;
  const int t = threadIdx.x & 255, lane = t & 63, wave = t >> 6;
  const int n = lane & 15, grp = lane >> 4;
  const uint32_t nqb = (T + QB - 1) / QB;
  const uint32_t h = blockIdx.x % kvh;             // consecutive workgroups go to different XCDs
  const uint32_t qb = nqb - 1 - blockIdx.x / kvh;  // the longest blocks first
  const uint32_t head = h * G + wave % G;
  const uint32_t tq0 = qb * QB + (wave / G) * 16;  // the wave's first query row
  const uint32_t tq = tq0 + n;                     // this lane's query row
  const bool qlive = tq < T;
  const uint32_t qpos = start + tq;
  const uint32_t wmax = start + min(tq0 + 15, T - 1);  // the wave's last position
  // a tile needs the causal mask from this key on (or always, when the wave has rows past T)
  const uint32_t wfull = tq0 + 16 <= T ? start + tq0 : 0;
  const uint32_t last = start + min(qb * QB + QB, T);  // keys [0, last) seen by the block
  const uint32_t tiles = (last + KT - 1) / KT;
  const u32x4 *kh = kc + (size_t)h * cap * 16, *vh = vc + (size_t)h * cap * 16;

  half8 qv[4];
#pragma unroll
  for (int s = 0; s < 4; s++)
    qv[s] = half8_of(qlive ? q[((size_t)tq * heads + head) * 16 + s * 4 + grp] : (u32x4){0u, 0u, 0u, 0u});

  // the chunks thread t moves: c = t + 256 i of a tile (key c/16, 16-byte chunk c%16)
  uint32_t gofs[PER], kst[PER], vst[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const uint32_t c = t + 256 * i, key = c / 16, ch = c % 16;
    gofs[i] = c;
    kst[i] = key * KROW + ch * 16;
    vst[i] = KBYTES + key * VROW + ch * 16;
  }
  // loads of tile `it` into r (K chunks, then V chunks); chunks past the keys [0, last) are clamped
  // to the last one (in bounds, finite, masked out of the scores), and tiles past the end reload the
  // last one, so that every load is unconditional
  const uint32_t lim = last * 16 - 1;
  auto load = [&](u32x4 *r, uint32_t it) __attribute__((always_inline)) {
    const uint32_t base = min(it, tiles - 1) * KT * 16;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const uint32_t c = min(base + gofs[i], lim);
      r[i] = kh[c];
      r[PER + i] = vh[c];
    }
  };
  // the lane's operand addresses in a stage: K rows kt*16 + n, chunks s*4 + grp; the V^T transpose
  // reads: source lane s of group g addresses key g*4 + s/4 (+16 for the second read), dims
  // d*16 + 4*(s%4) .. +3
  const uint32_t kofs = n * KROW + grp * 16;
  const uint32_t vofs = KBYTES + (grp * 4 + n / 4) * VROW + (n % 4) * 8;

  floatx4 acc[8];
#pragma unroll
  for (int d = 0; d < 8; d++) acc[d] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
  float m = -__builtin_inff(), l = 0.0f;

  // S^T of a tile (scj below): keys it*32 + kt*16 + grp*4 + r of this lane's query n (skipped, as the
  // update, for a tile wholly past the wave's queries)
  // the online softmax over tile `it`'s scores, then O^T += V^T P^T
  auto update = [&](const floatx4 *sc, uint32_t it, uint32_t stage) __attribute__((always_inline)) {
    const uint32_t key0 = it * KT;
    if (key0 > wmax) return;
    float s2[2][4], tmax = -__builtin_inff();
    if (key0 + KT - 1 >= wfull) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t key = key0 + kt * 16 + grp * 4 + r;
          s2[kt][r] = (qlive && key <= qpos) ? sc[kt][r] * scale_log2 : -__builtin_inff();
        }
    } else {  // every key of the tile is at or before every query of the wave
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) s2[kt][r] = sc[kt][r] * scale_log2;
    }
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 4; r++) tmax = fmaxf(tmax, s2[kt][r]);
    tmax = row_groups_max(tmax);
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
    psum = row_groups_sum(psum);
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
    if (__ballot(alpha != 1.0f)) {  // scaling by 1 is exact: skipped when no lane's max moved
#pragma unroll
      for (int d = 0; d < 8; d++) acc[d] *= alpha;
    }
    const lds_char *vb = (const lds_char *)lds + stage * STAGE + vofs;
#pragma unroll
    for (int d = 0; d < 8; d++) {
      const short4v a0 = tr_read(vb + d * 32);
      const short4v a1 = tr_read(vb + d * 32 + 16 * VROW);
      const half8 av = __builtin_bit_cast(half8, __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7));
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bhi, acc[d], 0, 0, 0);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, blo, acc[d], 0, 0, 0);
    }
  };

  // A group's step j's tile is in LDS stage j % 3 from the end of step j-2 on. Step j computes step
  // j+1's scores (so that their MFMAs run beside this tile's softmax), updates with step j's tile, and
  // stores step j+2's tile, loaded into ra during step j-1, into the stage step j-1 left (read for the
  // last time in step j-1), then loads step j+3's tile into ra.
  // with S groups the steps are the group's own tiles: local step j is tile j * S + gi (stage j % 3);
  // every group runs as many steps as group 0 (a step past a group's last tile loads, stores and
  // computes nothing that is used), so that all waves meet at the same barriers
  u32x4 ra[2 * PER];
  floatx4 sa[2], sb[2];
  const uint32_t steps = (tiles + S - 1) / S;
  auto T_ = [&](uint32_t j) { return j * S + gi; };
  auto ld = [&](u32x4 *r, uint32_t j) __attribute__((always_inline)) { load(r, T_(j)); };
  auto stj = [&](const u32x4 *r, uint32_t j) __attribute__((always_inline)) {
    char *st = lds + (j % NST) * STAGE;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      *(u32x4 *)(st + kst[i]) = r[i];
      *(u32x4 *)(st + vst[i]) = r[PER + i];
    }
  };
  auto scj = [&](floatx4 *sc, uint32_t j) __attribute__((always_inline)) {
    const uint32_t it = T_(j);
    if (it >= tiles || it * KT > wmax) return;
    const char *kb = lds + (j % NST) * STAGE + kofs;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      sc[kt] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; s++)
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(half8_of(*(const u32x4 *)(kb + kt * 16 * KROW + s * 64)),
                                                        qv[s], sc[kt], 0, 0, 0);
    }
  };
  auto upj = [&](const floatx4 *sc, uint32_t j) __attribute__((always_inline)) {
    if (T_(j) >= tiles) return;
    update(sc, T_(j), j % NST);
  };
  ld(ra, 0);
  stj(ra, 0);
  ld(ra, 1);
  stj(ra, 1);
  ld(ra, 2);
  __syncthreads();
  scj(sa, 0);
  for (uint32_t j = 0; j < steps; j += 2) {
    scj(sb, j + 1);
    upj(sa, j);
    stj(ra, j + 2);  // loaded in the step before; its stage left by step j-1
    ld(ra, j + 3);
    __syncthreads();
    if (j + 1 >= steps) break;
    scj(sa, j + 2);
    upj(sb, j + 1);
    stj(ra, j + 3);
    ld(ra, j + 4);
    __syncthreads();
  }
  if constexpr (S > 1) {
    // groups 1 .. S-1's states to group 0 through the stages (every tile is consumed: the last barrier
    // above follows the last update), group 0 merges: weights 2^(m - top), as the Merge rule
    float *xo = (float *)lds_all + (size_t)(wave * 64 + lane) * 34;
    constexpr size_t GX = 256 * 34;  // floats a group's states take
    if (gi > 0) {
      float *xg = xo + (gi - 1) * GX;
#pragma unroll
      for (int d = 0; d < 8; d++)
#pragma unroll
        for (int r = 0; r < 4; r++) xg[d * 4 + r] = acc[d][r];
      xg[32] = m;
      xg[33] = l;
    }
    __syncthreads();
    if (gi > 0) return;
    float mg[S], ag[S];
    mg[0] = m;
    float top = m;
#pragma unroll
    for (int g = 1; g < S; g++) {
      mg[g] = xo[(g - 1) * GX + 32];
      top = fmaxf(top, mg[g]);
    }
#pragma unroll
    for (int g = 0; g < S; g++) ag[g] = top == -__builtin_inff() ? 0.0f : exp2f(mg[g] - top);
    l = l * ag[0];
#pragma unroll
    for (int g = 1; g < S; g++) l = l + xo[(g - 1) * GX + 33] * ag[g];
#pragma unroll
    for (int d = 0; d < 8; d++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float v = acc[d][r] * ag[0];
#pragma unroll
        for (int g = 1; g < S; g++) v = v + xo[(g - 1) * GX + d * 4 + r] * ag[g];
        acc[d][r] = v;
      }
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
  const dim3 grid((tokens + QB - 1) / QB * p->kv_heads);
  // two key groups a workgroup once the longest block has a few tiles (8 waves a CU: the longest
  // blocks walk half their tiles each), three past 256 keys
  const bool two = start + tokens > 128;
  const bool three = start + tokens > 256;
  const float scale_log2 = hwk::f32_of_bits(p->scale_bits) * kLog2e;
  hipStream_t st = (hipStream_t)stream;
#define HWK_PF2(GG, SS)                                                                                             \
  hipLaunchKernelGGL((k_attn_prefill<GG, SS>), grid, dim3(256 * SS), 0, st, (const u32x4 *)q, (const u32x4 *)k, \
                     (const u32x4 *)v, out, (int)p->out_mode, tokens, start, p->heads, p->kv_heads, p->capacity, scale_log2)
#define HWK_PF(GG)                        \
  do {                                    \
    if (three)                            \
      HWK_PF2(GG, 3);                     \
    else if (two)                         \
      HWK_PF2(GG, 2);                     \
    else                                  \
      HWK_PF2(GG, 1);                     \
  } while (0)
  if (G == 1) HWK_PF(1);
  else if (G == 2) HWK_PF(2);
  else HWK_PF(4);
#undef HWK_PF
#undef HWK_PF2
  return hwk::launched("hwk_attn_prefill");
}

}  // extern "C"
