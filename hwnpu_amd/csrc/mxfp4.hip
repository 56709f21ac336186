// MXFP4 weights on gfx950: dequantization, the batch-1 GEMV (K1) and the encoder.
//
// K1 streams each weight row once with 128-bit loads (a lane takes a 32-value block: 16 code
// bytes and its scale byte), turns codes into fp16 pairs in registers with the hardware fp4
// conversion (exact at scale 1), multiplies them against x in fp16 pairs with fp32 accumulation
// (v_dot2), applies the block's power-of-two scale to the block's fp32 sum (exact), and sums the
// lanes of a row with cross-lane shuffles. x stays in registers for all of a wave's rows.
#include "hwk_common.h"
#include "internal.h"
#include "mxfp4_gemv.h"
#include "synth.h"

namespace {

// e2m1's values by their 4 bits; code 8 is -0 (reference internal/mxfp4/mxfp4.go:17)
__constant__ float kE2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

__global__ void k_mxfp4_dequant_f16(const uint8_t *__restrict__ w, const uint8_t *__restrict__ e,
                                    uint32_t *__restrict__ out, uint64_t nbytes) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nbytes) return;
  uint8_t by = w[i];
  float s = e8m0_scale(e[i >> 4]);
  h2 v;
  v.x = (f16)(kE2M1[by & 15] * s);
  v.y = (f16)(kE2M1[by >> 4] * s);
  out[i] = __builtin_bit_cast(uint32_t, v);
}

// LPR lanes share a row (RS = 64/LPR rows side by side in a wave), a lane takes BPL blocks of a
// pass, and a wave runs RPW such row sets. Passes cover nb blocks LPR*BPL at a time; with one
// pass (the configurations of the model) x is loaded into registers once for all the rows.
template <int LPR, int BPL, int RPW>
__global__ __launch_bounds__(256) void k_mxfp4_gemv(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                    const uint4 *__restrict__ x, void *__restrict__ y,
                                                    uint32_t n, uint32_t nb, int mode) {
  constexpr int RS = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int l = lane % LPR, sub = lane / LPR;
  const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t row0 = wave * (RPW * RS) + sub;
  float acc[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) acc[i] = 0.0f;

  for (uint32_t base = 0; base < nb; base += LPR * BPL) {
    uint4 c[RPW][BPL];
    uint32_t s[RPW][BPL];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
#pragma unroll
      for (int j = 0; j < BPL; j++) {
        const uint32_t r = row0 + i * RS, b = base + j * LPR + l;
        if (r < n && b < nb) {
          const size_t blk = (size_t)r * nb + b;
          c[i][j] = load_stream(&w[blk]);
          s[i][j] = e[blk];
        } else {
          c[i][j] = make_uint4(0, 0, 0, 0);
          s[i][j] = 0;
        }
      }
    }
    uint4 xr[BPL][4];
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const uint32_t b = base + j * LPR + l;
#pragma unroll
      for (int q = 0; q < 4; q++) xr[j][q] = b < nb ? x[(size_t)b * 4 + q] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
#pragma unroll
      for (int j = 0; j < BPL; j++) {
        float d0 = 0.0f, d1 = 0.0f;
        const uint32_t cw[4] = {c[i][j].x, c[i][j].y, c[i][j].z, c[i][j].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<0>(cw[q]), h2_of_bits(xr[j][q].x), d0, false);
          d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<1>(cw[q]), h2_of_bits(xr[j][q].y), d1, false);
          d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<2>(cw[q]), h2_of_bits(xr[j][q].z), d0, false);
          d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<3>(cw[q]), h2_of_bits(xr[j][q].w), d1, false);
        }
        acc[i] += (d0 + d1) * e8m0_scale(s[i][j]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const float v = group_sum<LPR>(acc[i]);
    const uint32_t r = row0 + i * RS;
    if (l == 0 && r < n) store_out(y, r, v, mode);
  }
}

// One row set of a single-pass layout (nb <= LPR*BPL): the codes and scales of RPW rows.
template <int BPL, int RPW>
struct RowSet {
  uint4 c[RPW][BPL];
  uint32_t s[RPW][BPL];
};

template <int LPR, int BPL, int RPW>
__device__ __forceinline__ void load_rowset(RowSet<BPL, RPW> &rs, const uint4 *__restrict__ w,
                                            const uint8_t *__restrict__ e, uint32_t row0, uint32_t n,
                                            uint32_t nb, int l) {
  // Every load is issued, rows past n and blocks past nb reading the last row / block instead
  // (callers drop those rows and zero those blocks' terms): a predicated load would make the
  // compiler wait for it before issuing the next one.
  constexpr int RS = 64 / LPR;
#pragma unroll
  for (int i = 0; i < RPW; i++) {
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const uint32_t r = min(row0 + i * RS, n - 1), b = min((uint32_t)(j * LPR + l), nb - 1);
      const size_t blk = (size_t)r * nb + b;
      rs.c[i][j] = load_stream(&w[blk]);
      rs.s[i][j] = e[blk];
    }
  }
}

// A block's term of a row's dot product: its fp32 sum times the block scale; zero for a lane's
// block past the row's end (its codes and x are copies of the last block's).
__device__ __forceinline__ float block_term(float d0, float d1, uint32_t s, bool in_row) {
  return in_row ? (d0 + d1) * e8m0_scale(s) : 0.0f;
}

// The rows' old y values of an ADD-mode call (a non-ADD call reads x there instead, never used):
// loaded before the weights so that the sum at the end waits on no load.
template <int RPW>
struct YOld {
  float v[RPW];
};
template <int RPW, int RS>
__device__ __forceinline__ void y_prefetch(bool add, const void *y, const uint4 *x, uint32_t r0, uint32_t n,
                                           YOld<RPW> &yo) {
#pragma unroll
  for (int i = 0; i < RPW; i++)
    yo.v[i] = add ? ((const float *)y)[min(r0 + i * RS, n - 1)] : ((const float *)x)[i & 1];
}

// The single-pass GEMV over a grid sized to the device: a wave loads x once, then walks row sets
// wave_count apart, issuing the next set's loads before it computes the current one, so that
// every lane keeps 2*RPW*BPL 16-byte loads in flight while the grid streams the matrix.
template <int LPR, int BPL, int RPW>
__global__ __launch_bounds__(256) void k_mxfp4_gemv_stream(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                           const uint4 *__restrict__ x, void *__restrict__ y,
                                                           uint32_t n, uint32_t nb, int mode) {
  constexpr int RS = 64 / LPR;
  constexpr uint32_t ROWS = RPW * RS;  // rows of a row set
  const int lane = threadIdx.x & 63;
  const int l = lane % LPR, sub = lane / LPR;
  const uint32_t waves = gridDim.x * 4;
  uint32_t set = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t sets = (n + ROWS - 1) / ROWS;
  if (set >= sets) return;
  const bool add = mode == HWK_OUT_ADD_F32;
  YOld<RPW> yo, yn;
  y_prefetch<RPW, RS>(add, y, x, set * ROWS + sub, n, yo);
  RowSet<BPL, RPW> cur, nxt;
  load_rowset<LPR, BPL, RPW>(cur, w, e, set * ROWS + sub, n, nb, l);
  uint4 xr[BPL][4];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const uint32_t b = min((uint32_t)(j * LPR + l), nb - 1);
#pragma unroll
    for (int q = 0; q < 4; q++) xr[j][q] = x[(size_t)b * 4 + q];
  }
  for (;;) {
    const uint32_t next = set + waves;
    if (next < sets) {
      y_prefetch<RPW, RS>(add, y, x, next * ROWS + sub, n, yn);
      load_rowset<LPR, BPL, RPW>(nxt, w, e, next * ROWS + sub, n, nb, l);
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < BPL; j++) {
        float d0 = 0.0f, d1 = 0.0f;
        const uint32_t cw[4] = {cur.c[i][j].x, cur.c[i][j].y, cur.c[i][j].z, cur.c[i][j].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<0>(cw[q]), h2_of_bits(xr[j][q].x), d0, false);
          d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<1>(cw[q]), h2_of_bits(xr[j][q].y), d1, false);
          d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<2>(cw[q]), h2_of_bits(xr[j][q].z), d0, false);
          d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<3>(cw[q]), h2_of_bits(xr[j][q].w), d1, false);
        }
        acc += block_term(d0, d1, cur.s[i][j], (uint32_t)(j * LPR + l) < nb);
      }
      const float v = group_sum<LPR>(acc);
      const uint32_t r = set * ROWS + sub + i * RS;
      if (l == 0 && r < n) {
        if (add)
          ((float *)y)[r] = yo.v[i] + v;
        else
          store_out(y, r, v, mode);
      }
    }
    if (next >= sets) break;
    set = next;
    cur = nxt;
    yo = yn;
  }
}

// Sum of a float64 over the wave.
// Where the decode-step GEMV's x comes from.
enum XMode { X_F16 = 0, X_NORM = 1, X_MERGE = 2 };

struct XIn {
  const uint4 *x16;  // X_F16: x itself
  const float *h;    // X_NORM: the fp32 residual and the norm weights
  const float *nw;
  double eps;
  const float *ws;   // X_MERGE: attn_step's partials, o (slots, 128) | m (slots) | l (slots)
  uint32_t G, nchunk;  // query heads a kv head; chunks a kv head
};

// Chunks of attention partials the X_MERGE prologue loads at once when a thread merges more than 4
// values of x (more are loaded a chunk at a time); a thread of 4 values loads every chunk's at once.
constexpr int kMergeBatch = 8;
// The most chunks X_MERGE takes (LDS holds their m and l for every query head).
constexpr uint32_t kMergeMaxChunks = 16;

// The decode-step GEMV (64 lanes a row, BPL blocks a lane, nb <= 64*BPL): K1's shape (one row set a
// wave, the grid as large as the matrix, DPP reduction into lane 63) with x made by the workgroup: its
// inputs are loaded first, then the wave's weights, and while those are in flight x goes to LDS,
// copied (X_F16) or made from the fp32 residual h by RMSNorm (X_NORM: every workgroup sums h^2 itself,
// which hides behind its weight loads). SWIGLU: a wave's rows come in (gate, up) pairs and the output
// is fp16 silu(gate) * up at the pair's index; otherwise y per MODE.
//
// The arguments are flat and ordered so that everything the prologue needs lies in the first 56
// bytes, which the hardware preloads into SGPRs at wave launch (-amdgpu-kernarg-preload-count):
// xa is x (X_F16), the residual h (X_NORM) or the partials (X_MERGE); xb the norm weights (X_NORM);
// gn = G | nchunk << 16 (X_MERGE); eps (X_NORM), past them, is loaded when first used.
template <int BPL, int RPW, int XM, bool SWIGLU, int WPB, int MODE, int MBC>
__global__ __launch_bounds__(64 * WPB) void k_mxfp4_gemv_x(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                           const void *__restrict__ xa, void *__restrict__ y,
                                                           uint32_t n, uint32_t nb, const float *__restrict__ xb,
                                                           uint32_t gn, double eps) {
  static_assert(!SWIGLU || RPW % 2 == 0, "SwiGLU pairs rows");
  constexpr int NT = 64 * WPB;
  constexpr int PER = (64 * BPL * 32 + NT - 1) / NT;  // x values a thread makes (X_NORM)
  constexpr int XC = 64 * BPL * 4;                    // 16-byte chunks of x LDS holds
  constexpr int XD = (64 * BPL * 16 + NT - 1) / NT;   // dwords of x a thread copies (X_F16)
  constexpr int M4 = (64 * BPL * 32 / 4 + NT - 1) / NT;  // groups of 4 x values a thread merges (X_MERGE)
  // chunks' o a thread loads up front: MBC, the launch's chunk count rounded up to 4, for one group a
  // thread (a chunk past it would be a duplicate load of weight 0: 1,494 -> 1,516 tokens/s on the C5
  // decode step against loading 16), else kMergeBatch
  constexpr int MB = M4 <= 1 ? MBC : kMergeBatch;
  constexpr bool add = MODE == HWK_OUT_ADD_F32;
  __shared__ uint4 xs[NT * XD / 4];  // x (at least XC chunks)
  __shared__ double red[WPB];
  constexpr int MS = XM == X_MERGE ? 64 * BPL / 4 * kMergeMaxChunks : 1;  // (head, chunk) slots (X_MERGE)
  constexpr int MPER = (MS + NT - 1) / NT;                                 // slots a thread takes
  static_assert(kMergeMaxChunks == 16 && NT % 16 == 0, "a head's chunks are one 16-lane DPP group");
  __shared__ __align__(16) float ml[MS + 64];  // l of (head, chunk); past MS one spare slot a lane
  __shared__ __align__(16) float mw[MS + 64];  // weight of (head, chunk)
  kernarg_now(w, e, xa, y, n, nb, xb, gn);
  const XIn in{(const uint4 *)xa, (const float *)xa, xb, eps, (const float *)xa, gn & 0xffffu, gn >> 16};
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t k = nb * 32;
  const uint32_t r0 = (blockIdx.x * WPB + (t >> 6)) * RPW;
  // x's inputs first, then the old y of ADD mode, then the weights (loads complete in issue order
  // for the wait counter, so x is made while the weights are in flight)
  float hv[PER], wv[PER];
  uint32_t xv[XD];
  float4 ov[XM == X_MERGE ? M4 : 1][XM == X_MERGE ? MB : 1];
  float mv[XM == X_MERGE ? MPER : 1], lv[XM == X_MERGE ? MPER : 1];
  // every chunk of the partials is read: one past the step's position has l = 0 and weighs nothing
  const uint32_t live = XM == X_MERGE ? in.nchunk : 1;
  if constexpr (XM == X_MERGE) {
    // the partials: o of this thread's x values (4 consecutive dims of one query head a group), and
    // the m and l of (head, chunk) slots
    const uint32_t heads = k / 128, slots = heads * in.nchunk;
    const float *ws_m = in.ws + (size_t)slots * 128, *ws_l = ws_m + slots;
#pragma unroll
    for (int j = 0; j < M4; j++) {
      const uint32_t e = min((uint32_t)(t + j * NT), k / 4 - 1) * 4, hq = e / 128, d = e % 128;
#pragma unroll
      for (int c = 0; c < MB; c++) {
        const uint32_t cc = min((uint32_t)c, live - 1);
        const size_t slot = ((size_t)(hq / in.G) * in.nchunk + cc) * in.G + hq % in.G;
        ov[j][c] = *(const float4 *)(in.ws + slot * 128 + d);
      }
    }
    // slot i = t + j*NT is (head i/16, chunk i%16): 16 lanes a head, so that the head's top is a
    // 16-lane DPP max in registers (a chunk past live reads chunk live - 1 and a head past the last
    // the last head's, unused); used once the weight loads are issued, with no use under a branch (a
    // load whose only use sits under a branch would be sunk into it, behind the weight loads)
#pragma unroll
    for (int j = 0; j < MPER; j++) {
      const uint32_t i = t + j * NT, hq = min(i / kMergeMaxChunks, heads - 1);
      const uint32_t cc = min(i % kMergeMaxChunks, live - 1);
      const size_t slot = ((size_t)(hq / in.G) * in.nchunk + cc) * in.G + hq % in.G;
      mv[j] = ws_m[slot];
      lv[j] = ws_l[slot];
    }
  } else if constexpr (XM == X_NORM) {
#pragma unroll
    for (int j = 0; j < PER; j++) {
      const uint32_t i = min((uint32_t)(t + j * NT), k - 1);
      hv[j] = in.h[i];
      wv[j] = in.nw[i];
    }
  } else {
    // dwords t, t + NT, ... of x (past x's end the last dword again, into slots no lane reads)
    const uint32_t *xw = (const uint32_t *)in.x16;
#pragma unroll
    for (int j = 0; j < XD; j++) xv[j] = xw[min((uint32_t)(t + j * NT), nb * 16 - 1)];
  }
  float yo[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) yo[i] = add ? ((const float *)y)[min(r0 + i, n - 1)] : 0.0f;
  issue_order();
  RowSet<BPL, RPW> cur;
  load_rowset<64, BPL, RPW>(cur, w, e, r0, n, nb, lane);
  issue_order();  // every weight load issued before the waits for x's inputs
  f16 *xh = (f16 *)xs;
  if constexpr (XM == X_NORM) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; j++)
      if (t + j * NT >= k) hv[j] = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) ss += (double)hv[j] * (double)hv[j];
    ss = wave_sum_f64_to_63(ss);
    if (lane == 63) red[t >> 6] = ss;
    __syncthreads();
    // r by wave 0 alone (a float64 chain issued by one wave, not by every wave of the workgroup),
    // handed over in LDS; ss / k by an exponent shift when k is a power of two (the same value)
    __shared__ float rs;
    if (t < 64) {
      ss = 0.0;
#pragma unroll
      for (int i = 0; i < WPB; i++) ss += red[i];
      double mean;
      if ((k & (k - 1)) == 0)
        mean = __builtin_ldexp(ss, -__builtin_ctz(k));
      else
        mean = ss / (double)k;
      if (t == 0) rs = (float)(1.0 / sqrt(mean + in.eps));
    }
    __syncthreads();
    const float r = rs;
#pragma unroll
    for (int j = 0; j < PER; j++)
      if (t + j * NT < k) xh[t + j * NT] = (f16)f32_value((hv[j] * r) * wv[j]);
  } else if constexpr (XM == X_MERGE) {
    // the reference's Merge rule per query head: top = the largest m among chunks with l > 0, a chunk
    // weighs exp(m - top), x = fp16(sum(w * o) / sum(w * l)). Each slot's weight, and its l, into LDS
    // (a chunk past live, of l <= 0 or of a head with none weighs 0; a thread past the slots writes
    // its spare one)
    const uint32_t heads = k / 128;
#pragma unroll
    for (int j = 0; j < MPER; j++) {
      const uint32_t i = t + j * NT;
      const bool ok = (i < heads * kMergeMaxChunks) & (i % kMergeMaxChunks < live) & (lv[j] > 0.0f);
      const float top = group_max_dpp<kMergeMaxChunks>(ok ? mv[j] : -__builtin_inff());
      const uint32_t at = i < heads * kMergeMaxChunks ? i : MS + lane;
      mw[at] = ok & (top != -__builtin_inff()) ? expf(mv[j] - top) : 0.0f;
      ml[at] = lv[j];
    }
    __syncthreads();
    typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int j = 0; j < M4; j++) {
      const uint32_t e = (uint32_t)(t + j * NT) * 4;
      if (e >= k) continue;
      const uint32_t hq = e / 128, d = e % 128;
      const float *hw = mw + hq * kMergeMaxChunks, *hl = ml + hq * kMergeMaxChunks;
      // chunks in ascending order, the first MB with their weights and l read at once and no branch
      // (a chunk of weight 0 adds +0: its o and l, a duplicate for a chunk past live, are finite)
      f32x4 w4[MB / 4], l4[MB / 4];
#pragma unroll
      for (int q = 0; q < MB / 4; q++) {
        w4[q] = ((const f32x4 *)hw)[q];
        l4[q] = ((const f32x4 *)hl)[q];
      }
      float den = 0.0f, n0 = 0.0f, n1 = 0.0f, n2 = 0.0f, n3 = 0.0f;
#pragma unroll
      for (int c = 0; c < MB; c++) {
        const float wc = w4[c / 4][c % 4];
        const float4 o = ov[j][c];
        den += wc * l4[c / 4][c % 4];
        n0 += wc * o.x;
        n1 += wc * o.y;
        n2 += wc * o.z;
        n3 += wc * o.w;
      }
      for (uint32_t c = MB; c < live; c++) {
        const float wc = hw[c];
        if (wc > 0.0f) {
          const size_t slot = ((size_t)(hq / in.G) * in.nchunk + c) * in.G + hq % in.G;
          const float4 o = *(const float4 *)(in.ws + slot * 128 + d);
          den += wc * hl[c];
          n0 += wc * o.x;
          n1 += wc * o.y;
          n2 += wc * o.z;
          n3 += wc * o.w;
        }
      }
      const float r0 = den > 0.0f ? n0 / den : 0.0f, r1 = den > 0.0f ? n1 / den : 0.0f;
      const float r2 = den > 0.0f ? n2 / den : 0.0f, r3 = den > 0.0f ? n3 / den : 0.0f;
      xh[e] = (f16)f32_value(r0);
      xh[e + 1] = (f16)f32_value(r1);
      xh[e + 2] = (f16)f32_value(r2);
      xh[e + 3] = (f16)f32_value(r3);
    }
  } else {
    // every thread writes (a write under a branch would let the compiler sink x's load into it,
    // behind the weight loads, and wait for those too)
#pragma unroll
    for (int j = 0; j < XD; j++) ((uint32_t *)xs)[t + j * NT] = xv[j];
  }
  __syncthreads();
  uint4 xr[BPL][4];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const uint32_t b = min((uint32_t)(j * 64 + lane), nb - 1);
#pragma unroll
    for (int q = 0; q < 4; q++) xr[j][q] = xs[b * 4 + q];
  }
  float v[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const float term = mxfp4_block_dot(cur.c[i][j], xr[j]) * e8m0_scale(cur.s[i][j]);
      acc += (uint32_t)(j * 64 + lane) < nb ? term : 0.0f;
    }
    v[i] = wave_sum_to_63(acc);
  }
  if constexpr (SWIGLU) {
    // the workgroup's (gate, up) sums gathered in LDS, then wave 0 computes them a pair a lane: the
    // float64 exp is issued once for all the pairs, not by each wave with one lane active
    constexpr int NP = WPB * RPW / 2;
    static_assert(NP <= 64, "a pair a lane of wave 0");
    __shared__ float gus[2 * NP];
    if (lane == 63) {
#pragma unroll
      for (int i = 0; i < RPW; i += 2) {
        gus[2 * ((t >> 6) * (RPW / 2) + i / 2)] = v[i];
        gus[2 * ((t >> 6) * (RPW / 2) + i / 2) + 1] = v[i + 1];
      }
    }
    __syncthreads();
    const uint32_t pair = blockIdx.x * NP + t;
    if (t < NP && 2 * pair + 1 < n) {
#pragma clang fp contract(off)
      const float g = gus[2 * t], u = gus[2 * t + 1];
      ((f16 *)y)[pair] = (f16)f32_value(g / (1.0f + (float)exp(-(double)g)) * u);
    }
  } else if (lane == 63) {
    {
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        if (r0 + i >= n) continue;
        if constexpr (MODE == HWK_OUT_F16)
          ((f16 *)y)[r0 + i] = (f16)f32_value(v[i]);
        else if constexpr (add)
          ((float *)y)[r0 + i] = yo[i] + v[i];
        else
          ((float *)y)[r0 + i] = v[i];
      }
    }
  }
}

// K1r: the MXFP4 GEMV of T <= 8 vectors at once (speculative verify, a few tokens), every weight
// row read once for all of them, as the reference's mxfp4.Run serves several vectors from one read
// of a row (internal/mxfp4/matvec.go:33-160). The workgroup copies X (T, k) fp16 into LDS; its
// waves stream row sets as the batch-1 GEMV does (64 lanes a row, BPL blocks a lane), each lane
// taking its block's x of every vector from LDS. Y (T, n) per out_mode.
template <int BPL, int RPW, int TT>
__global__ __launch_bounds__(256) void k_mxfp4_gemv_rows(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                         const uint4 *__restrict__ x, void *__restrict__ y,
                                                         uint32_t n, uint32_t nb, int mode) {
  extern __shared__ uint4 xs[];  // (TT, nb * 4)
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t waves = gridDim.x * 4;
  uint32_t set = blockIdx.x * 4 + (t >> 6);
  const uint32_t sets = (n + RPW - 1) / RPW;
  const bool live = set < sets;
  // x's chunks (up to 8 a thread) loaded before the weights, the first row set's weight loads
  // issued unconditionally (a clamped set; a load under a branch is waited for where the branches
  // join), then x written to LDS (past x's end the last chunk again: the same value, into its own
  // slot) waiting on x only
  constexpr int XPT = (TT * 64 * BPL * 4 + 255) / 256, XF = XPT < 8 ? XPT : 8;
  const uint32_t xn = TT * nb * 4;
  uint4 xv[XF];
#pragma unroll
  for (int j = 0; j < XF; j++) xv[j] = x[min((uint32_t)(t + j * 256), xn - 1)];
  issue_order();
  RowSet<BPL, RPW> cur, nxt;
  load_rowset<64, BPL, RPW>(cur, w, e, min(set, sets - 1) * RPW, n, nb, lane);
  issue_order();
#pragma unroll
  for (int j = 0; j < XF; j++) xs[min((uint32_t)(t + j * 256), xn - 1)] = xv[j];
  for (uint32_t i = t + XF * 256; i < xn; i += 256) xs[i] = x[i];
  __syncthreads();
  if (!live) return;
  for (;;) {
    const uint32_t next = set + waves;
    if (next < sets) load_rowset<64, BPL, RPW>(nxt, w, e, next * RPW, n, nb, lane);
    float acc[RPW][TT];
#pragma unroll
    for (int i = 0; i < RPW; i++)
#pragma unroll
      for (int v = 0; v < TT; v++) acc[i][v] = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; j++) {
      const uint32_t b = j * 64 + lane;
      if (b >= nb) continue;
#pragma unroll
      for (int v = 0; v < TT; v++) {
        const uint4 *xv = xs + (size_t)v * nb * 4 + b * 4;
        const uint4 xr[4] = {xv[0], xv[1], xv[2], xv[3]};
#pragma unroll
        for (int i = 0; i < RPW; i++) {
          float d0 = 0.0f, d1 = 0.0f;
          const uint32_t cw[4] = {cur.c[i][j].x, cur.c[i][j].y, cur.c[i][j].z, cur.c[i][j].w};
#pragma unroll
          for (int q = 0; q < 4; q++) {
            d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<0>(cw[q]), h2_of_bits(xr[q].x), d0, false);
            d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<1>(cw[q]), h2_of_bits(xr[q].y), d1, false);
            d0 = __builtin_amdgcn_fdot2(fp4x2_to_h2<2>(cw[q]), h2_of_bits(xr[q].z), d0, false);
            d1 = __builtin_amdgcn_fdot2(fp4x2_to_h2<3>(cw[q]), h2_of_bits(xr[q].w), d1, false);
          }
          acc[i][v] += block_term(d0, d1, cur.s[i][j], true);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const uint32_t r = set * RPW + i;
#pragma unroll
      for (int v = 0; v < TT; v++) {
        const float sum = group_sum<64>(acc[i][v]);
        if (lane == 0 && r < n) store_out(y, (size_t)v * n + r, sum, mode);
      }
    }
    if (next >= sets) break;
    set = next;
    cur = nxt;
  }
}

// K1r on the matrix cores, for several vectors (T <= 8) and rows of a multiple of 16 blocks: a
// workgroup of 4 waves takes 16 rows; wave w takes blocks round*64 + w*16 .. +15. Per block one
// v_mfma_f32_16x16x32_f16 of the 16 rows' codes (A: lane (row l%16, group l/16) holds the block's
// codes group*8 .. +7 as exact fp16 e2m1 values) with the T vectors (B: lane (vector l%16, group)
// holds x[vector][block*32 + group*8 .. +7], zero past T) sums the block's 32 products per (row,
// vector); each lane's four (row, vector) sums are scaled by the rows' e8m0 block scales in fp32 and
// added in block order. All of a round's loads are issued before its first MFMA. The four waves'
// sums meet in LDS and wave 0 adds them in wave order and stores.
template <int TT>
__global__ __launch_bounds__(256) void k_mxfp4_gemv_rows_mfma(const uint32_t *__restrict__ w,
                                                              const uint8_t *__restrict__ e,
                                                              const f16 *__restrict__ x, void *__restrict__ y,
                                                              uint32_t n, uint32_t nb, int mode) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef float floatx4 __attribute__((ext_vector_type(4)));
  __shared__ floatx4 part[3][64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int c16 = lane & 15, g = lane >> 4;
  const uint32_t row0 = blockIdx.x * 16;
  const uint32_t arow = min(row0 + c16, n - 1);                    // the A row of this lane
  const uint32_t vec = min((uint32_t)c16, (uint32_t)TT - 1);      // the B vector of this lane
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};  // rows g*4 + r, vector c16
  for (uint32_t b0 = (uint32_t)wave * 16; b0 < nb; b0 += 64) {
    uint32_t cw[16];
    u32x4 xv[16], sv[4];
#pragma unroll
    for (int j = 0; j < 16; j++) cw[j] = w[((size_t)arow * nb + b0 + j) * 4 + g];
    if (c16 < TT) {  // lanes past the T vectors load nothing
#pragma unroll
      for (int j = 0; j < 16; j++) xv[j] = *(const u32x4 *)(x + (size_t)vec * nb * 32 + (b0 + j) * 32 + g * 8);
    } else {
#pragma unroll
      for (int j = 0; j < 16; j++) xv[j] = (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < 4; r++) sv[r] = *(const u32x4 *)(e + (size_t)min(row0 + g * 4 + r, n - 1) * nb + b0);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const u32x4 a = {__builtin_bit_cast(uint32_t, fp4x2_to_h2<0>(cw[j])), __builtin_bit_cast(uint32_t, fp4x2_to_h2<1>(cw[j])),
                       __builtin_bit_cast(uint32_t, fp4x2_to_h2<2>(cw[j])), __builtin_bit_cast(uint32_t, fp4x2_to_h2<3>(cw[j]))};
      const floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, xv[j]),
                                                               (floatx4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++) acc[r] += d[r] * e8m0_scale((sv[r][j / 4] >> (8 * (j % 4))) & 255u);
    }
  }
  if (wave > 0) part[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0 || c16 >= TT) return;
  acc = ((acc + part[0][lane]) + part[1][lane]) + part[2][lane];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t row = row0 + g * 4 + r;
    if (row < n) store_out(y, (size_t)c16 * n + row, acc[r], mode);
  }
}

// ---- the encoder (reference internal/mxfp4/encode.go:11-78), one thread a block, in float64
// with every product and sum rounded on its own, as the reference computes it ----

__device__ __forceinline__ uint8_t nearest_code(double x) {
#pragma clang fp contract(off)
  uint8_t sign = 0;
  if (x < 0) {
    sign = 8;
    x = -x;
  }
  // midpoints between consecutive e2m1 magnitudes; on a midpoint the even code wins
  const double mids[7] = {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0};
  uint8_t c = 7;
  for (int k = 0; k < 7; k++) {
    if (x < mids[k] || (x == mids[k] && k % 2 == 0)) {
      c = (uint8_t)k;
      break;
    }
    if (x == mids[k]) {
      c = (uint8_t)(k + 1);
      break;
    }
  }
  if (c == 0) return 0;
  return sign | c;
}

__device__ void encode_block(const float v[32], uint8_t *__restrict__ wout, uint8_t *__restrict__ eout) {
#pragma clang fp contract(off)
  float m = 0.0f;
  for (int j = 0; j < 32; j++) m = fmaxf(m, fabsf(v[j]));
  uint32_t best = 0;
  double best_err = __builtin_huge_val();
  if (m > 0.0f) {
    int ex;
    frexp((double)m, &ex);
    const int rule = ex - 1 - 2;
    for (int xx = rule - 1; xx <= rule + 1; xx++) {
      const int eb = xx + 127;
      if (eb < 1 || eb > 254) continue;
      const double s = (double)e8m0_scale((uint32_t)eb);
      double se = 0.0;
      for (int j = 0; j < 32; j++) {
        const double vv = (double)v[j];
        const double d = vv - (double)kE2M1[nearest_code(vv / s)] * s;
        se += d * d;
      }
      if (se < best_err) {
        best = (uint32_t)eb;
        best_err = se;
      }
    }
  }
  uint32_t words[4] = {0, 0, 0, 0};
  if (best != 0) {
    const double s = (double)e8m0_scale(best);
    for (int j = 0; j < 16; j++) {
      const uint32_t lo = nearest_code((double)v[2 * j] / s), hi = nearest_code((double)v[2 * j + 1] / s);
      words[j >> 2] |= (lo | hi << 4) << (8 * (j & 3));
    }
  }
  *(uint4 *)wout = make_uint4(words[0], words[1], words[2], words[3]);
  *eout = (uint8_t)best;
}

__global__ void k_mxfp4_encode(const float *__restrict__ x, uint8_t *__restrict__ w, uint8_t *__restrict__ e,
                               uint64_t nblocks) {
  uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
  const float4 *src = (const float4 *)(x + b * 32);
#pragma unroll
  for (int q = 0; q < 8; q++) {
    float4 f = src[q];
    v[4 * q] = f.x;
    v[4 * q + 1] = f.y;
    v[4 * q + 2] = f.z;
    v[4 * q + 3] = f.w;
  }
  encode_block(v, w + b * 16, e + b);
}

// Block b of a (rows, k) matrix of N(0, std) values: element i = b*32 + j of the normal stream,
// float32(z * std), then encoded. Row r of the matrix lands at row row0 + r*stride of the output
// (stride 1, row0 0: in place; stride 2: interleaved with another matrix's rows).
__global__ void k_synth_mxfp4(uint8_t *__restrict__ w, uint8_t *__restrict__ e, uint64_t nblocks, uint64_t key,
                              float stdv, uint32_t nb, uint32_t stride, uint32_t row0) {
  uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
  for (int j = 0; j < 32; j++) v[j] = (float)(hwk::normal_at(key, b * 32 + j) * (double)stdv);
  const uint64_t r = b / nb, d = ((uint64_t)row0 + r * stride) * nb + b % nb;
  encode_block(v, w + d * 16, e + d);
}

// Waves the streaming grid runs: 16 resident waves a CU times the current device's CUs (the
// fastest of 8-32 measured on C1's shape and the decode step's).
uint32_t stream_waves() {
  constexpr int kWavesPerCu = 16;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return (uint32_t)(kWavesPerCu * (cus > 0 ? cus : 256));
}

template <int LPR, int BPL, int RPW>
void launch_gemv(hipStream_t st, const void *w, const void *e, const void *x, void *y, uint32_t n, uint32_t nb,
                 int mode) {
  constexpr uint32_t rows_per_wave = RPW * (64 / LPR);
  const uint32_t sets = (n + rows_per_wave - 1) / rows_per_wave;
  if (nb <= (uint32_t)(LPR * BPL)) {
    uint32_t waves = sets < stream_waves() ? sets : stream_waves();
    hipLaunchKernelGGL((k_mxfp4_gemv_stream<LPR, BPL, RPW>), dim3((waves + 3) / 4), dim3(256), 0, st,
                       (const uint4 *)w, (const uint8_t *)e, (const uint4 *)x, y, n, nb, mode);
    return;
  }
  hipLaunchKernelGGL((k_mxfp4_gemv<LPR, BPL, RPW>), dim3((sets + 3) / 4), dim3(256), 0, st, (const uint4 *)w,
                     (const uint8_t *)e, (const uint4 *)x, y, n, nb, mode);
}

template <int LPR, int BPL>
void launch_rpw(hipStream_t st, const void *w, const void *e, const void *x, void *y, uint32_t n, uint32_t nb,
                int mode) {
  // one row set a lane group for matrices of fewer rows than half the streaming grid's waves, else 2
  if ((n + 1) / 2 < stream_waves() / 2) launch_gemv<LPR, BPL, 1>(st, w, e, x, y, n, nb, mode);
  else launch_gemv<LPR, BPL, 2>(st, w, e, x, y, n, nb, mode);
}

// K1 for rows of 33..256 blocks (64 lanes a row), one row a wave: the most waves in flight, which is
// what a single launch's read of a few MB needs (4 waves a workgroup for matrices of 4096 rows or
// more, measured fastest on C1: x's barrier then waits on 4 waves' loads, not 16; else 8 waves).
template <int BPL, int MODE>
void launch_lds_m(hipStream_t st, const void *w, const void *e, const void *x, void *y, uint32_t n, uint32_t nb) {
  if (n >= 4096) {
    hipLaunchKernelGGL((k_mxfp4_gemv_lds<4, 1, BPL, MODE>), dim3((n + 3) / 4), dim3(64 * 4), 0, st,
                       (const uint4 *)w, (const uint8_t *)e, (const uint4 *)x, y, n, nb);
  } else {
    hipLaunchKernelGGL((k_mxfp4_gemv_lds<8, 1, BPL, MODE>), dim3((n + 7) / 8), dim3(64 * 8), 0, st,
                       (const uint4 *)w, (const uint8_t *)e, (const uint4 *)x, y, n, nb);
  }
}

template <int BPL>
void launch_lds(hipStream_t st, const void *w, const void *e, const void *x, void *y, uint32_t n, uint32_t nb,
                int mode) {
  if (mode == HWK_OUT_F16) launch_lds_m<BPL, HWK_OUT_F16>(st, w, e, x, y, n, nb);
  else if (mode == HWK_OUT_ADD_F32) launch_lds_m<BPL, HWK_OUT_ADD_F32>(st, w, e, x, y, n, nb);
  else launch_lds_m<BPL, HWK_OUT_F32>(st, w, e, x, y, n, nb);
}

template <int LPR>
void launch_bpl(int bpl, hipStream_t st, const void *w, const void *e, const void *x, void *y, uint32_t n,
                uint32_t nb, int mode) {
  switch (bpl) {
    case 1: launch_rpw<LPR, 1>(st, w, e, x, y, n, nb, mode); break;
    case 2: launch_rpw<LPR, 2>(st, w, e, x, y, n, nb, mode); break;
    case 3: launch_rpw<LPR, 3>(st, w, e, x, y, n, nb, mode); break;
    default: launch_rpw<LPR, 4>(st, w, e, x, y, n, nb, mode); break;
  }
}

}  // namespace

// The lane layout for nb blocks a row: the fewest idle block slots over one pass when a pass can
// hold the row (ties to more lanes a row), else 64 lanes of 4 blocks over several passes.
static void gemv_layout(uint32_t nb, int *lpr, int *bpl) {
  int best_l = 64, best_b = 4;
  long best_waste = -1;
  const int lprs[4] = {64, 32, 16, 8};
  for (int li = 0; li < 4; li++)
    for (int b = 1; b <= 4; b++) {
      long slots = (long)lprs[li] * b;
      if (slots < (long)nb) continue;
      long waste = slots - nb;
      if (best_waste < 0 || waste < best_waste) {
        best_waste = waste;
        best_l = lprs[li];
        best_b = b;
      }
    }
  *lpr = best_l;
  *bpl = best_b;
}

extern "C" {

HWK_API char *hwk_mxfp4_dequant_f16(void *stream, const void *w, const void *e, void *out, uint32_t rows,
                                    uint32_t k) {
  HWK_CHECK(w && e && out, "hwk_mxfp4_dequant_f16: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_mxfp4_dequant_f16: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(hwk::aligned(out, 4), "hwk_mxfp4_dequant_f16: out not 4-byte aligned");
  if (rows == 0) return nullptr;
  const uint64_t nbytes = (uint64_t)rows * (k / 2);
  const uint64_t blocks = (nbytes + 255) / 256;
  hipLaunchKernelGGL(k_mxfp4_dequant_f16, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t *)w, (const uint8_t *)e, (uint32_t *)out, nbytes);
  return hwk::launched("hwk_mxfp4_dequant_f16");
}

HWK_API char *hwk_mxfp4_gemv(void *stream, const void *w, const void *e, const void *x, void *y, uint32_t n,
                             uint32_t k, int out_mode) {
  HWK_CHECK(w && e && x && y, "hwk_mxfp4_gemv: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_mxfp4_gemv: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_mxfp4_gemv: unknown out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(w, 16) && hwk::aligned(x, 16), "hwk_mxfp4_gemv: w and x must be 16-byte aligned");
  HWK_CHECK(hwk::aligned(y, out_mode == HWK_OUT_F16 ? 2 : 4), "hwk_mxfp4_gemv: y misaligned");
  if (n == 0) return nullptr;
  const uint32_t nb = k / 32;
  int lpr, bpl;
  gemv_layout(nb, &lpr, &bpl);
  hipStream_t st = (hipStream_t)stream;
  if (lpr == 64 && nb <= 256) {
    switch (bpl) {
      case 1: launch_lds<1>(st, w, e, x, y, n, nb, out_mode); break;
      case 2: launch_lds<2>(st, w, e, x, y, n, nb, out_mode); break;
      case 3: launch_lds<3>(st, w, e, x, y, n, nb, out_mode); break;
      default: launch_lds<4>(st, w, e, x, y, n, nb, out_mode); break;
    }
    return hwk::launched("hwk_mxfp4_gemv");
  }
  switch (lpr) {
    case 64: launch_bpl<64>(bpl, st, w, e, x, y, n, nb, out_mode); break;
    case 32: launch_bpl<32>(bpl, st, w, e, x, y, n, nb, out_mode); break;
    case 16: launch_bpl<16>(bpl, st, w, e, x, y, n, nb, out_mode); break;
    default: launch_bpl<8>(bpl, st, w, e, x, y, n, nb, out_mode); break;
  }
  return hwk::launched("hwk_mxfp4_gemv");
}

// The fewest vectors K1r takes to the matrix cores (fewer: T dot products a lane on the VALUs, which
// is faster up to T = 5 on C1's shape: 4.5 / 5.8 / 8.3 µs at T = 1 / 2 / 4 against 8.3-8.6 µs for the
// MFMA form, whose time barely grows with T: 9.2 µs at T = 8 against 12.6).
constexpr uint32_t kRowsMfmaMinTokens = 6;

HWK_API char *hwk_mxfp4_gemv_rows(void *stream, const void *w, const void *e, const void *x, void *y, uint32_t n,
                                  uint32_t k, uint32_t tokens, int out_mode) {
  HWK_CHECK(w && e && x && y, "hwk_mxfp4_gemv_rows: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0 && k <= 64 * 4 * 32, "hwk_mxfp4_gemv_rows: k=%u (a multiple of 32 up to 8192)", k);
  HWK_CHECK(tokens >= 1 && tokens <= 8, "hwk_mxfp4_gemv_rows: %u vectors (1..8)", tokens);
  HWK_CHECK((size_t)tokens * k * 2 <= 64 * 1024, "hwk_mxfp4_gemv_rows: %u x %u fp16 vectors exceed 64 KB", tokens, k);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "hwk_mxfp4_gemv_rows: out_mode %d", out_mode);
  HWK_CHECK(hwk::aligned(w, 16) && hwk::aligned(x, 16), "hwk_mxfp4_gemv_rows: w and x must be 16-byte aligned");
  HWK_CHECK(hwk::aligned(y, out_mode == HWK_OUT_F16 ? 2 : 4), "hwk_mxfp4_gemv_rows: y misaligned");
  if (n == 0) return nullptr;
  const uint32_t nb = k / 32;
  hipStream_t st = (hipStream_t)stream;
  if (tokens >= kRowsMfmaMinTokens && nb % 16 == 0 && hwk::aligned(e, 16)) {
#define HWK_ROWS_M(T)                                                                                          \
  hipLaunchKernelGGL((k_mxfp4_gemv_rows_mfma<T>), dim3((n + 15) / 16), dim3(256), 0, st, (const uint32_t *)w, \
                     (const uint8_t *)e, (const f16 *)x, y, n, nb, out_mode)
    switch (tokens) {
      case 6: HWK_ROWS_M(6); break;
      case 7: HWK_ROWS_M(7); break;
      default: HWK_ROWS_M(8); break;
    }
#undef HWK_ROWS_M
    return hwk::launched("hwk_mxfp4_gemv_rows");
  }
  constexpr int RPW = 2;
  const uint32_t sets = (n + RPW - 1) / RPW;
  const uint32_t waves = sets < stream_waves() ? sets : stream_waves();
  const dim3 grid((waves + 3) / 4), block(256);
  const size_t lds = (size_t)tokens * k * 2;
#define HWK_ROWS(B, T)                                                                                        \
  hipLaunchKernelGGL((k_mxfp4_gemv_rows<B, RPW, T>), grid, block, lds, st, (const uint4 *)w, (const uint8_t *)e, \
                     (const uint4 *)x, y, n, nb, out_mode)
#define HWK_ROWS_T(B)                \
  switch (tokens) {                  \
    case 1: HWK_ROWS(B, 1); break;   \
    case 2: HWK_ROWS(B, 2); break;   \
    case 3: HWK_ROWS(B, 3); break;   \
    case 4: HWK_ROWS(B, 4); break;   \
    case 5: HWK_ROWS(B, 5); break;   \
    case 6: HWK_ROWS(B, 6); break;   \
    case 7: HWK_ROWS(B, 7); break;   \
    default: HWK_ROWS(B, 8); break;  \
  }
  switch ((nb + 63) / 64) {
    case 1: HWK_ROWS_T(1) break;
    case 2: HWK_ROWS_T(2) break;
    case 3: HWK_ROWS_T(3) break;
    default: HWK_ROWS_T(4) break;
  }
#undef HWK_ROWS_T
#undef HWK_ROWS
  return hwk::launched("hwk_mxfp4_gemv_rows");
}

HWK_API char *hwk_mxfp4_encode(void *stream, const void *x, void *w, void *e, uint32_t rows, uint32_t k) {
  HWK_CHECK(x && w && e, "hwk_mxfp4_encode: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_mxfp4_encode: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(hwk::aligned(x, 16) && hwk::aligned(w, 16), "hwk_mxfp4_encode: x and w must be 16-byte aligned");
  const uint64_t nblocks = (uint64_t)rows * (k / 32);
  if (nblocks == 0) return nullptr;
  hipLaunchKernelGGL(k_mxfp4_encode, dim3((uint32_t)((nblocks + 127) / 128)), dim3(128), 0, (hipStream_t)stream,
                     (const float *)x, (uint8_t *)w, (uint8_t *)e, nblocks);
  return hwk::launched("hwk_mxfp4_encode");
}

HWK_API char *hwk_synth_mxfp4(void *stream, void *w, void *e, uint32_t rows, uint32_t k, uint64_t key,
                              uint32_t std_bits) {
  HWK_CHECK(w && e, "hwk_synth_mxfp4: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0, "hwk_synth_mxfp4: k=%u is not a positive multiple of 32", k);
  HWK_CHECK(hwk::aligned(w, 16), "hwk_synth_mxfp4: w must be 16-byte aligned");
  const uint64_t nblocks = (uint64_t)rows * (k / 32);
  if (nblocks == 0) return nullptr;
  hipLaunchKernelGGL(k_synth_mxfp4, dim3((uint32_t)((nblocks + 127) / 128)), dim3(128), 0, (hipStream_t)stream,
                     (uint8_t *)w, (uint8_t *)e, nblocks, key, hwk::f32_of_bits(std_bits), k / 32, 1u, 0u);
  return hwk::launched("hwk_synth_mxfp4");
}

}  // extern "C"

namespace hwk {

namespace {

// The decode-step GEMV's workgroups: 8 waves of 2 rows a pass (x is made once for 8 waves' rows, and
// the model's shapes still give every CU whole workgroups: qkv 2048 row sets, 256 workgroups;
// gate_up 6144, 768; measured against 4 and 16 waves, and 4 rows a pass).
template <int BPL, int XM, bool SWIGLU, int MODE>
void launch_x(hipStream_t st, const void *w, const void *e, const XIn &in, void *y, uint32_t n, uint32_t nb) {
  constexpr int WPB = 8, RPW = 2;
  const uint32_t sets = (n + RPW - 1) / RPW;
  const void *xa = XM == X_F16 ? (const void *)in.x16 : XM == X_NORM ? (const void *)in.h : (const void *)in.ws;
#define HWK_XL(MBC) hipLaunchKernelGGL((k_mxfp4_gemv_x<BPL, RPW, XM, SWIGLU, WPB, MODE, MBC>), dim3((sets + WPB - 1) / WPB), \
                     dim3(64 * WPB), 0, st, (const uint4 *)w, (const uint8_t *)e, xa, y, n, nb, in.nw,              \
                     in.G | in.nchunk << 16, in.eps)
  if constexpr (XM == X_MERGE) {
    if (in.nchunk <= 4) HWK_XL(4);
    else if (in.nchunk <= 8) HWK_XL(8);
    else if (in.nchunk <= 12) HWK_XL(12);
    else HWK_XL(16);
  } else {
    HWK_XL(16);
  }
#undef HWK_XL
}

template <int XM, bool SWIGLU, int MODE>
void launch_x_bpl(hipStream_t st, const void *w, const void *e, const XIn &in, void *y, uint32_t n, uint32_t nb) {
  switch ((nb + 63) / 64) {
    case 1: launch_x<1, XM, SWIGLU, MODE>(st, w, e, in, y, n, nb); break;
    case 2: launch_x<2, XM, SWIGLU, MODE>(st, w, e, in, y, n, nb); break;
    case 3: launch_x<3, XM, SWIGLU, MODE>(st, w, e, in, y, n, nb); break;
    default: launch_x<4, XM, SWIGLU, MODE>(st, w, e, in, y, n, nb); break;
  }
}

template <int XM>
void launch_x_mode(hipStream_t st, const void *w, const void *e, const XIn &in, void *y, uint32_t n, uint32_t nb,
                   int mode, bool swiglu) {
  if (swiglu) launch_x_bpl<XM, true, HWK_OUT_F16>(st, w, e, in, y, n, nb);
  else if (mode == HWK_OUT_F16) launch_x_bpl<XM, false, HWK_OUT_F16>(st, w, e, in, y, n, nb);
  else if (mode == HWK_OUT_ADD_F32) launch_x_bpl<XM, false, HWK_OUT_ADD_F32>(st, w, e, in, y, n, nb);
  else launch_x_bpl<XM, false, HWK_OUT_F32>(st, w, e, in, y, n, nb);
}

}  // namespace

char *mxfp4_gemv_x(hipStream_t st, const void *w, const void *e, const void *x16, const float *h, const float *nw,
                   double eps, void *y, uint32_t n, uint32_t k, int out_mode, bool swiglu) {
  HWK_CHECK(w && e && y && (h ? nw != nullptr : x16 != nullptr), "mxfp4_gemv_x: null pointer");
  HWK_CHECK(k % 32 == 0 && k > 0 && k <= 64 * 4 * 32, "mxfp4_gemv_x: k=%u (a multiple of 32 up to 8192)", k);
  HWK_CHECK(!swiglu || n % 2 == 0, "mxfp4_gemv_x: SwiGLU over %u rows (pairs)", n);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "mxfp4_gemv_x: out_mode %d", out_mode);
  HWK_CHECK(aligned(w, 16) && (h || aligned(x16, 16)), "mxfp4_gemv_x: w and x must be 16-byte aligned");
  if (n == 0) return nullptr;
  XIn in{(const uint4 *)x16, h, nw, eps, nullptr, 1, 1};
  const uint32_t nb = k / 32;
  if (h) launch_x_mode<X_NORM>(st, w, e, in, y, n, nb, out_mode, swiglu);
  else launch_x_mode<X_F16>(st, w, e, in, y, n, nb, out_mode, swiglu);
  return launched("mxfp4_gemv_x");
}

char *mxfp4_gemv_merge(hipStream_t st, const void *w, const void *e, const void *workspace, uint32_t heads, uint32_t G,
                       uint32_t nchunk, void *y, uint32_t n, int out_mode) {
  HWK_CHECK(w && e && workspace && y, "mxfp4_gemv_merge: null pointer");
  const uint32_t k = heads * 128;
  HWK_CHECK(heads >= 1 && k <= 64 * 4 * 32, "mxfp4_gemv_merge: %u heads of 128 (at most 8192 values)", heads);
  HWK_CHECK(G >= 1 && G < 65536 && heads % G == 0, "mxfp4_gemv_merge: G %u", G);
  HWK_CHECK(nchunk >= 1 && nchunk <= kMergeMaxChunks, "mxfp4_gemv_merge: %u chunks (at most %u)", nchunk,
            kMergeMaxChunks);
  HWK_CHECK(out_mode >= HWK_OUT_F32 && out_mode <= HWK_OUT_ADD_F32, "mxfp4_gemv_merge: out_mode %d", out_mode);
  HWK_CHECK(aligned(w, 16) && aligned(workspace, 16), "mxfp4_gemv_merge: w and the workspace 16-byte aligned");
  if (n == 0) return nullptr;
  XIn in{nullptr, nullptr, nullptr, 0.0, (const float *)workspace, G, nchunk};
  launch_x_mode<X_MERGE>(st, w, e, in, y, n, k / 32, out_mode, false);
  return launched("mxfp4_gemv_merge");
}

char *synth_mxfp4_rows(hipStream_t st, void *w, void *e, uint32_t rows, uint32_t k, uint64_t key, float stdv,
                       uint32_t stride, uint32_t row0) {
  HWK_CHECK(w && e && k % 32 == 0 && k > 0 && stride > 0, "synth_mxfp4_rows: bad arguments");
  const uint64_t nblocks = (uint64_t)rows * (k / 32);
  if (nblocks == 0) return nullptr;
  hipLaunchKernelGGL(k_synth_mxfp4, dim3((uint32_t)((nblocks + 127) / 128)), dim3(128), 0, st, (uint8_t *)w,
                     (uint8_t *)e, nblocks, key, stdv, k / 32, stride, row0);
  return launched("synth_mxfp4_rows");
}

}  // namespace hwk
