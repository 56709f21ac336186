// The device code of K3, the prefill / verify GEMM, shared by libhwk's kernels (gemm.hip) and the
// kernels of the library's code object (co/hwk_co.hip), so that both run the same instructions.
//
// Prefill / verify GEMM (K3) on gfx950: Y (M, N) = X (M, K) W^T, X fp16, W int8 per output channel
// or MXFP4, fp32 accumulation on the fp16 MFMA (v_mfma_f32_16x16x32_f16).
//
// A workgroup of 4 waves (one a SIMD, 2 x 2) computes a BM x BN tile of Y; a wave holds a
// (BM/2) x (BN/2) block of 16 x 16 accumulator tiles. K goes 128 at a time:
//   X: the tile's 128-column slab goes through LDS (two buffers, one barrier a step), 16-byte chunks
//      placed at chunk ^ (row & 15) so that the 16 rows one MFMA operand load touches fall in 16
//      different bank groups (a row is 256 bytes, the width of the 64 banks);
//   W: each wave loads its own columns' codes straight into registers (16 or 32 bytes a lane per 16
//      columns a step) and converts them there: int8 exactly to fp16 (the channel scale applied to
//      the fp32 result), MXFP4 by the hardware fp4 conversion with the block scale folded in.
// Loads run two steps ahead of the multiply (register stages), so a step's global latency hides
// behind the two steps before it. A lane's 32 values of K a step are the same set in its X and W
// operands, so each MFMA sums 32 true products (which lane holds which k is a free choice of the
// kernel, made for contiguous loads).
//
// MXFP4 exactness: a code times its block scale is an fp16 value when the scale's exponent is in
// [-23, 13]. A row (output channel) whose finite block exponents leave that range is shifted by a
// power of two s0 chosen per row (the largest exponent mapped to 13) and its fp32 result scaled back
// by 2^s0, which is exact; rows whose exponents span more than 36 lose the low bits of their
// smallest blocks (values below 2^-24 of the shifted scale). Scale e = 0 is 0 and e = 255 is +Inf,
// as in the reference's Dequantize (internal/mxfp4/mxfp4.go:77).
//
// Tile order is XCD-aware: the workgroups that share a weight panel run on the same XCD, so its L2
// holds the panel once; the host picks the tile shape that fills the 256 CUs best.
#pragma once

#include "hwk_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace hwk_gemm {

constexpr int KS = 128;     // K a step
constexpr int CH = KS / 8;  // 16-byte chunks of an X row a step
constexpr int KK = KS / 32;  // MFMAs a step for one (16-row, 16-column) tile
constexpr int NS = 2;       // register stages: loads run NS steps ahead
constexpr int kOutSwiGLU = HWK_OUT_SWIGLU_F16;

// 4 int8 codes (one dword) as 4 exact fp16 values (two dwords).
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const h2 bias = {(f16)1152.0f, (f16)1152.0f};
  const h2 lo = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
  const h2 hi = h2_of_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

// 8 int8 codes (two dwords) as a half8 operand.
__device__ __forceinline__ half8 i8x8_to_half8(uint32_t a, uint32_t b) {
  const uint2 p = i8x4_to_f16x4(a), q = i8x4_to_f16x4(b);
  const u32x4 v = {p.x, p.y, q.x, q.y};
  return __builtin_bit_cast(half8, v);
}

// 8 e2m1 codes (one dword, even element in the low nibble) times scale s as a half8 operand.
__device__ __forceinline__ half8 fp4x8_to_half8(uint32_t w, float s) {
  const u32x4 v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3))};
  return __builtin_bit_cast(half8, v);
}

__device__ __forceinline__ u32x4 load16(const void *p) { return *(const u32x4 *)p; }

// The X chunk (of CH a row a step) that MFMA kk of lane group q reads: the k offsets of a lane's
// operands in the step. int8: two 16-byte weight loads a lane at q*16 and 64 + q*16 (each 16 rows x 64
// contiguous bytes a load instruction); MXFP4: one 32-value block a lane at q*32.
template <bool MX>
__device__ __forceinline__ int xchunk(int q, int kk) {
  if constexpr (MX) return 4 * q + kk;
  return kk < 2 ? 2 * q + kk : 8 + 2 * q + (kk - 2);
}

// KG k groups of WM x WN waves: group g takes MFMAs g*KK/KG .. of every step of the whole tile, and
// the groups' accumulators are summed at the end (int8 only: 2 groups make an 8-wave workgroup of a
// tile that 4 waves would hold, so that a CU's SIMDs split the tile's k as well as its columns).
template <int BM, int BN, bool MX, int WM, int WN, int KG>
struct Cfg {
  static constexpr int NT = 64 * WM * WN * KG;              // threads: KG groups of WM x WN waves
  static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16 x 16 tiles a wave
  static constexpr int AL = BM * CH / NT;                   // X chunks a thread stages a step
  static constexpr int BL = MX ? 1 : 2 / KG;                // 16-byte weight loads a lane a step a tile
  static constexpr int KKG = KK / KG;                       // MFMAs a tile a step a wave
  static_assert(BM * CH % NT == 0 && TM * WM * 16 == BM && TN * WN * 16 == BN, "tile shape");
  static_assert(KG == 1 || KG == 2, "one or two k groups");
};

template <int BM, int BN, bool MX, int WM, int WN, int KG>
struct Stage {
  u32x4 a[Cfg<BM, BN, MX, WM, WN, KG>::AL];
  u32x4 b[Cfg<BM, BN, MX, WM, WN, KG>::TN][Cfg<BM, BN, MX, WM, WN, KG>::BL];
  uint32_t e[Cfg<BM, BN, MX, WM, WN, KG>::TN];  // MXFP4 block scale bytes
  uint32_t k0;                                  // the step's K offset
};

// Issue the global loads of the step at K offset k0 into s: X (load_x) and the weights (load_w).
// Out-of-range rows and columns read the last row/column (their results are not stored); K past the
// end reads in-range data, which zero_tail clears when the stage is consumed (a select here would wait
// for the load at once). Every load is issued unconditionally (a load under a branch would be waited
// for at the join).
template <int BM, int BN, bool MX, int WM, int WN, int KG>
__device__ __forceinline__ void load_x(Stage<BM, BN, MX, WM, WN, KG> &s, const u32x4 *__restrict__ X, uint32_t M,
                                       uint32_t K, uint32_t m0, uint32_t k0, int t) {
  using C = Cfg<BM, BN, MX, WM, WN, KG>;
  s.k0 = k0;
#pragma unroll
  for (int i = 0; i < C::AL; i++) {
    const int c = t + C::NT * i, row = c / CH, ch = c % CH;
    const uint32_t m = min(m0 + row, M - 1);
    s.a[i] = X[((size_t)m * K + min(k0 + ch * 8, K - 8)) / 8];
  }
}

// (int8: a k group's half of the step's 128 codes a row, h = g, when KG = 2)
template <int BM, int BN, bool MX, int WM, int WN, int KG>
__device__ __forceinline__ void load_w(Stage<BM, BN, MX, WM, WN, KG> &s, const uint8_t *__restrict__ W,
                                       const uint8_t *__restrict__ E, uint32_t K, uint32_t k0,
                                       const uint32_t (&brow)[Cfg<BM, BN, MX, WM, WN, KG>::TN], int q, int g) {
  using C = Cfg<BM, BN, MX, WM, WN, KG>;
  if constexpr (MX) {
    const uint32_t blk = min(k0 + q * 32, K - 32) / 32;
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
      const size_t bi = (size_t)brow[j] * (K / 32) + blk;
      s.b[j][0] = load16(W + bi * 16);
      s.e[j] = E[bi];
    }
  } else {
#pragma unroll
    for (int h = 0; h < C::BL; h++) {
      const uint32_t kc = min(k0 + (KG == 1 ? h : g) * 64 + q * 16, K - 16);
#pragma unroll
      for (int j = 0; j < C::TN; j++) s.b[j][h] = load16(W + (size_t)brow[j] * K + kc);
    }
  }
}

// A step reaching past K: its X chunks and weight loads past K become zeros (MXFP4: scale 0).
template <int BM, int BN, bool MX, int WM, int WN, int KG>
__device__ __forceinline__ void zero_tail(Stage<BM, BN, MX, WM, WN, KG> &s, uint32_t K, int t, int q, int g) {
  using C = Cfg<BM, BN, MX, WM, WN, KG>;
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < C::AL; i++)
    if (s.k0 + ((t + C::NT * i) % CH) * 8 >= K) s.a[i] = zero;
#pragma unroll
  for (int j = 0; j < C::TN; j++) {
    if constexpr (MX) {
      if (s.k0 + q * 32 >= K) {
        s.b[j][0] = zero;
        s.e[j] = 0u;
      }
    } else {
#pragma unroll
      for (int h = 0; h < C::BL; h++)
        if (s.k0 + (KG == 1 ? h : g) * 64 + q * 16 >= K) s.b[j][h] = zero;
    }
  }
}

// The block scale of exponent byte e in a row shifted by 2^-s0 (see the header): 0 for e = 0 or a
// shifted exponent below the float range, +Inf for e = 255.
__device__ __forceinline__ float shifted_scale(uint32_t e, int s0) {
  const float v = __uint_as_float((uint32_t)max((int)e - s0, 0) << 23);  // below the float range: +0
  return e == 255u ? __builtin_inff() : e == 0u ? 0.0f : v;
}

// The row shifts s0 of the tile's BN weight rows (n0 .. n0+BN-1, clamped to N-1): 0 for a row whose
// finite, nonzero block exponents are all in [-23, 13]; else the largest mapped to 13. The workgroup's
// threads scan the rows' scale bytes (16-byte chunks when every row starts 16-byte aligned, all of a
// thread's loads issued before any is used; bytes otherwise) and combine per row in LDS (hs: the
// largest exponent byte other than 255, ls: the smallest other than 0 and 255). hs and ls are set
// to 0 and 255 by the caller before a barrier; another barrier follows before they are read.
template <int BN, int NT>
__device__ __forceinline__ void scan_shifts(const uint8_t *__restrict__ E, uint32_t n0, uint32_t N, uint32_t nb,
                                            bool quads, int t, int *hs, int *ls) {
  auto take = [&](uint32_t e, uint32_t &h, uint32_t &l) {
    h = max(h, e == 255u ? 0u : e);
    l = min(l, (e == 0u || e == 255u) ? 255u : e);
  };
  if (quads) {
    const uint32_t nch = nb / 16, total = BN * nch;
    for (uint32_t base = 0; base < total; base += 4 * NT) {
      u32x4 v[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t c = min(base + t + NT * i, total - 1), row = c / nch;
        v[i] = *(const u32x4 *)(E + (size_t)min(n0 + row, N - 1) * nb + (c % nch) * 16);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t c = base + t + NT * i;
        if (c >= total) continue;
        uint32_t h = 0, l = 255;
#pragma unroll
        for (int w = 0; w < 4; w++)
#pragma unroll
          for (int b = 0; b < 4; b++) take((v[i][w] >> (8 * b)) & 255u, h, l);
        atomicMax(&hs[c / nch], (int)h);
        atomicMin(&ls[c / nch], (int)l);
      }
    }
  } else {
    for (uint32_t c = t; c < BN * nb; c += NT) {
      const uint32_t row = c / nb;
      uint32_t h = 0, l = 255;
      take(E[(size_t)min(n0 + row, N - 1) * nb + c % nb], h, l);
      atomicMax(&hs[row], (int)h);
      atomicMin(&ls[row], (int)l);
    }
  }
}

// The shift of a row from its scanned bytes.
__device__ __forceinline__ int shift_of(int hi, int lo) {
  if (hi == 0) return 0;  // no finite nonzero scale
  const int emax = hi - 127, emin = lo - 127;
  return (emax <= 13 && emin >= -23) ? 0 : emax - 13;
}

// Workgroup id -> tile: consecutive ids go round the XCDs, so ids x, x+8, x+16, ... share an XCD;
// those take the M tiles of one N panel in turn.
__device__ __forceinline__ void tile_of(uint32_t id, uint32_t mt, uint32_t nt, uint32_t &tm, uint32_t &tn) {
  const uint32_t total = mt * nt;
  const uint32_t xcd = id % 8, j = id / 8;
  uint32_t lin = id;
  if (total % 8 == 0) {
    const uint32_t per = total / 8;  // tiles an XCD runs
    lin = xcd * per + j;
  }
  tn = lin / mt;
  tm = lin % mt;
}

// The tile's store: D of MFMA tile (i, j) of the wave, lane (r16, q) holding rows q*4 + r of column
// r16; int8 results take the column's scale, MXFP4 results the row shift back (2^s0, exact).
template <int BM, int WM, int TM, int TN, bool MX>
__device__ __forceinline__ void store_tile(const floatx4 (&acc)[TM][TN], const int (&s0)[TN],
                                           const uint16_t *__restrict__ S, void *__restrict__ Y, uint32_t M,
                                           uint32_t N, uint32_t m0, uint32_t nw, int wm, int r16, int q, int mode) {
  if (mode == kOutSwiGLU) {
    // columns (2c, 2c+1) are (gate, up) of output c, held by lanes r16 and r16 ^ 1 for the same four
    // rows: the gate lane takes the up values of rows 0, 1 and computes those outputs, the up lane
    // takes the gate values of rows 2, 3 and computes those. Every lane joins the swaps; columns past
    // N (a tile wider than N) store nothing, and with N % 16 == 0 a pair is wholly below N or not.
    const bool gate = (r16 & 1) == 0;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const uint32_t n = nw + j * 16 + r16, c = n / 2;
      const float sc = MX ? 1.0f : (float)__builtin_bit_cast(f16, S[min(n, N - 1)]);
#pragma unroll
      for (int i = 0; i < TM; i++) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = MX ? ldexpf(acc[i][j][r], s0[j]) : acc[i][j][r] * sc;
        const float o0 = __shfl_xor(gate ? v[2] : v[0], 1, 64), o1 = __shfl_xor(gate ? v[3] : v[1], 1, 64);
        const uint32_t mr = m0 + wm * (BM / WM) + i * 16 + q * 4 + (gate ? 0 : 2);  // the lane's first row
        const float y0 = gate ? swiglu_value(v[0], o0) : swiglu_value(o0, v[2]);
        const float y1 = gate ? swiglu_value(v[1], o1) : swiglu_value(o1, v[3]);
        if (n < N && mr < M) ((f16 *)Y)[(size_t)mr * (N / 2) + c] = (f16)y0;
        if (n < N && mr + 1 < M) ((f16 *)Y)[(size_t)(mr + 1) * (N / 2) + c] = (f16)y1;
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const uint32_t n = nw + j * 16 + r16;
    if (n >= N) continue;
    const float sc = MX ? 1.0f : (float)__builtin_bit_cast(f16, S[n]);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t m = m0 + wm * (BM / WM) + i * 16 + q * 4 + r;
        if (m < M) store_out(Y, (size_t)m * N + n, MX ? ldexpf(acc[i][j][r], s0[j]) : acc[i][j][r] * sc, mode);
      }
  }
}

// The same stores through LDS: the wave's block (RW x CW) into its region st of LDS, as the values
// stored (fp16 rounded, or SwiGLU'd pairs, or scaled fp32), then 16-byte pieces of its rows to Y: an
// MFMA tile's lanes hold one column each, so a direct store instruction writes 2 or 4 bytes a lane.
// Every value is rounded and combined as store_tile does it. The fp32 rows are padded (P32 = CW + 4
// floats) so that the 4 row groups of a write land in different banks (P32 = CW where the padded
// block does not fit); the fp16 rows are not (padding them measured no faster: their reads of 16
// bytes a lane then conflict). Needs Y 16-byte aligned and N a multiple of the piece (4 fp32, 8 fp16
// or 16 SwiGLU columns): staged() tells.
__device__ __forceinline__ bool staged(const void *Y, uint32_t N, int mode) {
  const uint32_t piece = mode == kOutSwiGLU ? 16 : mode == HWK_OUT_F16 ? 8 : 4;
  return ((uintptr_t)Y & 15) == 0 && N % piece == 0;
}
template <int TM, int TN, int P32>
struct StageRows {
  static constexpr int RW = TM * 16, CW = TN * 16;
  static constexpr int P16 = CW, PH = CW / 2 + 8;  // fp16 rows: full width, SwiGLU half width (padded)
  static constexpr int FLOATS = RW * P32;              // a region, in floats (the largest of the three)
  static_assert(P32 == CW || P32 == CW + 4, "fp32 row stride");
  static_assert(RW * P16 * 2 <= FLOATS * 4 && RW * PH * 2 <= FLOATS * 4, "fp16 rows fit the region");
};
template <int BM, int WM, int TM, int TN, bool MX, int P32>
__device__ __forceinline__ void store_tile_staged(const floatx4 (&acc)[TM][TN], const int (&s0)[TN],
                                                  const uint16_t *__restrict__ S, void *__restrict__ Y, uint32_t M,
                                                  uint32_t N, uint32_t m0, uint32_t nw, int wm, int lane, int mode,
                                                  float *st) {
  using G = StageRows<TM, TN, P32>;
  constexpr int RW = G::RW, CW = G::CW;
  const int r16 = lane & 15, q = lane >> 4;
  const uint32_t r0 = m0 + wm * RW;
  auto value = [&](int i, int j, int r) __attribute__((always_inline)) {
    const float sc = MX ? 1.0f : (float)__builtin_bit_cast(f16, S[min(nw + j * 16 + r16, N - 1)]);
    return MX ? ldexpf(acc[i][j][r], s0[j]) : acc[i][j][r] * sc;
  };
  if (mode == kOutSwiGLU) {
    // the pairs as store_tile makes them: gate lane rows 0, 1 of its quad, up lane rows 2, 3
    f16 *h = (f16 *)st;
    const bool gate = (r16 & 1) == 0;
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int i = 0; i < TM; i++) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = value(i, j, r);
        const float o0 = __shfl_xor(gate ? v[2] : v[0], 1, 64), o1 = __shfl_xor(gate ? v[3] : v[1], 1, 64);
        const int row = i * 16 + q * 4 + (gate ? 0 : 2), c = (j * 16 + r16) / 2;
        h[row * G::PH + c] = (f16)(gate ? swiglu_value(v[0], o0) : swiglu_value(o0, v[2]));
        h[(row + 1) * G::PH + c] = (f16)(gate ? swiglu_value(v[1], o1) : swiglu_value(o1, v[3]));
      }
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // this wave's LDS writes done
    constexpr int CPR = CW / 16;  // 8 outputs a piece
    for (int c = lane; c < RW * CPR; c += 64) {
      const int row = c / CPR, k = c % CPR;
      const uint32_t m = r0 + row, n = nw + k * 16;
      if (m < M && n < N)
        *(u32x4 *)((f16 *)Y + (size_t)m * (N / 2) + n / 2) = *(const u32x4 *)(h + row * G::PH + k * 8);
    }
  } else if (mode == HWK_OUT_F16) {
    f16 *h = (f16 *)st;
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) h[(i * 16 + q * 4 + r) * G::P16 + j * 16 + r16] = (f16)f32_value(value(i, j, r));
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
    constexpr int CPR = CW / 8;
    for (int c = lane; c < RW * CPR; c += 64) {
      const int row = c / CPR, k = c % CPR;
      const uint32_t m = r0 + row, n = nw + k * 8;
      if (m < M && n < N) *(u32x4 *)((f16 *)Y + (size_t)m * N + n) = *(const u32x4 *)(h + row * G::P16 + k * 8);
    }
  } else {
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) st[(i * 16 + q * 4 + r) * P32 + j * 16 + r16] = value(i, j, r);
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
    constexpr int CPR = CW / 4;
    for (int c = lane; c < RW * CPR; c += 64) {
      const int row = c / CPR, k = c % CPR;
      const uint32_t m = r0 + row, n = nw + k * 4;
      if (m >= M || n >= N) continue;
      floatx4 v = *(const floatx4 *)(st + row * P32 + k * 4);
      floatx4 *y = (floatx4 *)((float *)Y + (size_t)m * N + n);
      if (mode == HWK_OUT_ADD_F32) v = *y + v;
      *y = v;
    }
  }
}

template <int BM, int BN, bool MX, int WM, int WN, int KG = 1>
__device__ __forceinline__ void gemm_wg(uint32_t bx, const u32x4 *__restrict__ X, const uint8_t *__restrict__ W,
                                        const uint8_t *__restrict__ E, const uint16_t *__restrict__ S,
                                        void *__restrict__ Y, uint32_t M, uint32_t N, uint32_t K, int mode,
                                        bool equads) {
  using C = Cfg<BM, BN, MX, WM, WN, KG>;
  constexpr int TM = C::TM, TN = C::TN, NT = C::NT, KKG = C::KKG;
  static_assert(KG == 1 || !MX, "k groups here: int8 only");
  static_assert(KG == 1 || BM * BN * 4 <= 2 * BM * CH * 16, "the k groups' sum goes through the X buffers");
  __shared__ __attribute__((aligned(16))) u32x4 As[2][BM * CH];
  __shared__ int hs[MX ? BN : 1], ls[MX ? BN : 1];  // the row shift scan (MXFP4)
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g = wave / (WM * WN), wl = wave % (WM * WN);  // k group, wave in the group
  const int wm = wl / WN, wn = wl % WN;
  const int r16 = lane & 15, q = lane >> 4;
  uint32_t tm, tn;
  tile_of(bx, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t nw = n0 + wn * (BN / WN);  // the wave's first column
  uint32_t brow[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) brow[j] = min(nw + j * 16 + r16, N - 1);

  const uint32_t steps = (K + KS - 1) / KS;
  auto kofs = [&](uint32_t j) -> uint32_t { return min(j, steps) * KS; };  // past the end: reads zeros
  Stage<BM, BN, MX, WM, WN, KG> st[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) {
    load_x<BM, BN, MX, WM, WN, KG>(st[s], X, M, K, m0, kofs(s), t);
    load_w<BM, BN, MX, WM, WN, KG>(st[s], W, E, K, kofs(s), brow, q, g);
  }
  int s0[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) s0[j] = 0;
  if constexpr (MX) {
    if (t < BN) {
      hs[t] = 0;
      ls[t] = 255;
    }
    __syncthreads();
    scan_shifts<BN, NT>(E, n0, N, K / 32, equads, t, hs, ls);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const uint32_t r = brow[j] - n0;
      s0[j] = shift_of(hs[r], ls[r]);
    }
  }

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};

  // Steps in groups of NS (a partial last group multiplies zeros: its loads read past K). A step:
  // its X slab into LDS, barrier, the next X loads of its stage, then for each kk its weight operands
  // converted next to the MFMAs that take them (the VALU work overlaps the matrix core), then the
  // next weight loads of its stage. Issue order is pinned: the wait counter is in order, so a stage
  // consumed before the loads behind it is waited for without waiting for them.
  for (uint32_t j0 = 0; j0 < steps; j0 += NS) {
#pragma unroll
    for (int s = 0; s < NS; s++) {
      const uint32_t j = j0 + s;
      u32x4 *buf = As[s & 1];  // NS is even: step j uses buffer j & 1
      if (st[s].k0 + KS > K) zero_tail<BM, BN, MX, WM, WN, KG>(st[s], K, t, q, g);  // uniform: only a ragged step
#pragma unroll
      for (int i = 0; i < C::AL; i++) {
        const int c = t + NT * i, row = c / CH, ch = c % CH;
        buf[row * CH + (ch ^ (row & 15))] = st[s].a[i];
      }
      __syncthreads();
      issue_order();
      load_x<BM, BN, MX, WM, WN, KG>(st[s], X, M, K, m0, kofs(j + NS), t);
      issue_order();
      float sc[TN];
#pragma unroll
      for (int jn = 0; jn < TN; jn++) sc[jn] = MX ? shifted_scale(st[s].e[jn], s0[jn]) : 0.0f;
      // the operands of kk + 1 (X from LDS, weights converted) are fetched before the MFMAs of kk; kk
      // counts the group's MFMAs (the step's MFMA g*KKG + kk)
      auto operands = [&](half8 (&af)[TM], half8 (&bf)[TN], int kk) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const int row = wm * (BM / WM) + i * 16 + r16;
          const int ch = KG == 1 ? xchunk<MX>(q, kk) : xchunk<MX>(q, g * KKG + kk);
          af[i] = __builtin_bit_cast(half8, buf[row * CH + (ch ^ (row & 15))]);
        }
#pragma unroll
        for (int jn = 0; jn < TN; jn++) {
          if constexpr (MX) {
            bf[jn] = fp4x8_to_half8(st[s].b[jn][0][kk], sc[jn]);
          } else {
            const u32x4 v = st[s].b[jn][kk >> 1];  // KG = 2: the group's half, loaded alone
            bf[jn] = i8x8_to_half8(v[(kk & 1) * 2], v[(kk & 1) * 2 + 1]);
          }
        }
      };
      half8 af[2][TM], bf[2][TN];
      operands(af[0], bf[0], 0);
#pragma unroll
      for (int kk = 0; kk < KKG; kk++) {
        if (kk + 1 < KKG) operands(af[(kk + 1) & 1], bf[(kk + 1) & 1], kk + 1);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int jn = 0; jn < TN; jn++)
            acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[kk & 1][i], bf[kk & 1][jn], acc[i][jn], 0, 0, 0);
      }
      issue_order();
      load_w<BM, BN, MX, WM, WN, KG>(st[s], W, E, K, kofs(j + NS), brow, q, g);
      issue_order();
    }
  }
  if constexpr (KG == 2) {
    // group 1's accumulators to group 0 through the X buffers (every wave is done with them after
    // the barrier), summed in group 0, which writes the tile
    floatx4 *red = (floatx4 *)&As[0][0];
    __syncthreads();
    if (g == 1) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) red[((wl * TM + i) * TN + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (g == 0) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] += red[((wl * TM + i) * TN + j) * 64 + lane];
    }
    __syncthreads();  // group 0 is done with the sums' buffers, which its stores reuse
    if (g == 1) return;
  }
  if (staged(Y, N, mode)) {
    // a wave's block in region wl of the X buffers (rows padded where that fits)
    constexpr int CW = TN * 16, PAD = WM * WN * TM * 16 * (CW + 4) <= 2 * BM * CH * 4 ? CW + 4 : CW;
    using G = StageRows<TM, TN, PAD>;
    static_assert(WM * WN * G::FLOATS <= 2 * BM * CH * 4, "the staged blocks fit the X buffers");
    if constexpr (KG == 1) __syncthreads();  // every wave is done with the X buffers
    store_tile_staged<BM, WM, TM, TN, MX, PAD>(acc, s0, S, Y, M, N, m0, nw, wm, lane, mode,
                                               (float *)&As[0][0] + wl * G::FLOATS);
    return;
  }
  store_tile<BM, WM, TM, TN, MX>(acc, s0, S, Y, M, N, m0, nw, wm, r16, q, mode);
}


// ---- The ring form (K a multiple of 128): X and the weights both go straight from memory into LDS ----
//
// Every global load of the main loop is a load into LDS (global_load_lds_dwordx4: lane i of an
// instruction writes 16 bytes at the instruction's LDS base + 16 i), into a ring of RS buffers a
// stream (a template parameter), issued RS-1 steps ahead of the MFMAs that read them, and waited for
// by an explicit count
// (the wait counter is in order, and every step issues the same number of loads: past the last step
// they reread in-range data into a buffer nobody reads). No load result lives in a register across
// steps, so the loop carries nothing for the compiler to wait on at its head. The swizzles are applied
// on the source side (which 16-byte chunk a lane fetches), so that the MFMA operand reads of 16
// lanes land in distinct banks:
//   X   slot p: row p / CH, chunk (p % CH) ^ (row & 15)                       (256-byte rows)
//   W   slot p: column p / WCH, chunk (p % WCH) ^ ((column / CPB) & (WCH-1))    (WCH chunks a column a
//       step: int8 8 = 128 codes, MXFP4 4 = 128 values; CPB columns share a 256-byte bank row)
//   E   (MXFP4) slot p: column p, the 4 scale bytes of the step (4-byte loads)
// An LDS buffer of BYTES, one variable per (BYTES, I, TAG): the buffers of a ring are distinct
// variables, so that the compiler can tell an LDS read of one from the loads into LDS in flight for
// the others.
template <typename T, int COUNT, int I, int TAG>
__device__ __forceinline__ T *lds_buf() {
  __shared__ __attribute__((aligned(16))) T b[COUNT];
  return b;
}
template <typename T, int COUNT, int TAG, int N>
struct RingBufs {
  static __device__ __forceinline__ void fill(T **p) {
    RingBufs<T, COUNT, TAG, N - 1>::fill(p);
    p[N - 1] = lds_buf<T, COUNT, N - 1, TAG>();
  }
};
template <typename T, int COUNT, int TAG>
struct RingBufs<T, COUNT, TAG, 0> {
  static __device__ __forceinline__ void fill(T **) {}
};

template <int BM, int BN, bool MX, int WM, int WN, int KG, int RS>
struct RCfg {
  using C = Cfg<BM, BN, MX, WM, WN, KG>;
  static constexpr int NT = C::NT, NW = NT / 64;
  static constexpr int WCH = MX ? 4 : 8;                             // 16-byte weight chunks a column a step
  static constexpr int CPB = 256 / (WCH * 16);                       // columns a 256-byte bank row
  static constexpr int AX = BM * CH / NT;                            // X loads a lane a step
  static constexpr int AW = (BN * WCH + NT - 1) / NT;                // weight loads a lane a step
  static constexpr int WSLOTS = AW * NT;                             // weight slots a buffer (padded)
  static constexpr int LS = AX + AW + (MX ? 1 : 0);                  // loads a lane a step (E: one)
  static_assert(BM * CH % NT == 0, "X loads a lane");
  static_assert(!MX || BN <= NT, "scale slots");
  static_assert((RS - 1) * LS <= 63, "loads in flight past the wait counter");
};

template <int N>
__device__ __forceinline__ void wait_loads() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// LDS writes and reads of this wave done (lgkmcnt 0; the other counters not waited for)
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }
// A workgroup barrier that waits for no memory counter (__syncthreads would wait for every load into
// LDS in flight, the ring's prefetches included): the caller has waited for its own part.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void lds_void;
// The loads into LDS as inline assembly, so that the compiler inserts no wait of its own for them: its
// wait insertion tracks the LDS targets of a few such loads only, and before an LDS read that none of
// those covers it waits for every load in flight (vmcnt(0): in the software-pipelined loop below,
// two steps of six drained the prefetch that way). The ring's explicit vmcnt waits and barriers order
// them instead; the "memory" clobber keeps LDS reads and the barriers on their side of each load.
// The LDS address (wave-uniform) goes in M0 as an operand the compiler sets, the s_nop the wait state
// between that write and the load; the global address is sbase (scalar) + voff (a lane's offset).
__device__ __forceinline__ void to_lds16(const void *sbase, uint32_t voff, void *lds) {
  const uint32_t l = (uint32_t)(uintptr_t)(lds_void *)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(l) : "memory");
}
__device__ __forceinline__ void to_lds4(const void *sbase, uint32_t voff, void *lds) {
  const uint32_t l = (uint32_t)(uintptr_t)(lds_void *)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(l) : "memory");
}

// The sources of a lane's loads into LDS: a uniform base (the operand's start plus the step's K
// offset, in scalar registers) and the lane's byte offset from it (computed once: the loads take the
// base + offset form, no per-lane address arithmetic a step). Out-of-range rows and columns read the
// last row/column. The offsets are 32-bit: the launcher takes this form for operands under 4 GiB.
template <int BM, int BN, bool MX, int WM, int WN, int KG, int RS>
struct RingSrc {
  using R = RCfg<BM, BN, MX, WM, WN, KG, RS>;
  const char *X, *W, *E;
  uint32_t xo[R::AX], wo[R::AW], eo;
  uint32_t K;
  __device__ __forceinline__ RingSrc(const u32x4 *X_, const uint8_t *W_, const uint8_t *E_, uint32_t M, uint32_t N,
                                     uint32_t K_, uint32_t m0, uint32_t n0, int wave, int lane)
      : X((const char *)X_), W((const char *)W_), E((const char *)E_), K(K_) {
#pragma unroll
    for (int a = 0; a < R::AX; a++) {
      const int p = (a * R::NW + wave) * 64 + lane, row = p / CH, ch = (p % CH) ^ (row & 15);
      xo[a] = (min(m0 + row, M - 1) * K + ch * 8) * 2;
    }
    const uint32_t rowb = MX ? K / 2 : K;  // weight bytes a column
#pragma unroll
    for (int a = 0; a < R::AW; a++) {
      const int p = (a * R::NW + wave) * 64 + lane, col = p / R::WCH;
      const int c = (p % R::WCH) ^ ((col / R::CPB) & (R::WCH - 1));
      wo[a] = min(n0 + col, N - 1) * rowb + c * 16;
    }
    eo = MX ? min(n0 + (uint32_t)(wave * 64 + lane), N - 1) * (K / 32) : 0u;  // slots past BN: padding
  }
  // The loads of the step at K offset k0 (clamped to the last step: a step past the end rereads it).
  __device__ __forceinline__ void load(u32x4 *xb, u32x4 *wb, uint32_t *eb, uint32_t k0, int wave) const {
    k0 = min(k0, K - KS);
#pragma unroll
    for (int a = 0; a < R::AX; a++) to_lds16(X + k0 * 2, xo[a], xb + (a * R::NW + wave) * 64);
#pragma unroll
    for (int a = 0; a < R::AW; a++) to_lds16(W + (MX ? k0 / 2 : k0), wo[a], wb + (a * R::NW + wave) * 64);
    if constexpr (MX) to_lds4(E + k0 / 32, eo, eb + wave * 64);
  }
};

template <int BM, int BN, bool MX, int WM, int WN, int KG, int RS>
__device__ __forceinline__ void gemm_ring_wg(uint32_t bx, const u32x4 *__restrict__ X, const uint8_t *__restrict__ W,
                                             const uint8_t *__restrict__ E, const uint16_t *__restrict__ S,
                                             void *__restrict__ Y, uint32_t M, uint32_t N, uint32_t K, int mode,
                                             bool equads) {
  using C = Cfg<BM, BN, MX, WM, WN, KG>;
  using R = RCfg<BM, BN, MX, WM, WN, KG, RS>;
  constexpr int TM = C::TM, TN = C::TN, NT = C::NT, KKG = C::KKG, LS = R::LS;
  static_assert(RS >= 2 && RS <= 6, "ring depth");
  // one LDS variable a stage: X, then the weights, then the MXFP4 scales
  constexpr int XB = BM * CH, WB = R::WSLOTS, EB = MX ? R::NW * 16 : 0;  // 16-byte slots
  u32x4 *sr[RS], *xr[RS], *wr[RS];
  uint32_t *er[RS];
  RingBufs<u32x4, XB + WB + EB, 0, RS>::fill(sr);
#pragma unroll
  for (int s = 0; s < RS; s++) {
    xr[s] = sr[s];
    wr[s] = sr[s] + XB;
    er[s] = (uint32_t *)(sr[s] + XB + WB);
  }
  __shared__ int hs[MX ? BN : 1], ls[MX ? BN : 1];  // the row shift scan (MXFP4)
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int g = wave / (WM * WN), wl = wave % (WM * WN);  // k group, wave in the group
  const int wm = wl / WN, wn = wl % WN;
  const int r16 = lane & 15, q = lane >> 4;
  uint32_t tm, tn;
  tile_of(bx, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t nw = n0 + wn * (BN / WN);  // the wave's first column
  const uint32_t steps = K / KS;
  const RingSrc<BM, BN, MX, WM, WN, KG, RS> src(X, W, E, M, N, K, m0, n0, wave, lane);
#pragma unroll
  for (int s = 0; s < RS - 1; s++) src.load(xr[s], wr[s], er[s], s * KS, wave);
  int s0[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) s0[j] = 0;
  if constexpr (MX) {
    if (t < BN) {
      hs[t] = 0;
      ls[t] = 255;
    }
    wait_lds();
    ring_barrier();
    scan_shifts<BN, NT>(E, n0, N, K / 32, equads, t, hs, ls);
    wait_lds();
    ring_barrier();
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const uint32_t r = min(nw + j * 16 + r16, N - 1) - n0;
      s0[j] = shift_of(hs[r], ls[r]);
    }
  }

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};

  // Software-pipelined steps: the operands of step j+1 are read from LDS (into the other register set)
  // before the MFMAs of step j, so that the LDS reads of one step run under the MFMAs of the other
  // (every operand of a step read at once: read one at a time before its MFMA, each read's latency
  // showed). Step j: wait for this wave's LDS reads of step j (in registers: buffer j % RS is free)
  // and its loads of step j+1, a barrier (every wave's loads of step j+1 have landed, every wave is
  // done with buffer j % RS), the reads of step j+1, the loads of step j+RS into buffer j % RS, then
  // the MFMAs of step j, each kk's weights converted next to the MFMAs that take them.
  struct Ops {
    u32x4 ax[KKG][TM];
    u32x4 wv[TN][C::BL];  // int8: the wave's codes of the step
    u32x2 wd[TN];         // MXFP4: the k group's dwords of block q (KG 2) or the first two (KG 1)
    u32x2 wd2[TN];        // MXFP4 KG 1: the last two
    uint32_t eb[TN];      // MXFP4: the block scale bytes of the step (4 a dword)
  };
  auto read_ops = [&](Ops &o, int b) __attribute__((always_inline)) {
    const u32x4 *xb = xr[b], *wb = wr[b];
#pragma unroll
    for (int jn = 0; jn < TN; jn++) {
      const int col = wn * (BN / WN) + jn * 16 + r16;
      if constexpr (MX) {
        const int slot = col * R::WCH + (q ^ ((col / R::CPB) & (R::WCH - 1)));
        if constexpr (KG == 1) {
          const u32x4 v = wb[slot];
          o.wd[jn] = (u32x2){v[0], v[1]};
          o.wd2[jn] = (u32x2){v[2], v[3]};
        } else {
          o.wd[jn] = *((const u32x2 *)&wb[slot] + g);
        }
        o.eb[jn] = er[b][col];
      } else {
#pragma unroll
        for (int h = 0; h < C::BL; h++) {
          const int c = (KG == 1 ? h : g) * 4 + q;
          o.wv[jn][h] = wb[col * R::WCH + (c ^ ((col / R::CPB) & (R::WCH - 1)))];
        }
      }
    }
#pragma unroll
    for (int kk = 0; kk < KKG; kk++)
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int row = wm * (BM / WM) + i * 16 + r16;
        const int ch = KG == 1 ? xchunk<MX>(q, kk) : xchunk<MX>(q, g * KKG + kk);
        o.ax[kk][i] = xb[row * CH + (ch ^ (row & 15))];
      }
  };
  auto mfma_ops = [&](const Ops &o) __attribute__((always_inline)) {
    float sc[TN];
    if constexpr (MX) {
#pragma unroll
      for (int jn = 0; jn < TN; jn++) sc[jn] = shifted_scale((o.eb[jn] >> (8 * q)) & 255u, s0[jn]);
    }
    auto bops = [&](half8 (&bf)[TN], int kk) __attribute__((always_inline)) {
#pragma unroll
      for (int jn = 0; jn < TN; jn++) {
        if constexpr (MX) {
          const uint32_t w = KG == 1 ? (kk < 2 ? o.wd[jn][kk] : o.wd2[jn][kk - 2]) : o.wd[jn][kk];
          bf[jn] = fp4x8_to_half8(w, sc[jn]);
        } else {
          const u32x4 v = o.wv[jn][kk >> 1];
          bf[jn] = i8x8_to_half8(v[(kk & 1) * 2], v[(kk & 1) * 2 + 1]);
        }
      }
    };
    half8 bf[2][TN];
    bops(bf[0], 0);
#pragma unroll
    for (int kk = 0; kk < KKG; kk++) {
      if (kk + 1 < KKG) bops(bf[(kk + 1) & 1], kk + 1);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int jn = 0; jn < TN; jn++)
          acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, o.ax[kk][i]), bf[kk & 1][jn],
                                                              acc[i][jn], 0, 0, 0);
    }
  };
  Ops P[2];
  wait_loads<(RS - 2) * LS>();  // step 0 (this wave's loads)
  ring_barrier();
  issue_order();
  src.load(xr[RS - 1], wr[RS - 1], er[RS - 1], (RS - 1) * KS, wave);
  issue_order();
  read_ops(P[0], 0);
  for (uint32_t j0 = 0; j0 < steps; j0 += 2 * RS) {
#pragma unroll
    for (int s = 0; s < 2 * RS; s++) {
      const uint32_t j = j0 + s;
      if (j >= steps) break;
      wait_lds();  // this wave's reads of step j (on both paths: the MFMAs below then wait for nothing)
      if (j + 1 < steps) {
        wait_loads<(RS - 2) * LS>();
        ring_barrier();
        issue_order();
        read_ops(P[(s + 1) & 1], (s + 1) % RS);
        issue_order();
        src.load(xr[s % RS], wr[s % RS], er[s % RS], (j + RS) * KS, wave);
        issue_order();
      }
      mfma_ops(P[s & 1]);
    }
  }
  wait_loads<0>();  // no load into LDS may land after the workgroup ends
  if constexpr (KG == 2) {
    // group 1's accumulators to group 0 through the X buffers, summed in group 0, which writes the
    // tile (BM x BN fp32: 2 buffers hold BM x 128)
    static_assert(BM * BN * 4 <= 2 * BM * CH * 16, "the k groups' sum goes through two X buffers");
    constexpr int HALF = BM * CH;  // float4 slots a buffer
    wait_lds();
    ring_barrier();
    if (g == 1) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          const int r = ((wl * TM + i) * TN + j) * 64;  // wave-uniform
          floatx4 *d = r < HALF ? (floatx4 *)xr[0] + r : (floatx4 *)xr[1] + (r - HALF);
          d[lane] = acc[i][j];
        }
    }
    wait_lds();
    ring_barrier();
    if (g == 0) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          const int r = ((wl * TM + i) * TN + j) * 64;
          const floatx4 *d = r < HALF ? (const floatx4 *)xr[0] + r : (const floatx4 *)xr[1] + (r - HALF);
          acc[i][j] += d[lane];
        }
    }
    wait_lds();
    ring_barrier();  // group 0 is done with the sums' buffers, which its stores reuse
    if (g == 1) return;
  }
  // staged stores where the waves' blocks fit the X buffers (a wave's block in region wl, PER regions
  // a buffer), else straight from the accumulators
  using G = StageRows<TM, TN, TN * 16 + 4>;
  constexpr int PER = BM * CH * 4 / G::FLOATS;
  if constexpr (PER >= 1 && (WM * WN + PER - 1) / PER <= RS) {
    if (staged(Y, N, mode)) {
      if constexpr (KG == 1) {
        wait_lds();
        ring_barrier();  // every wave is done with the ring's buffers
      }
      store_tile_staged<BM, WM, TM, TN, MX, TN * 16 + 4>(acc, s0, S, Y, M, N, m0, nw, wm, lane, mode,
                                                         (float *)xr[wl / PER] + (wl % PER) * G::FLOATS);
      return;
    }
  }
  store_tile<BM, WM, TM, TN, MX>(acc, s0, S, Y, M, N, m0, nw, wm, r16, q, mode);
}

}  // namespace hwk_gemm
