// Shared by libhwk's sources: error strings, launch checks and the device helpers every kernel
// uses (fp16 pairs, e8m0 scales, wave reductions). gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/hwk.h"

typedef _Float16 f16;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

namespace hwk {

// A malloc'd message for the C ABI (freed by hwk_free_error).
static inline char *errf(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  char buf[512];
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  size_t n = strlen(buf) + 1;
  char *out = (char *)malloc(n);
  if (out) memcpy(out, buf, n);
  return out;
}

static inline char *hip_err(const char *what, hipError_t e) {
  return errf("%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
}

// The launch's own error, if any (hipGetLastError clears it).
static inline char *launched(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_err(what, e);
  return nullptr;
}

static inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

static inline float f32_of_bits(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

}  // namespace hwk

#define HWK_TRY(what, call)                          \
  do {                                               \
    hipError_t e_ = (call);                          \
    if (e_ != hipSuccess) return hwk::hip_err(what, e_); \
  } while (0)

#define HWK_CHECK(cond, ...)                 \
  do {                                       \
    if (!(cond)) return hwk::errf(__VA_ARGS__); \
  } while (0)

// ---- device helpers ----

// e8m0 scale 2^(e-127) as the float whose bits are e<<23: e=0 is +0 and e=255 is +Inf, as the
// reference's scale (internal/mxfp4/mxfp4.go:77).
__device__ __forceinline__ float e8m0_scale(uint32_t e) { return __uint_as_float(e << 23); }

__device__ __forceinline__ h2 h2_of_bits(uint32_t b) { return __builtin_bit_cast(h2, b); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A 16-byte load of data read once (weights streamed from HBM): marked non-temporal so that it
// does not displace what is reused in the caches.
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
  const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Two e2m1 codes of byte `sel` of w, as fp16 (low nibble in .x): exact, the hardware's fp4
// conversion at scale 1.
template <int SEL>
__device__ __forceinline__ h2 fp4x2_to_h2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, SEL);
}

// The two permlane swaps: v_permlane16_swap exchanges the odd rows (16 lanes) of its first operand
// with the even rows of its second, v_permlane32_swap the upper half of the first with the lower
// half of the second. On two copies of v, the two results hold v and its row (half) partner in every
// lane. Issued as inline asm after two wait states (the hazard the compiler inserts before them):
// the compiler builtin's second result is not usable (it is folded into the first).
__device__ __forceinline__ void swap_rows16(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_rows32(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Sum / max over the 4 row groups (l, l^16, l^32, l^48); every lane gets the result.
__device__ __forceinline__ float row_groups_sum(float v) {
  float a = v, b = v;
  swap_rows16(a, b);
  v = a + b;
  a = v;
  b = v;
  swap_rows32(a, b);
  return a + b;
}
__device__ __forceinline__ float row_groups_max(float v) {
  float a = v, b = v;
  swap_rows16(a, b);
  v = fmaxf(a, b);
  a = v;
  b = v;
  swap_rows32(a, b);
  return fmaxf(a, b);
}

// Sum / max of v over aligned groups of G lanes (G = 8, 16, 32 or 64) with no LDS round trip: quad
// swaps, the half-row and row mirrors (DPP), then the row-group swaps. Each step adds a lane and its
// partner, so every lane of a group ends with the same bits.
#define HWK_DPP_ALL(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), ctrl, 0xf, 0xf, false))
template <int G>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(G == 8 || G == 16 || G == 32 || G == 64, "groups of 8, 16, 32 or 64 lanes");
  v += HWK_DPP_ALL(v, 0xb1);   // quad_perm [1, 0, 3, 2]
  v += HWK_DPP_ALL(v, 0x4e);   // quad_perm [2, 3, 0, 1]
  v += HWK_DPP_ALL(v, 0x141);  // row_half_mirror
  if constexpr (G >= 16) v += HWK_DPP_ALL(v, 0x140);  // row_mirror
  if constexpr (G >= 32) {
    float a = v, b = v;
    swap_rows16(a, b);
    v = a + b;
  }
  if constexpr (G == 64) {
    float a = v, b = v;
    swap_rows32(a, b);
    v = a + b;
  }
  return v;
}
template <int G>
__device__ __forceinline__ float group_max_dpp(float v) {
  static_assert(G == 8 || G == 16 || G == 32 || G == 64, "groups of 8, 16, 32 or 64 lanes");
  v = fmaxf(v, HWK_DPP_ALL(v, 0xb1));
  v = fmaxf(v, HWK_DPP_ALL(v, 0x4e));
  v = fmaxf(v, HWK_DPP_ALL(v, 0x141));
  if constexpr (G >= 16) v = fmaxf(v, HWK_DPP_ALL(v, 0x140));
  if constexpr (G >= 32) {
    float a = v, b = v;
    swap_rows16(a, b);
    v = fmaxf(a, b);
  }
  if constexpr (G == 64) {
    float a = v, b = v;
    swap_rows32(a, b);
    v = fmaxf(a, b);
  }
  return v;
}

// The best (value, index) of the 64 lanes, in every lane: the larger value, on a tie the lower index
// (a NaN never replaces a pair and the pairs a thread's scan leaves hold none, so each step's choice
// between a lane's pair and its partner's is the same in both lanes), by DPP and permlane swaps.
__device__ __forceinline__ void best_of(float &bv, uint32_t &bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}
__device__ __forceinline__ void wave_best(float &bv, uint32_t &bi) {
#define HWK_BEST_STEP(ctrl) \
  best_of(bv, bi, HWK_DPP_ALL(bv, ctrl), __builtin_bit_cast(uint32_t, HWK_DPP_ALL(__builtin_bit_cast(float, bi), ctrl)))
  HWK_BEST_STEP(0xb1);   // quad_perm [1, 0, 3, 2]
  HWK_BEST_STEP(0x4e);   // quad_perm [2, 3, 0, 1]
  HWK_BEST_STEP(0x141);  // row_half_mirror
  HWK_BEST_STEP(0x140);  // row_mirror
#undef HWK_BEST_STEP
  {
    float va = bv, vb = bv, ia = __builtin_bit_cast(float, bi), ib = ia;
    swap_rows16(va, vb);  // (even row's, odd row's) of each row pair, in both rows
    swap_rows16(ia, ib);
    bv = va;
    bi = __builtin_bit_cast(uint32_t, ia);
    best_of(bv, bi, vb, __builtin_bit_cast(uint32_t, ib));
  }
  {
    float va = bv, vb = bv, ia = __builtin_bit_cast(float, bi), ib = ia;
    swap_rows32(va, vb);  // (lower half's, upper half's), in both halves
    swap_rows32(ia, ib);
    bv = va;
    bi = __builtin_bit_cast(uint32_t, ia);
    best_of(bv, bi, vb, __builtin_bit_cast(uint32_t, ib));
  }
}

// Sum of a value over groups of G lanes (G a power of two up to 64), every lane gets its group's: by
// DPP and permlane swaps from 8 lanes up, else by LDS shuffles.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 8) {
    return group_sum_dpp<G>(v);
  } else {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
  }
}

// Sum of a value over the 64 lanes by DPP row shifts and row broadcasts (no LDS traffic): lane 63
// ends with the total (the other lanes hold partial sums).
#define HWK_DPP_F32(v, ctrl, row_mask, bound_ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), ctrl, row_mask, 0xf, bound_ctrl))
__device__ __forceinline__ float wave_sum_to_63(float v) {
  v += HWK_DPP_F32(v, 0x111, 0xf, true);   // row_shr:1
  v += HWK_DPP_F32(v, 0x112, 0xf, true);   // row_shr:2
  v += HWK_DPP_F32(v, 0x114, 0xf, true);   // row_shr:4
  v += HWK_DPP_F32(v, 0x118, 0xf, true);   // row_shr:8: lane 15 of each row of 16 holds the row's sum
  v += HWK_DPP_F32(v, 0x142, 0xa, false);  // row_bcast:15 into rows 1 and 3
  v += HWK_DPP_F32(v, 0x143, 0xc, false);  // row_bcast:31 into rows 2 and 3
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// *p by a vector load (its index an opaque zero), for a value that later loads must not wait on: a
// scalar load shares its wait counter with LDS traffic and the kernel arguments' loads, so waits for
// those would wait for it too, while vector loads complete in issue order (a load issued first is
// waited for without waiting on the loads after it). readfirstlane of the result gives it as a scalar
// where it is used.
__device__ __forceinline__ int32_t load_first(const int32_t *p) {
  uint32_t z = 0;
  asm volatile("" : "+v"(z));
  return p[z];
}

// v as a float32 value of its own: instruction selection cannot see through the empty asm, so a
// conversion to fp16 that follows rounds this float32 (twice rounded, as the reference's fp16
// storage of a float32 result). Without it the backend folds a product and the conversion into
// one mixed-precision FMA that rounds the exact product to fp16 once.
__device__ __forceinline__ float f32_value(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// SwiGLU of one (gate, up) pair: silu(g) * u with silu(g) = g / (1 + float(exp(-g))), exp in float64,
// each step rounded to float32 on its own (the reference's SiLU, internal/llm/blocks/blocks.go:395-401).
__device__ __forceinline__ float swiglu_value(float g, float u) {
#pragma clang fp contract(off)
  return f32_value(g / (1.0f + (float)exp(-(double)g)) * u);
}

// A scheduling barrier: the instruction scheduler moves nothing across it, so loads written before
// it are issued before those written after it (no wait is implied: the wait counter still waits
// only where a value is used).
__device__ __forceinline__ void issue_order() { __builtin_amdgcn_sched_barrier(0); }

// Loads the named kernel arguments into SGPRs here, all in one batch with one wait: otherwise the
// compiler loads each argument where it is first used, and a load issued after an issue_order()
// fence waits for its argument with a round trip of its own before the global loads behind it issue.
template <typename T>
__device__ __forceinline__ int kernarg_one(const T &v) {
  asm volatile("" ::"s"(v));
  return 0;
}
template <typename... T>
__device__ __forceinline__ void kernarg_now(const T &...v) {
  const int d[] = {kernarg_one(v)...};
  (void)d;
}

// Store one GEMV/GEMM output per out_mode.
__device__ __forceinline__ void store_out(void *y, size_t i, float v, int mode) {
  if (mode == HWK_OUT_F16)
    ((f16 *)y)[i] = (f16)f32_value(v);
  else if (mode == HWK_OUT_ADD_F32)
    ((float *)y)[i] += v;
  else
    ((float *)y)[i] = v;
}
