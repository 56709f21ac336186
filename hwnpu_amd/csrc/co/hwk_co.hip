// The gfx950 code object libhwk's runtime calls load (hwk_module_load): kernels with C names and a
// launch manifest, built with `hipcc --genco` into lib/hwk_gfx950.hsaco. Each kernel runs the same
// device code as the library's entry point it names (mxfp4_gemv.h, attn_kernels.h, gemm_kernels.h,
// moe_kernels.h); the caller sets every argument by index and the grid follows from the argument the
// manifest names. A kernel whose shape arguments are outside what it is built for writes NaN to its
// outputs (rows, tiles) instead of a wrong value. It holds
//   hwk_co_mxfp4_gemv        K1, the batch-1 MXFP4 GEMV (hwk_mxfp4_gemv for rows of up to 64
//                            blocks): y fp16 (n) = W (n, nb*32) x
//   hwk_co_stream_read       a read of n16 16-byte chunks, one a lane, nothing written unless the
//                            data's XOR hits a fixed value: the time one launch takes to stream a buffer
//   hwk_co_attn_decode_f16_g1/g2/g4, hwk_co_attn_decode_i8_g4
//                            K4, the split-K GQA decode attention (hwk_attn_decode) with G query heads
//                            a kv head, fp16 or int8 KV: one workgroup a (kv head, chunk), 4 waves of
//                            kpw keys; partials (o | m | l, slots = heads * nchunk) or, with one chunk,
//                            the output itself
//   hwk_co_attn_merge        the merge of those partials (up to 64 chunks): one wave a (query head,
//                            16 dims)
//   hwk_co_i8_gemm, hwk_co_mxfp4_gemm
//                            K3, the prefill GEMM (hwk_i8_gemm / hwk_mxfp4_gemm) in 128 x 128 tiles
//   hwk_co_moe_route, hwk_co_moe_gate_up, hwk_co_moe_down
//                            K5a routing (hwk_moe_route) and K5b's two stages (hwk_moe_experts) for
//                            hidden <= 2048 and intermediate <= 768
#include "../attn_kernels.h"
#include "../co_manifest.h"
#include "../gemm_kernels.h"
#include "../moe_kernels.h"
#include "../mxfp4_gemv.h"

extern "C" {

// Argument indices the grids follow (see each kernel's signature).
__attribute__((used)) __constant__ hwk_co_geometry hwk_co_manifest[12] = {
    // 8 waves of 2 rows: grid.x = ceil(n / 16), n is argument 4
    {"hwk_co_mxfp4_gemv", 512, 4, 16, 0, 0, 0, {0, 0}},
    // a lane a chunk: grid.x = ceil(n16 / 256), n16 is argument 1
    {"hwk_co_stream_read", 256, 1, 256, 0, 0, 0, {0, 0}},
    // a workgroup a (kv head, chunk): grid.x = groups (argument 7) = kv_heads * nchunk
    {"hwk_co_attn_decode_f16_g1", 256, 7, 1, 0, 0, 0, {0, 0}},
    {"hwk_co_attn_decode_f16_g2", 256, 7, 1, 0, 0, 0, {0, 0}},
    {"hwk_co_attn_decode_f16_g4", 256, 7, 1, 0, 0, 0, {0, 0}},
    // int8 caches: two scale arrays more, groups is argument 9
    {"hwk_co_attn_decode_i8_g4", 256, 9, 1, 0, 0, 0, {0, 0}},
    // a wave a (query head, 16 dims): grid.x = groups (argument 4) = heads * 8
    {"hwk_co_attn_merge", 64, 4, 1, 0, 0, 0, {0, 0}},
    // a workgroup a 128 x 128 tile: grid.x = tiles (argument 8) = ceil(m / 128) * ceil(n / 128)
    {"hwk_co_i8_gemm", 256, 8, 1, 0, 0, 0, {0, 0}},
    {"hwk_co_mxfp4_gemm", 256, 8, 1, 0, 0, 0, {0, 0}},
    // a wave a row: grid.x = ceil(rows / 4), rows is argument 4
    {"hwk_co_moe_route", 256, 4, 4, 0, 0, 1u << 1, {0, 0}},  // bias may be null
    // a workgroup a (8 row pairs, chosen expert): grid.x = groups (argument 14) = ceil(inter / 8) *
    // min(tokens * k, experts)
    {"hwk_co_moe_gate_up", 256, 14, 1, 0, 0, 1u << 4, {0, 0}},  // gb may be null
    // a workgroup of 8 waves a tile of 8 output rows: grid.x = ceil(hidden / 8), hidden is argument 8
    {"hwk_co_moe_down", 512, 8, 8, 0, 0, 1u << 5, {0, 0}},  // db may be null
};
__attribute__((used)) __constant__ uint32_t hwk_co_manifest_count = 12;

__global__ __launch_bounds__(512) void hwk_co_mxfp4_gemv(const uint4 *__restrict__ w, const uint8_t *__restrict__ e,
                                                         const uint4 *__restrict__ x, f16 *__restrict__ y, uint32_t n,
                                                         uint32_t nb) {
  if (n == 0) return;        // nothing to read (the runtime launches no grid for n = 0)
  if (nb == 0 || nb > 64) {  // uniform: the whole grid takes this branch
    const uint32_t r = blockIdx.x * 16 + threadIdx.x;
    if (threadIdx.x < 16 && r < n) y[r] = (f16)__builtin_nanf("");
    return;
  }
  mxfp4_gemv_lds<8, 2, 1, HWK_OUT_F16>(w, e, x, y, n, nb);
}

__global__ __launch_bounds__(256) void hwk_co_stream_read(const uint4 *__restrict__ p, uint32_t n16,
                                                          uint32_t *__restrict__ sink) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (n16 == 0) return;
  const uint4 v = load_stream(&p[min(i, n16 - 1)]);
  const uint32_t a = v.x ^ v.y ^ v.z ^ v.w;
  if (a == 0x9e3779b9u && i < n16) sink[blockIdx.x] = a;
}

}  // extern "C"

namespace {

// The decode attention's shape checks: 4 waves of kpw keys (a multiple of 16) a chunk, the chunks
// covering len <= cap keys. A bad shape writes NaN to the workgroup's kv head's G output rows.
template <int G>
__device__ __forceinline__ bool attn_shape_ok(void *out, int mode, uint32_t kv_heads, uint32_t len, uint32_t cap,
                                              uint32_t chunk, uint32_t nchunk, uint32_t kpw) {
  const bool ok = kv_heads > 0 && kpw >= 16 && kpw % 16 == 0 && chunk == 4 * kpw && nchunk >= 1 && len <= cap &&
                  (uint64_t)chunk * nchunk >= len && (mode == HWK_OUT_F32 || mode == HWK_OUT_F16);
  if (!ok && blockIdx.x < kv_heads && (mode == HWK_OUT_F32 || mode == HWK_OUT_F16))
    for (uint32_t i = threadIdx.x; i < (uint32_t)G * 128; i += 256)
      store_out(out, (size_t)blockIdx.x * G * 128 + i, __builtin_nanf(""), mode);
  return ok;
}

template <int G>
__device__ __forceinline__ void co_attn_f16(const f16 *q, const void *k, const void *v, float *ws_o, float *ws_m,
                                            float *ws_l, void *out, uint32_t kv_heads, uint32_t mode, uint32_t len,
                                            uint32_t cap, uint32_t chunk, uint32_t nchunk, uint32_t kpw,
                                            uint32_t scale_bits) {
  if (!attn_shape_ok<G>(out, (int)mode, kv_heads, len, cap, chunk, nchunk, kpw)) return;
  if (blockIdx.x >= kv_heads * nchunk) return;
  hwk_attn::attn_decode_wg<G, false, 4>(blockIdx.x, q, k, v, nullptr, nullptr, ws_o, ws_m, ws_l, out, (int)mode,
                                        nullptr, len, cap, chunk, nchunk, kpw,
                                        __uint_as_float(scale_bits) * hwk_attn::kLog2e);
}


template <bool MX>
__device__ __forceinline__ void co_gemm(const uint32_t *X, const uint8_t *W, const uint8_t *E, const uint16_t *S,
                                        void *Y, uint32_t m, uint32_t n, uint32_t k, uint32_t mode) {
  const uint32_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
  if (blockIdx.x >= tiles) return;
  const bool ok = k > 0 && k % 32 == 0 && mode <= HWK_OUT_SWIGLU_F16 && (mode != HWK_OUT_SWIGLU_F16 || n % 16 == 0);
  if (!ok) {
    if (mode > HWK_OUT_ADD_F32) return;  // no defined output layout to mark
    uint32_t tm, tn;
    hwk_gemm::tile_of(blockIdx.x, (m + 127) / 128, (n + 127) / 128, tm, tn);
    for (uint32_t i = threadIdx.x; i < 128 * 128; i += 256) {
      const uint32_t r = tm * 128 + i / 128, c = tn * 128 + i % 128;
      if (r < m && c < n) store_out(Y, (size_t)r * n + c, __builtin_nanf(""), mode == HWK_OUT_F16 ? mode : HWK_OUT_F32);
    }
    return;
  }
  const bool equads = MX && (k / 32) % 16 == 0 && ((uintptr_t)E & 15) == 0;
  hwk_gemm::gemm_wg<128, 128, MX, 2, 2>(blockIdx.x, (const u32x4 *)X, W, E, S, Y, m, n, k, (int)mode, equads);
}

__device__ __forceinline__ hwk_moe::MoeArgs moe_args(uint32_t T, uint32_t H, uint32_t I, uint32_t E, uint32_t k,
                                                     uint32_t act, uint32_t alpha_bits, uint32_t limit_bits,
                                                     uint32_t mode) {
  hwk_moe::MoeArgs a;
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.k = k;
  a.act = (int)act;
  a.score = HWK_SCORE_SOFTMAX;
  a.norm = 1;
  a.alpha = __uint_as_float(alpha_bits);
  a.limit = __uint_as_float(limit_bits);
  a.scale = 0.0f;
  a.mode = (int)mode;
  return a;
}

// The MoE kernels' shapes: 1..8 tokens, experts <= 64, k <= experts, tokens*k <= 64, hidden a multiple
// of 32 up to 2048, inter a multiple of 32 up to 768.
__device__ __forceinline__ bool moe_shape_ok(uint32_t T, uint32_t H, uint32_t I, uint32_t E, uint32_t k) {
  return T >= 1 && T <= 8 && E >= 1 && E <= 64 && k >= 1 && k <= E && T * k <= 64 && H % 32 == 0 && H > 0 &&
         H <= 2048 && I % 32 == 0 && I > 0 && I <= 768;
}
}  // namespace

extern "C" {

// q fp16 (kv_heads * G, 128); k, v fp16 (kv_heads, cap, 128); ws_o (slots, 128), ws_m, ws_l (slots)
// float with slots = kv_heads * G * nchunk; out (kv_heads * G, 128) fp16 or fp32 per mode, written
// here when nchunk is 1 (else by hwk_co_attn_merge); the keys [0, len); scale_bits the float bits of
// the score scale.
#define HWK_CO_ATTN(GG)                                                                                             \
  __global__ __launch_bounds__(256) void hwk_co_attn_decode_f16_g##GG(                                            \
      const f16 *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v, float *__restrict__ ws_o, \
      float *__restrict__ ws_m, float *__restrict__ ws_l, void *__restrict__ out, uint32_t groups,                 \
      uint32_t kv_heads, uint32_t mode, uint32_t len, uint32_t cap, uint32_t chunk, uint32_t nchunk, uint32_t kpw, \
      uint32_t scale_bits) {                                                                                      \
    (void)groups;                                                                                                 \
    co_attn_f16<GG>(q, k, v, ws_o, ws_m, ws_l, out, kv_heads, mode, len, cap, chunk, nchunk, kpw, scale_bits);    \
  }
HWK_CO_ATTN(1)
HWK_CO_ATTN(2)
HWK_CO_ATTN(4)
#undef HWK_CO_ATTN

// The int8 form: k, v int8 (kv_heads, cap, 128) with fp16 scales ks, vs (kv_heads, cap).
__global__ __launch_bounds__(256) void hwk_co_attn_decode_i8_g4(const f16 *__restrict__ q, const void *__restrict__ k,
                                                                const void *__restrict__ v,
                                                                const uint16_t *__restrict__ ks,
                                                                const uint16_t *__restrict__ vs,
                                                                float *__restrict__ ws_o, float *__restrict__ ws_m,
                                                                float *__restrict__ ws_l, void *__restrict__ out,
                                                                uint32_t groups, uint32_t kv_heads, uint32_t mode,
                                                                uint32_t len, uint32_t cap, uint32_t chunk,
                                                                uint32_t nchunk, uint32_t kpw, uint32_t scale_bits) {
  (void)groups;
  if (!attn_shape_ok<4>(out, (int)mode, kv_heads, len, cap, chunk, nchunk, kpw)) return;
  if (blockIdx.x >= kv_heads * nchunk) return;
  hwk_attn::attn_decode_wg<4, true, 4>(blockIdx.x, q, k, v, ks, vs, ws_o, ws_m, ws_l, out, (int)mode, nullptr, len,
                                       cap, chunk, nchunk, kpw, __uint_as_float(scale_bits) * hwk_attn::kLog2e);
}

// The partials' merge (the reference's Merge rule): out (heads, 128) from o, m, l of chunks <= 64
// chunks a query head, G query heads a kv head; groups = heads * 8.
__global__ __launch_bounds__(64) void hwk_co_attn_merge(const float *__restrict__ o, const float *__restrict__ m,
                                                        const float *__restrict__ l, void *__restrict__ out,
                                                        uint32_t groups, uint32_t chunks, uint32_t G, uint32_t mode) {
  const uint32_t row = blockIdx.x / 8, slice = blockIdx.x % 8;
  if (blockIdx.x >= groups || (mode != HWK_OUT_F32 && mode != HWK_OUT_F16)) return;
  if (chunks == 0 || chunks > 64 || G == 0) {
    if (threadIdx.x < 16) store_out(out, (size_t)row * 128 + slice * 16 + threadIdx.x, __builtin_nanf(""), (int)mode);
    return;
  }
  hwk_attn::attn_merge_wave_wg<16>(row, slice, o, m, l, out, chunks, G, (int)mode);
}


// Y (m, n) = X (m, k) W^T: X fp16, W int8 (n, k) with fp16 row scales s (hwk_i8_gemm), or MXFP4
// codes (n, k/32, 16) with E8M0 scales e (hwk_mxfp4_gemm); mode HWK_OUT_F32 / F16 / ADD_F32 /
// SWIGLU_F16; tiles = ceil(m / 128) * ceil(n / 128). k must be a positive multiple of 32 (and n of 16
// for SwiGLU): otherwise the tile is NaN.
__global__ __launch_bounds__(256) void hwk_co_i8_gemm(const uint32_t *__restrict__ x, const uint8_t *__restrict__ w,
                                                      const uint16_t *__restrict__ s, void *__restrict__ y, uint32_t m,
                                                      uint32_t n, uint32_t k, uint32_t mode, uint32_t tiles) {
  (void)tiles;
  co_gemm<false>(x, w, nullptr, s, y, m, n, k, mode);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void hwk_co_mxfp4_gemm(
    const uint32_t *__restrict__ x, const uint8_t *__restrict__ w, const uint8_t *__restrict__ e, void *__restrict__ y,
    uint32_t m, uint32_t n, uint32_t k, uint32_t mode, uint32_t tiles) {
  (void)tiles;
  co_gemm<true>(x, w, e, nullptr, y, m, n, k, mode);
}

// Routing.Choose of rows of experts <= 64 fp32 logits (softmax, or sigmoid plus an optional bias),
// top k: idx (rows, k) int32, w (rows, k) fp32, scale_bits the float bits of a weight scale (0: none).
__global__ __launch_bounds__(256) void hwk_co_moe_route(const float *__restrict__ logits, const float *__restrict__ bias,
                                                        int32_t *__restrict__ idx, float *__restrict__ w, uint32_t rows,
                                                        uint32_t experts, uint32_t k, uint32_t score, uint32_t norm,
                                                        uint32_t scale_bits) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  if (experts == 0 || experts > 64 || k == 0 || k > experts || score > HWK_SCORE_SIGMOID) {
    if ((threadIdx.x & 63) < k && k <= 64) {
      idx[(size_t)row * k + (threadIdx.x & 63)] = -1;
      w[(size_t)row * k + (threadIdx.x & 63)] = __builtin_nanf("");
    }
    return;
  }
  hwk_moe::choose_wave(logits + (size_t)row * experts, bias, experts, k, (int)score, (int)norm,
                       __uint_as_float(scale_bits), idx + (size_t)row * k, w + (size_t)row * k);
}


// The chosen experts' gate_up (rows interleaved gate 2j, up 2j+1: (E, 2I, H/32, 16) codes, (E, 2I, H/32)
// scales, optional fp32 biases (E, 2I)) against x fp16 (T, H) for idx (T, k): act (T, k, I) fp32 the
// gated unit (act HWK_ACT_SILU, or HWK_ACT_GPTOSS with alpha, limit). A bad shape makes act NaN.
__global__ __launch_bounds__(256) void hwk_co_moe_gate_up(const uint4 *__restrict__ x, const int32_t *__restrict__ idx,
                                                          const uint4 *__restrict__ gw, const uint8_t *__restrict__ ge,
                                                          const float *__restrict__ gb, float *__restrict__ act,
                                                          uint32_t T, uint32_t H, uint32_t I, uint32_t E, uint32_t k,
                                                          uint32_t act_kind, uint32_t alpha_bits, uint32_t limit_bits,
                                                          uint32_t groups) {
  (void)groups;
  if (!moe_shape_ok(T, H, I, E, k) || act_kind > HWK_ACT_GPTOSS) {
    if (blockIdx.x == 0 && T >= 1 && T <= 8 && k >= 1 && k <= 64 && I <= 8192)
      for (uint32_t i = threadIdx.x; i < T * k * I; i += 256) act[i] = __builtin_nanf("");
    return;
  }
  const uint32_t gx = (I + 7) / 8;
  hwk_moe::moe_gate_up_wg<1, 2, false>(blockIdx.x % gx, blockIdx.x / gx, x, nullptr, nullptr, const_cast<int32_t *>(idx),
                                       nullptr, gw, ge, gb, act, moe_args(T, H, I, E, k, act_kind, alpha_bits, limit_bits, 0));
}

// down (E, H, I/32, 16) codes, (E, H, I/32) scales, optional fp32 biases (E, H), of act (T, k, I):
// out (T, H) fp32 = (mode HWK_OUT_ADD_F32: out +) the sum over each token's experts in ascending id
// of w * (y + bias).
__global__ __launch_bounds__(512) void hwk_co_moe_down(const float *__restrict__ act, const int32_t *__restrict__ idx,
                                                       const float *__restrict__ w, const uint4 *__restrict__ dw,
                                                       const uint8_t *__restrict__ de, const float *__restrict__ db,
                                                       float *__restrict__ out, uint32_t T, uint32_t H, uint32_t I,
                                                       uint32_t E, uint32_t k, uint32_t mode) {
  if (!moe_shape_ok(T, H, I, E, k) || (mode != HWK_OUT_F32 && mode != HWK_OUT_ADD_F32)) {
    const uint32_t r = blockIdx.x * 8 + (threadIdx.x & 7), t = threadIdx.x >> 3;
    if (T <= 8 && t < T && r < H && H <= 8192) out[(size_t)t * H + r] = __builtin_nanf("");
    return;
  }
  hwk_moe::moe_down_wg<8, 3, 2, false, 8>(blockIdx.x, act, idx, w, dw, de, db, out,
                                          moe_args(T, H, I, E, k, HWK_ACT_SILU, 0, 0, mode));
}

}  // extern "C"
