/*
 * hwk.h - libhwk, the MI355X (gfx950) kernel library behind hwnpu's backend API.
 *
 * A C ABI in the style of hwnpu's XRT shim (reference native/xrtshim/xrtshim.h:1-113) so that Go
 * without cgo binds it through purego (reference internal/dl/dl.go:23-64,
 * internal/backend/amdxrt/shim.go:47-80):
 *   - every call that can fail returns NULL on success, or a malloc'd message that the caller
 *     frees with hwk_free_error;
 *   - objects are opaque and freed by their *_free;
 *   - arguments are integers and pointers only: no float scalars (they travel as uint32 bit
 *     patterns) and no structs by value (reference docs/design/architecture.md:145-152);
 *   - no callbacks.
 *
 * Device memory is plain device pointers (`const void *` / `void *`); a stream is a hipStream_t
 * passed as `void *` (NULL: the null stream). Every op is asynchronous on its stream. There is
 * no CPU fallback: an op this library cannot run on the GPU returns an error.
 */
#ifndef HWNPU_HWK_H
#define HWNPU_HWK_H

#include <stddef.h>
#include <stdint.h>

#define HWK_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* The ABI version: a binding refuses a library of another (reference xrtshim.h:25-26, the XS_ABI
 * check of internal/backend/amdxrt/shim.go:25-26). */
#define HWK_ABI 4

typedef struct hwk_device hwk_device;
typedef struct hwk_buf hwk_buf;
typedef struct hwk_module hwk_module;
typedef struct hwk_run hwk_run;

/* Buffer kinds of hwk_buf_alloc (reference internal/types BufferKind): a device allocation with a
 * pinned host mirror synced explicitly (hwnpu Buffer.Bytes/SyncToDevice/SyncFromDevice), or a
 * device allocation alone. */
enum { HWK_BUF_MIRRORED = 0, HWK_BUF_DEVICE = 1 };

/* Directions of hwk_buf_sync. */
enum { HWK_SYNC_TO_DEVICE = 0, HWK_SYNC_FROM_DEVICE = 1 };

/* Keys of hwk_device_info. */
enum { HWK_INFO_NAME = 0, HWK_INFO_ARCH = 1, HWK_INFO_PCI_BUS = 2, HWK_INFO_CUS = 3, HWK_INFO_MEM_BYTES = 4 };

/* Event states of hwk_event_wait. */
enum { HWK_STATE_DONE = 0, HWK_STATE_PENDING = 1 };

/* Output modes of the GEMV/GEMM ops: fp32 or fp16 (RNE of the fp32 accumulator), or the fp32
 * result added into y (y += W x), for a residual stream. HWK_OUT_SWIGLU_F16 (the GEMMs only): y is
 * (m, n/2) fp16 with y[:, c] = fp16(silu(g) * u) of the fp32 result's column pairs (g, u) = (2c, 2c+1),
 * silu as hwk_silu_mul's (internal/llm/blocks/blocks.go:395-401), n a multiple of 16: a gate/up
 * projection with interleaved rows and its SwiGLU in one launch. */
enum { HWK_OUT_F32 = 0, HWK_OUT_F16 = 1, HWK_OUT_ADD_F32 = 2, HWK_OUT_SWIGLU_F16 = 3 };

HWK_API int hwk_abi(void);
HWK_API void hwk_free_error(char *err);

/* ---- devices (reference Provider.Enumerate/Open, internal/backend/backend.go:13-19) ---- */
HWK_API char *hwk_device_count(uint32_t *count);
/* Fails unless the device is gfx950: the code objects in this library are built for it alone. */
HWK_API char *hwk_device_open(uint32_t index, hwk_device **out);
HWK_API void hwk_device_free(hwk_device *d);
/* The device's value for key (an HWK_INFO_* string: name, gfx arch, PCI bus id, CU count, memory
 * bytes), copied into buf (n bytes, always terminated when n > 0); *need receives the bytes the whole
 * string takes, its terminating zero included, so a caller can size buf and ask again. */
HWK_API char *hwk_device_info(hwk_device *d, int key, char *buf, size_t n, size_t *need);
HWK_API char *hwk_device_synchronize(hwk_device *d);

/* ---- buffers (reference Device.AllocBuffer, Buffer, backend.go:54-67) ---- */
HWK_API char *hwk_buf_alloc(hwk_device *d, size_t size, int kind, hwk_buf **out);
HWK_API void hwk_buf_free(hwk_buf *b);
/* The pinned host mirror (NULL for HWK_BUF_DEVICE) and the device address. */
HWK_API void *hwk_buf_host_ptr(hwk_buf *b);
HWK_API void *hwk_buf_dev_ptr(hwk_buf *b);
HWK_API size_t hwk_buf_size(hwk_buf *b);
/* Copies n bytes from byte off between the mirror and the device, synchronously. */
HWK_API char *hwk_buf_sync(hwk_buf *b, int dir, size_t off, size_t n);

/* ---- streams and events (reference Run.Submit -> Fence.Wait/Done, graph.go:144-150) ---- */
HWK_API char *hwk_stream_new(hwk_device *d, void **stream);
HWK_API void hwk_stream_free(void *stream);
HWK_API char *hwk_stream_sync(void *stream);
HWK_API char *hwk_event_new(hwk_device *d, void **event);
HWK_API void hwk_event_free(void *event);
HWK_API char *hwk_event_record(void *event, void *stream);
/* Waits up to timeout_ms (0: poll once) and writes HWK_STATE_DONE or HWK_STATE_PENDING. */
HWK_API char *hwk_event_wait(void *event, uint32_t timeout_ms, int *state);
/* The time between two recorded events, in nanoseconds. */
HWK_API char *hwk_event_elapsed_ns(void *start, void *end, uint64_t *ns);

/* ---- code objects (reference KernelDevice.LoadProgram, Program.Kernels/NewRun, Run, Fence;
 * internal/backend/backend.go:27-46, internal/types/kernel.go:22-36, kernel.go:109-254) ----
 * A gfx950 code object (an ELF, or a clang offload bundle holding one) loaded with hipModuleLoadData.
 * Its kernels and their arguments are read from the object's AMDGPU metadata; the launch geometry of
 * each kernel from the object's own manifest (the `hwk_co_manifest` constant array: workgroup size,
 * and grid.x as a function of one 4-byte argument), so that no call takes grid or block sizes. The
 * library's own code object is lib/hwk_gfx950.hsaco: the batch-1 MXFP4 GEMV, the split-K decode
 * attention and its merge, the int8 and MXFP4 prefill GEMMs, the MoE route, gate_up and down, and a
 * streaming read (the same device code as the entry points below). */

/* A kernel of a loaded module (reference types.KernelInfo). */
typedef struct hwk_kernel_info {
  char name[64];
  uint32_t args;          /* explicit arguments (hidden ones are the runtime's) */
  uint32_t kernarg_bytes; /* bytes the explicit arguments span */
  uint32_t block;         /* threads a workgroup (the manifest's); 0 without a manifest entry */
  uint32_t max_block;     /* the kernel's largest workgroup (its launch bounds) */
  uint32_t lds_bytes;     /* LDS a workgroup: static (metadata) + dynamic (manifest) */
  uint32_t cus;           /* compute units of the module's device; 0 for an inspection-only module */
  uint32_t runnable;      /* 1 when the manifest gives the kernel's launch geometry */
  uint32_t reserved;
} hwk_kernel_info;

/* An explicit argument of a kernel (reference types.KernelArg). */
typedef struct hwk_kernel_arg {
  uint32_t index;  /* position in the kernel's signature */
  uint32_t offset; /* byte offset in the argument buffer */
  uint32_t size;   /* bytes */
  uint32_t buffer; /* 1: a device address, set with hwk_run_set_buffer*; 0: a value, hwk_run_set_arg */
  uint32_t nullable; /* a buffer argument the kernel accepts as null (hwk_run_set_null), per the manifest */
  char name[64];
  char type[32];   /* "void *" for a buffer, else "uint8_t", "uint16_t", "uint32_t", "uint64_t" or "bytes" */
} hwk_kernel_arg;

/* Loads a code object on device d; with d NULL the module only lists its kernels (no HIP call). */
HWK_API char *hwk_module_load(hwk_device *d, const void *image, size_t n, hwk_module **out);
HWK_API void hwk_module_free(hwk_module *m);
HWK_API char *hwk_module_kernel_count(hwk_module *m, uint32_t *count);
HWK_API char *hwk_module_kernel_info(hwk_module *m, uint32_t kernel, hwk_kernel_info *out);
HWK_API char *hwk_module_kernel_arg(hwk_module *m, uint32_t kernel, uint32_t arg, hwk_kernel_arg *out);
/* An invocation of a kernel; arguments start zeroed (reference Kernel.NewRun). */
HWK_API char *hwk_run_new(hwk_module *m, const char *kernel, hwk_run **out);
/* A value argument from its little-endian bytes: an unknown index, a buffer argument or a size other
 * than the argument's is an error (reference internal/backend/amd/device.go:349-363). The first
 * setter error is kept: hwk_run_err returns it and hwk_run_submit refuses (kernel.go:135-199). */
HWK_API char *hwk_run_set_arg(hwk_run *r, uint32_t index, const void *value, size_t n);
/* A buffer argument: the device address of b (plus off), b allocated on the module's device; a
 * value argument or a range past the buffer is an error (device.go:367-394). */
HWK_API char *hwk_run_set_buffer(hwk_run *r, uint32_t index, hwk_buf *b);
HWK_API char *hwk_run_set_buffer_at(hwk_run *r, uint32_t index, hwk_buf *b, size_t off, size_t n);
/* A buffer argument the kernel's manifest marks as optional set to the null address (an absent bias,
 * say); any other argument is an error. No counterpart in the reference, whose NPU kernels take no
 * optional buffers: a code object's kernels here do (the MoE biases, the router bias). A buffer
 * argument left unset refuses hwk_run_submit. */
HWK_API char *hwk_run_set_null(hwk_run *r, uint32_t index);
/* The first error a setter recorded (a copy), or NULL. */
HWK_API char *hwk_run_err(hwk_run *r);
/* Launches on the stream with the manifest's geometry. An error while the run's previous
 * submission is still running (device.go:396-401). Sync input buffers to the device first. */
HWK_API char *hwk_run_submit(hwk_run *r, void *stream);
/* The run's fence: waits up to timeout_ms (0: poll once) and writes HWK_STATE_DONE or
 * HWK_STATE_PENDING; the submission keeps running when the wait gives up (graph.go:144-150). */
HWK_API char *hwk_run_wait(hwk_run *r, uint32_t timeout_ms, int *state);
/* Waits for a running submission, then releases the run (reference Run.Close). */
HWK_API char *hwk_run_free(hwk_run *r);

/* ---- MXFP4 weights: rows of k values, blocks of 32; codes (rows, k/32, 16) bytes with the even
 * value in the low nibble, e8m0 scales (rows, k/32) (reference internal/mxfp4/mxfp4.go:1-20,
 * internal/llm/experts/host.go:21-27). ---- */

/* Dequantize into fp16 (rows, k): RNE(Values[code] * 2^(e-127)) with e=0 giving 0 and e=255
 * Inf (replaces reference mxfp4.Dequantize, internal/mxfp4/mxfp4.go:120-128). */
HWK_API char *hwk_mxfp4_dequant_f16(void *stream, const void *w, const void *e, void *out,
                                    uint32_t rows, uint32_t k);
/* K1: y (n) = W (n, k) x (k), x fp16, fp32 accumulation; y per out_mode (replaces the MXFP4
 * GEMV of reference internal/mxfp4/matvec.go:33-160 with mxfp4.go:80-117, and milcpu's
 * dequantize + linear, internal/milcpu/ops.go:940-956). k a multiple of 32; w 16-byte aligned. */
HWK_API char *hwk_mxfp4_gemv(void *stream, const void *w, const void *e, const void *x, void *y,
                             uint32_t n, uint32_t k, int out_mode);

/* K1r: Y (tokens, n) = X (tokens, k) W^T for tokens <= 8 fp16 vectors (tokens * k * 2 <= 64 KB), every
 * weight row read once for all of them (replaces mxfp4.Run serving several vectors from one read of
 * a row, reference internal/mxfp4/matvec.go:33-160; speculative verify, internal/llm/decode/decode.go:
 * 1235-1261). Y per out_mode, row t at y + t*n. */
HWK_API char *hwk_mxfp4_gemv_rows(void *stream, const void *w, const void *e, const void *x, void *y,
                                  uint32_t n, uint32_t k, uint32_t tokens, int out_mode);

/* ---- int8 per-output-channel weights: codes (n, k) int8 row-major, scales (n) fp16
 * (reference internal/milcpu/ops.go:1589-1610 constexpr_blockwise_shift_scale, the
 * mlpackage.Int8Scaled layout internal/mlpackage/program.go:421-461). ---- */

/* K2: y (n) = scale * (Q (n, k) x (k)), x fp16, fp32 accumulation (replaces shiftScale +
 * sgemm of reference internal/milcpu/ops.go:940-956 at one row). k a multiple of 16. */
HWK_API char *hwk_i8_gemv(void *stream, const void *q, const void *scale16, const void *x,
                          void *y, uint32_t n, uint32_t k, int out_mode);

/* ---- K3: prefill and verify GEMM, Y (m, n) = X (m, k) W^T, X fp16 row-major, fp32 accumulation on
 * the fp16 MFMA, the weights dequantized to fp16 in LDS; Y per out_mode (fp32, fp16 = RNE of the
 * fp32 accumulator, or added into fp32 Y). k a multiple of 32. ---- */

/* int8 W (n, k) with fp16 per-row scales (replaces milcpu's shiftScale + linear,
 * internal/milcpu/ops.go:940-956,1589-1610, over a whole prompt). */
HWK_API char *hwk_i8_gemm(void *stream, const void *x, const void *q, const void *scale16, void *y, uint32_t m,
                          uint32_t n, uint32_t k, int out_mode);
/* MXFP4 W (n, k): codes (n, k/32, 16), scales (n, k/32) (replaces mxfp4.Dequantize + sgemm,
 * internal/mxfp4/mxfp4.go:120-128 with internal/sgemm/sgemm.go:127-163). The block scale is folded
 * into the fp16 dequantization; a row whose finite block exponents leave [-23, 13] is shifted by a
 * power of two and scaled back in fp32, exact while its exponents span at most 36. */
HWK_API char *hwk_mxfp4_gemm(void *stream, const void *x, const void *w, const void *e, void *y, uint32_t m,
                             uint32_t n, uint32_t k, int out_mode);

/* ---- fp16 weights (reference internal/llm/blocks/blocks.go:135-184, format "fp16") ---- */

/* K7: y (n) = W (n, k) x (k), W and x fp16, fp32 accumulation: the tied head (reference
 * internal/llm/qwen3/build.go:107-109). k a multiple of 8. */
HWK_API char *hwk_f16_gemv(void *stream, const void *w, const void *x, void *y, uint32_t n,
                           uint32_t k, int out_mode);
/* K7r: Y (T, n) = X (T, k) W^T for fp16 W (n, k) and T <= 8 fp16 vectors, each row of W read once
 * for all of them: the tied head over the rows of a speculative verify (the head of
 * internal/llm/qwen3/build.go:107-109 on every row, as decode.Session.Speculate asks for the logits
 * after each token, internal/llm/decode/decode.go:1235-1261). k a multiple of 8, T*k*2 <= 64 KB. */
HWK_API char *hwk_f16_gemv_rows(void *stream, const void *w, const void *x, void *y, uint32_t n,
                                uint32_t k, uint32_t tokens, int out_mode);

/* ---- the decoder's small ops (K6): what the reference's graph runs between the linears
 * (internal/llm/blocks/blocks.go, internal/llm/qwen3/build.go:107-311). Float scalars travel as
 * float64 bit patterns. ---- */

/* RoPE tables of positions start .. start+n-1, on the HOST: cos_out/sin_out (n, head_dim/2) float32
 * of float64 cos/sin of p * theta^(-2j/head_dim) (reference internal/llm/qwen3/config.go:152-159,
 * blocks.go:412-425: the cat(freqs, freqs) table stored once). Touches no device. */
HWK_API char *hwk_rope_tables(uint64_t theta_bits, uint32_t start, uint32_t n, uint32_t head_dim,
                              float *cos_out, float *sin_out);
/* out (rows, n) = (x * r) * w, r = float(1/sqrt(mean(x^2) + eps)) with the sum in float64; x, w fp32,
 * out fp16 or fp32 (reference blocks.go:351-395, RMSNormWith). */
HWK_API char *hwk_rmsnorm(void *stream, const void *x, const void *w, void *out, uint32_t rows, uint32_t n,
                          uint64_t eps_bits, int out_mode);
/* x (tokens, heads, 128) fp32: each head's RMSNorm with norm_w (128) when norm_w is not NULL (Qwen3's
 * q/k norm before RoPE), then RoPE at position pos0 + token with rotate_half over tables from
 * hwk_rope_tables (device copies of table_rows rows); out fp16 or fp32 (reference blocks.go:427-445,
 * ApplyRope). */
HWK_API char *hwk_rope(void *stream, const void *x, const void *norm_w, const void *cos_t, const void *sin_t,
                       void *out, uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t pos0,
                       uint32_t table_rows, uint64_t eps_bits, int out_mode);
/* Copies k, v (tokens, kv_heads, head_dim) fp16 into rows pos0 .. pos0+tokens-1 of the caches
 * (kv_heads, capacity, head_dim) (reference decode.go:1668, writeRows); k and v may be NULL when
 * tokens is 0. */
HWK_API char *hwk_kv_append(void *stream, const void *k, const void *v, void *k_cache, void *v_cache,
                            uint32_t tokens, uint32_t kv_heads, uint32_t head_dim, uint32_t capacity,
                            uint32_t pos0);
/* out[i] = g / (1 + float(exp(-g))) * u, exp in float64, g = gate[i*stride], u = up[i*stride], fp32
 * in, fp16 or fp32 out (reference blocks.go:395-401 SiLU, SwiGLU; interleaved gate/up rows: gate =
 * base, up = base + 1, stride 2). */
HWK_API char *hwk_silu_mul(void *stream, const void *gate, const void *up, void *out, uint64_t n,
                           uint32_t stride, int out_mode);
/* y[i] += x[i], fp32 (the residual add). */
HWK_API char *hwk_add(void *stream, void *y, const void *x, uint64_t n);
/* out (tokens, hidden) fp32 = rows ids[t] (int32, device) of the fp16 table (vocab, hidden); a row
 * whose id is outside [0, vocab) is NaN (reference qwen3 build.go embedding gather). */
HWK_API char *hwk_embed(void *stream, const void *table, const void *ids, void *out, uint32_t tokens,
                        uint32_t hidden, uint32_t vocab);
/* Greedy pick a row: out[r] (int32, device) = the lowest index of the largest of x (rows, n) fp32, NaNs
 * never chosen except a NaN at index 0, which is kept (strict >, reference internal/chat/sample.go:
 * 80-87). Two launches over a workspace of hwk_argmax_workspace_bytes(rows). */
HWK_API size_t hwk_argmax_workspace_bytes(uint32_t rows);
HWK_API char *hwk_argmax(void *stream, const void *x, void *out, uint32_t rows, uint64_t n, void *workspace,
                         size_t workspace_bytes);

/* ---- decode attention (K4): one query token per head over a KV cache, split over the context
 * and merged as Flash-Decoding does (reference internal/llm/paged/paged.go:70-310, the per-chunk
 * program and Merge, driven by internal/llm/decode/decode.go:1435-1483). ---- */
typedef struct hwk_attn_params {
  uint32_t heads;      /* query heads (a multiple of kv_heads; heads/kv_heads in {1, 2, 4}) */
  uint32_t kv_heads;   /* KV heads */
  uint32_t head_dim;   /* 128 */
  uint32_t len;        /* keys in use, positions 0 .. len-1 (all visible to the query) */
  uint32_t capacity;   /* positions a head's cache holds: K[h] at k + h*capacity*head_dim */
  uint32_t kv_int8;    /* 0: fp16 K/V; 1: int8 K/V with an fp16 scale per (kv head, position) */
  uint32_t scale_bits; /* the score scale as float32 bits (1/sqrt(head_dim) for the models here) */
  uint32_t out_mode;   /* HWK_OUT_F32 or HWK_OUT_F16 */
  uint32_t split;      /* keys a split takes (a multiple of 64), 0 for the library's choice */
} hwk_attn_params;

/* Bytes of device workspace hwk_attn_decode needs for these parameters (the chunks' partial
 * outputs; no initial contents needed). Calls that overlap on one workspace race. */
HWK_API size_t hwk_attn_workspace_bytes(const hwk_attn_params *p);
/* out (heads, head_dim) = softmax(q k^T * scale) v per head, head h on kv head h/(heads/kv_heads)
 * (GQA, reference internal/llm/blocks/blocks.go:516-540). q fp16 (heads, head_dim). fp16 caches:
 * k, v (kv_heads, capacity, head_dim); int8 caches: the same in int8 with k_scale, v_scale fp16
 * (kv_heads, capacity), value = code * scale (reference internal/probe/kv.go:147-156). Returns an
 * error for an unsupported shape; there is no CPU path. */
HWK_API char *hwk_attn_decode(void *stream, const void *q, const void *k, const void *v, const void *k_scale,
                              const void *v_scale, void *out, void *workspace, size_t workspace_bytes,
                              const hwk_attn_params *p);
/* hwk_attn_decode without a workspace, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart in
 * the reference. The split-K partials go to a scratch array the library keeps in each device's
 * memory (HWK_ATTN_SCRATCH_BYTES, held until the process ends); parameters whose
 * hwk_attn_workspace_bytes exceed it are refused with an error. It allocates nothing. Every call on
 * one device shares that device's scratch: calls that overlap on one device (two streams, or two
 * threads) race. Results equal hwk_attn_decode's bit for bit. */
#define HWK_ATTN_SCRATCH_BYTES (4u << 20)
HWK_API char *hwk_attn_decode_noalloc(void *stream, const void *q, const void *k, const void *v,
                                      const void *k_scale, const void *v_scale, void *out,
                                      const hwk_attn_params *p);
/* The int8 KV rule, per row of head_dim values (one kv head at one position): scale =
 * fp16(absmax/127) (1 for a row of zeros), codes = RoundToEven(value/scale) clamped to +-127
 * (reference internal/llm/experts/weights.go:229-252 with internal/vecops/vecops.go:179-185).
 * x fp16 (rows, head_dim); q int8 (rows, head_dim); scale fp16 (rows). */
HWK_API char *hwk_kv_quantize_i8(void *stream, const void *x, void *q, void *scale, uint32_t rows,
                                 uint32_t head_dim);
/* Causal attention of a prompt: tokens query rows at positions start .. start+tokens-1, q fp16
 * (tokens, heads, head_dim), each seeing the keys at or before its own position in fp16 caches k,
 * v (kv_heads, capacity, head_dim) that already hold them; p->len = start + tokens. out (tokens,
 * heads, head_dim) per p->out_mode (replaces the prompt form of the reference's chunk program with
 * its causal mask, internal/llm/paged/paged.go:70-203 at tokens > 1, as decode.Session.Step runs a
 * prompt through it, internal/llm/decode/decode.go:1391-1483). */
HWK_API char *hwk_attn_prefill(void *stream, const void *q, const void *k, const void *v, void *out,
                               uint32_t tokens, uint32_t start, const hwk_attn_params *p);
/* Merge chunk outputs as the reference's Merge does (paged.go:227-310): o (chunks, rows, dim)
 * fp32, each chunk normalized over its own keys, m and l (chunks, rows) fp32 (a chunk whose l is
 * not positive is skipped); out (rows, dim) per out_mode, zero for a row no chunk saw. */
HWK_API char *hwk_attn_merge(void *stream, const void *o, const void *m, const void *l, void *out,
                             uint32_t chunks, uint32_t rows, uint32_t dim, int out_mode);

/* ---- MoE (K5) ---- */

/* Score functions of hwk_moe_route. */
enum { HWK_SCORE_SOFTMAX = 0, HWK_SCORE_SIGMOID = 1 };

/* K5a: per row of router logits (rows, experts) fp32 (experts <= 64), the k experts of the
 * largest scores and their weights, as the reference's Routing.Choose computes them
 * (internal/llm/experts/weights.go:33-81): softmax scores in float32 with exp in float64, or
 * sigmoid; a stable descending order (ties to the lower index); with norm the chosen scores over
 * their float32 sum plus 1e-6; times scale (float32 bits) unless 0. bias (experts) fp32 or NULL
 * moves the choice, not the weights. idx int32 (rows, k); w fp32 (rows, k). */
HWK_API char *hwk_moe_route(void *stream, const void *logits, const void *bias, void *idx, void *w, uint32_t rows,
                            uint32_t experts, uint32_t k, int score, int norm, uint32_t scale_bits);

/* Gated units of the experts (reference internal/llm/experts/host.go:44-57). */
enum { HWK_ACT_SILU = 0, HWK_ACT_GPTOSS = 1 };

typedef struct hwk_moe_params {
  uint32_t tokens;     /* rows of x (1..8) */
  uint32_t hidden;     /* H, a multiple of 32, at most 8192 */
  uint32_t inter;      /* I, a multiple of 32, at most 8192 */
  uint32_t experts;    /* E (<= 64) */
  uint32_t k;          /* experts a token (tokens * k <= 64) */
  uint32_t out_mode;   /* HWK_OUT_F32 (out = the experts' sum) or HWK_OUT_ADD_F32 (out += it) */
  uint32_t act;        /* HWK_ACT_SILU: silu(g)*u; HWK_ACT_GPTOSS: g = min(g, limit),
                        * u = clamp(u, -limit, limit), g*sigmoid(alpha*g)*(u+1) (host.go:516-527) */
  uint32_t alpha_bits; /* float32 bits of alpha (gpt-oss 1.702) */
  uint32_t limit_bits; /* float32 bits of limit (gpt-oss 7) */
  uint32_t score;      /* hwk_moe_layer's routing: HWK_SCORE_SOFTMAX or HWK_SCORE_SIGMOID */
  uint32_t norm;       /* hwk_moe_layer's routing: 1 to normalize the chosen weights */
  uint32_t scale_bits; /* hwk_moe_layer's routing: float32 bits of the weights' scale (0: none) */
} hwk_moe_params;

/* Device workspace of hwk_moe_experts / hwk_moe_layer: the gated activations, fp32 (tokens*k, I). */
HWK_API size_t hwk_moe_workspace_bytes(const hwk_moe_params *p);
/* K5b: the chosen experts of each token (reference experts.Host.Run / runRow, host.go:478-579,
 * 723-882): gate_up MXFP4 (E, 2I, H/32, 16) codes + (E, 2I, H/32) scales with the gate on the even
 * rows, plus the bias gu_b fp32 (E, 2I) (NULL: none); act = the gated unit of (gate, up) in fp32;
 * down MXFP4 (E, H, I/32, 16) + (E, H, I/32); out[t] (+)= sum over its experts in ascending expert
 * id of w * (down act + dn_b) with dn_b fp32 (E, H) (NULL: none). An expert's rows are read once for
 * all the tokens that chose it. Two launches. x fp16 (tokens, H); idx int32 and w fp32 (tokens, k)
 * as hwk_moe_route writes them; out fp32 (tokens, H). */
HWK_API char *hwk_moe_experts(void *stream, const void *x, const void *idx, const void *w, const void *gu_w,
                              const void *gu_e, const void *gu_b, const void *dn_w, const void *dn_e,
                              const void *dn_b, void *out, void *workspace, size_t workspace_bytes,
                              const hwk_moe_params *p);
/* The MoE layer as chain.moe.runHost runs it (internal/llm/chain/moe.go:582-610): Routing.Choose of
 * the router logits fp32 (tokens, E) with router_bias (E) or NULL, per p's score, norm and scale
 * (as hwk_moe_route), then hwk_moe_experts, in two launches: the route is folded into the gate_up
 * launch. idx and w (tokens, k) are written for the caller. */
HWK_API char *hwk_moe_layer(void *stream, const void *x, const void *logits, const void *router_bias, void *idx,
                            void *w, const void *gu_w, const void *gu_e, const void *gu_b, const void *dn_w,
                            const void *dn_e, const void *dn_b, void *out, void *workspace,
                            size_t workspace_bytes, const hwk_moe_params *p);

/* ---- the Qwen3 decoder on the device (the shape of reference internal/llm/qwen3, build.go:107-311,
 * driven the way internal/llm/iron/model.go:578 Step(token, pos) -> logits drives a device-resident
 * model). Weights, KV cache, token history and position live on the device; a decode step is one
 * captured HIP graph that reads its token and position on the device and writes the greedy next
 * token there, so that steps replay without the host. ---- */
typedef struct hwk_qwen3 hwk_qwen3;

typedef struct hwk_qwen3_config {
  uint32_t layers;       /* 28 */
  uint32_t hidden;       /* 2048: a multiple of 32, at most 8192 */
  uint32_t heads;        /* 16 query heads */
  uint32_t kv_heads;     /* 8 (heads/kv_heads in {1, 2, 4}) */
  uint32_t head_dim;     /* 128 only */
  uint32_t inter;        /* 6144: the SwiGLU width, a multiple of 32, at most 8192 */
  uint32_t vocab;        /* 151936: rows of the tied fp16 embedding / head */
  uint32_t max_ctx;      /* positions the KV cache holds */
  uint32_t max_prompt;   /* rows a prefill call takes at once (longer prompts go in pieces) */
  uint32_t pad;
  uint64_t theta_bits;   /* RoPE theta as float64 bits (1e6) */
  uint64_t eps_bits;     /* RMSNorm epsilon as float64 bits (1e-6) */
} hwk_qwen3_config;

/* Allocates the model on the current device (weights uninitialized). */
HWK_API char *hwk_qwen3_new(const hwk_qwen3_config *cfg, hwk_qwen3 **out);
HWK_API void hwk_qwen3_free(hwk_qwen3 *m);
/* Fills every weight with the synthetic checkpoint: each linear N(0, std) drawn under its Hugging
 * Face name (model.layers.{i}.self_attn.q_proj.weight, ...) and encoded to MXFP4, the embedding
 * fp16(N(0, std)) under model.embed_tokens.weight, every norm weight 1. std as float32 bits. */
HWK_API char *hwk_qwen3_synth(hwk_qwen3 *m, void *stream, uint64_t seed, uint32_t std_bits);
/* A weight's device memory by its name in this layout, for a loader:
 *   layers.{i}.qkv.blocks/.scales      MXFP4 (q, k, v rows stacked: heads*hd + 2*kv_heads*hd, hidden)
 *   layers.{i}.o.blocks/.scales        MXFP4 (hidden, heads*hd)
 *   layers.{i}.gate_up.blocks/.scales  MXFP4 (2*inter, hidden), gate row j at 2j, up row j at 2j+1
 *   layers.{i}.down.blocks/.scales     MXFP4 (hidden, inter)
 *   layers.{i}.input_norm, .post_norm  fp32 (hidden); layers.{i}.q_norm, .k_norm fp32 (head_dim)
 *   norm fp32 (hidden); embed fp16 (vocab, hidden)
 *   layers.{i}.k_cache, .v_cache       fp16 (kv_heads, max_ctx, head_dim)
 * blocks are (rows, cols/32, 16) bytes, scales (rows, cols/32) e8m0. */
HWK_API char *hwk_qwen3_tensor(hwk_qwen3 *m, const char *name, void **ptr, size_t *bytes);
/* The device state: logits fp32 (vocab) of the last processed row; the token history int32
 * (max_ctx + 1), hist[p] the token at position p; pos int32, the position the next step takes. */
HWK_API char *hwk_qwen3_state(hwk_qwen3 *m, void **logits, void **hist, void **pos);
/* Runs a prompt of n host token ids at positions start .. start+n-1 (KV written there), then the
 * head on its last row: logits, and the greedy next token into hist[start+n]; pos = start+n.
 * Synchronous on the host for the token copy, asynchronous for the compute. */
HWK_API char *hwk_qwen3_prefill(hwk_qwen3 *m, void *stream, const int32_t *tokens, uint32_t n, uint32_t start);
/* One decode step, eagerly: the token hist[pos] at position pos -> logits, hist[pos+1] = the
 * greedy token (strict >, ties to the lowest id, reference internal/chat/sample.go:80-87), pos+1. */
HWK_API char *hwk_qwen3_step(hwk_qwen3 *m, void *stream);
/* steps decode steps as replays of the captured step graphs (one of 8 steps, one of 1 step;
 * each captured on its first use unless hwk_qwen3_capture captured it before). */
HWK_API char *hwk_qwen3_decode(hwk_qwen3 *m, void *stream, uint32_t steps);
/* Captures and instantiates both step graphs now, without running them, so that a later
 * hwk_qwen3_decode only replays (no capture inside a caller's timed region). */
HWK_API char *hwk_qwen3_capture(hwk_qwen3 *m);

/* ---- the session's cache and position (reference decode.Session, internal/llm/decode/
 * decode.go:1107-1210, 1849-1968; the prompt store's rows, internal/chat/store.go) ---- */

/* Bytes of one position's rows in hwk_qwen3_export_rows: K and V of every layer, kv_heads x
 * head_dim fp16 each (RowBytes, decode.go:1849-1855). */
HWK_API char *hwk_qwen3_row_bytes(hwk_qwen3 *m, size_t *bytes);
/* Packs the cache rows of positions [from, to) into dst (device memory, (to-from) x row_bytes):
 * per position, the caches in the order of their reference names kv_k_N_new / kv_v_N_new sorted as
 * strings (kv_k_0, kv_k_1, kv_k_10, ...; decode.go:484), each kv_heads rows of head_dim fp16
 * (ExportRows, decode.go:1857-1881). to <= max_ctx. */
HWK_API char *hwk_qwen3_export_rows(hwk_qwen3 *m, void *stream, uint32_t from, uint32_t to, void *dst);
/* Writes rows packed as export_rows packs them (bytes a multiple of row_bytes, device memory) at
 * positions from on; the position does not move (ImportRows, decode.go:1883-1914). */
HWK_API char *hwk_qwen3_import_rows(hwk_qwen3 *m, void *stream, uint32_t from, const void *src,
                                   size_t bytes);
/* The position the next step takes: a mark of the sequence (Mark, decode.go:1120-1137; the model
 * has no rings or windows, so a mark is its position). */
HWK_API char *hwk_qwen3_position(hwk_qwen3 *m, uint32_t *pos);
/* Moves the sequence to position pos (< max_ctx - 1): the next step takes hist[pos] at pos, and
 * next_token >= 0 is first written there. Back to a mark (Rewind, decode.go:1190-1203: the rows
 * before pos must be those of the mark), or, after import_rows, to the end of imported rows
 * (Resume, decode.go:1930-1968). */
HWK_API char *hwk_qwen3_rewind(hwk_qwen3 *m, void *stream, uint32_t pos, int32_t next_token);
/* Speculative verify (Speculate, decode.go:1235-1261; ironSession.SpeculateTokens,
 * internal/chat/iron.go:169): runs n host tokens (1..8, at most max_prompt; the first is the
 * token the next step would take, the rest drafts) at positions pos .. pos+n-1, writing their K/V,
 * and gives the logits after each row (*logits: fp32 (n, vocab)) and each row's greedy token
 * (*argmax: int32 (n)), device memory valid until the next verify. The position does not move
 * until hwk_qwen3_keep. */
HWK_API char *hwk_qwen3_verify(hwk_qwen3 *m, void *stream, const int32_t *tokens, uint32_t n,
                               void **logits, void **argmax);
/* Keeps the first kept (1..n) rows of the last verify: pos moves past them, hist[pos] = the greedy
 * token of row kept-1 and the state's logits are that row's. The K/V of the rows not kept are
 * never read: the steps after write each position before they attend to it. */
HWK_API char *hwk_qwen3_keep(hwk_qwen3 *m, void *stream, uint32_t kept);

/* ---- synthetic inputs, reproducible from (seed, name) alone: splitmix64 counter streams keyed
 * by seed ^ fnv64a(name) (the role of reference internal/llm/synth.go:12-56). Each element i
 * reads draw i (normals: draws 2i/2i+1 of pair i/2 through Box-Muller in float64). ---- */

/* n bytes, each the low byte of its draw */
HWK_API char *hwk_synth_bytes(void *stream, void *out, uint64_t n, uint64_t key);
/* n ints uniform in [lo, lo+span) (multiply-high of the draw's top 32 bits), stored as bytes
 * (elem_size 1) or int32 (elem_size 4) */
HWK_API char *hwk_synth_uniform(void *stream, void *out, uint64_t n, uint64_t key, int32_t lo,
                                uint32_t span, int elem_size);
/* n normals N(0, std) as fp16 (f64 -> f32 -> f16, RNE) or fp32; std as float32 bits */
HWK_API char *hwk_synth_normal(void *stream, void *out, uint64_t n, uint64_t key,
                               uint32_t std_bits, int out_f16);
/* rows x k normals N(0, std) encoded to MXFP4 as the reference's Encode does (least-error scale
 * among OCP's rule and its neighbours, nearest code, ties to even; reference
 * internal/mxfp4/encode.go:11-78), never materialized in fp32. */
HWK_API char *hwk_synth_mxfp4(void *stream, void *w, void *e, uint32_t rows, uint32_t k,
                              uint64_t key, uint32_t std_bits);
/* The reference's own synthetic checkpoint values (llm.Synthetic.Get, internal/llm/synth.go:17-35):
 * n values of the tensor called name (a NUL-terminated string), seeded by FNV-64a(name) and
 * stepped by the MMIX LCG, uniform in [-0.2, 0.2) (the code's range; its comment says +-0.1),
 * as fp32 or fp16 (RNE of the fp32 value). */
HWK_API char *hwk_synth_reference(void *stream, void *out, uint64_t n, const char *name, int out_f16);
/* Encode an fp32 matrix (rows, k) to MXFP4 (reference internal/mxfp4/encode.go:11-78). */
HWK_API char *hwk_mxfp4_encode(void *stream, const void *x, void *w, void *e, uint32_t rows,
                               uint32_t k);

/* ---- measurement (no counterpart in the reference) ---- */

/* The read floor: one launch that reads bytes (a multiple of 16, 16-byte aligned) from src once in
 * 16-byte loads and computes nothing, with waves_per_cu (1..32) waves a CU each holding
 * loads_per_lane (1, 2, 4 or 8) loads in flight; *out (device) is written only for data that
 * practically never occurs. Its time is the shortest in which a single launch streams that many
 * bytes, the bound for the batch-1 GEMV (K1) of the same bytes. */
HWK_API char *hwk_read_floor(void *stream, const void *src, size_t bytes, uint32_t *out,
                             uint32_t waves_per_cu, uint32_t loads_per_lane);

#ifdef __cplusplus
}
#endif

#endif
