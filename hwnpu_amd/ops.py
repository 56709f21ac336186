"""The hot-path ops on torch tensors, each a call through libhwk's C ABI.

torch supplies device memory and the stream (its current stream); every computation is one of
libhwk's HIP kernels. Shapes, dtypes and devices are checked here before any launch, so that a
kernel never sees operands that disagree with its grid. Nothing falls back to the CPU: without
libhwk or a GPU, every op raises.
"""
from __future__ import annotations

import struct

import torch

from . import hwk

OUT_MODES = {"f32": hwk.OUT_F32, "f16": hwk.OUT_F16, "add": hwk.OUT_ADD_F32, "swiglu": hwk.OUT_SWIGLU_F16}


def f32_bits(v: float) -> int:
    """A float32 scalar as the uint32 bit pattern the ABI takes."""
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need(t: torch.Tensor, name: str, dtype, shape=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: must be on the GPU (no CPU path)")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, want {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, want {tuple(shape)}")


def _out(y, n, mode, device):
    dt = torch.float16 if mode == "f16" else torch.float32
    if y is None:
        if mode == "add":
            raise ValueError("out_mode 'add' needs y")
        return torch.empty(n, dtype=dt, device=device)
    _need(y, "y", dt, (n,))
    return y


def mxfp4_dequant_f16(w: torch.Tensor, e: torch.Tensor) -> torch.Tensor:
    """fp16 (rows, k) of MXFP4 codes w (rows, k/2) and scales e (rows, k/32)."""
    rows, half = w.shape
    k = half * 2
    _need(w, "w", torch.uint8, (rows, half))
    _need(e, "e", torch.uint8, (rows, k // 32))
    out = torch.empty((rows, k), dtype=torch.float16, device=w.device)
    hwk.load().hwk_mxfp4_dequant_f16(_stream(), w.data_ptr(), e.data_ptr(), out.data_ptr(), rows, k)
    return out


def mxfp4_gemv(w, e, x, out_mode="f32", y=None):
    """y = W x for MXFP4 W (n, k): codes w (n, k/2), scales e (n, k/32); x fp16 (k)."""
    n, half = w.shape
    k = half * 2
    _need(w, "w", torch.uint8, (n, half))
    _need(e, "e", torch.uint8, (n, k // 32))
    _need(x, "x", torch.float16, (k,))
    y = _out(y, n, out_mode, w.device)
    hwk.load().hwk_mxfp4_gemv(_stream(), w.data_ptr(), e.data_ptr(), x.data_ptr(), y.data_ptr(), n, k,
                              OUT_MODES[out_mode])
    return y


def mxfp4_gemv_rows(w, e, x, out_mode="f32", y=None):
    """Y (T, n) = X W^T for MXFP4 W (n, k) and T <= 8 fp16 vectors X (T, k), W read once for all."""
    n, half = w.shape
    k = half * 2
    T = x.shape[0]
    _need(w, "w", torch.uint8, (n, half))
    _need(e, "e", torch.uint8, (n, k // 32))
    _need(x, "x", torch.float16, (T, k))
    y = _out2(y, T, n, out_mode, w.device)
    hwk.load().hwk_mxfp4_gemv_rows(_stream(), w.data_ptr(), e.data_ptr(), x.data_ptr(), y.data_ptr(), n, k, T,
                                   OUT_MODES[out_mode])
    return y


def i8_gemv(q, scale16, x, out_mode="f32", y=None):
    """y = scale * (Q x) for int8 Q (n, k) and fp16 per-row scales; x fp16 (k)."""
    n, k = q.shape
    _need(q, "q", torch.int8, (n, k))
    _need(scale16, "scale", torch.float16, (n,))
    _need(x, "x", torch.float16, (k,))
    y = _out(y, n, out_mode, q.device)
    hwk.load().hwk_i8_gemv(_stream(), q.data_ptr(), scale16.data_ptr(), x.data_ptr(), y.data_ptr(), n, k,
                           OUT_MODES[out_mode])
    return y


def f16_gemv(w, x, out_mode="f32", y=None):
    """y = W x for fp16 W (n, k) and x (k)."""
    n, k = w.shape
    _need(w, "w", torch.float16, (n, k))
    _need(x, "x", torch.float16, (k,))
    y = _out(y, n, out_mode, w.device)
    hwk.load().hwk_f16_gemv(_stream(), w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k, OUT_MODES[out_mode])
    return y


def f16_gemv_rows(w, x, out_mode="f32", y=None):
    """Y (T, n) = X W^T for fp16 W (n, k) and T <= 8 fp16 vectors X (T, k), W read once for all."""
    n, k = w.shape
    T = x.shape[0]
    _need(w, "w", torch.float16, (n, k))
    _need(x, "x", torch.float16, (T, k))
    y = _out2(y, T, n, out_mode, w.device)
    hwk.load().hwk_f16_gemv_rows(_stream(), w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k, T, OUT_MODES[out_mode])
    return y


def _out2(y, m, n, mode, device):
    dt = torch.float16 if mode in ("f16", "swiglu") else torch.float32
    if mode == "swiglu":
        n //= 2
    if y is None:
        if mode == "add":
            raise ValueError("out_mode 'add' needs y")
        return torch.empty((m, n), dtype=dt, device=device)
    _need(y, "y", dt, (m, n))
    return y


def i8_gemm(x, q, scale16, out_mode="f32", y=None):
    """Y (m, n) = X W^T for fp16 X (m, k) and int8 W (n, k) with fp16 per-row scales; out_mode "swiglu":
    Y (m, n/2) fp16, the SwiGLU of the column pairs."""
    m, k = x.shape
    n = q.shape[0]
    _need(x, "x", torch.float16, (m, k))
    _need(q, "q", torch.int8, (n, k))
    _need(scale16, "scale", torch.float16, (n,))
    y = _out2(y, m, n, out_mode, x.device)
    hwk.load().hwk_i8_gemm(_stream(), x.data_ptr(), q.data_ptr(), scale16.data_ptr(), y.data_ptr(), m, n, k,
                           OUT_MODES[out_mode])
    return y


def mxfp4_gemm(x, w, e, out_mode="f32", y=None):
    """Y (m, n) = X W^T for fp16 X (m, k) and MXFP4 W: codes w (n, k/2), scales e (n, k/32); out_mode
    "swiglu": Y (m, n/2) fp16, the SwiGLU of the column pairs."""
    m, k = x.shape
    n = w.shape[0]
    _need(x, "x", torch.float16, (m, k))
    _need(w, "w", torch.uint8, (n, k // 2))
    _need(e, "e", torch.uint8, (n, k // 32))
    y = _out2(y, m, n, out_mode, x.device)
    hwk.load().hwk_mxfp4_gemm(_stream(), x.data_ptr(), w.data_ptr(), e.data_ptr(), y.data_ptr(), m, n, k,
                              OUT_MODES[out_mode])
    return y


def mxfp4_encode(x: torch.Tensor):
    """MXFP4 codes (rows, k/2) and scales (rows, k/32) of fp32 x (rows, k)."""
    rows, k = x.shape
    _need(x, "x", torch.float32, (rows, k))
    w = torch.empty((rows, k // 2), dtype=torch.uint8, device=x.device)
    e = torch.empty((rows, k // 32), dtype=torch.uint8, device=x.device)
    hwk.load().hwk_mxfp4_encode(_stream(), x.data_ptr(), w.data_ptr(), e.data_ptr(), rows, k)
    return w, e


def attn_params(heads, kv_heads, length, capacity, kv_int8=False, scale=None, out_mode="f32", split=0,
                head_dim=128):
    p = hwk.AttnParams()
    p.heads, p.kv_heads, p.head_dim = heads, kv_heads, head_dim
    p.len, p.capacity, p.kv_int8 = length, capacity, 1 if kv_int8 else 0
    p.scale_bits = f32_bits(head_dim ** -0.5 if scale is None else scale)
    p.out_mode = OUT_MODES[out_mode]
    p.split = split
    return p


def attn_workspace(p) -> torch.Tensor:
    """A workspace for hwk_attn_decode with parameters p (reusable across calls in stream order)."""
    n = hwk.load().hwk_attn_workspace_bytes(p)
    return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")


def attn_decode(q, k, v, length, k_scale=None, v_scale=None, out_mode="f32", scale=None, split=0, out=None,
                workspace=None):
    """out (heads, d) for one query token per head over caches k, v (kv_heads, capacity, d): fp16, or
    int8 with fp16 scales (kv_heads, capacity)."""
    heads, d = q.shape
    kvh, cap, d2 = k.shape
    if d2 != d:
        raise ValueError("head_dim of q and k differ")
    i8 = k.dtype == torch.int8
    _need(q, "q", torch.float16, (heads, d))
    _need(k, "k", torch.int8 if i8 else torch.float16, (kvh, cap, d))
    _need(v, "v", torch.int8 if i8 else torch.float16, (kvh, cap, d))
    if i8:
        _need(k_scale, "k_scale", torch.float16, (kvh, cap))
        _need(v_scale, "v_scale", torch.float16, (kvh, cap))
    p = attn_params(heads, kvh, length, cap, i8, scale, out_mode, split, d)
    ws = attn_workspace(p) if workspace is None else workspace
    dt = torch.float16 if out_mode == "f16" else torch.float32
    if out is None:
        out = torch.empty((heads, d), dtype=dt, device=q.device)
    else:
        _need(out, "out", dt, (heads, d))
    hwk.load().hwk_attn_decode(_stream(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               k_scale.data_ptr() if i8 else None, v_scale.data_ptr() if i8 else None,
                               out.data_ptr(), ws.data_ptr(), ws.numel(), p)
    return out


def attn_decode_noalloc(q, k, v, length, k_scale=None, v_scale=None, out_mode="f32", scale=None, split=0, out=None):
    """attn_decode through hwk_attn_decode_noalloc: no workspace (the library's per-device scratch
    holds the partials), so that nothing is allocated when `out` is given."""
    heads, d = q.shape
    kvh, cap, d2 = k.shape
    if d2 != d:
        raise ValueError("head_dim of q and k differ")
    i8 = k.dtype == torch.int8
    _need(q, "q", torch.float16, (heads, d))
    _need(k, "k", torch.int8 if i8 else torch.float16, (kvh, cap, d))
    _need(v, "v", torch.int8 if i8 else torch.float16, (kvh, cap, d))
    if i8:
        _need(k_scale, "k_scale", torch.float16, (kvh, cap))
        _need(v_scale, "v_scale", torch.float16, (kvh, cap))
    p = attn_params(heads, kvh, length, cap, i8, scale, out_mode, split, d)
    dt = torch.float16 if out_mode == "f16" else torch.float32
    if out is None:
        out = torch.empty((heads, d), dtype=dt, device=q.device)
    else:
        _need(out, "out", dt, (heads, d))
    hwk.load().hwk_attn_decode_noalloc(_stream(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       k_scale.data_ptr() if i8 else None, v_scale.data_ptr() if i8 else None,
                                       out.data_ptr(), p)
    return out


def attn_prefill(q, k, v, start, out_mode="f32", scale=None, out=None):
    """Causal attention of tokens query rows q (tokens, heads, d) at positions start .. start+tokens-1
    over fp16 caches k, v (kv_heads, capacity, d) that hold their keys: out (tokens, heads, d)."""
    tokens, heads, d = q.shape
    kvh, cap, d2 = k.shape
    if d2 != d:
        raise ValueError("head_dim of q and k differ")
    _need(q, "q", torch.float16, (tokens, heads, d))
    _need(k, "k", torch.float16, (kvh, cap, d))
    _need(v, "v", torch.float16, (kvh, cap, d))
    p = attn_params(heads, kvh, start + tokens, cap, False, scale, out_mode, 0, d)
    dt = torch.float16 if out_mode == "f16" else torch.float32
    if out is None:
        out = torch.empty((tokens, heads, d), dtype=dt, device=q.device)
    else:
        _need(out, "out", dt, (tokens, heads, d))
    hwk.load().hwk_attn_prefill(_stream(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), tokens, start, p)
    return out


def kv_quantize_i8(x: torch.Tensor):
    """int8 codes and fp16 scales of fp16 rows x (..., d) by the int8 KV rule."""
    d = x.shape[-1]
    _need(x, "x", torch.float16)
    rows = x.numel() // d
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[:-1], dtype=torch.float16, device=x.device)
    hwk.load().hwk_kv_quantize_i8(_stream(), x.data_ptr(), q.data_ptr(), s.data_ptr(), rows, d)
    return q, s


def attn_merge(o, m, l, out_mode="f32"):
    """The reference's Merge over chunks: o (chunks, rows, dim), m and l (chunks, rows), fp32."""
    chunks, rows, dim = o.shape
    _need(o, "o", torch.float32, (chunks, rows, dim))
    _need(m, "m", torch.float32, (chunks, rows))
    _need(l, "l", torch.float32, (chunks, rows))
    out = torch.empty((rows, dim), dtype=torch.float16 if out_mode == "f16" else torch.float32, device=o.device)
    hwk.load().hwk_attn_merge(_stream(), o.data_ptr(), m.data_ptr(), l.data_ptr(), out.data_ptr(), chunks, rows,
                              dim, OUT_MODES[out_mode])
    return out


def moe_route(logits, k, score="softmax", norm=True, scale=0.0, bias=None):
    """idx int32 (rows, k) and w fp32 (rows, k) of router logits fp32 (rows, experts)."""
    rows, E = logits.shape
    _need(logits, "logits", torch.float32, (rows, E))
    if bias is not None:
        _need(bias, "bias", torch.float32, (E,))
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((rows, k), dtype=torch.float32, device=logits.device)
    hwk.load().hwk_moe_route(_stream(), logits.data_ptr(), None if bias is None else bias.data_ptr(), idx.data_ptr(),
                             w.data_ptr(), rows, E, k, hwk.SCORE_SOFTMAX if score == "softmax" else hwk.SCORE_SIGMOID,
                             1 if norm else 0, f32_bits(scale))
    return idx, w


def _moe_params(T, H, I, E, k, out_mode, act, alpha, limit, score="softmax", norm=True, scale=0.0):
    if act not in ("silu", "gptoss"):
        raise ValueError(f"act {act!r}: 'silu' or 'gptoss'")
    p = hwk.MoeParams()
    p.tokens, p.hidden, p.inter, p.experts, p.k = T, H, I, E, k
    p.out_mode = OUT_MODES[out_mode]
    p.act = hwk.ACT_SILU if act == "silu" else hwk.ACT_GPTOSS
    p.alpha_bits, p.limit_bits = f32_bits(alpha), f32_bits(limit)
    p.score = hwk.SCORE_SOFTMAX if score == "softmax" else hwk.SCORE_SIGMOID
    p.norm, p.scale_bits = 1 if norm else 0, f32_bits(scale)
    return p


def _moe_operands(x, gu_w, gu_e, dn_w, dn_e, gu_b, dn_b):
    T, H = x.shape
    E, I2 = gu_e.shape[0], gu_e.shape[1]
    I = I2 // 2
    _need(x, "x", torch.float16, (T, H))
    _need(gu_w, "gu_w", torch.uint8, (E, I2, H // 32, 16))
    _need(gu_e, "gu_e", torch.uint8, (E, I2, H // 32))
    _need(dn_w, "dn_w", torch.uint8, (E, H, I // 32, 16))
    _need(dn_e, "dn_e", torch.uint8, (E, H, I // 32))
    if gu_b is not None:
        _need(gu_b, "gu_b", torch.float32, (E, I2))
    if dn_b is not None:
        _need(dn_b, "dn_b", torch.float32, (E, H))
    return T, H, I, E


def _moe_out(out, out_mode, T, H, device):
    if out is None:
        if out_mode == "add":
            raise ValueError("out_mode 'add' needs out")
        return torch.empty((T, H), dtype=torch.float32, device=device)
    _need(out, "out", torch.float32, (T, H))
    return out


def _ptr(t):
    return None if t is None else t.data_ptr()


def moe_experts(x, idx, w, gu_w, gu_e, dn_w, dn_e, out=None, out_mode="f32", workspace=None, gu_b=None, dn_b=None,
                act="silu", alpha=1.702, limit=7.0):
    """The chosen experts' gated FFNs: x fp16 (T, H); gu_w uint8 (E, 2I, H/32, 16), gu_e (E, 2I, H/32);
    dn_w (E, H, I/32, 16), dn_e (E, H, I/32); optional fp32 biases gu_b (E, 2I), dn_b (E, H); act 'silu'
    or 'gptoss' (alpha, limit); out fp32 (T, H)."""
    T, H, I, E = _moe_operands(x, gu_w, gu_e, dn_w, dn_e, gu_b, dn_b)
    k = idx.shape[1]
    _need(idx, "idx", torch.int32, (T, k))
    _need(w, "w", torch.float32, (T, k))
    p = _moe_params(T, H, I, E, k, out_mode, act, alpha, limit)
    out = _moe_out(out, out_mode, T, H, x.device)
    n = hwk.load().hwk_moe_workspace_bytes(p)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=x.device) if workspace is None else workspace
    hwk.load().hwk_moe_experts(_stream(), x.data_ptr(), idx.data_ptr(), w.data_ptr(), gu_w.data_ptr(), gu_e.data_ptr(),
                               _ptr(gu_b), dn_w.data_ptr(), dn_e.data_ptr(), _ptr(dn_b), out.data_ptr(),
                               ws.data_ptr(), ws.numel(), p)
    return out


def moe_layer(x, logits, k, gu_w, gu_e, dn_w, dn_e, out=None, out_mode="f32", workspace=None, gu_b=None, dn_b=None,
              act="silu", alpha=1.702, limit=7.0, score="softmax", norm=True, scale=0.0, router_bias=None):
    """Route (Routing.Choose of fp32 logits (T, E)) and run the chosen experts in two launches;
    returns (out, idx, w)."""
    T, H, I, E = _moe_operands(x, gu_w, gu_e, dn_w, dn_e, gu_b, dn_b)
    _need(logits, "logits", torch.float32, (T, E))
    if router_bias is not None:
        _need(router_bias, "router_bias", torch.float32, (E,))
    p = _moe_params(T, H, I, E, k, out_mode, act, alpha, limit, score, norm, scale)
    out = _moe_out(out, out_mode, T, H, x.device)
    idx = torch.empty((T, k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, k), dtype=torch.float32, device=x.device)
    n = hwk.load().hwk_moe_workspace_bytes(p)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=x.device) if workspace is None else workspace
    hwk.load().hwk_moe_layer(_stream(), x.data_ptr(), logits.data_ptr(), _ptr(router_bias), idx.data_ptr(),
                             w.data_ptr(), gu_w.data_ptr(), gu_e.data_ptr(), _ptr(gu_b), dn_w.data_ptr(),
                             dn_e.data_ptr(), _ptr(dn_b), out.data_ptr(), ws.data_ptr(), ws.numel(), p)
    return out, idx, w


# ---------------- the decoder's small ops (K6) ----------------

def f64_bits(v: float) -> int:
    """A float64 scalar as the uint64 bit pattern the ABI takes."""
    return struct.unpack("<Q", struct.pack("<d", float(v)))[0]


def _f_out(shape, mode, device):
    if mode not in ("f32", "f16"):
        raise ValueError(f"out_mode {mode!r}: 'f32' or 'f16'")
    return torch.empty(shape, dtype=torch.float16 if mode == "f16" else torch.float32, device=device)


def rope_tables(theta: float, start: int, n: int, head_dim: int = 128):
    """Host RoPE tables (n, head_dim/2) float32 of positions start .. start+n-1, on the GPU."""
    import numpy as np

    c = np.empty((n, head_dim // 2), np.float32)
    s = np.empty((n, head_dim // 2), np.float32)
    hwk.load().hwk_rope_tables(f64_bits(theta), start, n, head_dim, c.ctypes.data, s.ctypes.data)
    return torch.from_numpy(c).cuda(), torch.from_numpy(s).cuda()


def rmsnorm(x, w, eps: float, out_mode="f16"):
    """RMSNorm of the rows of x (rows, n) fp32 with weights w (n) fp32."""
    rows, n = x.shape
    _need(x, "x", torch.float32, (rows, n))
    _need(w, "w", torch.float32, (n,))
    out = _f_out((rows, n), out_mode, x.device)
    hwk.load().hwk_rmsnorm(_stream(), x.data_ptr(), w.data_ptr(), out.data_ptr(), rows, n, f64_bits(eps),
                           OUT_MODES[out_mode])
    return out


def rope(x, cos_t, sin_t, pos0: int, norm_w=None, eps: float = 1e-6, out_mode="f16"):
    """Per-head RMSNorm (when norm_w is given) then RoPE of x (T, heads, 128) fp32 at positions pos0+t."""
    T, heads, d = x.shape
    _need(x, "x", torch.float32, (T, heads, d))
    _need(cos_t, "cos_t", torch.float32)
    _need(sin_t, "sin_t", torch.float32, tuple(cos_t.shape))
    if norm_w is not None:
        _need(norm_w, "norm_w", torch.float32, (d,))
    out = _f_out((T, heads, d), out_mode, x.device)
    hwk.load().hwk_rope(_stream(), x.data_ptr(), 0 if norm_w is None else norm_w.data_ptr(), cos_t.data_ptr(),
                        sin_t.data_ptr(), out.data_ptr(), T, heads, d, pos0, cos_t.shape[0], f64_bits(eps),
                        OUT_MODES[out_mode])
    return out


def kv_append(k, v, k_cache, v_cache, pos0: int):
    """Write k, v (T, kv_heads, d) fp16 into rows pos0.. of the caches (kv_heads, capacity, d)."""
    T, kvh, d = k.shape
    cap = k_cache.shape[1]
    _need(k, "k", torch.float16, (T, kvh, d))
    _need(v, "v", torch.float16, (T, kvh, d))
    _need(k_cache, "k_cache", torch.float16, (kvh, cap, d))
    _need(v_cache, "v_cache", torch.float16, (kvh, cap, d))
    hwk.load().hwk_kv_append(_stream(), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), T, kvh, d,
                             cap, pos0)


def silu_mul(gate, up, out_mode="f16", stride: int = 1, n=None):
    """silu(gate) * up elementwise over n values taken every `stride` floats of gate and up."""
    if n is None:
        n = gate.numel() // stride
    if gate.dtype != torch.float32 or up.dtype != torch.float32 or not gate.is_cuda or not up.is_cuda:
        raise TypeError("gate, up: fp32 tensors on the GPU")
    for t, name in ((gate, "gate"), (up, "up")):
        end = t.storage_offset() + (n - 1) * stride + 1
        if n and end > t.untyped_storage().nbytes() // 4:
            raise ValueError(f"{name}: {n} values at stride {stride} run past the tensor's storage")
    out = _f_out((n,), out_mode, gate.device)
    hwk.load().hwk_silu_mul(_stream(), gate.data_ptr(), up.data_ptr(), out.data_ptr(), n, stride, OUT_MODES[out_mode])
    return out


def add_(y, x):
    """y += x in fp32."""
    _need(y, "y", torch.float32)
    _need(x, "x", torch.float32, tuple(y.shape))
    hwk.load().hwk_add(_stream(), y.data_ptr(), x.data_ptr(), y.numel())
    return y


def embed(table, ids):
    """Rows ids (T) int32 of the fp16 table (vocab, hidden), as fp32 (T, hidden)."""
    vocab, hidden = table.shape
    _need(table, "table", torch.float16, (vocab, hidden))
    _need(ids, "ids", torch.int32)
    out = torch.empty((ids.numel(), hidden), dtype=torch.float32, device=table.device)
    hwk.load().hwk_embed(_stream(), table.data_ptr(), ids.data_ptr(), out.data_ptr(), ids.numel(), hidden, vocab)
    return out


def argmax(x):
    """The greedy pick of each row of x (rows, n) fp32, int32 (rows)."""
    if x.dim() == 1:
        x = x.view(1, -1)
    rows, n = x.shape
    _need(x, "x", torch.float32, (rows, n))
    out = torch.empty(rows, dtype=torch.int32, device=x.device)
    ws = torch.empty(max(16, hwk.load().hwk_argmax_workspace_bytes(rows)), dtype=torch.uint8, device=x.device)
    hwk.load().hwk_argmax(_stream(), x.data_ptr(), out.data_ptr(), rows, n, ws.data_ptr(), ws.numel())
    return out
